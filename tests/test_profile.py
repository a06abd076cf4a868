"""The ROCm-aware profiler (autokernel_amd/profile.py): kernel classification, rocprofv3 CSV
ingestion and the profile_report.json layout on the CPU; a live profile of a small LLaMA on the GPU."""
from __future__ import annotations

import csv
import json

import pytest

from autokernel_amd import profile as P
from autokernel_amd.harness import GPUSpec

# (kernel name as ROCm tools print it, expected op type)
NAMES = [
    # hipBLASLt / Tensile GEMMs carry none of the reference's vendor fragments
    ("Cijk_Ailk_Bljk_BBS_BH_Bias_HA_S_SAV_UserArgs_MT256x256x64_MI16x16x1_SN_LDSB1_AFC1", "matmul"),
    ("Cijk_Alik_Bljk_HHS_BH_MT128x128x32_MI32x32x8x1_SN_1LDSB0_APM1", "matmul"),
    ("rocblas_gemm_ex_kernel", "matmul"),
    # aotriton / CK attention
    ("attn_fwd", "flash_attention"),
    ("ck_tile::FmhaFwdKernel<...>", "flash_attention"),
    # libak355
    ("void ak::fa_fwd2<ak::TF16, 128, 1>(unsigned short const*, unsigned short const*)", "flash_attention"),
    ("void ak::fa_fwd2<ak::TBF16, 64, 2>(unsigned short const*, unsigned short const*)", "flash_attention"),
    ("void ak::gemm_dma<ak::TBF16, 256, 128, 2, 4, 2, 1, 64, 2, false>(unsigned short const*)", "fused_mlp"),
    ("void ak::gemm_dma<ak::TBF16, 256, 256, 2, 4, 1, 0, 64, 2, true>(unsigned short const*)", "matmul"),
    ("void ak::gemm_mfma<ak::TF16, true, true, 256, 128, 2, 4, 2, 1>(unsigned short const*)", "fused_mlp"),
    ("void ak::gemm_f32<true>(float const*, float const*, float*, int, int, int)", "matmul"),
    ("void ak::ce_rows<ak::TF16, 1024, 4>(ak::TF16::S const*, long const*, float*)", "cross_entropy"),
    ("void ak::ce_mean<ak::TF16>(float const*, long const*, ak::TF16::S*, long, long)", "cross_entropy"),
    ("void ak::rope_f32t_vec<ak::TF16>(ak::TF16::S const*, float const*)", "rotary_embedding"),
    ("void ak::rmsnorm_rows<ak::TF16, 128, 4, 1>(ak::TF16::S const*)", "rmsnorm"),
    ("void ak::layernorm_rows<ak::TF16, 64, 4>(ak::TF16::S const*)", "layernorm"),
    ("void ak::softmax_rows<ak::TF16, 256, 4>(ak::TF16::S const*, ak::TF16::S*, long, int)", "softmax"),
    ("void ak::reduce_rows<ak::TF16, 512, 2, false>(ak::TF16::S const*)", "reduce"),
    # PyTorch-ROCm native kernels
    ("void at::native::(anonymous namespace)::cunn_SoftMaxForward<8, c10::Half, float, float>", "softmax"),
    ("void at::native::(anonymous namespace)::vectorized_layer_norm_kernel<c10::Half, float>", "layernorm"),
    ("void at::native::(anonymous namespace)::RowwiseMomentsCUDAKernel<float, float>", "layernorm"),
    ("void at::native::vectorized_elementwise_kernel<4, at::native::CUDAFunctor_add<c10::Half>>", "other"),
    # the reference's own rules still hold (profile.py:44-55, :459-463)
    ("sm90_xmma_gemm_f16f16_f16f32_f32_tn_n_tilesize128x128x64", "matmul"),
    ("flash_fwd_kernel<Flash_fwd_kernel_traits<128, 64, 64, 4>>", "flash_attention"),
    ("void rms_norm_kernel<c10::Half>", "rmsnorm"),
    ("silu_and_mul_kernel", "fused_mlp"),
    ("aten::mm", "matmul"),
    ("command_queue_drain", "other"),
]


@pytest.mark.parametrize("name,op", NAMES)
def test_classify_rocm_and_reference_names(name, op):
    assert P.classify_kernel(name) == op


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_kernel_trace_csv_aggregates_launches(tmp_path):
    trace = tmp_path / "trace_kernel_trace.csv"
    gemm = "Cijk_Ailk_Bljk_BBS_BH_MT256x256x64_MI16x16x1"
    _write(trace, ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp"], [
        ["KERNEL_DISPATCH", gemm, 1000, 101000],           # 100 us
        ["KERNEL_DISPATCH", "attn_fwd", 200000, 250000],    # 50 us
        ["KERNEL_DISPATCH", gemm, 300000, 400000],          # 100 us
        ["KERNEL_DISPATCH", "void ak::softmax_rows<ak::TF16, 256, 4>(x)", 500000, 525000],  # 25 us
    ])
    recs = P.read_rocprof_csv(str(trace))
    assert [(r.op_type, r.call_count, round(r.gpu_time_us)) for r in recs] == [
        ("matmul", 2, 200), ("flash_attention", 1, 50), ("softmax", 1, 25)]


def test_kernel_stats_csv(tmp_path):
    stats = tmp_path / "trace_kernel_stats.csv"
    _write(stats, ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"], [
        ["void ak::rope_vec<ak::TF16>(x)", 4, 40000, 10000, 20.0],
        ["Cijk_Alik_Bljk_HHS_BH_MT128x128x32", 2, 160000, 80000, 80.0],
    ])
    recs = P.read_rocprof_csv(str(stats))
    assert [(r.op_type, r.call_count, r.gpu_time_us) for r in recs] == [
        ("matmul", 2, 160.0), ("rotary_embedding", 4, 40.0)]


def test_unknown_csv_is_rejected(tmp_path):
    bad = tmp_path / "x.csv"
    _write(bad, ["a", "b"], [[1, 2]])
    with pytest.raises(ValueError):
        P.read_rocprof_csv(str(bad))


def test_report_layout_ranking_and_amdahl():
    recs = [P.KernelRecord("Cijk_gemm", "matmul", 500.0, 5),
            P.KernelRecord("elementwise_add", "other", 300.0, 30),
            P.KernelRecord("attn_fwd", "flash_attention", 200.0, 2)]
    gpu = GPUSpec(name="AMD Instinct MI355X", peak_tflops_fp16=2516.6, peak_bandwidth_gb_s=8000.0)
    rep = P.build_report(recs, {"model": "m", "class_name": None, "input_shape": [1, 8], "dtype": "float16"},
                         gpu, 10)
    json.dumps(rep)  # serialisable
    # the reference's profile_report.json keys (profile.py:717-742)
    for key in ("model", "class_name", "input_shape", "dtype", "gpu_name", "gpu_peak_tflops_fp16",
                "gpu_peak_bandwidth_gb_s", "total_gpu_time_ms", "total_kernels", "profile_iters",
                "top_kernels", "optimization_summary"):
        assert key in rep
    k0 = rep["top_kernels"][0]
    for key in ("rank", "name", "op_type", "shape_info", "gpu_time_ms", "call_count", "avg_time_us",
                "pct_total", "cumulative_pct", "roofline", "autokernel_supported", "optimization_priority"):
        assert key in k0
    assert [k["rank"] for k in rep["top_kernels"]] == [1, 2, 3]
    assert [k["pct_total"] for k in rep["top_kernels"]] == [50.0, 30.0, 20.0]
    assert rep["top_kernels"][-1]["cumulative_pct"] == 100.0
    assert [k["autokernel_supported"] for k in rep["top_kernels"]] == [True, False, True]
    assert rep["top_kernels"][0]["roofline"] == "compute-bound"
    assert rep["top_kernels"][1]["roofline"] == "likely compute-bound"  # other, > 100 us
    assert rep["top_kernels"][0]["optimization_priority"] == "HIGH"
    # f = 0.7 supported, 3x each: 1 / (0.3 + 0.7 / 3) = 1.875
    assert rep["optimization_summary"]["supported_kernels_pct"] == 70.0
    assert rep["optimization_summary"]["estimated_max_speedup"].startswith("1.9x")
    assert rep["total_gpu_time_ms"] == 1.0
    assert rep["op_type_summary"]["matmul"]["pct_total"] == 50.0


@pytest.mark.gpu
def test_live_profile_small_llama(gpu, tmp_path):
    out = tmp_path / "report.json"
    for kernels in ("none", "all"):
        assert P.main(["--model", "small", "--input-shape", "1,256", "--kernels", kernels,
                       "--output", str(out)]) == 0
        rep = json.loads(out.read_text())
        ops = rep["op_type_summary"]
        # device kernels only: the host op that launched a kernel is not counted a second time
        assert not [k["name"] for k in rep["top_kernels"] if k["name"].startswith(("aten::", "hipLaunch"))]
        assert ops.get("matmul", {}).get("gpu_time_ms", 0) > 0, ops
        if kernels == "all":
            names = [k["name"] for k in rep["top_kernels"]]
            ak = [n for n in names if "ak::" in n]
            assert ak, names[:10]
            assert all(P.classify_kernel(n) != "other" for n in ak)
            assert ops.get("flash_attention", {}).get("gpu_time_ms", 0) > 0
