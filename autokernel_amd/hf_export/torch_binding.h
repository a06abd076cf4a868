// torch_binding.h -- tensor-level torch ops over libak355's C ABI (include/ak355.h), for the
// HuggingFace Kernels ROCm package that autokernel_amd/export_hf.py writes.
//
// One op per C entry point. Outputs (and the cross-entropy workspace) are caller-allocated and
// passed first, as mutable arguments; the Python layer (_host.py) allocates them and does the
// reference kernel_fn's shape handling. Every op launches on torch's current HIP stream of the
// input's device and raises (TORCH_CHECK) on a bad argument or a failed launch.
#pragma once

#include <optional>

#include <ATen/core/Tensor.h>

void ak_op_rmsnorm(at::Tensor& y, const at::Tensor& x, const at::Tensor& weight, double eps);
void ak_op_layernorm(at::Tensor& y, const at::Tensor& x, const std::optional<at::Tensor>& weight,
                     const std::optional<at::Tensor>& bias, double eps);
void ak_op_softmax(at::Tensor& y, const at::Tensor& x);
void ak_op_rope(at::Tensor& y, const at::Tensor& x, const at::Tensor& cos, const at::Tensor& sin,
                int64_t rep_inner);
void ak_op_cross_entropy(at::Tensor& out, at::Tensor& row_loss, const at::Tensor& logits,
                         const at::Tensor& targets, int64_t ignore_index);
void ak_op_reduce_sum(at::Tensor& y, const at::Tensor& x, int64_t outer, int64_t reduce, int64_t inner);
void ak_op_reduce_max(at::Tensor& y, const at::Tensor& x, int64_t outer, int64_t reduce, int64_t inner);
void ak_op_gemm(at::Tensor& c, const at::Tensor& a, const at::Tensor& b, bool b_trans,
                const std::optional<at::Tensor>& workspace);
void ak_op_gemm_batched(at::Tensor& c, const at::Tensor& a, const at::Tensor& b, bool b_trans);
int64_t ak_op_gemm_workspace_bytes(int64_t dtype, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                   int64_t ldc, bool b_trans);
void ak_op_mlp_gate_up(at::Tensor& h, const at::Tensor& x, const at::Tensor& w_gate,
                       const at::Tensor& w_up, int64_t activation);
void ak_op_flash_attn_fwd(at::Tensor& o, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                          bool causal, double sm_scale);
