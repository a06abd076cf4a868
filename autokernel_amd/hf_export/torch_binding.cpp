// torch_binding.cpp -- registers libak355's entry points as torch ops (the HuggingFace Kernels
// ROCm package written by autokernel_amd/export_hf.py). Each op checks devices, dtypes and the
// layout its C entry point assumes, makes the input's device current, launches on torch's current
// HIP stream and turns a non-OK ak_status into a RuntimeError. Shape handling of the reference's
// kernel_fn (row flattening, dim moves, allocation) is done by the package's _host.py.
#include "torch_binding.h"

#include <algorithm>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "../include/ak355.h"
#include "registration.h"

namespace {

int dtype_code(const at::Tensor& t, const char* op) {
  switch (t.scalar_type()) {
    case at::kFloat: return AK_F32;
    case at::kHalf: return AK_F16;
    case at::kBFloat16: return AK_BF16;
    default: break;
  }
  TORCH_CHECK(false, op, ": dtype ", t.scalar_type(), " unsupported (float32, float16, bfloat16)");
  return -1;
}

// t lives on ref's GPU (and has ref's dtype unless same_dtype is false)
void on_gpu(const at::Tensor& t, const at::Tensor& ref, const char* op, const char* name,
            bool same_dtype = true) {
  TORCH_CHECK(t.is_cuda(), op, ": ", name, " must be a GPU tensor (libak355 has no CPU path)");
  TORCH_CHECK(t.device() == ref.device(), op, ": ", name, " is on ", t.device(), ", expected ", ref.device());
  if (same_dtype)
    TORCH_CHECK(t.scalar_type() == ref.scalar_type(), op, ": ", name, " dtype ", t.scalar_type(),
                " differs from ", ref.scalar_type());
}

void dense(const at::Tensor& t, const char* op, const char* name) {
  TORCH_CHECK(t.is_contiguous(), op, ": ", name, " must be contiguous");
}

void rows2d(const at::Tensor& t, const char* op, const char* name) {
  TORCH_CHECK(t.dim() == 2, op, ": ", name, " must be 2-D [rows, cols], got ", t.dim(), "-D");
  dense(t, op, name);
}

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_status(int st, const char* fn) {
  if (st == AK_OK) return;
  if (st == AK_EHIP) TORCH_CHECK(false, fn, " failed: ", ak_status_string(st), ": ", ak_last_hip_error_string());
  TORCH_CHECK(false, fn, " failed: ", ak_status_string(st));
}

}  // namespace

void ak_op_rmsnorm(at::Tensor& y, const at::Tensor& x, const at::Tensor& weight, double eps) {
  const char* op = "rmsnorm";
  on_gpu(x, x, op, "x");
  on_gpu(weight, x, op, "weight");
  on_gpu(y, x, op, "y");
  rows2d(x, op, "x");
  dense(weight, op, "weight");
  dense(y, op, "y");
  TORCH_CHECK(y.sizes() == x.sizes(), op, ": y shape ", y.sizes(), " != x shape ", x.sizes());
  TORCH_CHECK(weight.numel() == x.size(1), op, ": weight has ", weight.numel(), " elements, rows have ", x.size(1));
  const c10::DeviceGuard g(x.device());
  check_status(ak_rmsnorm(dtype_code(x, op), x.data_ptr(), weight.data_ptr(), y.data_ptr(), x.size(0),
                          x.size(1), (float)eps, stream_of(x)),
               "ak_rmsnorm");
}

void ak_op_layernorm(at::Tensor& y, const at::Tensor& x, const std::optional<at::Tensor>& weight,
                     const std::optional<at::Tensor>& bias, double eps) {
  const char* op = "layernorm";
  on_gpu(x, x, op, "x");
  on_gpu(y, x, op, "y");
  rows2d(x, op, "x");
  dense(y, op, "y");
  TORCH_CHECK(y.sizes() == x.sizes(), op, ": y shape ", y.sizes(), " != x shape ", x.sizes());
  const void* wp = nullptr;
  const void* bp = nullptr;
  if (weight.has_value()) {
    on_gpu(*weight, x, op, "weight");
    dense(*weight, op, "weight");
    TORCH_CHECK(weight->numel() == x.size(1), op, ": weight has ", weight->numel(), " elements, rows have ", x.size(1));
    wp = weight->data_ptr();
  }
  if (bias.has_value()) {
    on_gpu(*bias, x, op, "bias");
    dense(*bias, op, "bias");
    TORCH_CHECK(bias->numel() == x.size(1), op, ": bias has ", bias->numel(), " elements, rows have ", x.size(1));
    bp = bias->data_ptr();
  }
  const c10::DeviceGuard g(x.device());
  check_status(ak_layernorm(dtype_code(x, op), x.data_ptr(), wp, bp, y.data_ptr(), x.size(0), x.size(1),
                            (float)eps, stream_of(x)),
               "ak_layernorm");
}

void ak_op_softmax(at::Tensor& y, const at::Tensor& x) {
  const char* op = "softmax";
  on_gpu(x, x, op, "x");
  on_gpu(y, x, op, "y");
  rows2d(x, op, "x");
  dense(y, op, "y");
  TORCH_CHECK(y.sizes() == x.sizes(), op, ": y shape ", y.sizes(), " != x shape ", x.sizes());
  const c10::DeviceGuard g(x.device());
  check_status(ak_softmax(dtype_code(x, op), x.data_ptr(), y.data_ptr(), x.size(0), x.size(1), stream_of(x)),
               "ak_softmax");
}

void ak_op_rope(at::Tensor& y, const at::Tensor& x, const at::Tensor& cos, const at::Tensor& sin,
                int64_t rep_inner) {
  const char* op = "rotary_embedding";
  on_gpu(x, x, op, "x");
  on_gpu(cos, x, op, "cos");
  on_gpu(sin, x, op, "sin");
  on_gpu(y, x, op, "y");
  rows2d(x, op, "x");
  rows2d(cos, op, "cos");
  rows2d(sin, op, "sin");
  dense(y, op, "y");
  TORCH_CHECK(y.sizes() == x.sizes(), op, ": y shape ", y.sizes(), " != x shape ", x.sizes());
  TORCH_CHECK(x.size(1) % 2 == 0, op, ": head_dim ", x.size(1), " is odd");
  TORCH_CHECK(cos.sizes() == sin.sizes() && cos.size(1) == x.size(1) / 2, op, ": tables ", cos.sizes(),
              " / ", sin.sizes(), " do not fit head_dim ", x.size(1));
  TORCH_CHECK(rep_inner >= 1, op, ": rep_inner must be >= 1");
  const c10::DeviceGuard g(x.device());
  check_status(ak_rope(dtype_code(x, op), x.data_ptr(), cos.data_ptr(), sin.data_ptr(), y.data_ptr(),
                       x.size(0), x.size(1), cos.size(0), rep_inner, stream_of(x)),
               "ak_rope");
}

void ak_op_cross_entropy(at::Tensor& out, at::Tensor& row_loss, const at::Tensor& logits,
                         const at::Tensor& targets, int64_t ignore_index) {
  const char* op = "cross_entropy";
  on_gpu(logits, logits, op, "logits");
  on_gpu(out, logits, op, "out");
  on_gpu(targets, logits, op, "targets", false);
  on_gpu(row_loss, logits, op, "row_loss", false);
  rows2d(logits, op, "logits");
  dense(targets, op, "targets");
  dense(row_loss, op, "row_loss");
  TORCH_CHECK(targets.scalar_type() == at::kLong, op, ": targets must be int64");
  TORCH_CHECK(row_loss.scalar_type() == at::kFloat, op, ": row_loss must be float32");
  TORCH_CHECK(out.numel() == 1, op, ": out must hold one element");
  const int64_t rows = logits.size(0);
  TORCH_CHECK(targets.numel() == rows, op, ": ", rows, " rows of logits but ", targets.numel(), " targets");
  TORCH_CHECK(row_loss.numel() >= std::max<int64_t>(rows, 1), op, ": row_loss needs ", std::max<int64_t>(rows, 1),
              " elements");
  const c10::DeviceGuard g(logits.device());
  check_status(ak_cross_entropy(dtype_code(logits, op), logits.data_ptr(), targets.data_ptr<int64_t>(),
                                row_loss.data_ptr<float>(), out.data_ptr(), rows, logits.size(1), ignore_index,
                                stream_of(logits)),
               "ak_cross_entropy");
}

static void reduce_common(at::Tensor& y, const at::Tensor& x, int64_t outer, int64_t reduce, int64_t inner,
                          bool is_max) {
  const char* op = is_max ? "reduce_max" : "reduce_sum";
  on_gpu(x, x, op, "x");
  on_gpu(y, x, op, "y");
  dense(x, op, "x");
  dense(y, op, "y");
  TORCH_CHECK(outer >= 0 && reduce >= 0 && inner >= 0, op, ": negative extent");
  TORCH_CHECK(x.numel() == outer * reduce * inner, op, ": x has ", x.numel(), " elements, expected ",
              outer, " x ", reduce, " x ", inner);
  TORCH_CHECK(y.numel() == outer * inner, op, ": y has ", y.numel(), " elements, expected ", outer * inner);
  const c10::DeviceGuard g(x.device());
  const int code = dtype_code(x, op);
  if (is_max)
    check_status(ak_reduce_max(code, x.data_ptr(), y.data_ptr(), outer, reduce, inner, stream_of(x)), "ak_reduce_max");
  else
    check_status(ak_reduce_sum(code, x.data_ptr(), y.data_ptr(), outer, reduce, inner, stream_of(x)), "ak_reduce_sum");
}

void ak_op_reduce_sum(at::Tensor& y, const at::Tensor& x, int64_t outer, int64_t reduce, int64_t inner) {
  reduce_common(y, x, outer, reduce, inner, false);
}

void ak_op_reduce_max(at::Tensor& y, const at::Tensor& x, int64_t outer, int64_t reduce, int64_t inner) {
  reduce_common(y, x, outer, reduce, inner, true);
}

// c [M, N] = a [M, K] @ op(b): b is stored [K, N] (b_trans false) or [N, K] (b_trans true, an
// nn.Linear weight). Every operand needs a unit stride along its last dim; row strides are passed.
void ak_op_gemm(at::Tensor& c, const at::Tensor& a, const at::Tensor& b, bool b_trans,
                const std::optional<at::Tensor>& workspace) {
  const char* op = "matmul";
  on_gpu(a, a, op, "a");
  on_gpu(b, a, op, "b");
  on_gpu(c, a, op, "c");
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2 && c.dim() == 2, op, ": a, b, c must be 2-D");
  const int64_t M = a.size(0), K = a.size(1);
  const int64_t N = b_trans ? b.size(0) : b.size(1);
  TORCH_CHECK((b_trans ? b.size(1) : b.size(0)) == K, op, ": shapes ", a.sizes(), " and ", b.sizes(),
              (b_trans ? " (transposed)" : ""), " do not align");
  TORCH_CHECK(c.size(0) == M && c.size(1) == N, op, ": c shape ", c.sizes(), " != [", M, ", ", N, "]");
  const at::Tensor* operands[] = {&a, &b, &c};
  for (const at::Tensor* t : operands)
    TORCH_CHECK(t->size(1) <= 1 || t->stride(1) == 1, op, ": operands need a unit stride along their last dim");
  auto ld = [](const at::Tensor& t) { return t.size(0) > 1 ? t.stride(0) : std::max<int64_t>(t.size(1), 1); };
  const c10::DeviceGuard g(a.device());
  const int code = dtype_code(a, op);
  // a workspace (fp32, sized by gemm_workspace_bytes) lets under-filled grids split K
  if (workspace.has_value() && workspace->numel() > 0) {
    on_gpu(*workspace, a, op, "workspace", false);
    dense(*workspace, op, "workspace");
    TORCH_CHECK(workspace->scalar_type() == at::kFloat, op, ": workspace must be float32");
    check_status(ak_gemm_ws(code, a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, ld(a), ld(b), ld(c),
                            b_trans ? 1 : 0, workspace->data_ptr(), workspace->numel() * 4, stream_of(a)),
                 "ak_gemm_ws");
    return;
  }
  check_status(ak_gemm(code, a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, ld(a), ld(b), ld(c),
                       b_trans ? 1 : 0, stream_of(a)),
               "ak_gemm");
}

// c [Z, M, N] = a [Z, M, K] @ op(b) per batch item (torch.matmul's batched product): b is stored
// [Z, K, N] (b_trans false) or [Z, N, K] (true). Unit stride along each last dim; row and batch
// strides are passed (a batch stride of 0 shares an operand across the batch).
void ak_op_gemm_batched(at::Tensor& c, const at::Tensor& a, const at::Tensor& b, bool b_trans) {
  const char* op = "matmul";
  on_gpu(a, a, op, "a");
  on_gpu(b, a, op, "b");
  on_gpu(c, a, op, "c");
  TORCH_CHECK(a.dim() == 3 && b.dim() == 3 && c.dim() == 3, op, ": batched a, b, c must be 3-D");
  const int64_t Z = a.size(0), M = a.size(1), K = a.size(2);
  const int64_t N = b_trans ? b.size(1) : b.size(2);
  TORCH_CHECK(b.size(0) == Z && (b_trans ? b.size(2) : b.size(1)) == K, op, ": shapes ", a.sizes(), " and ",
              b.sizes(), (b_trans ? " (transposed)" : ""), " do not align");
  TORCH_CHECK(c.size(0) == Z && c.size(1) == M && c.size(2) == N, op, ": c shape ", c.sizes(), " != [", Z, ", ",
              M, ", ", N, "]");
  const at::Tensor* operands[] = {&a, &b, &c};
  for (const at::Tensor* t : operands)
    TORCH_CHECK(t->size(2) <= 1 || t->stride(2) == 1, op, ": operands need a unit stride along their last dim");
  auto ld = [](const at::Tensor& t) { return t.size(1) > 1 ? t.stride(1) : std::max<int64_t>(t.size(2), 1); };
  const c10::DeviceGuard g(a.device());
  check_status(ak_gemm_batched(dtype_code(a, op), a.data_ptr(), b.data_ptr(), c.data_ptr(), Z, M, N, K, ld(a),
                               ld(b), ld(c), a.stride(0), b.stride(0), c.stride(0), b_trans ? 1 : 0, stream_of(a)),
               "ak_gemm_batched");
}

int64_t ak_op_gemm_workspace_bytes(int64_t dtype, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                   int64_t ldc, bool b_trans) {
  return ak_gemm_workspace_bytes((int)dtype, M, N, K, lda, ldb, ldc, b_trans ? 1 : 0);
}

void ak_op_mlp_gate_up(at::Tensor& h, const at::Tensor& x, const at::Tensor& w_gate,
                       const at::Tensor& w_up, int64_t activation) {
  const char* op = "fused_mlp";
  on_gpu(x, x, op, "x");
  on_gpu(w_gate, x, op, "w_gate");
  on_gpu(w_up, x, op, "w_up");
  on_gpu(h, x, op, "h");
  rows2d(x, op, "x");
  rows2d(w_gate, op, "w_gate");
  rows2d(w_up, op, "w_up");
  rows2d(h, op, "h");
  const int64_t M = x.size(0), D = x.size(1), H = w_gate.size(0);
  TORCH_CHECK(w_gate.size(1) == D && w_up.sizes() == w_gate.sizes(), op, ": weights ", w_gate.sizes(), " / ",
              w_up.sizes(), " do not fit x ", x.sizes());
  TORCH_CHECK(h.size(0) == M && h.size(1) == H, op, ": h shape ", h.sizes(), " != [", M, ", ", H, "]");
  const c10::DeviceGuard g(x.device());
  check_status(ak_mlp_gate_up(dtype_code(x, op), x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), h.data_ptr(),
                              M, H, D, (int)activation, stream_of(x)),
               "ak_mlp_gate_up");
}

void ak_op_flash_attn_fwd(at::Tensor& o, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                          bool causal, double sm_scale) {
  const char* op = "flash_attention";
  on_gpu(q, q, op, "Q");
  on_gpu(k, q, op, "K");
  on_gpu(v, q, op, "V");
  on_gpu(o, q, op, "O");
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4 && o.dim() == 4, op, ": Q, K, V, O must be 4-D [B, H, S, D]");
  TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(3) == q.size(3), op, ": shapes Q",
              q.sizes(), " K", k.sizes(), " V", v.sizes());
  TORCH_CHECK(o.sizes() == q.sizes(), op, ": O shape ", o.sizes(), " != Q shape ", q.sizes());
  const at::Tensor* operands[] = {&q, &k, &v, &o};
  for (const at::Tensor* t : operands)
    TORCH_CHECK(t->stride(3) == 1, op, ": head_dim must be contiguous");
  const int64_t qs[3] = {q.stride(0), q.stride(1), q.stride(2)};
  const int64_t ks[3] = {k.stride(0), k.stride(1), k.stride(2)};
  const int64_t vs[3] = {v.stride(0), v.stride(1), v.stride(2)};
  const int64_t os[3] = {o.stride(0), o.stride(1), o.stride(2)};
  const c10::DeviceGuard g(q.device());
  check_status(ak_flash_attn_fwd(dtype_code(q, op), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                 q.size(0), q.size(1), k.size(1), q.size(2), k.size(2), q.size(3), qs, ks, vs, os,
                                 causal ? 1 : 0, (float)sm_scale, stream_of(q)),
               "ak_flash_attn_fwd");
}

TORCH_LIBRARY_EXPAND(TORCH_EXTENSION_NAME, ops) {
  ops.def("rmsnorm(Tensor! y, Tensor x, Tensor weight, float eps) -> ()");
  ops.impl("rmsnorm", c10::kCUDA, &ak_op_rmsnorm);
  ops.def("layernorm(Tensor! y, Tensor x, Tensor? weight, Tensor? bias, float eps) -> ()");
  ops.impl("layernorm", c10::kCUDA, &ak_op_layernorm);
  ops.def("softmax(Tensor! y, Tensor x) -> ()");
  ops.impl("softmax", c10::kCUDA, &ak_op_softmax);
  ops.def("rope(Tensor! y, Tensor x, Tensor cos, Tensor sin, int rep_inner) -> ()");
  ops.impl("rope", c10::kCUDA, &ak_op_rope);
  ops.def("cross_entropy(Tensor! out, Tensor! row_loss, Tensor logits, Tensor targets, int ignore_index) -> ()");
  ops.impl("cross_entropy", c10::kCUDA, &ak_op_cross_entropy);
  ops.def("reduce_sum(Tensor! y, Tensor x, int outer, int reduce, int inner) -> ()");
  ops.impl("reduce_sum", c10::kCUDA, &ak_op_reduce_sum);
  ops.def("reduce_max(Tensor! y, Tensor x, int outer, int reduce, int inner) -> ()");
  ops.impl("reduce_max", c10::kCUDA, &ak_op_reduce_max);
  ops.def("gemm(Tensor! c, Tensor a, Tensor b, bool b_trans, Tensor(w!)? workspace) -> ()");
  ops.impl("gemm", c10::kCUDA, &ak_op_gemm);
  ops.def("gemm_batched(Tensor! c, Tensor a, Tensor b, bool b_trans) -> ()");
  ops.impl("gemm_batched", c10::kCUDA, &ak_op_gemm_batched);
  ops.def("gemm_workspace_bytes(int dtype, int M, int N, int K, int lda, int ldb, int ldc, bool b_trans) -> int");
  ops.impl("gemm_workspace_bytes", &ak_op_gemm_workspace_bytes);
  ops.def("mlp_gate_up(Tensor! h, Tensor x, Tensor w_gate, Tensor w_up, int activation) -> ()");
  ops.impl("mlp_gate_up", c10::kCUDA, &ak_op_mlp_gate_up);
  ops.def("flash_attn_fwd(Tensor! o, Tensor q, Tensor k, Tensor v, bool causal, float sm_scale) -> ()");
  ops.impl("flash_attn_fwd", c10::kCUDA, &ak_op_flash_attn_fwd);
}

REGISTER_EXTENSION(TORCH_EXTENSION_NAME)
