/*
 * ak355.h -- C ABI of libak355.so, the MI355X (gfx950) kernels behind AutoKernel's nine-op suite.
 *
 * Every entry point:
 *   - takes device pointers, element counts and scalars only (no framework types);
 *   - launches asynchronously on the caller's HIP stream `stream` (pass torch's current stream);
 *   - never allocates, frees or synchronises; every buffer (outputs, workspaces) is the caller's
 *     (ak_cross_entropy_noalloc alone keeps its workspace in a fixed device array, see there);
 *   - keeps no mutable global state, so concurrent calls on different streams are safe (the
 *     one per-thread setting, ak_set_launch_events, affects only its own thread's next launch;
 *     ak_cross_entropy_noalloc's calls on one device share its array);
 *   - returns AK_OK or an ak_status code; AK_EHIP means a HIP launch error
 *     (its text is available from ak_last_hip_error_string() on the calling thread).
 *
 * Tensors are dense and row-major unless a leading-dimension / stride argument says otherwise.
 * Element types are given by an ak_dtype code; f16 and bf16 are IEEE binary16 and bfloat16.
 *
 * The "replaces" notes name the reference interface each entry point stands in for
 * (paths relative to RightNow-AI/autokernel).
 */
#ifndef AK355_H
#define AK355_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum ak_dtype {
    AK_F32 = 0,
    AK_F16 = 1,
    AK_BF16 = 2
} ak_dtype;

typedef enum ak_status {
    AK_OK = 0,
    AK_EINVAL = 1,        /* bad argument: null pointer, negative size, bad dtype */
    AK_EUNSUPPORTED = 2,  /* valid request this build has no kernel for (e.g. head_dim 320) */
    AK_EHIP = 3           /* kernel launch failed; see ak_last_hip_error_string() */
} ak_status;

typedef enum ak_activation {
    AK_ACT_SILU = 0,   /* x * sigmoid(x)                 (reference.py:49-50) */
    AK_ACT_GELU = 1,   /* exact erf GELU, F.gelu default (reference.py:51-52) */
    AK_ACT_RELU2 = 2,  /* relu(x)^2                      (reference.py:53-54) */
    AK_ACT_NONE = 3    /* identity: gate passed through  (reference.py: unknown activation string) */
} ak_activation;

/* Library identity and diagnostics. */
const char* ak_version(void);
const char* ak_status_string(int status);
const char* ak_last_hip_error_string(void);

/*
 * Measurement hook: the calling thread's next timed launch (ak_softmax, ak_copy) records `start`
 * and `stop` (created HIP events, or NULL) as part of its kernel dispatch, at the kernel's start
 * and end, through hipExtLaunchKernel; the setting is then cleared. Event pairs recorded this way
 * time the kernel alone, without the gap a separate hipEventRecord leaves before the dispatch.
 * Per thread, so calls on other threads are unaffected. No counterpart in the reference: the
 * benchmark's per-launch roofline timing.
 */
int ak_set_launch_events(hipEvent_t start, hipEvent_t stop);

/*
 * RMSNorm over the last dim: y = (x / sqrt(mean(x*x) + eps)) * w, each step rounded to the
 * element type as the reference's tensor op sequence does.
 * x, y: [rows, cols]; w: [cols].
 * Replaces: reference.py:26-29 rmsnorm_ref; kernels/cuda/rmsnorm.py:132-158 rmsnorm_cuda;
 *           kernels/rmsnorm.py:45 kernel_fn(x, weight, eps).
 */
int ak_rmsnorm(int dtype, const void* x, const void* w, void* y,
               int64_t rows, int64_t cols, float eps, hipStream_t stream);

/*
 * RMSNorm in the form a LLaMA block's module computes it: y = x * rsqrt(mean(x*x) + eps) * w,
 * each step a tensor op rounded to the element type (the rsqrt factor included).
 * Replaces: models/llama_7b.py:28-30 RMSNorm.forward (the model plug-in's norm replacement).
 */
int ak_rmsnorm_rsqrt(int dtype, const void* x, const void* w, void* y,
                     int64_t rows, int64_t cols, float eps, hipStream_t stream);

/*
 * LayerNorm over the last dim with fp32 statistics: y = (x - mean) * rsqrt(var + eps) * w + b.
 * w or b may be NULL (treated as ones / zeros). x, y: [rows, cols]; w, b: [cols].
 * Replaces: reference.py:20-23 layernorm_ref; kernels/cuda/layernorm.py:268-307 layernorm_cuda.
 */
int ak_layernorm(int dtype, const void* x, const void* w, const void* b, void* y,
                 int64_t rows, int64_t cols, float eps, hipStream_t stream);

/*
 * Softmax over the last dim with fp32 internals, one output rounding. x, y: [rows, cols].
 * Replaces: reference.py:15-17 softmax_ref; kernels/cuda/softmax.py:187-232 softmax_cuda.
 */
int ak_softmax(int dtype, const void* x, void* y, int64_t rows, int64_t cols, hipStream_t stream);

/*
 * Interleaved rotary embedding. x, y: [rows, head_dim]; cos, sin: [table_rows, head_dim/2].
 * Row r of x uses table row (r / rep_inner) % table_rows, which covers the [.., S, D] layout
 * (rep_inner = 1) and the [B, S, H, D] layout (rep_inner = H).
 *   y[2i]   = x[2i]*cos[i] - x[2i+1]*sin[i]
 *   y[2i+1] = x[2i]*sin[i] + x[2i+1]*cos[i]   (every product and sum rounded to the element type)
 * Replaces: reference.py:63-69 rotary_embedding_ref; kernels/cuda/rotary_embedding.py:100-125.
 */
int ak_rope(int dtype, const void* x, const void* cos_t, const void* sin_t, void* y,
            int64_t rows, int64_t head_dim, int64_t table_rows, int64_t rep_inner,
            hipStream_t stream);

/*
 * Rotary embedding in the form a LLaMA block applies it: x (f16 / bf16) rotated by fp32 tables
 * with fp32 arithmetic and one rounding to x's dtype; cos_t, sin_t: fp32 [table_rows, head_dim/2].
 * x holds rows / rep_inner tokens of rep_inner heads; token t starts at element t * x_tok_stride
 * (rep_inner * head_dim when dense; larger for a column slice of a fused QKV projection) and
 * uses table row t % table_rows. y is dense [rows, head_dim]. head_dim and x_tok_stride multiples
 * of 8, x and y 16-byte aligned.
 * Replaces: models/llama_7b.py:40-48 apply_rotary_emb (complex multiply in fp32, type_as(x)).
 */
int ak_rope_f32_tables(int dtype, const void* x, const float* cos_t, const float* sin_t, void* y,
                       int64_t rows, int64_t head_dim, int64_t table_rows, int64_t rep_inner,
                       int64_t x_tok_stride, hipStream_t stream);

/*
 * Mean cross-entropy over rows: out = mean_r( logsumexp(x_r) - x_r[t_r] ), rows whose target is
 * ignore_index excluded from sum and count (F.cross_entropy semantics). A target outside
 * [0, vocab) that is not ignore_index makes the result NaN.
 * logits: [rows, vocab]; targets: int64 [rows]; row_loss: fp32 workspace [rows] (caller-owned);
 * out: one element of the logits' dtype.
 * Replaces: reference.py:58-60 cross_entropy_ref; kernels/cuda/cross_entropy.py:116-138.
 */
int ak_cross_entropy(int dtype, const void* logits, const int64_t* targets, float* row_loss,
                     void* out, int64_t rows, int64_t vocab, int64_t ignore_index,
                     hipStream_t stream);

/*
 * Cross-entropy that allocates nothing: the result of ak_cross_entropy (same arguments except the
 * row_loss workspace, same kernels, bit-identical output), with the per-row losses kept in a
 * fixed device array of AK_CE_NOALLOC_MAX_ROWS floats (4 MiB) that the library holds on each
 * device it runs on until the process ends. rows above AK_CE_NOALLOC_MAX_ROWS: AK_EINVAL.
 * Calls that overlap on one device (concurrent streams or threads) share that array and race:
 * serialise them. The device is the stream's (the current device for the null stream).
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 */
#define AK_CE_NOALLOC_MAX_ROWS (1 << 20)
int ak_cross_entropy_noalloc(int dtype, const void* logits, const int64_t* targets, void* out,
                             int64_t rows, int64_t vocab, int64_t ignore_index, hipStream_t stream);

/*
 * Sum / max over the middle dim of x viewed as [outer, reduce, inner]; y: [outer, inner].
 * Sum accumulates in fp32 with a fixed order (deterministic); max propagates NaN like torch.max.
 * Replaces: reference.py:72-78 reduce_sum_ref / reduce_max_ref; kernels/cuda/reduce.py:79-98;
 *           kernels/reduce.py:51-140 kernel_fn(x, dim).
 */
int ak_reduce_sum(int dtype, const void* x, void* y, int64_t outer, int64_t reduce,
                  int64_t inner, hipStream_t stream);
int ak_reduce_max(int dtype, const void* x, void* y, int64_t outer, int64_t reduce,
                  int64_t inner, hipStream_t stream);

/*
 * GEMM with fp32 accumulation and one output rounding: C[M,N] = A[M,K] * op(B).
 *   b_trans = 0: B is [K, N] with row stride ldb  (torch.matmul(A, B), reference.py:10-12)
 *   b_trans = 1: B is [N, K] with row stride ldb  (x @ W.T for an nn.Linear weight W)
 * lda / ldc are the row strides of A and C in elements.
 * Replaces: reference.py:10-12 matmul_ref; kernels/cuda/matmul.py:210-233 matmul_cuda;
 *           verify.py:429-430 (the Linear path, without its per-call weight transpose copy).
 */
int ak_gemm(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
            int64_t lda, int64_t ldb, int64_t ldc, int b_trans, hipStream_t stream);

/*
 * Batched GEMM: for z in [0, batch), C_z = A_z * op(B_z) as ak_gemm computes each product, where
 * X_z starts stride_x elements after X_{z-1}. A stride of 0 shares A or B across the batch (a
 * broadcast operand). C's items must not overlap. One launch for the whole batch (the batch is the
 * grid's third dimension), for fp32 as for f16 / bf16.
 * Replaces: reference.py:10-12 matmul_ref for operands with batch dimensions (torch.matmul's
 *           broadcast batched product), one launch instead of one per batch item.
 */
int ak_gemm_batched(int dtype, const void* A, const void* B, void* C, int64_t batch, int64_t M,
                    int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t stride_a,
                    int64_t stride_b, int64_t stride_c, int b_trans, hipStream_t stream);

/*
 * Split-K GEMM for grids that leave most compute units idle (few output tiles, long K), e.g.
 * 1024 x 1024 x 8192. Same arguments and result semantics as ak_gemm (fp32 accumulation, one output
 * rounding; deterministic), plus a caller-owned fp32 workspace.
 *   ak_gemm_workspace_bytes: bytes of workspace ak_gemm_ws uses for this problem; 0 when it would
 *     not split (fp32, grids that fill the GPU, K too short), and then needs none.
 *   ak_gemm_ws: splits K into slices that run side by side, each storing fp32 partial tiles to the
 *     workspace ([slices][M][N]), then adds the slices in a fixed order and rounds once. With too
 *     small a workspace (or NULL), or unaligned operands, it runs ak_gemm instead.
 * Replaces: reference.py:10-12 matmul_ref for the reference harness's under-filled shapes
 *           (bench.py:336-345: tiny .. medium, deep_k); no counterpart in the starters.
 */
int64_t ak_gemm_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                                int64_t ldc, int b_trans);
int ak_gemm_ws(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
               int64_t lda, int64_t ldb, int64_t ldc, int b_trans, void* workspace, int64_t workspace_bytes,
               hipStream_t stream);

/*
 * GEMM with the residual add of a transformer block in its epilogue: C = R + A * op(B), with
 * A, B, b_trans, lda, ldb as in ak_gemm. The product is rounded to the element type, R is added
 * and the sum rounded again, so C equals ak_gemm followed by a separate element-type add, bit for
 * bit. R [M, N] has C's row stride ldc and must not overlap C. f16 / bf16 (fp32: AK_EUNSUPPORTED).
 * Replaces: models/llama_7b.py:110-111 (x = x + attention(...), x = x + feed_forward(...)): the
 *           output projections' GEMM plus the add kernel that follows it.
 */
int ak_gemm_residual(int dtype, const void* A, const void* B, const void* R, void* C, int64_t M,
                     int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int b_trans,
                     hipStream_t stream);

/*
 * GEMM with nn.Linear's bias fused: C = A * op(B) + bias, the bias [N] (element type) added to the
 * fp32 accumulator and the sum rounded once, as torch's addmm does for a biased nn.Linear (one
 * rounding, not two). Arguments as in ak_gemm. f16 / bf16 (fp32: AK_EUNSUPPORTED).
 * Replaces: verify.py:429-434 (the Linear wrapper's kernel_fn(x, weight.t()) + bias) for the
 *           biased projections of models/gpt2.py:27-28, :60-62 and models/bert_base.py:23-26, :47-48.
 */
int ak_gemm_bias(int dtype, const void* A, const void* B, const void* bias, void* C, int64_t M,
                 int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int b_trans,
                 hipStream_t stream);

/*
 * ak_gemm_bias followed by exact GELU: C = gelu(A * op(B) + bias), the biased product rounded to
 * the element type as ak_gemm_bias rounds it, then x * 0.5 * (1 + erf(x / sqrt(2))) in fp32 and
 * rounded again: nn.Linear then nn.GELU (torch's addmm, then its GELU kernel in fp32), bit for bit.
 * Arguments as in ak_gemm_bias. f16 / bf16 (fp32: AK_EUNSUPPORTED).
 * Replaces: models/gpt2.py:60-62 and models/bert_base.py:47-48 (c_fc / dense1 followed by the MLP's
 *           GELU): the first MLP projection plus the GELU kernel that follows it.
 */
int ak_gemm_bias_gelu(int dtype, const void* A, const void* B, const void* bias, void* C, int64_t M,
                      int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int b_trans,
                      hipStream_t stream);

/*
 * ak_gemm_bias plus a residual: C = R + (A * op(B) + bias), the biased product rounded to the
 * element type, R added and the sum rounded again: torch's `x + linear(y)` for a biased Linear, bit
 * for bit. R [M, N] has C's row stride ldc and must not overlap C. f16 / bf16.
 * Replaces: models/gpt2.py:63-65 (x + attn(...), x + mlp(...)) and models/bert_base.py:60-62
 *           (x + attention(x), x + mlp(x) before each LayerNorm): the output projections' GEMM plus
 *           the add kernel that follows it.
 */
int ak_gemm_bias_residual(int dtype, const void* A, const void* B, const void* bias, const void* R,
                          void* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                          int64_t ldc, int b_trans, hipStream_t stream);

/*
 * GEMM with the model's rotary embedding in its epilogue: C = A * op(B) (arguments as in ak_gemm),
 * the product rounded to the element type; then, in columns [0, rot_cols), every head of head_dim
 * columns has its (even, odd) pairs rotated in fp32 by cos / sin [seq_len, head_dim / 2] (fp32,
 * contiguous; row m of C is token m % seq_len) and rounded once: y0 = x0 c - x1 s, y1 = x0 s + x1 c,
 * each product and sum rounded in fp32. Columns from rot_cols on (v of a fused QKV projection)
 * are plain products. Equals ak_gemm followed by ak_rope_f32_tables on those columns, bit for bit.
 * head_dim a multiple of 4, rot_cols a multiple of head_dim and at most N; cos / sin 8-byte
 * aligned. f16 / bf16.
 * Replaces: models/llama_7b.py:67-71 (the wq / wk / wv projections and apply_rotary_emb,
 *           models/llama_7b.py:40-48): the QKV GEMM plus the RoPE kernel that follows it.
 */
int ak_gemm_rope(int dtype, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                 int64_t lda, int64_t ldb, int64_t ldc, int b_trans, const float* cos_t,
                 const float* sin_t, int64_t seq_len, int64_t head_dim, int64_t rot_cols,
                 hipStream_t stream);

/*
 * Device copy of `bytes` bytes (a multiple of 16, 16-byte aligned src and dst), one 16-byte vector
 * per thread. No counterpart in the reference: the bandwidth reference the benchmark times beside
 * the HBM-bound ops (the practical ceiling at a given size). A timed launch (ak_set_launch_events).
 */
int ak_copy(const void* src, void* dst, int64_t bytes, hipStream_t stream);

/*
 * Fused gate/up projection of the SwiGLU MLP:
 *   h = round(act(round(x @ w_gate.T))) * round(x @ w_up.T), rounded to the element type.
 * x: [M, D]; w_gate, w_up: [H, D] (nn.Linear layout); h: [M, H].
 * The down projection is ak_gemm(h, w_down, b_trans = 1).
 * Replaces: reference.py:45-55 fused_mlp_ref (gate/up/activation/product);
 *           kernels/cuda/fused_mlp.py:115-157 fused_mlp_cuda.
 */
int ak_mlp_gate_up(int dtype, const void* x, const void* w_gate, const void* w_up, void* h,
                   int64_t M, int64_t H, int64_t D, int activation, hipStream_t stream);

/*
 * Flash-attention forward: O = softmax(Q K^T * sm_scale [+ causal mask]) V per (batch, head).
 * Q, O: [B, Hq, Sq, D]-indexed, K, V: [B, Hkv, Sk, D]-indexed, each given by element strides
 * (batch, head, seq); the last dim is contiguous. Hq must be a multiple of Hkv (grouped-query
 * attention: query head h reads KV head h / (Hq / Hkv)). causal masks key j > query i
 * (top-left aligned, as torch.triu(ones(Sq, Sk), 1) does). f16 / bf16 with D 64 or 128 and
 * 16-byte aligned rows run the MFMA kernels; fp32, any other D from 1 to 256 and unaligned rows run
 * a general kernel that keeps the reference's roundings (scores and their scaled value in the
 * element type, softmax output rounded, P V accumulated in fp32). D above 256: AK_EUNSUPPORTED.
 * Replaces: reference.py:32-42 flash_attention_ref; kernels/cuda/flash_attention.py:207-235;
 *           kernels/flash_attention.py:130 kernel_fn(Q, K, V, causal, sm_scale).
 */
int ak_flash_attn_fwd(int dtype, const void* Q, const void* K, const void* V, void* O,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                      const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides,
                      int causal, float sm_scale, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AK355_H */
