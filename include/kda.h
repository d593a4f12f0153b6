/*
 * kda.h -- C ABI of the MI355X (gfx950) operator library.
 *
 * One entry point per operator of the reference's NKIBench operator set.  Each
 * replaces the NKI `kernel(...)` that the reference's adapter assembles and its
 * profiler runs (adapter/nkibench_case.py:105-166, `kernel_fn="kernel"` :177);
 * the argument order follows the reference kernel's HBM-tensor order, which is
 * the order of the numpy `forward(...)` parameters (adapter/nkibench_case.py:199-216).
 *
 * Conventions (all entry points):
 *   - Every pointer is a device pointer the caller owns (allocated with hipMalloc
 *     or by PyTorch).  The library never allocates, frees or retains them.
 *   - Tensors are dense and row-major in the "natural" layout of the numpy
 *     reference (every NKIBench transform_to_nki_inputs is a pure reshape).
 *   - bf16 tensors are passed as `kda_bf16*` (raw 16-bit storage, IEEE bfloat16).
 *   - `stream` is a hipStream_t cast to void*; NULL means the default stream.
 *     Launches are asynchronous; no entry point synchronises the host.
 *   - Return value: KDA_OK (0) on success, otherwise a KDA_ERR_* code; the
 *     message for the last failure on the calling thread is kda_last_error().
 *     Nothing is launched when a call fails argument validation.
 */
#ifndef KDA_H_
#define KDA_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t kda_bf16;

enum {
  KDA_OK = 0,
  KDA_ERR_INVALID_ARG = 1,  /* null pointer, bad size, misaligned pointer       */
  KDA_ERR_UNSUPPORTED = 2,  /* shape outside what the kernel was written for    */
  KDA_ERR_HIP = 3           /* a HIP runtime call failed (launch, attribute...) */
};

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int kda_version(void);

/* Message describing the most recent failure on the calling thread ("" if none). */
const char* kda_last_error(void);

/* ---------------------------------------------------------------- elementwise */

/* SiLU, y = x / (1 + exp(-x)), fp32, n elements.
 * Replaces kernel(v1) of workspaces/silu/runs/silu_v3_s7.py:31-71
 * (forward `y = x/(1+exp(-x))`, prompts/_gen_prompts.py:25).  x and y may alias. */
int kda_silu_f32(const float* x, float* y, int64_t n, void* stream);

/* AdamW step (decoupled weight decay), fp32, n elements:
 *   p' = p*(1 - lr*wd);  m' = b1*m + (1-b1)*g;  v' = b2*v + (1-b2)*g*g
 *   p'' = p' - (lr/(1-b1^step)) * m' / (sqrt(v')/sqrt(1-b2^step) + eps)
 * Reads param_in/grad/m_in/v_in; writes param_out (may equal param_in for the
 * in-place step) and, when non-NULL, m_out / v_out (may equal m_in / v_in).
 * Replaces kernel(v1..v4) = (theta, g, m, v) of workspaces/adamw/runs/adamw_v1.py:50-97,
 * whose forward is this update at step 1, lr 1e-3, wd 1e-2, eps 1e-8
 * (workspaces/adamw/docs/draft-phase1.md:20-26) returning only the new theta. */
int kda_adamw_f32(const float* param_in, const float* grad, const float* m_in,
                  const float* v_in, float* param_out, float* m_out, float* v_out,
                  int64_t n, float lr, float beta1, float beta2, float eps,
                  float weight_decay, int64_t step, void* stream);

/* Half-split rotary embedding applied along axis 0 of x (D rows, S columns):
 *   out[d]       = x[d]*cos[d] - x[d+D/2]*sin[d]        d < D/2
 *   out[d + D/2] = x[d]*sin[d] + x[d+D/2]*cos[d]
 * x, out: (D, S) fp32; cos, sin: (D/2, S) fp32; D even.  Rounded exactly like the
 * numpy reference (two products, then one add/sub; no fused multiply-add).
 * Replaces kernel(x_in, cos, sin) of
 * workspaces/rope_single_freq_apply/runs/rope_v1.py:32-80. */
int kda_rope_f32(const float* x, const float* cos_t, const float* sin_t, float* out,
                 int64_t d, int64_t s, void* stream);

/* ---------------------------------------------------------------- workspaces
 * Entry points that stage intermediates (bf16 hi/lo planes of fp32 operands,
 * normalised activations, row statistics) take a caller-owned device buffer
 * `workspace` of at least kda_workspace_size(op, ...) bytes, 16-byte aligned.
 * The library never allocates. */
enum {
  KDA_OP_MATMUL_F32 = 1,
  KDA_OP_TRANSPOSE_MATMUL_F32 = 2,
  KDA_OP_BMM_F32 = 3,
  KDA_OP_LORA_F32 = 4,
  KDA_OP_RMSNORM_MATMUL_F32 = 5,
  KDA_OP_ADD_RMSNORM_MATMUL_F32 = 6,
  KDA_OP_MATMUL_ADD_RMSNORM_F32 = 7,
  KDA_OP_SWIGLU_F32 = 8,          /* n = F (intermediate width) */
  KDA_OP_RMSNORM_MATMUL_BF16 = 9,
  KDA_OP_BMM_SOFTMAX_F32 = 10,
  KDA_OP_GQA_F32 = 11,            /* batch = B, m = S, k = Hq, n = Hkv */
  KDA_OP_SWIGLU_BF16 = 12,        /* m = M, k = K: optional split-K partials */
  KDA_OP_ADD_RMSNORM_MATMUL_BF16 = 13,
  KDA_OP_MATMUL_ADD_RMSNORM_BF16 = 14
};

/* Workspace bytes for operator `op` at the given sizes (unused sizes: 0);
 * -1 for an unknown op, a negative size, or sizes whose workspace does not fit
 * in int64 (every product and sum is overflow-checked); entry points refuse such
 * sizes with KDA_ERR_UNSUPPORTED.  The sizes depend only on the arguments, not on
 * the device. */
int64_t kda_workspace_size(int op, int64_t batch, int64_t m, int64_t k, int64_t n, int64_t r);

/* ---------------------------------------------------------------- bf16 GEMMs
 * bf16 storage, fp32 accumulation on MFMA, bf16 output.  Shape limits: K and N
 * multiples of 8 (16-byte rows); all pointers 16-byte aligned; any M. */

/* c[M,N] = a[M,K] @ b[K,N].  The GEMM core of workspaces/matmul/runs/matmul_v1.py:10-111
 * (kernel(v1=lhs, v2=rhs)), at bf16 precision. */
int kda_matmul_bf16(const kda_bf16* a, const kda_bf16* b, kda_bf16* c, int64_t m, int64_t k,
                    int64_t n, void* stream);

/* y[M,N] = (x * rsqrt(mean_k(x^2) + eps) * gamma) @ w, x [M,K], gamma [K] (16-byte
 * aligned), w [K,N].  A streaming pre-pass reads x once and writes the per-row
 * 1/rms (fp32) and bf16(x * gamma) into `workspace`; the GEMM applies 1/rms to
 * its accumulators in the epilogue.  Workspace: KDA_OP_RMSNORM_MATMUL_BF16.
 * Replaces kernel(v1=x, v2=w) of workspaces/rmsnorm_matmul/runs/rmsnorm_matmul_v1.py:10-138
 * (which has no gain and no eps) and the x+z-free part of
 * workspaces/add_rmsnorm_matmul/runs/add_rmsnorm_matmul_v1.py:8-146 (gain g, eps). */
int kda_rmsnorm_matmul_bf16(const kda_bf16* x, const kda_bf16* gamma, const kda_bf16* w,
                            kda_bf16* y, int64_t m, int64_t k, int64_t n, float eps,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* The residual variant of kda_rmsnorm_matmul_bf16, in the argument order of
 * forward(x, w, eps, z, g) of workspaces/add_rmsnorm_matmul/runs/add_rmsnorm_matmul_v1.py:8-146
 * (fp32 there): y = x + z (summed in fp32, not rounded); out[M,N] =
 * (y / sqrt(sum_k(y^2 / K) + eps) * g) @ w with x, z [M,K], g [K], w [K,N].  The
 * pre-pass reads x and z once and writes 1/rms and bf16(y * g); the GEMM applies
 * 1/rms in its epilogue.  Workspace: KDA_OP_ADD_RMSNORM_MATMUL_BF16 (2*M*K + 4*M
 * bytes, as KDA_OP_RMSNORM_MATMUL_BF16). */
int kda_add_rmsnorm_matmul_bf16(const kda_bf16* x, const kda_bf16* w, float eps, const kda_bf16* z,
                                const kda_bf16* g, kda_bf16* out, int64_t m, int64_t k, int64_t n,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* y = x @ w + z; out[M,N] = y * g / sqrt(mean_n(y^2) + eps) with x [M,K], w [K,N],
 * z [M,N], g [N], all bf16; argument order of forward(x, w, eps, z, g) of
 * workspaces/matmul_add_rmsnorm/runs/matmul_add_rmsnorm_v2_bf16_split.py:8-212
 * (fp32 there).  The GEMM epilogue adds z to the fp32 accumulators, writes
 * bf16(y) into out and per-row partial sums of the fp32 y^2; a row kernel then
 * scales out in place (so y is rounded to bf16 once before the scaling).
 * Workspace: KDA_OP_MATMUL_ADD_RMSNORM_BF16 (4*M*ceil(N/32) bytes). */
int kda_matmul_add_rmsnorm_bf16(const kda_bf16* x, const kda_bf16* w, float eps, const kda_bf16* z,
                                const kda_bf16* g, kda_bf16* out, int64_t m, int64_t k, int64_t n,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of the per-device static buffer behind kda_rmsnorm_matmul_bf16_noalloc. */
#define KDA_NOALLOC_SCRATCH_BYTES (64LL << 20)

/* kda_rmsnorm_matmul_bf16 without a workspace argument and without any allocation:
 * no counterpart in the reference; for callers that cannot allocate (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * workspace is a file-scope device buffer of KDA_NOALLOC_SCRATCH_BYTES that every
 * device the library runs on holds until the process ends; its address is looked
 * up once per device (no allocation).  Sizes whose workspace (2*M*K + 4*M bytes)
 * exceeds it are rejected with KDA_ERR_UNSUPPORTED before any launch.  All calls
 * on one device share the buffer: calls that overlap on one device (different
 * streams, or host threads without ordering) race and must not be issued.
 * Results equal kda_rmsnorm_matmul_bf16's bit for bit. */
int kda_rmsnorm_matmul_bf16_noalloc(const kda_bf16* x, const kda_bf16* gamma, const kda_bf16* w,
                                    kda_bf16* y, int64_t m, int64_t k, int64_t n, float eps,
                                    void* stream);

/* y[M,K] = (silu(x @ w_gate) * (x @ w_up)) @ w_down with x [M,K], w_up/w_gate [K,F],
 * w_down [F,K].  h is caller-provided scratch of M*F bf16 (the gated activation,
 * written by the first kernel and read by the second).  `workspace` (optional:
 * NULL or too small disables it) of kda_workspace_size(KDA_OP_SWIGLU_BF16, 1, M,
 * K, F, 0) = 8*M*K bytes lets the down GEMM split F in two when its output tiles
 * fill at most half the device (fp32 partials, summed into y).  Argument order follows
 * kernel(v1=x, v2=w_up, v3=w_down, v4=w_gate) of workspaces/swiglu/runs/swiglu_v1.py:38-146. */
int kda_swiglu_bf16(const kda_bf16* x, const kda_bf16* w_up, const kda_bf16* w_down,
                    const kda_bf16* w_gate, kda_bf16* h, kda_bf16* y, int64_t m, int64_t k,
                    int64_t f, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- fp32 GEMMs
 * The reference's fp32 NKIBench operators.  fp32 in, fp32 out, computed on bf16
 * MFMA through a three-product split (x = hi + lo in bf16; A@B ~= Ah@Bh + Ah@Bl +
 * Al@Bh, fp32 accumulation; relative-L2 ~5e-6 on N(0,1) data), the same scheme
 * as workspaces/matmul/runs/matmul_v3_bf16_split.py:21-33.  K (and every
 * contraction extent) must be a multiple of 32, N a multiple of 8; pointers
 * 16-byte aligned.  All arrays dense row-major. */

/* out[M,N] = lhs[M,K] @ rhs[K,N].  Replaces kernel(v1=lhs, v2=rhs) of
 * workspaces/matmul/runs/matmul_v3_bf16_split.py:10-161 (forward lhs @ rhs). */
int kda_matmul_f32(const float* lhs, const float* rhs, float* out, int64_t m, int64_t k,
                   int64_t n, void* workspace, int64_t workspace_bytes, void* stream);

/* out[M,N] = lhs^T @ rhs with lhs [K,M], rhs [K,N]; M a multiple of 8.  Replaces
 * kernel(v1=lhs, v2=rhs) of workspaces/transpose_matmul/runs/tmm_v3_mblk16_bf16_split.py:10-41
 * (forward transpose(lhs) @ rhs). */
int kda_transpose_matmul_f32(const float* lhs, const float* rhs, float* out, int64_t m,
                             int64_t k, int64_t n, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* out[b] = lhs[b] @ rhs[b], lhs [B,M,K], rhs [B,K,N], out [B,M,N].  Replaces
 * kernel(lhs, rhs) of workspaces/bmm/runs/bmm_v2.py:10-41. */
int kda_bmm_f32(const float* lhs, const float* rhs, float* out, int64_t batch, int64_t m,
                int64_t k, int64_t n, void* workspace, int64_t workspace_bytes, void* stream);

/* out[M,N] = x[M,K] @ w[K,N] + (x @ a[K,R]) @ b[R,N], both terms in one
 * accumulation.  Replaces kernel(x, w, a, b) of workspaces/lora/runs/lora_v3_bf16_split.py:10-64. */
int kda_lora_f32(const float* x, const float* w, const float* a, const float* b, float* out,
                 int64_t m, int64_t k, int64_t n, int64_t r, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* out[M,N] = (x / sqrt(sum_k(x^2 / K))) @ w (no eps, no gain).  Replaces
 * kernel(v1=x, v2=w) of workspaces/rmsnorm_matmul/runs/rmsnorm_matmul_v1.py:10-138. */
int kda_rmsnorm_matmul_f32(const float* x, const float* w, float* out, int64_t m, int64_t k,
                           int64_t n, void* workspace, int64_t workspace_bytes, void* stream);

/* y = x + z; out[M,N] = (y / sqrt(sum_k(y^2 / K) + eps) * g) @ w with x, z [M,K],
 * g [K], w [K,N].  Argument order of forward(x, w, eps, z, g) /
 * workspaces/add_rmsnorm_matmul/runs/add_rmsnorm_matmul_v1.py:8-146. */
int kda_add_rmsnorm_matmul_f32(const float* x, const float* w, float eps, const float* z,
                               const float* g, float* out, int64_t m, int64_t k, int64_t n,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* y = x @ w + z; out[M,N] = y * g / sqrt(mean_n(y^2) + eps) with x [M,K], w [K,N],
 * z [M,N], g [N].  The GEMM epilogue adds z and writes per-row partial sums of
 * squares; a row kernel applies the norm in place.  Argument order of
 * forward(x, w, eps, z, g) / workspaces/matmul_add_rmsnorm/runs/matmul_add_rmsnorm_v2_bf16_split.py:8-212. */
int kda_matmul_add_rmsnorm_f32(const float* x, const float* w, float eps, const float* z,
                               const float* g, float* out, int64_t m, int64_t k, int64_t n,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* out[M,K] = (silu(x @ w_gate) * (x @ w_up)) @ w_down, fp32, x [M,K], w_up/w_gate
 * [K,F], w_down [F,K]; workspace KDA_OP_SWIGLU_F32 with n = F.  Argument order of
 * kernel(v1=x, v2=w_up, v3=w_down, v4=w_gate) of workspaces/swiglu/runs/swiglu_v1.py:38-146. */
int kda_swiglu_f32(const float* x, const float* w_up, const float* w_down, const float* w_gate,
                   float* out, int64_t m, int64_t k, int64_t f, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* out[b, m, :] = softmax_n(lhs[b, m, :] @ rhs[b, :, :]) (max-shifted), fp32; lhs
 * [B,M,K], rhs [B,K,N], out [B,M,N]; K <= 64, N a multiple of 64.  Scores on
 * fp16 MFMA from a two-limb split of both operands after power-of-two scaling
 * per lhs row and per 64-column rhs tile (three products, ~22 significant bits:
 * the softmax turns score errors into relative output errors); one fused
 * kernel computes online row statistics, then recomputes the scores and writes
 * the probabilities once.  Workspace: KDA_OP_BMM_SOFTMAX_F32.
 * Replaces kernel(lhs, rhs) of workspaces/bmm_softmax/runs/bmm_softmax_v4.py:10-181
 * (forward workspaces/bmm_softmax/docs/draft-phase1.md:14-23). */
int kda_bmm_softmax_f32(const float* lhs, const float* rhs, float* out, int64_t batch, int64_t m,
                        int64_t k, int64_t n, void* workspace, int64_t workspace_bytes,
                        void* stream);

/* ---------------------------------------------------------------- selective scan */

/* Mamba selective scan, fp32:
 *   dA = exp(delta[c,m] * a[c,s]);  dBu = (delta[c,m] * b[s,m]) * u[c,m]
 *   h[c,s,m] = dA * h[c,s,m-1] + dBu  (h = 0 before m = 0);  out[c,m] = sum_s c[s,m] h[c,s,m]
 * delta, u, out [C,M]; a [C,S]; b, c [S,M]; 1 <= S <= 16; any alignment.
 * A chunked parallel scan: one workgroup per channel, one wave per state, 8-step
 * chunks per lane folded into (prod dA, h) pairs and scanned across the wave in
 * fp64, then re-run from their entry states; the states are summed in order
 * s = 0..S-1 and exp is numpy's float32 exp bit for bit.  Not bit-identical to
 * the sequential evaluation (each chunk's entry state is rounded once to fp32):
 * ~2e-6 relative-L2 at C256 M7168 S16 on N(0, 0.05) inputs; bit-identical when
 * M <= 8.  Scratch: none.
 * Replaces kernel(delta, u, a, b, c) of workspaces/mamba/runs/mamba_v4_s4unroll.py:7-117
 * (forward workspaces/mamba/docs/draft-phase1.md:24-30). */
int kda_mamba_f32(const float* delta, const float* u, const float* a, const float* b,
                  const float* c, float* out, int64_t channels, int64_t seq, int64_t states,
                  void* stream);

/* ---------------------------------------------------------------- attention */

/* Grouped-query softmax attention forward, bf16 in/out, fp32 online softmax:
 *   out[b,s,h,:] = softmax_j(q[b,s,h,:] . k[b,j,h/G,:] * scale) @ v[b,j,h/G,:]
 * q [B,S,Hq,D], k/v [B,S,Hkv,D] dense (BSHD); D = 128; any G = Hq/Hkv >= 1 (a
 * workgroup serves the largest power of two up to 8 dividing G of the group's heads).
 * causal != 0 masks keys j > s.  The output element (b,s,h,d) is written at
 * out + b*out_stride_b + s*out_stride_s + h*out_stride_h + d (strides in elements,
 * multiples of 4): BSHD (S*Hq*D, Hq*D, D) or BHSD (Hq*S*D, D, S*D).
 * KDA_ERR_UNSUPPORTED for Hkv > 266305, and for causal launches with Hq > 541200
 * (32-bit DMA offsets of a key tile and of a wave's staged q rows).
 * Replaces kernel(v1=q, v2=k, v3=v) of
 * workspaces/gqa_full/runs/gqa_full_v7a_exp_from_psum.py:15-220 (non-causal, BHSD out). */
int kda_gqa_fwd_bf16(const kda_bf16* q, const kda_bf16* k, const kda_bf16* v, kda_bf16* out,
                     int64_t batch, int64_t seq, int64_t hq, int64_t hkv, int64_t head_dim,
                     float scale, int causal, int64_t out_stride_b, int64_t out_stride_s,
                     int64_t out_stride_h, void* stream);

/* The same attention for fp32 q/k/v/out with fp32-class accuracy: q, k and v are
 * scaled by powers of two (q per row, k per 64-key tile, v per kv head) and split
 * into two fp16 limbs; QK^T and PV each take three fp16 MFMA products (~22
 * significant bits).  D = 128, any G = Hq/Hkv >= 1; output strides as above.
 * Workspace: KDA_OP_GQA_F32 (limb planes and scales).
 * Replaces kernel(v1=q, v2=k, v3=v) of
 * workspaces/gqa_full/runs/gqa_full_v7a_exp_from_psum.py:15-220 at its own fp32
 * inputs (B1 S4096 Hq16 Hkv8 D128, non-causal, BHSD out). */
int kda_gqa_fwd_f32(const float* q, const float* k, const float* v, float* out, int64_t batch,
                    int64_t seq, int64_t hq, int64_t hkv, int64_t head_dim, float scale,
                    int causal, int64_t out_stride_b, int64_t out_stride_s, int64_t out_stride_h,
                    void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KDA_H_ */
