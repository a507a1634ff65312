/*
 * lthc.h — C ABI of the MI355X (gfx950) Local Token Hyper-Connection interface.
 *
 * The library replaces the device side of the reference's LTHC interface: the
 * shared channel-wise read from the high-resolution NHWC residual stream into
 * the workspace, the per-layer channel-wise write with its lazy workspace
 * recurrence, and the single final materialisation, forward and backward.
 * The reference exposes these as torch.library ops (namespace `jit_thc`) in
 * flowmatching_lthc/models/local_thc_triton_kernels.py and as module hooks in
 * flowmatching_lthc/models/local_thc.py; each entry point below names the
 * reference op, kernel or hook it replaces.
 *
 * Conventions shared by every entry point
 *   - All tensors are dense, row-major, in device memory of the current HIP
 *     device.  Activation pointers must be aligned to 4 elements (8 bytes for
 *     16-bit types, 16 bytes for fp32), weight pointers to 16 bytes, and C
 *     must be a multiple of 4.
 *   - Geometry: B batch, G workspace grid side, s cell side (taps K = s*s),
 *     C channels.  High-resolution grid side H = G*s.  Cells M = G*G.
 *       x  (high-res)  [B, H, H, C]   (NHWC; cell view [B, M, K, C] is logical)
 *       z  (workspace) [B, M, C]
 *       w  (weights)   [C, K]         (alpha = read weights, beta_l = write weights)
 *     Tap k = sy*s + sx of cell m = gy*G + gx lives at h = gy*s + sy,
 *     w = gx*s + sx (local_thc_triton_kernels.py:355-363).
 *     Only s == 4 is implemented (K = 16, the B/4 model and the 512px
 *     stress configuration); other values return LTHC_ERR_UNSUPPORTED.
 *   - dtype codes: LTHC_F32, LTHC_BF16, LTHC_F16.  Activations share one
 *     dtype per call; weights are fp32 or the activation dtype (other pairs
 *     return LTHC_ERR_UNSUPPORTED; lthc_gamma takes any).  All arithmetic is fp32
 *     (fused multiply-add), results are rounded once (round-to-nearest-even)
 *     to the output dtype.
 *   - Every call is asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream), performs no host synchronisation and no device allocation.
 *     Entry points that need scratch memory take a caller-provided workspace
 *     whose size is given by the matching *_workspace_bytes function.
 *   - Return value: LTHC_OK (0) or an error code; lthc_last_error() then
 *     returns a thread-local description.  A call with an empty batch
 *     (B == 0 or rows == 0) is a no-op that returns LTHC_OK (the weight
 *     gradients are then written as zeros).
 */
#ifndef LTHC_H_
#define LTHC_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LTHC_F32 0
#define LTHC_BF16 1
#define LTHC_F16 2

#define LTHC_OK 0
#define LTHC_ERR_INVALID 1     /* bad argument: shape, dtype, alignment, null pointer */
#define LTHC_ERR_UNSUPPORTED 2 /* valid but not implemented (s != 4, L too large) */
#define LTHC_ERR_HIP 3         /* a HIP runtime call failed (launch error, no device) */

/* Largest depth L accepted by the multi-layer entry points. */
#define LTHC_MAX_LAYERS 48

/* Thread-local text of the last error raised on this thread ("" if none). */
const char* lthc_last_error(void);

/* ABI version of this library (incremented on any signature change). */
int lthc_abi_version(void);

/*
 * READ   z[b,m,c] = sum_k alpha[c,k] * x[b,m,k,c]
 * Replaces jit_thc::local_write_traceable (local_thc_triton_kernels.py:2673-2683,
 * kernel _write_fwd_kernel :27-60; the legacy name "write" is the algorithmic
 * read) and the eager SharedLocalRead.read (local_thc.py:1211-1223).
 * Accumulation order k = 0..K-1, acc = fma(x, alpha, acc), as in :51-55.
 */
int lthc_read_fwd(const void* x, int x_dtype, const void* alpha, int w_dtype, void* z,
                  int64_t B, int64_t G, int64_t s, int64_t C, void* stream);

/*
 * MULTI-WEIGHT READ   out_l[b,m,c] = sum_k w_l[c,k] * g[b,m,k,c],  l < L
 * Replaces jit_thc::final_accumulate_b4_12_grad_dz_ptr
 * (local_thc_triton_kernels.py:1800-1845, kernel :512-595) and
 * jit_thc::final_accumulate_b4_grad_dz (:1601-1621, kernel :241-277): the
 * gradient of the materialisation with respect to each dZ_l.
 * `w` and `out` are host arrays of L device pointers.
 */
int lthc_read_multi_fwd(const void* g, int x_dtype, const void* const* w, int w_dtype,
                        void* const* out, int64_t B, int64_t G, int64_t s, int64_t C, int L,
                        void* stream);

/*
 * MATERIALISE / WRITE
 *   out[b,m,k,c] = base[b,m,k,c] + sum_{l<L} beta_l[c,k] * dz_l[b,m,c]
 * `base` may be NULL (treated as zero) when L == 1 — the plain write — and for
 * L <= 24 when the tensors are below 4 GiB (the sum of writes, which is the
 * adjoint of a multi-weight read: jit_thc::all_base_b4_12_grad_x,
 * local_thc_triton_kernels.py:2532-2550).  `dz`
 * and `beta` are host arrays of L
 * device pointers ([B,M,C] and [C,K]).  Accumulation: acc = base, then
 * acc = fma(beta_l, dz_l, acc) for l = 0..L-1, one rounding at the store.
 * Replaces
 *   jit_thc::final_accumulate_b4_12_traceable (local_thc_triton_kernels.py:1669-1736,
 *     kernel _final_accumulate_b4_12_fwd_kernel :317-405)            base = x0, L = 12
 *   jit_thc::final_accumulate_b4_traceable (:1578-1598, kernel :202-238)  any L
 *   jit_thc::local_read_traceable (:2686-2696, kernel _read_fwd_kernel :63-95)
 *     and the read backward dX = R^T gZ (:1409, :2726-2729)         base = NULL, L = 1
 *   LayerLocalWrite.write / write_add (local_thc.py:1261-1276) and the
 *     final_accumulate_reference loop (local_thc.py:1368-1372).
 */
int lthc_materialise_fwd(const void* base, const void* const* dz, int x_dtype,
                         const void* const* beta, int w_dtype, void* out,
                         int64_t B, int64_t G, int64_t s, int64_t C, int L, void* stream);

/*
 * CELL WEIGHT GRADIENT (deterministic two-stage fp32 reduction)
 *   gw[l,c,k] = sum_{b,m} high[b,m,k,c] * low_l[b,m,c]      gw: fp32 [L,C,K]
 * Replaces jit_thc::local_weight_grad_traceable (local_thc_triton_kernels.py:2699-2710,
 * kernel _cell_weight_grad_kernel :167-199) — d(alpha) of the read with
 * high = x, low = gZ, and d(weight) of the write with high = gX, low = z —
 * and jit_thc::final_accumulate_b4_12_grad_beta_ptr (:1848-1894, kernel :598-680),
 * jit_thc::final_accumulate_b4_grad_beta (:1624-1644): d(beta_l) of the
 * materialisation with high = grad_out, low_l = dz_l.  The reference reduces
 * with relaxed fp32 atomics; this library sums per-block partials in a fixed
 * order, so results are bitwise reproducible run to run.
 */
size_t lthc_weight_grad_workspace_bytes(int64_t B, int64_t G, int64_t s, int64_t C, int L);
int lthc_weight_grad(const void* high, const void* const* low, int x_dtype, float* gw,
                     int64_t B, int64_t G, int64_t s, int64_t C, int L,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * MATERIALISE BACKWARD (gdZ and gbeta in one pass over G)
 *   gdz_l[cell, c]  = sum_k beta_l[c,k] G[cell,k,c]      (x_dtype, fp32 accumulation, k in order)
 *   gbeta[l, c, k]  = sum_cells G[cell,k,c] dz_l[cell,c] (fp32 [L, C, 16], fixed-order reduction)
 * Replaces final_accumulate_b4_12_grad_dz_ptr + final_accumulate_b4_12_grad_beta_ptr
 * (local_thc_triton_kernels.py:512-680, 1800-1894): the same two results as
 * lthc_read_multi_fwd(G, beta) and lthc_weight_grad(G, dz), but G (the
 * largest tensor) is read once instead of twice.  gdz is bitwise equal to
 * lthc_read_multi_fwd's.  One LDS-staged tile kernel (gbeta on the matrix
 * cores) for 16-bit activations with L <= 24, C % 64 == 0, G % 8 == 0 and
 * 16-byte aligned dz and gdz; otherwise one
 * register kernel when L <= 24, C % 64 == 0 and G is below 4 GiB; otherwise
 * the two separate passes.  `dz`, `beta`, `gdz` are host arrays of L device
 * pointers; the workspace holds the fp32 partials.
 */
size_t lthc_materialise_bwd_workspace_bytes(int64_t B, int64_t G, int64_t s, int64_t C, int L);
int lthc_materialise_bwd(const void* g, int x_dtype, const void* const* dz, const void* const* beta, int w_dtype,
                         void* const* gdz, float* gbeta, int64_t B, int64_t G, int64_t s, int64_t C, int L,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * MATERIALISE BACKWARD WITHOUT A WORKSPACE: lthc_materialise_bwd with the fp32
 * partial sums in a scratch array the library holds on every GPU it runs on
 * (lthc_noalloc_scratch_bytes() = 64 MiB, kept until the process ends).  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  It
 * calls no allocator.  Shapes whose partials need more than the scratch array
 * (lthc_materialise_bwd_workspace_bytes() > 64 MiB) return LTHC_ERR_UNSUPPORTED.
 * All calls on one GPU share the array, which keeps the last call's contents:
 * calls that overlap on one GPU race; the caller serialises them.  The first
 * call on a device looks up that device's scratch address and the launch
 * plans (occupancy queries): make it outside graph capture; later calls may be
 * captured and replayed.
 */
size_t lthc_noalloc_scratch_bytes(void);
int lthc_materialise_bwd_noalloc(const void* g, int x_dtype, const void* const* dz, const void* const* beta,
                                 int w_dtype, void* const* gdz, float* gbeta, int64_t B, int64_t G, int64_t s,
                                 int64_t C, int L, void* stream);

/*
 * GAMMA   gamma_l[c] = sum_k alpha[c,k] * beta_l[c,k]   (written in out_dtype)
 * Replaces LayerLocalWrite.gamma_from_alpha (local_thc.py:1278-1283), computed
 * here in fp32 from the given weights.  `beta` is a host array of L device
 * pointers; `gamma` is [L,C].
 */
int lthc_gamma(const void* alpha, const void* const* beta, int w_dtype, void* gamma, int out_dtype,
               int64_t C, int64_t K, int L, void* stream);

/*
 * GAMMA WITH THE EAGER DTYPE SEQUENCE, all layers in one launch: for the
 * block hook LayerLocalWrite.gamma_from_alpha(shared_read.alpha(dz.dtype))
 * (local_thc.py:1278-1283, :1325-1327) evaluated in out_dtype,
 *   gamma[l, c] = r(sum_k r(r(alpha[c,k]) * r(beta_l[c,k])))
 * with r = round to out_dtype (identity for fp32) and the sum in fp32 over
 * k = 0..K-1.  alpha [C, K] in a_dtype (e.g. the fp32 softmax of the read
 * logits), beta_l [C, K] in b_dtype, gamma [L, C] in out_dtype.
 */
int lthc_gamma_rounded(const void* alpha, int a_dtype, const void* const* beta, int b_dtype, void* gamma,
                       int out_dtype, int64_t C, int64_t K, int L, void* stream);

/*
 * Backward of lthc_gamma_rounded: the values eager autograd gives for that
 * sequence.  With a = r(alpha), b_l = r(beta_l), g_l = grad[l, c] (grad
 * [L, C] in out_dtype):
 *   gbeta_l[c,k] = r(g_l * a[c,k])                     written in b_dtype
 *   galpha[c,k]  = the L products r(g_l * b_l[c,k]) summed in out_dtype,
 *                  last layer first, each partial sum rounded (the order
 *                  autograd accumulates a's gradient in)   written in a_dtype
 * galpha may be NULL; gbeta may be NULL or hold NULL entries (no output).
 */
int lthc_gamma_rounded_bwd(const void* grad, const void* alpha, int a_dtype, const void* const* beta, int b_dtype,
                           void* galpha, void* const* gbeta, int out_dtype, int64_t C, int64_t K, int L,
                           void* stream);

/*
 * LAZY WORKSPACE RECURRENCE STEP   z_next[r,c] = z[r,c] + gamma[c] * dz[r,c]
 * Replaces SharedReadLocalTHCSharedAdaLNJiTBlock.lazy_workspace_update
 * (local_thc.py:1325-1328); rows = B*M.  Computed as fma(gamma, dz, z).
 */
int lthc_recur_fwd(const void* z, const void* dz, int x_dtype, const void* gamma, int g_dtype,
                   void* z_next, int64_t rows, int64_t C, void* stream);

/*
 * RECURRENCE BACKWARD (given g = dL/dz_next)
 *   gdz[r,c]   = gamma[c] * g[r,c] (+ gdz_add[r,c])   (x_dtype; one rounding)
 *   ggamma[c]  = sum_r g[r,c] * dz[r,c]               (fp32, deterministic)
 * dL/dz = g itself, as in eager autograd of local_thc.py:1328.  gdz_add may
 * be NULL; when given it is added before the single rounding, so a caller
 * whose dz also feeds the final materialisation gets the whole gradient of
 * dz (that use's contribution, from lthc_read_multi_fwd, plus this one) in
 * one pass instead of a separate add.
 */
size_t lthc_recur_bwd_workspace_bytes(int64_t rows, int64_t C);
int lthc_recur_bwd(const void* g, const void* dz, const void* gdz_add, int x_dtype, const void* gamma,
                   int g_dtype, void* gdz, float* ggamma, int64_t rows, int64_t C,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * RECURRENCE BACKWARD WITH THE BRANCH GRADIENT
 *   g_sum[r,c] = g[r,c] + g_branch[r,c]                (x_dtype; one rounding)
 *   then lthc_recur_bwd with g_sum in place of g.
 * z_next feeds two consumers in the lazy forward, the next recurrence step
 * and the next block's branch (local_thc.py:1383-1385); eager autograd adds
 * their gradients in a separate pass before the recurrence backward of
 * local_thc.py:1328 sees them.  Here the add happens in the same pass, with
 * the same rounding, and g_sum (= dL/dz_next, which is also dL/dz) is
 * written for the previous step.  ggamma is the fp32 sum rounded once to
 * gg_dtype (gamma's own dtype saves the caller a cast).  Same workspace as
 * lthc_recur_bwd.
 */
int lthc_recur_bwd_sum(const void* g, const void* g_branch, const void* dz, const void* gdz_add, int x_dtype,
                       const void* gamma, int g_dtype, void* g_sum, void* gdz, void* ggamma, int gg_dtype,
                       int64_t rows, int64_t C, void* workspace, size_t workspace_bytes, void* stream);

/*
 * WORKSPACE ACCUMULATION (non-shared / triangular lazy interface)
 *   out[r,c] = base[r,c] + sum_{i<L} gamma[i,c] * dz_i[r,c]        gamma [L, C], L <= 24
 * With a separate read per layer, layer l's workspace input is
 * z_l = R_l(x0) + sum_{j<l} gamma[l,j] * dz_j (local_thc.py:1434-1451).
 * Replaces jit_thc::triangular_accumulate_traceable, the 12-pointer and
 * active-prefix forms (local_thc_triton_kernels.py:684-711, 1922-2488).
 * `dz` is a host array of L device pointers; fp32 accumulation, one rounding.
 */
int lthc_ws_accumulate_fwd(const void* base, const void* const* dz, int x_dtype, const void* gamma, int g_dtype,
                           void* out, int64_t rows, int64_t C, int L, void* stream);

/*
 * Its backward, given g = dL/dout:
 *   gdz_i[r,c] = gamma[i,c] * g[r,c]       (x_dtype; skipped when gdz is NULL)
 *   ggamma[i,c] = sum_r g[r,c] * dz_i[r,c] (fp32 [L,C], deterministic; skipped when NULL)
 * (dL/dbase = g itself.)  Replaces the _grad_dz / _grad_gamma ops of the same
 * family (:713-762).  The workspace is needed only for ggamma.
 */
size_t lthc_ws_accumulate_bwd_workspace_bytes(int64_t rows, int64_t C, int L);
int lthc_ws_accumulate_bwd(const void* g, const void* const* dz, int x_dtype, const void* gamma, int g_dtype,
                           void* const* gdz, float* ggamma, int64_t rows, int64_t C, int L, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * FINAL-LAYER RMSNORM + ADALN MODULATE (the consumer of the materialisation)
 *   inv[t]  = rsqrt(mean_c x[t,c]^2 + eps)                           fp32 [B*N] (may be NULL)
 *   y[t,c]  = r(r(r((x*inv)*weight[c]) * r(1 + scale[b,c])) + shift[b,c])
 * for token t = b*N + n of x [B, N, C], r = round to x_dtype (identity for
 * fp32).  shift and scale are per-sample rows of C values in x_dtype, row b
 * at element offset b * mod_ld (mod_ld >= C, a multiple of 4: e.g. chunks of
 * the shared [B, 6C] AdaLN vector); weight [C] is fp32 or w_dtype, aligned
 * to 4 elements.
 * Replaces FinalLayerSharedAdaLN's norm_final + modulate
 * (local_thc.py:870-873, RMSNorm jit_shared_adaln.py:26-30, modulate
 * local_thc.py:37-38), which eager PyTorch evaluates as about eight passes
 * over the [B, N, C] tensor; here one read and one write.  C <= 2048.
 */
int lthc_norm_modulate_fwd(const void* x, int x_dtype, const void* weight, int w_dtype, const void* shift,
                           const void* scale, int64_t mod_ld, void* y, float* inv, int64_t B, int64_t N, int64_t C,
                           float eps, void* stream);

/*
 * Its backward, given gy = dL/dy and the forward's inv:
 *   gx (x_dtype), gweight fp32 [C], gshift fp32 [B,C], gscale fp32 [B,C]
 * (the fp32 gradient of the function above; reductions in a fixed order).
 */
size_t lthc_norm_modulate_bwd_workspace_bytes(int64_t B, int64_t N, int64_t C);
int lthc_norm_modulate_bwd(const void* gy, const void* x, int x_dtype, const void* weight, int w_dtype,
                           const void* scale, int64_t mod_ld, const float* inv, void* gx, float* gweight,
                           float* gshift, float* gscale, int64_t B, int64_t N, int64_t C, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Q/K RMSNORM + 2-D ROPE of the branch's attention (no reference op: the
 * reference evaluates WorkspaceAttention.forward's q_norm/k_norm + rope,
 * local_thc.py:246-249 with RMSNorm jit_shared_adaln.py:26-30 and
 * VisionRotaryEmbeddingFast jit_shared_adaln.py:57-59, as about twenty
 * eager passes per block).  For qkv [B, N, 3, H, D] (the projection, x_dtype)
 * and x = its q or k part:
 *   n   = r((x * rsqrt(mean_d x^2 + eps)) * weight[d])              weight fp32 [D]
 *   out = r(r(n * r(cos[n,d])) + r(rot(n) * r(sin[n,d])))           rot(n)_{2i} = -n_{2i+1}, rot(n)_{2i+1} = n_{2i}
 * written to q_out / k_out [B, N, H, D] (x_dtype); cos / sin are fp32
 * [N, D] (table_dtype; the table rounded to x_dtype first, as RoPE's
 * .to(x.dtype)); weights [D] in w_dtype; w_dtype and table_dtype are fp32 or
 * x_dtype; r = round to x_dtype.  D must be 64; every pointer 16-byte aligned.
 */
int lthc_qk_norm_rope(const void* qkv, int x_dtype, const void* q_weight, const void* k_weight, int w_dtype,
                      const void* cos_table, const void* sin_table, int table_dtype, void* q_out, void* k_out, int64_t B,
                      int64_t N, int64_t H, int64_t D, float eps, void* stream);

/*
 * Q/K RMSNORM + ROPE FUSED WITH THE ATTENTION (no reference op: the reference
 * evaluates WorkspaceAttention.forward, local_thc.py:246-251, as the q/k
 * norms, RoPE and F.scaled_dot_product_attention).  For qkv [B, N, 3, H, D]:
 *   q_n, k_n = the normalised q and k of lthc_qk_norm_rope (bit-identical)
 *   out[b, n, h, :] = sum_m softmax_m(scale * q_n . k_m) v[b, m, h, :]
 * written as [B, N, H, D] (x_dtype, the [B, N, C] layout of the output
 * projection's input).  Scores, softmax and the output accumulate in fp32;
 * the probabilities are rounded to x_dtype before they multiply V (as flash
 * attention does) and the output is divided by the fp32 row sum and rounded
 * once.  x_dtype bf16 or fp16; D == 64; N a multiple of 64, at most 256;
 * scale > 0 (F.scaled_dot_product_attention's default is 1 / sqrt(D));
 * weights, tables and alignment as lthc_qk_norm_rope.  No dropout.
 */
int lthc_qk_norm_rope_attention(const void* qkv, int x_dtype, const void* q_weight, const void* k_weight, int w_dtype,
                                const void* cos_table, const void* sin_table, int table_dtype, void* out, int64_t B,
                                int64_t N, int64_t H, int64_t D, float eps, float scale, void* stream);

/*
 * DECODER HEAD (no reference op: FinalLayerSharedAdaLN.forward and
 * unpatchify, local_thc.py:865-873 and :972-980, are eager torch).  For the
 * materialised x [B, h*w, C] (x_dtype bf16 or fp16):
 *   y   = RMSNorm + modulate of x as lthc_norm_modulate_fwd (the same roundings)
 *   o   = r(sum_c y[t,c] * r(W[j,c]) + r(bias[j]))        j < 48 = P*P*CO
 *   img[b, ci, hp*P + p1, wp*P + p2] = o[hp*w + wp, (p1*P + p2)*CO + ci]
 * written to img [B, CO, h*P, w*P] (x_dtype).  The product accumulates in
 * fp32 (matrix cores); W and bias are rounded to x_dtype first, as autocast
 * casts them.  norm_weight [C], lin_weight [48, C] and lin_bias [48] are fp32
 * or x_dtype; shift / scale rows [B, C] at row stride mod_ld, x_dtype.
 * C a multiple of 32 up to 768; h*w a multiple of 64; P == 4 and CO == 3;
 * x and lin_weight 16-byte aligned.
 */
int lthc_decoder_fwd(const void* x, int x_dtype, const void* norm_weight, int nw_dtype, const void* shift,
                     const void* scale, int64_t mod_ld, const void* lin_weight, int lw_dtype, const void* lin_bias,
                     int lb_dtype, void* img, int64_t B, int64_t h, int64_t w, int64_t C, int64_t P, int64_t CO,
                     float eps, void* stream);

/*
 * MATERIALISATION WITH THE DECODER FRONT IN ITS EPILOGUE (no-grad forwards;
 * no reference op: the final materialisation, local_thc.py:1368-1372, followed
 * by FinalLayerSharedAdaLN.forward and unpatchify, :865-873 and :972-980).
 * X_L = x0 + sum_l P_l(dz[l]) is formed per token in registers, rounded to
 * x_dtype as the materialisation rounds it, and never written; for each token
 *   o[j] = r(inv * sum_c x[c] M_b[j,c] + Q_b[j]),  inv = 1/sqrt(mean_c x[c]^2 + eps)
 *   M_b[j,c] = r(norm_weight[c] * r(1 + scale[b,c]) * r(W[j,c])),
 *   Q_b[j] = sum_c shift[b,c] r(W[j,c]) + r(bias[j])  (fp32),
 * r() the rounding to x_dtype; img[b, ci, hp*P + p1, wp*P + p2] =
 * o[(hp, wp), (p1*P + p2)*CO + ci] in x_dtype, img [B, CO, 4G*P, 4G*P].
 * This is modulate(RMSNorm(x)) @ W^T + bias without the eager sequence's
 * roundings of the normalised and modulated rows (compare with the exact
 * function, not bit for bit).  x_dtype bf16 or fp16; beta fp32 [C,16]
 * (16-byte aligned); norm_weight, lin_weight [48, C], lin_bias fp32 or
 * x_dtype; shift / scale rows [B, C] at row stride mod_ld, x_dtype.  s == 4,
 * C % 256 == 0, G % 16 == 0, L <= 12, P == 4 and CO == 3, x0 below 4 GiB, img
 * 16-byte aligned.  The caller workspace (256-byte aligned) holds M_b, Q_b's
 * partial sums and the per-slab fp32 partial rows (3 KiB per cell and 256
 * channels).
 */
size_t lthc_materialise_decoder_workspace_bytes(int64_t B, int64_t G, int64_t s, int64_t C);
int lthc_materialise_decoder_fwd(const void* x0, int x_dtype, const void* const* dz, const void* const* beta,
                                 int w_dtype, const void* norm_weight, int nw_dtype, const void* shift,
                                 const void* scale, int64_t mod_ld, const void* lin_weight, int lw_dtype,
                                 const void* lin_bias, int lb_dtype, void* img, int64_t B, int64_t G, int64_t s,
                                 int64_t C, int L, int64_t P, int64_t CO, float eps, void* workspace,
                                 size_t workspace_bytes, void* stream);

/*
 * BATCHED WEIGHT CONVERSION (no reference op: autocast converts each fp32
 * weight in its own kernel on every forward).  entries: device array of
 * {const float* src; int64_t numel; int64_t dst_offset; int64_t first_block}
 * (32 bytes each, 8-byte aligned); block_map: device int32 [nblocks], the
 * entry of each block.  Block b converts elements
 * [(b - first_block) * 2048, +2048) of its entry to dst_dtype (bf16 or fp16,
 * round to nearest even) at dst + dst_offset.  dst 16-byte aligned, every
 * dst_offset a multiple of 8 elements.
 */
int lthc_cast_many(const void* entries, const void* block_map, int64_t nblocks, void* dst, int dst_dtype,
                   void* stream);

/*
 * SWIGLU GATE (no reference op: SwiGLUFFN.forward's chunk + silu + mul,
 * local_thc.py:267-269, three eager passes):
 *   out[r, f] = r(r(a / (1 + exp(-a))) * v),  a = x[r, f], v = x[r, F + f]
 * for x [rows, 2F] and out [rows, F] in x_dtype.  F % 8 == 0; x and out
 * 16-byte aligned.
 */
int lthc_swiglu(const void* x, int x_dtype, void* out, int64_t rows, int64_t F, void* stream);

/*
 * GATED RESIDUALS OF THE BRANCH (no reference op: WorkspaceSharedAdaLNBranch.forward,
 * local_thc.py:319-323, evaluates them as eager multiplies and adds).  For
 * tokens t = b*N + n of [B, N, C] tensors and per-sample [B, C] gates:
 *   lthc_gate_add_norm_modulate_fwd:  d = r(gate * a),  x = r(z + d),  then the
 *     RMSNorm + modulate of x as lthc_norm_modulate_fwd (y, inv); d is written
 *     to d_out.  (dz_attn, z_tmp and the second pre-norm in one pass.)
 *   lthc_gate_residual:  out = r(d + r(gate * m))   (dz_attn + gate_mlp * mlp);
 *     C % 8 == 0, gate_ld % 8 == 0, every pointer 16-byte aligned.
 * Row b of a per-sample vector is at element offset b * mod_ld (gate_ld).  All
 * tensors in x_dtype except the weight [C] (w_dtype) and inv [B*N] (fp32, may
 * be NULL).
 */
int lthc_gate_add_norm_modulate_fwd(const void* z, const void* a, const void* gate, int x_dtype, const void* weight,
                                    int w_dtype, const void* shift, const void* scale, int64_t mod_ld, void* d_out,
                                    void* y, float* inv, int64_t B, int64_t N, int64_t C, float eps, void* stream);
int lthc_gate_residual(const void* d, const void* gate, int64_t gate_ld, const void* m, int x_dtype, void* out,
                       int64_t B, int64_t N, int64_t C, void* stream);

/*
 * BLOCK TAIL (inference): one block's last gated residual, the lazy
 * recurrence step and the next block's first pre-norm in one pass.  Per token
 * t of sample b, channel c (z = Z_l, a = the attention's gated residual
 * g_a * attn, m = the MLP output, gate = g_m):
 *   dz[t,c]     = r(a[t,c] + r(gate[b,c] * m[t,c]))     (lthc_gate_residual)
 *   z_next[t,c] = r(fma(gamma[c], dz[t,c], z[t,c]))       (lthc_recur_fwd)
 *   y[t,:]      = lthc_norm_modulate_fwd of z_next with weight, shift, scale
 * (local_thc.py:319-323 of block l, :1325-1328, :315-317 of block l + 1),
 * each value bitwise that of the three entry points in sequence.  gate,
 * shift and scale are rows of stride mod_ld; gamma is [C] in g_dtype.
 */
int lthc_block_tail_fwd(const void* z, const void* a, const void* m, const void* gate, int x_dtype, const void* gamma,
                        int g_dtype, const void* weight, int w_dtype, const void* shift, const void* scale,
                        int64_t mod_ld, void* dz, void* z_next, void* y, int64_t B, int64_t N, int64_t C, float eps,
                        void* stream);

/*
 * RECURRENCE OVER ALL LAYERS (one pass; the all-L form of lthc_recur_fwd):
 *   z_out[l] = Z_{l+1} = Z_l + gamma[l] * dz[l],  Z_0 = z0,  l = 0..L-1
 * each step rounded to x_dtype as lthc_recur_fwd rounds it (bitwise equal to
 * L calls), Z_0 read once.  gamma is [L, C] in g_dtype; dz and z_out are host
 * arrays of L device pointers.  For callers that hold every dZ_l at once; the
 * lazy forward of local_thc.py:1376-1385 has a branch between the steps.
 */
int lthc_recur_fwd_prefix(const void* z0, const void* const* dz, int x_dtype, const void* gamma, int g_dtype,
                          void* const* z_out, int64_t rows, int64_t C, int L, void* stream);

/*
 * READ BACKWARD (autograd of SharedLocalRead.read, local_thc.py:1211-1223;
 * jit_thc::local_read_add_traceable + local_weight_grad_traceable,
 * local_thc_triton_kernels.py:2713-2764):
 *   dx[cell,k,c]  = g_base[cell,k,c] + alpha[c,k] gz[cell,c]   (g_base may be NULL: zero)
 *   dalpha[c,k]   = sum_cells x[cell,k,c] gz[cell,c]            (fp32, fixed order)
 * dx or dalpha may be NULL to skip that output.
 */
size_t lthc_read_bwd_workspace_bytes(int64_t B, int64_t G, int64_t s, int64_t C);
int lthc_read_bwd(const void* gz, const void* x, int x_dtype, const void* alpha, int w_dtype, const void* g_base,
                  void* dx, float* dalpha, int64_t B, int64_t G, int64_t s, int64_t C, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * WHOLE INTERFACE, every branch update given (local_thc.py:1376-1385 with the
 * dZ_l known in advance; docs/model.md:54-108):
 *   forward:  z[0] = R(x0); gamma_l = sum_k alpha beta_l (fp32);
 *             z[l+1] = z[l] + gamma_l * dz[l]; x_out = x0 + sum_l P_l(dz[l])
 *             (z holds L + 1 outputs)
 *   backward: given gx = dL/dX_L and gz[l] = dL/dZ_l for l < L (NULL entries
 *             are zero; Z_L feeds nothing), with S_l = sum_{j >= l} gz[j]:
 *             dx0 = gx + R^T S_0;  ddz[l] = P_l^T gx + gamma_l S_{l+1};
 *             dbeta[l] = sum gx dz_l + (sum S_{l+1} dz_l) alpha;
 *             dalpha = sum x0 S_0 + sum_l (sum S_{l+1} dz_l) beta_l
 *             (dalpha [C,16], dbeta [L,C,16] fp32; fixed-order reductions).
 * The forward is one pass over x0 and the dz stack for 16-bit activations
 * with L <= 12 and C % 256 == 0, or L == 24 and any C (one kernel writes
 * z[0..L] and x_out, bitwise the per-op entry points' values), and otherwise
 * composes them (read, gamma, recurrence prefix, materialise).  The backward is one pass over gx and the dz and gz
 * stacks for 16-bit activations with L <= 24, C % 64 == 0, G % 8 == 0 and
 * 16-byte aligned gx, dx0, alpha and dz, gz and ddz entries (one tile kernel forms gamma, writes
 * ddz, dx0 and S_0 and the partial sums of dbeta and of the gamma terms; then
 * dalpha's pass over x0 and S_0 and one launch of the reductions), and otherwise a composition (materialise backward; the
 * recurrence steps in one pass over H, dZ and gdZ up to depth 24, one
 * lthc_recur_bwd or lthc_recur_bwd_sum per step above; read backward).  Both
 * give the per-step entry points' ddz and dx0 bit for bit (local_thc_triton_kernels.py:512-680,
 * 1800-1919 and the eager autograd of local_thc.py:1211-1223, 1325-1328).
 * One caller workspace of lthc_interface_workspace_bytes() serves both.
 */
size_t lthc_interface_workspace_bytes(int64_t B, int64_t G, int64_t s, int64_t C, int L);
int lthc_interface_fwd(const void* x0, int x_dtype, const void* alpha, const void* const* beta, int w_dtype,
                       const void* const* dz, void* const* z, void* x_out, int64_t B, int64_t G, int64_t s, int64_t C,
                       int L, void* workspace, size_t workspace_bytes, void* stream);
int lthc_interface_bwd(const void* gx, const void* const* gz, int x_dtype, const void* x0, const void* const* dz,
                       const void* alpha, const void* const* beta, int w_dtype, void* dx0, void* const* ddz,
                       float* dalpha, float* dbeta, int64_t B, int64_t G, int64_t s, int64_t C, int L, void* workspace,
                       size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LTHC_H_ */
