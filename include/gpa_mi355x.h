/*
 * gpa_mi355x.h — C ABI of the MI355X (gfx950) GPA-VGGT merging hot path.
 *
 * Eight entry points (two of them with an fp16 twin, the attention also
 * with an allocation-free variant) sit behind this boundary:
 *
 *   gpa_sim_argmax_bf16   — fused cosine-similarity row max / argmax between
 *                           source and destination token metrics
 *                           (replaces merging/fused_similarity.py:81-112,
 *                            the Triton `_sim_argmax_kernel` at :33-78).
 *   gpa_attn_keybias_bf16 — flash attention with a per-key additive bias
 *                           (replaces merging/fused_attention.py:130-180,
 *                            the Triton `_attn_keybias_kernel` at :70-127).
 *   gpa_merge_heads       — deterministic segmented mean/sum of token rows,
 *                           the K/V merge (replaces the scatter_reduce_ of
 *                           merging/merge.py:234-250).
 *   gpa_lse_combine_bf16  — merge of two partial attentions by their log2
 *                           LSE (replaces vggt/layers/attention.py:166-176).
 *   gpa_qk_norm_rope_bf16 (and _f16) — qk LayerNorm + 2D RoPE + cast of a block's
 *                           attention operands (replaces the torch op
 *                           sequence of vggt/layers/attention.py:210-220).
 *   gpa_pool_shared_bf16 (and _f16) — pooled summaries of the frame-special shared
 *                           K/V set (replaces vggt/layers/attention.py:113-140).
 *   gpa_merge_metric_bf16 — the merge's metric projection, normalisation and
 *                           dst/src split (replaces merging/merge.py:180-187).
 *   gpa_residual_layernorm_bf16 (and _f16) — residual + LayerScale + LayerNorm of the
 *                           caller's blocks (replaces vggt/layers/block.py:84-96
 *                           torch ops).
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are device pointers owned by the caller.  The
 *     library allocates nothing and keeps no reference after returning
 *     (gpa_attn_keybias_bf16_noalloc uses the library's one static device
 *     array instead of a caller workspace).
 *   - Element strides are in elements (not bytes).  The innermost (feature)
 *     dimension has unit stride; row pointers must be 16-byte aligned.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL is the
 *     legacy default stream).  Functions return GPA_OK (0) after a successful
 *     launch or a negative GPA_E* code; gpa_last_error() then holds a
 *     message for the calling thread.
 *   - The library is reentrant and keeps no per-call state (except for the
 *     shared scratch of gpa_attn_keybias_bf16_noalloc): tile shapes are a
 *     deterministic function of the problem shape and, for the similarity,
 *     of the current device's CU count (read once per device and cached;
 *     query gpa_sim_argmax_workspace_bytes with the launch's device
 *     current).  No autotuning.
 */
#ifndef GPA_MI355X_H
#define GPA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPA_ABI_VERSION 15

enum {
  GPA_OK = 0,
  GPA_E_INVALID = -1,      /* null pointer, negative size, bad stride/alignment */
  GPA_E_UNSUPPORTED = -2,  /* shape outside what the kernels implement */
  GPA_E_WORKSPACE = -3,    /* workspace missing or too small */
  GPA_E_LAUNCH = -4        /* the HIP runtime rejected the launch */
};

/* Bias element types accepted by gpa_attn_keybias_bf16 / _f16. */
enum { GPA_BIAS_NONE = 0, GPA_BIAS_F32 = 1, GPA_BIAS_BF16 = 2, GPA_BIAS_F16 = 3 };

/* Element types and reductions of gpa_merge_heads. */
enum { GPA_DTYPE_F32 = 0, GPA_DTYPE_BF16 = 1, GPA_DTYPE_F16 = 2 };
enum { GPA_MERGE_SUM = 0, GPA_MERGE_MEAN = 1 };

/* ABI version of the loaded library (GPA_ABI_VERSION at build time). */
int gpa_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* gpa_last_error(void);

/* Bytes of device workspace gpa_sim_argmax_bf16 needs for this shape on
 * the current device (0 when the kernel writes its outputs directly).  The
 * workspace passed to the call must be 16-byte aligned. */
size_t gpa_sim_argmax_workspace_bytes(int64_t B, int64_t M, int64_t N, int64_t D);

/*
 * Fused similarity row max / argmax.
 *   a [B, M, D] bf16 (source metric), b [B, N, D] bf16 (destination metric)
 *   out_max[b*omax_sb + m] = max_n  sum_d a[b,m,d] * b[b,n,d]   (fp32 accumulate)
 *   out_idx[b*oidx_sb + m] = the lowest n attaining that maximum (int64)
 * out_max holds max_dtype elements: GPA_DTYPE_F32, or GPA_DTYPE_BF16 /
 * GPA_DTYPE_F16 (the fp32 max rounded to nearest even), so the reference's
 * `node_max` in a's dtype (fused_similarity.py:112) needs no separate cast.
 * Replaces merging/fused_similarity.py:81-112 (`fused_similarity_argmax`);
 * the index tie rule follows the kernel's strict `>` at
 * merging/fused_similarity.py:73 together with tl.argmax's first index.
 * D must be a multiple of 32 and at most 4096 (above 256 GEMM-tiled kernels
 * loop over the features: the unprojected 1024-d metric); N >= 1.
 * NaN scores never win (an all-NaN row yields -inf and index 0).
 */
int gpa_sim_argmax_bf16(const void* a, const void* b,
                        void* out_max, int max_dtype, int64_t* out_idx,
                        int64_t B, int64_t M, int64_t N, int64_t D,
                        int64_t a_sb, int64_t a_sm,
                        int64_t b_sb, int64_t b_sn,
                        int64_t omax_sb, int64_t oidx_sb,
                        void* workspace, size_t workspace_bytes,
                        void* stream);

/* The same on fp16 a and b (v_mfma_f32_16x16x32_f16; same arguments, same
 * workspace).  Replaces fused_similarity.py:81-112 for fp16 operands, which
 * the reference passes to its kernel as they are (only an fp32 `a` is cast,
 * to bf16). */
int gpa_sim_argmax_f16(const void* a, const void* b,
                       void* out_max, int max_dtype, int64_t* out_idx,
                       int64_t B, int64_t M, int64_t N, int64_t D,
                       int64_t a_sb, int64_t a_sm,
                       int64_t b_sb, int64_t b_sn,
                       int64_t omax_sb, int64_t oidx_sb,
                       void* workspace, size_t workspace_bytes,
                       void* stream);

/* Bytes of device workspace gpa_attn_keybias_bf16 needs: per (batch, head)
 * one 144-byte record per 32-key tile, holding the keys' bias/sm_scale
 * (padded past N) and two per-tile maxima the kernel bounds its scores with,
 * 16 bytes of row maxima and means, and one flag byte per 64 queries.  The
 * reference wrapper allocates the analogous padded bias buffer
 * (merging/fused_attention.py:159-160).  At head dims 128 and 256 the call
 * writes one fp32 bias row per (batch, head) there instead (4 bytes per key,
 * rounded up to 32 keys), which the same size holds. */
size_t gpa_attn_keybias_workspace_bytes(int64_t B, int64_t H, int64_t M, int64_t N);

/*
 * Attention with a per-key additive bias, head_dim D in {16, 32, 64, 128,
 * 256} (the reference kernel's HEAD_DIM, fused_attention.py:82, 97, 177).
 * D = 64 (VGGT) runs the tuned kernel with a certified fixed softmax
 * offset; D = 128 and 256 a tiled kernel with a lazily moved offset, D = 16
 * and 32 a running-max kernel, all with the same contract.
 *   o[b,h,m,:] = softmax_n( q[b,h,m,:].k[b,h,n,:] * sm_scale + bias[b,h,n] ) . v[b,h,n,:]
 *   lse[b,h,m] = log2( sum_n 2^( (q.k*sm_scale + bias) * log2(e) ) )   (if lse != NULL)
 * Replaces merging/fused_attention.py:130-180 (`attention_keybias`) and the
 * Triton kernel at merging/fused_attention.py:70-127, including its log2
 * log-sum-exp output (:123-127).  q/k/v/o are bf16; the softmax runs in fp32
 * and P is rounded to bf16 for the P.V product, as in the reference kernel.
 * bias_kind is GPA_BIAS_NONE (bias ignored), GPA_BIAS_F32 or GPA_BIAS_BF16;
 * bias strides may be 0 (e.g. one bias row shared by every head).
 * workspace: 16-byte aligned device memory of at least
 * gpa_attn_keybias_workspace_bytes(...) bytes, overwritten by the call.
 */
int gpa_attn_keybias_bf16(const void* q, const void* k, const void* v,
                          const void* bias, int bias_kind,
                          int64_t bias_sb, int64_t bias_sh, int64_t bias_sn,
                          void* o, float* lse,
                          int64_t B, int64_t H, int64_t M, int64_t N, int64_t D,
                          int64_t q_sb, int64_t q_sh, int64_t q_sm,
                          int64_t k_sb, int64_t k_sh, int64_t k_sn,
                          int64_t v_sb, int64_t v_sh, int64_t v_sn,
                          int64_t o_sb, int64_t o_sh, int64_t o_sm,
                          int64_t lse_sb, int64_t lse_sh,
                          void* workspace, size_t workspace_bytes,
                          float sm_scale, void* stream);

/* The same on fp16 q, k, v and o (fp16 MFMA; P rounded to fp16 for P.V,
 * fp32 softmax and accumulation; same arguments and workspace).  The fixed
 * offset sits 15 below the score bound, so P <= 2^15 fits fp16, and is
 * certified only where every row max is within 16 of the bound; a wave that
 * cannot certify it continues with an offset that moves lazily, whenever a
 * tile's row max rises above the offset + 15.  Replaces
 * fused_attention.py:130-180 under fp16 autocast (its :139-144 cast). */
int gpa_attn_keybias_f16(const void* q, const void* k, const void* v,
                         const void* bias, int bias_kind,
                         int64_t bias_sb, int64_t bias_sh, int64_t bias_sn,
                         void* o, float* lse,
                         int64_t B, int64_t H, int64_t M, int64_t N, int64_t D,
                         int64_t q_sb, int64_t q_sh, int64_t q_sm,
                         int64_t k_sb, int64_t k_sh, int64_t k_sn,
                         int64_t v_sb, int64_t v_sh, int64_t v_sn,
                         int64_t o_sb, int64_t o_sh, int64_t o_sm,
                         int64_t lse_sb, int64_t lse_sh,
                         void* workspace, size_t workspace_bytes,
                         float sm_scale, void* stream);

/* Bytes of the device-resident scratch array behind
 * gpa_attn_keybias_bf16_noalloc (one per GPU, held until the process ends). */
#define GPA_ATTN_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * gpa_attn_keybias_bf16 without the workspace arguments: the workspace is a
 * static device array of GPA_ATTN_NOALLOC_SCRATCH_BYTES in the library, so
 * the call allocates nothing (no hipMalloc/hipFree, no allocating library
 * routine).  No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation).  Same arguments, semantics and kernels otherwise.
 * Shapes whose gpa_attn_keybias_workspace_bytes(B, H, M, N) exceeds the
 * array are refused with GPA_E_UNSUPPORTED.  The array is resolved on the
 * current device at its first call there; `stream` must belong to the
 * current device.  Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (other threads, other streams) race.
 */
int gpa_attn_keybias_bf16_noalloc(const void* q, const void* k, const void* v,
                                  const void* bias, int bias_kind,
                                  int64_t bias_sb, int64_t bias_sh, int64_t bias_sn,
                                  void* o, float* lse,
                                  int64_t B, int64_t H, int64_t M, int64_t N, int64_t D,
                                  int64_t q_sb, int64_t q_sh, int64_t q_sm,
                                  int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                  int64_t v_sb, int64_t v_sh, int64_t v_sn,
                                  int64_t o_sb, int64_t o_sh, int64_t o_sm,
                                  int64_t lse_sb, int64_t lse_sh,
                                  float sm_scale, void* stream);

/*
 * Deterministic segmented reduction of token rows: the K/V merge.
 *   out[b,h,s,:] = reduce over n in tokens[offsets[b*S+s] .. offsets[b*S+s+1])
 *                  of t[b,h,n,:]                  (GPA_MERGE_SUM or GPA_MERGE_MEAN)
 * fp32 accumulation in list order, one rounding to `dtype` (t and out share
 * it).  Token values are positions in [0, N) of batch b; every slot's list is
 * its own token followed by the tokens merged into it.  size_out /
 * log_size_out (nullable, fp32 [B*S]) receive the list lengths and their
 * natural logs.  Out-of-range tokens or offsets make that slot NaN (no
 * out-of-bounds access).  Rows: unit feature stride, 16-byte aligned; D a
 * multiple of 4 (fp32) or 8 (bf16, fp16).
 * Replaces merging/merge.py:234-250 (`merge.heads`, and `merge` with H = 1),
 * whose scatter_reduce_ sums in a run-dependent order, and the size of
 * merging/merge.py:211-217 with the log-count bias of
 * vggt/layers/attention.py:250-260.
 */
int gpa_merge_heads(const void* t, int dtype, void* out,
                    const int64_t* offsets, const int64_t* tokens,
                    int64_t B, int64_t H, int64_t N, int64_t S, int64_t D,
                    int64_t t_sb, int64_t t_sh, int64_t t_sn,
                    int64_t o_sb, int64_t o_sh, int64_t o_sn,
                    int mode, float* size_out, float* log_size_out, void* stream);

/*
 * Merge of two attentions over a partition of the keys by their log2 LSE,
 * written in the token-major projection layout:
 *   m = max(la, lb), wa = 2^(la-m), wb = 2^(lb-m)
 *   y[b, n, h*D + d] = (oa[b,h,n,d]*wa + ob[b,h,n,d]*wb) / (wa + wb)     (fp32, bf16 out)
 * Every operand is addressed per (b, h, s, p) with token n = s*P + p (element
 * strides *_b, *_h, *_s, *_p), so the own-frame output [B*S, H, P, D] and the
 * shared-set output [B, H, N, D] are both plain strides; y has strides
 * (y_b, y_n, y_h) and unit feature stride.  N must be a multiple of P,
 * D a multiple of 8, rows 16-byte aligned.
 * Replaces the combine of the frame-special split path,
 * vggt/layers/attention.py:166-176 (with the final transpose to [B, N, C]).
 */
int gpa_lse_combine_bf16(const void* oa, const float* la, const void* ob, const float* lb,
                         void* y, int64_t B, int64_t H, int64_t N, int64_t P, int64_t D,
                         int64_t oa_b, int64_t oa_h, int64_t oa_s, int64_t oa_p,
                         int64_t la_b, int64_t la_h, int64_t la_s, int64_t la_p,
                         int64_t ob_b, int64_t ob_h, int64_t ob_s, int64_t ob_p,
                         int64_t lb_b, int64_t lb_h, int64_t lb_s, int64_t lb_p,
                         int64_t y_b, int64_t y_n, int64_t y_h, void* stream);

/* The same on fp16 oa, ob and y (the combine under fp16 autocast, where the
 * reference combines in the fp16 activation dtype, attention.py:166-176);
 * weights and sums in fp32, one rounding to fp16. */
int gpa_lse_combine_f16(const void* oa, const float* la, const void* ob, const float* lb,
                        void* y, int64_t B, int64_t H, int64_t N, int64_t P, int64_t D,
                        int64_t oa_b, int64_t oa_h, int64_t oa_s, int64_t oa_p,
                        int64_t la_b, int64_t la_h, int64_t la_s, int64_t la_p,
                        int64_t ob_b, int64_t ob_h, int64_t ob_s, int64_t ob_p,
                        int64_t lb_b, int64_t lb_h, int64_t lb_s, int64_t lb_p,
                        int64_t y_b, int64_t y_n, int64_t y_h, void* stream);

/*
 * qk LayerNorm + 2D rotary embedding + cast, from the QKV projection rows.
 * For each token n < N of batch b and head h < H (D must be 64):
 *   x = qkv[b*qkv_sb + n*qkv_sn + h*64 .. +64]              (q; k at + k_offset)
 *   y = (x - mean) / sqrt(var + eps) * w + beta              (fp32; biased variance)
 *   within each 32-feature half (first: row coordinate, second: column
 *   coordinate of pos[(n mod period)*2 + half]), for j < 16:
 *     out[j] = y[j] c - y[j+16] s,  out[j+16] = y[j+16] c + y[j] s
 *   with (c, s) = rope_cs[(p*16 + j)*2 + {0,1}] (positions clamped to
 *   [0, npos)); pos == NULL skips the rotation.
 * ln_weight / ln_bias hold 128 floats each: q's 64, then k's 64.  q_out and
 * k_out are contiguous [B, H, N, 64] of q_dtype / k_dtype (GPA_DTYPE_F32 or
 * GPA_DTYPE_BF16).  qkv rows: bf16, unit feature stride, 16-byte aligned,
 * each holding at least k_offset + H*64 elements (k_offset >= H*64).
 * Replaces q_norm / k_norm and the RoPE of vggt/layers/attention.py:216-220
 * (vggt/layers/rope.py:167-209) and the fp32 -> bf16 cast of
 * merging/fused_attention.py:139-144; the reference module interface has no
 * such entry point (it runs these as separate torch ops).
 */
int gpa_qk_norm_rope_bf16(const void* qkv, int64_t B, int64_t N, int64_t H, int64_t D,
                          int64_t qkv_sb, int64_t qkv_sn, int64_t k_offset,
                          const float* ln_weight, const float* ln_bias, float eps,
                          const int32_t* pos, int64_t period,
                          const float* rope_cs, int64_t npos,
                          void* q_out, int q_dtype, void* k_out, int k_dtype, void* stream);

/* The same on an fp16 projection (the fp16-autocast stack): q_dtype /
 * k_dtype GPA_DTYPE_F32 or GPA_DTYPE_F16; the arithmetic is the same fp32.
 * Replaces the same reference lines under fp16 autocast (the cast of
 * fused_attention.py:139-144 then goes to fp16). */
int gpa_qk_norm_rope_f16(const void* qkv, int64_t B, int64_t N, int64_t H, int64_t D,
                         int64_t qkv_sb, int64_t qkv_sn, int64_t k_offset,
                         const float* ln_weight, const float* ln_bias, float eps,
                         const int32_t* pos, int64_t period,
                         const float* rope_cs, int64_t npos,
                         void* q_out, int q_dtype, void* k_out, int k_dtype, void* stream);

/*
 * Pooled summaries of the frame-special shared K/V set.  For every
 * (b, h, frame s) and its patch keys x_p = k[b, h, s*P + pts + p, :]
 * (p < grid_h*grid_w on a grid_h-row, grid_w-column patch grid, row-major;
 * D = 64):
 *   seeds y_g: the patches (gy*kp, gx*kp), g = gy*nw + gx, nh = ceil(grid_h/kp),
 *              nw = ceil(grid_w/kp), npool = nh*nw (any kp >= 1)
 *   assign a_p = argmax_g bf16(bf16(x_p/max(|x_p|,1e-6)) . bf16(y_g/max(|y_g|,1e-6)))
 *              (fp32 dots rounded to bf16; the lowest g wins ties)
 *   size[b,h,s,g]         = #{p : a_p = g}                                (fp32)
 *   pooled_k[b,h,s*npool+g,:] = sum_{a_p=g} k_p / max(size, 1)           (bf16)
 *   pooled_v likewise from v (same token positions).
 * pooled_k / pooled_v are contiguous [B, H, S*npool, 64], size [B, H, S, npool];
 * assign (nullable) receives a_p as int32 [B, H, S, grid_h*grid_w].  k and v
 * rows 16-byte aligned, unit feature stride; grid_h*grid_w <= 4096 (else
 * GPA_E_UNSUPPORTED).  Up to 64 seeds per frame they stay in registers;
 * above, they are scored and summed in super-chunks of 64 (K read twice and
 * V once per chunk).  The sums run in fp32 in a fixed order,
 * so the means are deterministic (the reference's scatter_add_ sums with
 * atomics in a run-dependent order).
 * Replaces `_pool` of vggt/layers/attention.py:113-140 (ph = grid_h,
 * pw = grid_w; the einsum at :130 under bf16 autocast) and the pool sizes
 * behind the bias of :142-146; the reference module interface has no such
 * entry point (it runs these as torch ops).
 */
int gpa_pool_shared_bf16(const void* k, const void* v, void* pooled_k, void* pooled_v,
                         float* size, int32_t* assign, int64_t B, int64_t H, int64_t S,
                         int64_t P, int64_t pts, int64_t grid_h, int64_t grid_w, int64_t kp,
                         int64_t D, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                         int64_t v_sb, int64_t v_sh, int64_t v_sn, void* stream);

/* The same on fp16 k and v (the pooling under fp16 autocast: fp16
 * normalised rows and fp16 scores; fp16 pooled outputs). */
int gpa_pool_shared_f16(const void* k, const void* v, void* pooled_k, void* pooled_v,
                        float* size, int32_t* assign, int64_t B, int64_t H, int64_t S,
                        int64_t P, int64_t pts, int64_t grid_h, int64_t grid_w, int64_t kp,
                        int64_t D, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                        int64_t v_sb, int64_t v_sh, int64_t v_sn, void* stream);

/*
 * Front end of the bipartite merge: for every batch b and output row j,
 * with t = order[j] (order == NULL: t = j),
 *   y = bf16( bf16(metric[b, t, :]) @ proj )   C -> P, fp32 accumulation
 *   n = sqrt(sum y^2) in fp32; norm_mode 1 rounds n to bf16
 *   out[b, j, :] = bf16(y / n)                  (no epsilon: a zero row gives NaN)
 * norm_mode 2 is the chain under fp16 autocast: the metric (fp32 only) and
 * proj (then fp16 bits) are rounded to fp16, y = fp16(...) on the fp16 MFMA,
 * and n, the division and the output as in mode 0.
 * metric: [B, N, C] of metric_dtype (GPA_DTYPE_F32 or GPA_DTYPE_BF16), unit
 * feature stride, 16-byte aligned rows, C in {256, 512, 768, 1024}; proj:
 * contiguous [C][P] bf16, P = 128; order: int64 [N]; out: contiguous
 * [B, N, P] bf16.  With order = [dst positions | src positions] the output
 * holds the similarity operands b then a.
 * Replaces merging/merge.py:180-187 as it runs under bf16 autocast
 * (norm_mode 0: `metric @ proj` in bf16, the norm in fp32, the division
 * promoted to fp32, then the bf16 cast of fused_similarity.py:90-95) or on
 * a bf16 metric without autocast (norm_mode 1); the reference runs it as
 * torch ops (projection, norm, division, two index gathers).
 */
int gpa_merge_metric_bf16(const void* metric, int metric_dtype, int64_t B, int64_t N, int64_t C,
                          int64_t m_sb, int64_t m_sn, const void* proj, int64_t P,
                          const int64_t* order, int norm_mode, void* out, void* stream);

/*
 * Residual + LayerScale + LayerNorm of a pre-LN block, bf16 rows of C
 * features (C a multiple of 512, <= 4096), one pass:
 *   h   = bf16(x + bf16(gamma * y))                     (y given; else h = x)
 *   out = bf16((h - mean) * rsqrt(var + eps) * w + b)    fp32 moments, biased var
 * h_out (only with y) and ln_out are each optional, but one is required.
 * Rows are x + r*x_sn (likewise y, h_out, ln_out); rows and gamma / w / b
 * 16-byte aligned.  Replaces `x + self.ls1(attn_out)` / `self.norm2(x)` of
 * vggt/layers/block.py:84-96 under bf16 autocast (bf16 multiply and add,
 * fp32 layer_norm, the cast to bf16 before the next Linear); the reference
 * module interface has no such entry point (it runs these as torch ops).
 */
int gpa_residual_layernorm_bf16(const void* x, const void* y, const void* gamma,
                                const void* ln_weight, const void* ln_bias, float eps,
                                int64_t rows, int64_t C, int64_t x_sn, int64_t y_sn,
                                void* h_out, int64_t h_sn, void* ln_out, int64_t ln_sn,
                                void* stream);

/* The same on fp16 rows and parameters: the chain under fp16 autocast on an
 * fp16 model (the reference's accuracy-evaluation stack, eval/eval_co3d.py:
 * 152 and :226), every bf16 rounding above an fp16 rounding. */
int gpa_residual_layernorm_f16(const void* x, const void* y, const void* gamma,
                               const void* ln_weight, const void* ln_bias, float eps,
                               int64_t rows, int64_t C, int64_t x_sn, int64_t y_sn,
                               void* h_out, int64_t h_sn, void* ln_out, int64_t ln_sn,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GPA_MI355X_H */
