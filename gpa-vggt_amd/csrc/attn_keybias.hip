// Flash attention with a per-key additive bias for gfx950 (CDNA4), head_dim 64.
//
//   o[m,:]  = sum_n softmax_n(q_m.k_n * sm_scale + bias_n) v_n
//   lse[m]  = log2 sum_n 2^((q_m.k_n * sm_scale + bias_n) * log2 e)
//
// Semantics follow merging/fused_attention.py:70-127: scores in the exp2
// domain, fp32 online softmax, P rounded to bf16 for the P.V product, fp32
// accumulation, log2 log-sum-exp output.
//
// Mapping onto CDNA4
//   * A workgroup owns 256 queries of one (batch, head): 8 waves of 32
//     queries, about 128 VGPRs each, so four waves share a SIMD and the
//     hardware overlaps one wave's MFMAs with another's softmax.  K, V^T and
//     the bias stream through double-buffered LDS tiles of 32 keys, fed by
//     range-checked buffer loads one tile ahead.
//   * Scores are computed transposed, S^T = K . Q^T, on
//     v_mfma_f32_32x32x16_bf16: a lane owns one query and 16 of the tile's
//     32 keys (the other 16 sit in lane^32), so the running max, the sum and
//     the rescale factor are per-lane scalars; the two halves meet through
//     v_permlane32_swap.
//   * The bias rides in a fifth k-step of the score MFMA: each key carries
//     bias/sm_scale split into a bf16 hi/lo pair, multiplied by a constant
//     (1, 1) column of Q, so
//       s = q.k + bias/sm_scale,  x = s * (sm_scale*log2 e) - m
//     costs no VALU work and one 4-byte LDS read per lane per tile (instead
//     of four 16-byte broadcast reads of an fp32 bias row).  Q stays
//     unscaled: rounding q*sm_scale*log2(e) to bf16 would perturb sharp
//     logits by ~2^-9 of their size.
//   * P^T leaves the score MFMA already in the B-operand register layout of
//     the next MFMA, O^T = V^T . P^T, provided the V^T A-operand enumerates
//     keys in the same order; V is transposed into LDS when staged.  O^T
//     keeps one query per lane, so a rescale is a per-lane multiply.
//   * The running max moves lazily: only when a tile's max exceeds it by more
//     than kTau (log2 units), so P stays <= 2^kTau and the rescale (a rare,
//     wave-uniform branch) runs on a handful of tiles per row.
//   * Row sums: when the log-sum-exp is requested they accumulate the fp32
//     probabilities (before their bf16 rounding), as the reference does.
//     Otherwise they sum the bf16 P the P.V product uses with
//     v_dot2_f32_bf16 (exact fp32 sums of bf16 pairs, 8 instead of 16 VALU
//     instructions per tile), normalising O by exactly the weights it was
//     built from.
#include "gpa_common.h"

#include <math.h>

namespace gpa {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kQPerWG = kWaves * 32;          // 256 queries per workgroup
constexpr int kKT = 32;                       // keys per tile
constexpr int kHD = 64;                       // head dim
constexpr int kVTS = kKT + 4;                 // padded V^T row (elements)
constexpr float kTau = 8.0f;                  // lazy rescale threshold (log2)
constexpr float kPadBias = -1.0e30f;          // bias of keys past N
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const void* bias;
  int bias_kind;
  int H;
  uint16_t* o;
  float* lse;
  int64_t M, N;
  int64_t q_sb, q_sh, q_sm, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sm;
  int64_t bias_sb, bias_sh, bias_sn, lse_sb, lse_sh;
  uint32_t k_bytes, v_bytes, bias_bytes;  // extent of one (batch, head) slice
  float c;         // sm_scale * log2(e)
  float bias_mul;  // log2(e) / c, i.e. 1 / sm_scale
};

// One LDS tile: K rows (16-byte chunks XOR-swizzled by key), V transposed
// (feature-major, padded rows), and per key the bias/sm_scale as a packed
// bf16 (hi, lo) pair; slot kKT stays zero for the lanes whose fifth-k-step
// operand is empty.
struct alignas(16) Tile {
  uint16_t k[kKT * kHD];
  uint16_t vt[kHD * kVTS];
  uint32_t bias[kKT + 1];
};

// XOR swizzle of K's 16-byte chunks: lanes reading one logical chunk of 16
// consecutive keys hit 16 distinct 16-byte bank groups (64 banks), and any
// 8 consecutive keys hit 8 distinct ones (32 banks).
__device__ __forceinline__ int k_chunk(int key, int ch) {
  return ch ^ (key & 7) ^ ((key >> 3) & 1);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

template <int BIAS, bool LSE>
__global__ __launch_bounds__(kThreads, 4) void attn_keybias_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) Tile ring[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, hi = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q_row = (int64_t)blockIdx.x * kQPerWG + wave * 32 + l32;
  const float c = p.c;

  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* V = p.v + b * p.v_sb + h * p.v_sh;

  // Q^T as the B-operand of S^T = K . Q^T: lane supplies query (lane%32),
  // features 16*ks + 8*hi .. +8.
  bf16x8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = q_row < p.M ? *reinterpret_cast<const bf16x8*>(Q + q_row * p.q_sm + ks * 16 + hi * 8)
                         : bf16x8{};
  // Fifth k-step: Q supplies (1, 1) against each key's (bias_hi, bias_lo),
  // on the low half only (k = 64, 65).
  bf16x8 q_bias = bf16x8{};
  if (hi == 0) {
    q_bias[0] = (__bf16)1.0f;
    q_bias[1] = (__bf16)1.0f;
  }
  const int bias_slot = hi == 0 ? l32 : kKT;  // slot kKT holds zero

  // Tile staging through range-checked buffer loads (keys past N read as
  // zeros).  Waves 0-3 fetch K rows as 16-byte chunks (thread -> key t/8,
  // chunk t%8); waves 4-7 fetch V as 2 keys x 4 features per thread,
  // transposed on the way into LDS; threads 0-31 fetch the raw bias.
  const int ntiles = (int)((p.N + kKT - 1) / kKT);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(K, p.k_bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, p.v_bytes);
  const __amdgpu_buffer_rsrc_t brs =
      make_rsrc(BIAS == GPA_BIAS_NONE ? nullptr
                                      : static_cast<const char*>(p.bias) +
                                            (b * p.bias_sb + h * p.bias_sh) *
                                                (BIAS == GPA_BIAS_F32 ? 4 : 2),
                BIAS == GPA_BIAS_NONE ? 0u : p.bias_bytes);
  const uint32_t k_row = (uint32_t)p.k_sn * 2u, v_row = (uint32_t)p.v_sn * 2u;
  const uint32_t b_step = (uint32_t)p.bias_sn * (BIAS == GPA_BIAS_F32 ? 4u : 2u);
  const bool k_loader = tid < 256;
  const int u = tid & 255;
  const int k_key = u >> 3, k_ch = u & 7;
  const int v_kp = u >> 4, v_dq = u & 15;
  u32x4 stg = u32x4{};  // K chunk (waves 0-3) or two V half-rows (waves 4-7)
  uint32_t braw = 0;

  // Per-lane byte offsets are fixed; the tile advance goes in soffset.
  const uint32_t k_voff = k_key * k_row + k_ch * 16;
  const uint32_t v_voff = 2 * v_kp * v_row + v_dq * 8;
  const uint32_t b_voff = tid * b_step;
  auto load_tile = [&](int t) {
    const uint32_t n0 = (uint32_t)t * kKT;
    if (k_loader) {
      stg = buf_load16(krs, k_voff, n0 * k_row);
    } else {
      const u32x2 v0 = buf_load8(vrs, v_voff, n0 * v_row);
      const u32x2 v1 = buf_load8(vrs, v_voff + v_row, n0 * v_row);
      stg = u32x4{v0.x, v0.y, v1.x, v1.y};
    }
    if (BIAS == GPA_BIAS_F32 && tid < kKT)
      braw = __builtin_amdgcn_raw_buffer_load_b32(brs, b_voff, n0 * b_step, 0);
    if (BIAS == GPA_BIAS_BF16 && tid < kKT)
      braw = __builtin_amdgcn_raw_buffer_load_b16(brs, b_voff, n0 * b_step, 0);
  };
  auto store_tile = [&](int t, Tile& T) {
    if (k_loader) {
      *reinterpret_cast<u32x4*>(&T.k[k_key * kHD + (k_chunk(k_key, k_ch) << 3)]) = stg;
    } else {
      // stg.xy = key 2kp: (f0|f1, f2|f3); stg.zw = key 2kp+1.  Emit, per
      // feature, the pair (key 2kp, key 2kp+1) into row `feature` of V^T.
      uint32_t* vt = reinterpret_cast<uint32_t*>(T.vt);
      const int f0 = 4 * v_dq;
      vt[((f0 + 0) * kVTS) / 2 + v_kp] = __builtin_amdgcn_perm(stg.z, stg.x, 0x05040100u);
      vt[((f0 + 1) * kVTS) / 2 + v_kp] = __builtin_amdgcn_perm(stg.z, stg.x, 0x07060302u);
      vt[((f0 + 2) * kVTS) / 2 + v_kp] = __builtin_amdgcn_perm(stg.w, stg.y, 0x05040100u);
      vt[((f0 + 3) * kVTS) / 2 + v_kp] = __builtin_amdgcn_perm(stg.w, stg.y, 0x07060302u);
    }
    if (tid < kKT) {
      float bv = 0.f;
      if (BIAS == GPA_BIAS_F32) bv = __uint_as_float(braw) * p.bias_mul;
      if (BIAS == GPA_BIAS_BF16) bv = bf16_bits_to_f32(braw) * p.bias_mul;
      bv = tid < (int)min((int64_t)kKT, p.N - (int64_t)t * kKT) ? bv : kPadBias;
      const __bf16 bhi = (__bf16)bv;
      const __bf16 blo = (__bf16)(bv - (float)bhi);
      T.bias[tid] = (uint32_t)__builtin_bit_cast(uint16_t, bhi) |
                    ((uint32_t)__builtin_bit_cast(uint16_t, blo) << 16);
    }
  };

  float m_run = -INFINITY;  // running max in log2 units (moved lazily)
  float l_run = 0.f;        // LSE variant: fp32 row sum of this lane's keys
  f32x16 o_acc[2] = {f32x16{}, f32x16{}};
  const bf16x2 ones2 = {(__bf16)1.0f, (__bf16)1.0f};

  // One tile: scores, softmax, P.V; then stage tile t+1 into `Tn` (last read
  // before the previous barrier) and synchronise.  Both ring slots are
  // compile-time objects in the unrolled loop below, so every LDS address
  // is a loop-invariant register plus an immediate offset.
  auto step = [&](const Tile& T, Tile& Tn, const int t) {
    if (t + 1 < ntiles) load_tile(t + 1);

    // Scores s = q.k + bias/sm_scale (rows 8g + 4hi + j of the 32x32 result).
    f32x16 sv = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 kf =
          *reinterpret_cast<const bf16x8*>(&T.k[l32 * kHD + (k_chunk(l32, 2 * ks + hi) << 3)]);
      sv = mfma32x32x16(kf, qf[ks], sv);
    }
    {
      const uint32_t pair = T.bias[bias_slot];
      const u32x4 kb = {pair, 0u, 0u, 0u};
      sv = mfma32x32x16(__builtin_bit_cast(bf16x8, kb), q_bias, sv);
    }

    float mx = fmaxf(fmaxf(sv[0], sv[1]), sv[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, sv[r]), sv[r + 1]);
    mx = fmaxf(mx, sv[15]);
    const float ms = max_halves(mx) * c;
    const bool need = t == 0 || ms > m_run + kTau;
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      // Move m up to this tile's max and rescale what has been accumulated.
      const float m_new = need ? ms : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
      o_acc[0] *= alpha;
      o_acc[1] *= alpha;
    }

    const float neg_m = -m_run;
    bf16x8 pb[2];
    float lsum = 0.f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[8 * half + e], c, neg_m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[8 * half + e + 1], c, neg_m));
        const bf16x2 pp = {(__bf16)p0, (__bf16)p1};
        pb[half][e] = pp[0];
        pb[half][e + 1] = pp[1];
        if (LSE)
          lsum = (half == 0 && e == 0) ? p0 + p1 : lsum + (p0 + p1);
        else
          lsum = __builtin_amdgcn_fdot2_f32_bf16(pp, ones2, lsum, false);
      }
    }
    l_run += lsum;

    // O^T += V^T . P^T.  V^T A-operand for k-step s: feature row d, keys
    // 16s+4hi+{0..3} and 16s+8+4hi+{0..3} -- the keys whose probabilities
    // this lane holds in its score registers 8s..8s+7.
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint16_t* row = &T.vt[(db * 32 + l32) * kVTS + 16 * s + 4 * hi];
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(row);
        const bf16x4 up = *reinterpret_cast<const bf16x4*>(row + 8);
        const bf16x8 vf = {lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
        o_acc[db] = mfma32x32x16(vf, pb[s], o_acc[db]);
      }

    if (t + 1 < ntiles) store_tile(t + 1, Tn);
    __syncthreads();
  };

  if (tid == 0) {
    ring[0].bias[kKT] = 0u;
    ring[1].bias[kKT] = 0u;
  }
  load_tile(0);
  store_tile(0, ring[0]);
  __syncthreads();
  int t = 0;
  for (; t + 2 <= ntiles; t += 2) {
    step(ring[0], ring[1], t);
    step(ring[1], ring[0], t + 1);
  }
  if (t < ntiles) step(ring[0], ring[1], t);

  // Epilogue: combine the two key halves of the row sum, normalise, store.
  uint16_t* O = p.o + b * p.o_sb + h * p.o_sh;
  const float l_tot = sum_halves(l_run);
  const float inv = 1.0f / l_tot;
  if (q_row < p.M) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hi;
        const bf16x4 ov = {(__bf16)(o_acc[db][4 * g + 0] * inv),
                           (__bf16)(o_acc[db][4 * g + 1] * inv),
                           (__bf16)(o_acc[db][4 * g + 2] * inv),
                           (__bf16)(o_acc[db][4 * g + 3] * inv)};
        *reinterpret_cast<bf16x4*>(O + q_row * p.o_sm + d0) = ov;
      }
    if (p.lse && hi == 0) p.lse[b * p.lse_sb + h * p.lse_sh + q_row] = m_run + __log2f(l_tot);
  }
}

}  // namespace
}  // namespace gpa

using namespace gpa;

extern "C" int gpa_attn_keybias_bf16(const void* q, const void* k, const void* v, const void* bias,
                                     int bias_kind, int64_t bias_sb, int64_t bias_sh,
                                     int64_t bias_sn, void* o, float* lse, int64_t B, int64_t H,
                                     int64_t M, int64_t N, int64_t D, int64_t q_sb, int64_t q_sh,
                                     int64_t q_sm, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                     int64_t v_sb, int64_t v_sh, int64_t v_sn, int64_t o_sb,
                                     int64_t o_sh, int64_t o_sm, int64_t lse_sb, int64_t lse_sh,
                                     float sm_scale, void* stream) {
  gpa_clear_error();
  if (B < 0 || H < 0 || M < 0 || N < 0 || D < 0) {
    gpa_set_error("gpa_attn_keybias_bf16: negative size");
    return GPA_E_INVALID;
  }
  if (B == 0 || H == 0 || M == 0) return GPA_OK;
  if (N == 0) {
    gpa_set_error("gpa_attn_keybias_bf16: empty key set (N=0)");
    return GPA_E_INVALID;
  }
  if (D != kHD) {
    gpa_set_error("gpa_attn_keybias_bf16: head_dim %lld unsupported (only 64)", (long long)D);
    return GPA_E_UNSUPPORTED;
  }
  if (!q || !k || !v || !o) {
    gpa_set_error("gpa_attn_keybias_bf16: null tensor pointer");
    return GPA_E_INVALID;
  }
  if (bias_kind != GPA_BIAS_NONE && bias_kind != GPA_BIAS_F32 && bias_kind != GPA_BIAS_BF16) {
    gpa_set_error("gpa_attn_keybias_bf16: unknown bias kind %d", bias_kind);
    return GPA_E_INVALID;
  }
  if (bias_kind != GPA_BIAS_NONE && !bias) {
    gpa_set_error("gpa_attn_keybias_bf16: bias kind %d with a null bias pointer", bias_kind);
    return GPA_E_INVALID;
  }
  if (!(sm_scale > 0.f) || !isfinite(sm_scale)) {
    gpa_set_error("gpa_attn_keybias_bf16: sm_scale must be positive and finite");
    return GPA_E_INVALID;
  }
  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) &&
                       ((uintptr_t)v % 8 == 0) && ((uintptr_t)o % 8 == 0) && q_sm % 8 == 0 &&
                       q_sb % 8 == 0 && q_sh % 8 == 0 && k_sn % 8 == 0 && k_sb % 8 == 0 &&
                       k_sh % 8 == 0 && v_sn % 4 == 0 && v_sb % 4 == 0 && v_sh % 4 == 0 &&
                       o_sm % 4 == 0 && o_sb % 4 == 0 && o_sh % 4 == 0;
  if (!aligned || q_sm < D || k_sn < D || v_sn < D || o_sm < D) {
    gpa_set_error("gpa_attn_keybias_bf16: rows must have unit feature stride, q/k rows 16-byte "
                  "and v/o rows 8-byte aligned");
    return GPA_E_INVALID;
  }
  if (B * H > 65535) {
    gpa_set_error("gpa_attn_keybias_bf16: B*H=%lld exceeds the grid limit", (long long)(B * H));
    return GPA_E_UNSUPPORTED;
  }
  const int64_t gx = (M + kQPerWG - 1) / kQPerWG;
  // Buffer offsets are 32-bit: one (batch, head) slice of K, V and the bias,
  // plus one tile of overrun, must stay below 2^31 bytes.
  const int64_t span = N + kKT;
  const int64_t bias_esize = bias_kind == GPA_BIAS_F32 ? 4 : 2;
  if (gx > 0x7fffffff || span * k_sn * 2 >= ((int64_t)1 << 31) ||
      span * v_sn * 2 >= ((int64_t)1 << 31) ||
      (bias_kind != GPA_BIAS_NONE && span * bias_sn * bias_esize >= ((int64_t)1 << 31))) {
    gpa_set_error("gpa_attn_keybias_bf16: one head's K/V/bias slice exceeds 2 GiB");
    return GPA_E_UNSUPPORTED;
  }
  if (bias_kind != GPA_BIAS_NONE && N > 1 && bias_sn <= 0) {
    gpa_set_error("gpa_attn_keybias_bf16: bias key stride must be positive");
    return GPA_E_INVALID;
  }

  AttnArgs p{};
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.bias = bias;
  p.bias_kind = bias_kind;
  p.H = (int)H;
  p.o = (uint16_t*)o;
  p.lse = lse;
  p.M = M;
  p.N = N;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_sm = q_sm;
  p.k_sb = k_sb; p.k_sh = k_sh; p.k_sn = k_sn;
  p.v_sb = v_sb; p.v_sh = v_sh; p.v_sn = v_sn;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_sm = o_sm;
  p.bias_sb = bias_sb; p.bias_sh = bias_sh; p.bias_sn = bias_sn;
  p.lse_sb = lse_sb; p.lse_sh = lse_sh;
  p.k_bytes = (uint32_t)(((N - 1) * k_sn + D) * 2);
  p.v_bytes = (uint32_t)(((N - 1) * v_sn + D) * 2);
  p.bias_bytes = bias_kind == GPA_BIAS_NONE ? 0u : (uint32_t)(((N - 1) * bias_sn + 1) * bias_esize);
  p.c = sm_scale * kLog2e;
  p.bias_mul = 1.0f / sm_scale;

  const dim3 grid((unsigned)gx, (unsigned)(B * H)), block(kThreads);
  hipStream_t s = (hipStream_t)stream;
  const bool want_lse = lse != nullptr;
#define GPA_ATTN_LAUNCH(KIND)                                                          \
  if (want_lse)                                                                        \
    hipLaunchKernelGGL((attn_keybias_kernel<KIND, true>), grid, block, 0, s, p);       \
  else                                                                                 \
    hipLaunchKernelGGL((attn_keybias_kernel<KIND, false>), grid, block, 0, s, p);
  switch (bias_kind) {
    case GPA_BIAS_F32:
      GPA_ATTN_LAUNCH(GPA_BIAS_F32);
      break;
    case GPA_BIAS_BF16:
      GPA_ATTN_LAUNCH(GPA_BIAS_BF16);
      break;
    default:
      GPA_ATTN_LAUNCH(GPA_BIAS_NONE);
      break;
  }
#undef GPA_ATTN_LAUNCH
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("gpa_attn_keybias_bf16: launch failed: %s", hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}
