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
//   * A workgroup owns 256 queries of one (batch, head): 4 waves x 2 blocks
//     of 32 queries.  Q stays in VGPRs for the whole kernel.  K, V^T and the
//     bias stream through double-buffered LDS tiles of 32 keys.
//   * Scores are computed transposed, S^T = K . Q^T, on
//     v_mfma_f32_32x32x16_bf16: a lane owns one query and 16 of the tile's
//     32 keys (the other 16 sit in lane^32), so the running max, the sum and
//     the rescale factor are per-lane scalars.
//   * The bias enters through the accumulator input of the first QK^T MFMA
//     (pre-divided by the exp2 scale), so adding it costs no VALU work:
//       s = q.k + bias/sm_scale,  x = s * (sm_scale*log2 e) - m.
//   * P^T leaves the score MFMA already in the B-operand register layout of
//     the next MFMA, O^T = V^T . P^T, provided the V^T A-operand enumerates
//     keys in the same order; V is transposed into LDS when staged.  The
//     output O^T also keeps one query per lane, so rescaling is a per-lane
//     multiply.
//   * The running max is updated lazily: it only moves when a tile's max
//     exceeds it by more than kTau (log2 units), so P stays <= 2^kTau and the
//     O rescale runs on a handful of tiles per row instead of every tile.
//   * Row sums are accumulated from the bf16 P with v_dot2_f32_bf16 (half a
//     VALU op per score).
#include "gpa_common.h"

#include <math.h>

namespace gpa {
namespace {

constexpr int kWaves = 4;
constexpr int kQB = 2;                        // 32-query blocks per wave
constexpr int kQPerWG = kWaves * kQB * 32;    // 256 queries per workgroup
constexpr int kKT = 32;                       // keys per tile
constexpr int kHD = 64;                       // head dim
constexpr int kVTS = kKT + 4;                 // padded V^T row (elements)
constexpr float kTau = 8.0f;                  // lazy rescale threshold (log2)
constexpr float kPadBias = -1.0e30f;          // bias of keys past N

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
  float c;         // sm_scale * log2(e)
  float bias_mul;  // log2(e) / c, i.e. 1 / sm_scale
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

__global__ __launch_bounds__(256, 2) void attn_keybias_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kKT * kHD];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][kHD * kVTS];
  __shared__ __attribute__((aligned(16))) float Bs[2][kKT];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, hi = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q_wave = (int64_t)blockIdx.x * kQPerWG + wave * (kQB * 32);

  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* V = p.v + b * p.v_sb + h * p.v_sh;

  // Q^T as the B-operand of S^T = K . Q^T: lane supplies query (lane%32),
  // features 16*ks + 8*hi .. +8.
  bf16x8 qf[kQB][4];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int64_t row = q_wave + qb * 32 + l32;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[qb][ks] = row < p.M ? *reinterpret_cast<const bf16x8*>(Q + row * p.q_sm + ks * 16 + hi * 8)
                             : bf16x8{};
  }

  float m_run[kQB], l_run[kQB];
  f32x16 o_acc[kQB][2];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
    o_acc[qb][0] = f32x16{};
    o_acc[qb][1] = f32x16{};
  }

  // Tile staging: K rows as 16-byte chunks (thread -> key tid/8, chunk tid%8);
  // V as 2 keys x 4 features per thread, transposed on the way into LDS;
  // bias for 32 keys, already multiplied by bias_mul.
  const int ntiles = (int)((p.N + kKT - 1) / kKT);
  u32x4 kreg;
  u32x2 vreg0, vreg1;
  float breg = 0.f;
  const int k_key = tid >> 3, k_ch = tid & 7;
  const int v_kp = tid >> 4, v_dq = tid & 15;

  auto load_tile = [&](int t) {
    const int64_t n0 = (int64_t)t * kKT;
    {
      const int64_t n = n0 + k_key;
      kreg = n < p.N ? *reinterpret_cast<const u32x4*>(K + n * p.k_sn + k_ch * 8) : u32x4{};
    }
    {
      const int64_t n = n0 + 2 * v_kp;
      vreg0 = n < p.N ? *reinterpret_cast<const u32x2*>(V + n * p.v_sn + v_dq * 4) : u32x2{};
      vreg1 = n + 1 < p.N ? *reinterpret_cast<const u32x2*>(V + (n + 1) * p.v_sn + v_dq * 4)
                          : u32x2{};
    }
    if (tid < kKT) {
      const int64_t n = n0 + tid;
      float bv = kPadBias;
      if (n < p.N) {
        const int64_t off = b * p.bias_sb + h * p.bias_sh + n * p.bias_sn;
        if (p.bias_kind == GPA_BIAS_F32)
          bv = static_cast<const float*>(p.bias)[off] * p.bias_mul;
        else if (p.bias_kind == GPA_BIAS_BF16)
          bv = bf16_bits_to_f32(static_cast<const uint16_t*>(p.bias)[off]) * p.bias_mul;
        else
          bv = 0.f;
      }
      breg = bv;
    }
  };
  auto store_tile = [&](int buf) {
    *reinterpret_cast<u32x4*>(&Ks[buf][k_key * kHD + ((k_ch ^ (k_key & 7)) << 3)]) = kreg;
    // vreg0 = key 2kp: (f0|f1, f2|f3); vreg1 = key 2kp+1.  Emit, per feature,
    // the pair (key 2kp, key 2kp+1) into row `feature` of V^T.
    uint32_t* vt = reinterpret_cast<uint32_t*>(&Vt[buf][0]);
    const int col = v_kp;  // 32-bit column = key pair
    const int f0 = 4 * v_dq;
    vt[((f0 + 0) * kVTS) / 2 + col] = (vreg0.x & 0xffffu) | (vreg1.x << 16);
    vt[((f0 + 1) * kVTS) / 2 + col] = (vreg0.x >> 16) | (vreg1.x & 0xffff0000u);
    vt[((f0 + 2) * kVTS) / 2 + col] = (vreg0.y & 0xffffu) | (vreg1.y << 16);
    vt[((f0 + 3) * kVTS) / 2 + col] = (vreg0.y >> 16) | (vreg1.y & 0xffff0000u);
    if (tid < kKT) Bs[buf][tid] = breg;
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();

  const float c = p.c;
  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1);

    // Accumulator input of the first score MFMA: the bias of the keys this
    // lane's registers cover (rows 8g + 4hi + j of the 32x32 tile).
    f32x16 cinit;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(&Bs[cur][8 * g + 4 * hi]);
      cinit[4 * g + 0] = bv[0];
      cinit[4 * g + 1] = bv[1];
      cinit[4 * g + 2] = bv[2];
      cinit[4 * g + 3] = bv[3];
    }
    bf16x8 kf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kf[ks] = *reinterpret_cast<const bf16x8*>(
          &Ks[cur][l32 * kHD + (((2 * ks + hi) ^ (l32 & 7)) << 3)]);
    // V^T A-operand for k-step s: feature row d, keys 16s+4hi+{0..3} and
    // 16s+8+4hi+{0..3} -- the keys whose probabilities this lane holds in
    // its score registers 8s..8s+7.
    bf16x8 vf[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint16_t* row = &Vt[cur][(db * 32 + l32) * kVTS + 16 * s + 4 * hi];
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(row);
        const bf16x4 up = *reinterpret_cast<const bf16x4*>(row + 8);
        vf[db][s] = bf16x8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
      }

#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      f32x16 s = mfma32x32x16(kf[0], qf[qb][0], cinit);
      s = mfma32x32x16(kf[1], qf[qb][1], s);
      s = mfma32x32x16(kf[2], qf[qb][2], s);
      s = mfma32x32x16(kf[3], qf[qb][3], s);

      float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
      for (int r = 3; r < 16; r += 2) mx = fmaxf(fmaxf(mx, s[r]), s[r + 1 < 16 ? r + 1 : r]);
      mx = fmaxf(mx, xor32(mx));
      const float ms = mx * c;
      const bool need = ms > m_run[qb] + kTau;
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float mnew = need ? ms : m_run[qb];
        const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - mnew);
        m_run[qb] = mnew;
        l_run[qb] *= alpha;
        o_acc[qb][0] *= alpha;
        o_acc[qb][1] *= alpha;
      }
      const float neg_m = -m_run[qb];
      bf16x8 pb[2];
      float lsum = l_run[qb];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * half + e], c, neg_m));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * half + e + 1], c, neg_m));
          const bf16x2 pp = {(__bf16)p0, (__bf16)p1};
          pb[half][e] = pp[0];
          pb[half][e + 1] = pp[1];
          lsum = __builtin_amdgcn_fdot2_f32_bf16(pp, bf16x2{(__bf16)1.0f, (__bf16)1.0f}, lsum,
                                                 false);
        }
      }
      l_run[qb] = lsum;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        o_acc[qb][db] = mfma32x32x16(vf[db][0], pb[0], o_acc[qb][db]);
        o_acc[qb][db] = mfma32x32x16(vf[db][1], pb[1], o_acc[qb][db]);
      }
    }

    if (t + 1 < ntiles) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: combine the two key halves of each row's sum, normalise, store.
  uint16_t* O = p.o + b * p.o_sb + h * p.o_sh;
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const float l_tot = l_run[qb] + xor32(l_run[qb]);
    const float inv = 1.0f / l_tot;
    const int64_t row = q_wave + qb * 32 + l32;
    if (row < p.M) {
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = db * 32 + 8 * g + 4 * hi;
          const bf16x4 ov = {(__bf16)(o_acc[qb][db][4 * g + 0] * inv),
                             (__bf16)(o_acc[qb][db][4 * g + 1] * inv),
                             (__bf16)(o_acc[qb][db][4 * g + 2] * inv),
                             (__bf16)(o_acc[qb][db][4 * g + 3] * inv)};
          *reinterpret_cast<bf16x4*>(O + row * p.o_sm + d0) = ov;
        }
      if (p.lse && hi == 0)
        p.lse[b * p.lse_sb + h * p.lse_sh + row] = m_run[qb] + __log2f(l_tot);
    }
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
  if (gx > 0x7fffffff || N > ((int64_t)1 << 40)) {
    gpa_set_error("gpa_attn_keybias_bf16: problem too large");
    return GPA_E_UNSUPPORTED;
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
  const float log2e = 1.4426950408889634f;
  p.c = sm_scale * log2e;
  p.bias_mul = 1.0f / sm_scale;

  hipLaunchKernelGGL(attn_keybias_kernel, dim3((unsigned)gx, (unsigned)(B * H)), dim3(256), 0,
                     (hipStream_t)stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("gpa_attn_keybias_bf16: launch failed: %s", hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}
