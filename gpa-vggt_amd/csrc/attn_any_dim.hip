// Biased flash attention for head dims other than 64 (16, 32, 128, 256):
// the same contract as attn_main_kernel (scores q.k * sm_scale + bias in the
// exp2 domain, fp32 online softmax, P rounded to the operand format for the
// P.V product, fp32 accumulation, log2 LSE), computed with the reference
// kernel's own softmax scheme (merging/fused_attention.py:103-118): a
// running row max, the accumulator and row sum rescaled by exp2(m - m_new)
// on every tile, and the row sum of the fp32 probabilities.  The reference
// kernel takes HEAD_DIM as a constexpr (fused_attention.py:82, 89, 97) and
// its wrapper reads it from q (:146, 177); VGGT uses 64, which the tuned
// main kernel serves, so this kernel favours a simple schedule over speed.
//
// Mapping onto CDNA4
//   * A workgroup owns 128 queries of one (batch, head): 4 waves of one
//     32-query block each; one wave per SIMD pair of slots is left to the
//     register budget (HD 256 holds 64 Q and 128 O registers per lane).
//   * Keys stream through a two-slot LDS ring of 32-key tiles loaded with
//     plain 16-byte loads: the next tile's loads are issued into registers
//     before the current tile is computed and written to the other slot
//     after it, one barrier per tile.  K stays row-major (padded rows); V is
//     stored transposed, each 16-key step's keys in the order the score
//     MFMA's result registers enumerate them, so the A operand of
//     O^T = V^T . P^T is one 16-byte LDS read and P^T is used in place.
//   * Scores are computed transposed, S^T = K . Q^T, on
//     v_mfma_f32_32x32x16 (HD / 16 k-steps): a lane owns one query and 16 of
//     the tile's 32 keys (the other 16 sit in lane^32); the accumulator
//     starts from the keys' bias / sm_scale (-inf past N).
//   * HD 16: the P.V product runs on a 32-feature block whose upper 16
//     features are zero and never stored.
#include "gpa_common.h"

#include <math.h>

#include "attn_any_dim.h"

namespace gpa {
namespace {

constexpr int kAWaves = 4;
constexpr int kAThreads = kAWaves * 64;
constexpr int kAQ = kAWaves * 32;            // queries per workgroup
constexpr int kAKT = 32;                      // keys per tile

// Position of key k (0..31) of a tile in the transposed V rows: step s =
// k / 16 holds, in lane-half order, the keys the score MFMA's result
// registers 8s .. 8s+7 of lanes 0-31 (hi = 0) and 32-63 (hi = 1) hold:
// register r of half hi is key 8 (r / 4) + 4 hi + r % 4.
__device__ __forceinline__ int vt_pos(int k) {
  return (k & ~15) + ((k >> 2) & 1) * 8 + ((k >> 3) & 1) * 4 + (k & 3);
}

template <int KIND>
__device__ __forceinline__ float any_bias(const void* bias, int64_t off) {
  if constexpr (KIND == GPA_BIAS_F32) return static_cast<const float*>(bias)[off];
  else if constexpr (KIND == GPA_BIAS_BF16)
    return __uint_as_float((uint32_t)static_cast<const uint16_t*>(bias)[off] << 16);
  else if constexpr (KIND == GPA_BIAS_F16)
    return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(bias)[off]);
  else return 0.f;
}

template <int HD, bool F16, int KIND>
__global__ __launch_bounds__(kAThreads, HD >= 256 ? 1 : 2) void attn_any_dim_kernel(AnyDimArgs p) {
  constexpr int KS = HD / 16;                 // k-steps of the score product
  constexpr int DB = HD >= 32 ? HD / 32 : 1;  // 32-feature blocks of O
  constexpr int KROW = HD + 8;                // padded K row (elements)
  constexpr int VROW = kAKT + 8;              // padded transposed V row
  constexpr int CH = HD / 8;                  // 16-byte chunks per key row
  constexpr int NCH = kAKT * CH;              // chunks per tile and tensor
  constexpr int CPT = (NCH + kAThreads - 1) / kAThreads;
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[2][kAKT * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][DB * 32 * VROW];
  __shared__ __attribute__((aligned(16))) float bias_lds[2][kAKT];

  const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5, l32 = lane & 31;
  const int wave = tid >> 6;
  const int64_t bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
  const int64_t q_row = (int64_t)blockIdx.x * kAQ + wave * 32 + l32;
  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* V = p.v + b * p.v_sb + h * p.v_sh;
  const int64_t boff = b * p.bias_sb + h * p.bias_sh;
  const float c = p.c;

  if constexpr (HD == 16) {                   // the zero upper half of the O block
    for (int i = tid; i < 2 * 32 * VROW; i += kAThreads) {
      const int sl = i / (32 * VROW), r = i % (32 * VROW);
      if (r >= 16 * VROW) vt_lds[sl][r] = 0;
    }
  }

  bf16x8 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qf[ks] = q_row < p.M ? *reinterpret_cast<const bf16x8*>(Q + q_row * p.q_sm + 16 * ks + 8 * hi)
                         : bf16x8{};

  // One tile's K and V chunks and bias, into registers (zeros / -inf past N).
  u32x4 kreg[CPT], vreg[CPT];
  float breg = -INFINITY;
  auto load_tile = [&](int t) {
    const int64_t n0 = (int64_t)t * kAKT;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int cidx = tid + i * kAThreads;
      const int key = cidx / CH, ch = cidx % CH;
      const bool ok = cidx < NCH && n0 + key < p.N;
      kreg[i] = ok ? *reinterpret_cast<const u32x4*>(K + (n0 + key) * p.k_sn + 8 * ch) : u32x4{};
      vreg[i] = ok ? *reinterpret_cast<const u32x4*>(V + (n0 + key) * p.v_sn + 8 * ch) : u32x4{};
    }
    if (tid < kAKT)
      breg = n0 + tid < p.N ? any_bias<KIND>(p.bias, boff + (n0 + tid) * p.bias_sn) * p.mul
                            : -INFINITY;
  };
  auto store_tile = [&](int sl) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int cidx = tid + i * kAThreads;
      if (cidx < NCH) {
        const int key = cidx / CH, ch = cidx % CH;
        *reinterpret_cast<u32x4*>(&ks_lds[sl][key * KROW + 8 * ch]) = kreg[i];
        const int pos = vt_pos(key);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vt_lds[sl][(8 * ch + 2 * e) * VROW + pos] = (uint16_t)(vreg[i][e] & 0xffffu);
          vt_lds[sl][(8 * ch + 2 * e + 1) * VROW + pos] = (uint16_t)(vreg[i][e] >> 16);
        }
      }
    }
    if (tid < kAKT) bias_lds[sl][tid] = breg;
  };

  float m = -1.0e30f, l = 0.f;                // finite: a tile of -inf biases scores 0
  f32x16 o_acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o_acc[db] = f32x16{};

  const int ntiles = (int)((p.N + kAKT - 1) / kAKT);
  load_tile(0);
  store_tile(0);
  for (int t = 0; t < ntiles; ++t) {
    const int sl = t & 1;
    __syncthreads();                          // slot sl written; slot sl^1 free
    if (t + 1 < ntiles) load_tile(t + 1);
    // S^T = K . Q^T + bias / sm_scale
    f32x16 sv;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(&bias_lds[sl][8 * g + 4 * hi]);
      sv[4 * g + 0] = bv[0];
      sv[4 * g + 1] = bv[1];
      sv[4 * g + 2] = bv[2];
      sv[4 * g + 3] = bv[3];
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&ks_lds[sl][l32 * KROW + 16 * ks + 8 * hi]);
      sv = mfma32x32x16_t<F16>(kf, qf[ks], sv);
    }
    // Online softmax: running max, rescale, P in the operand format.
    float mx = sv[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sv[r]);
    const float m_new = fmaxf(m, max_halves(mx) * c);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int db = 0; db < DB; ++db) o_acc[db] *= alpha;
    bf16x8 pb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[8 * s + e], c, -m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[8 * s + e + 1], c, -m));
        l += p0 + p1;
        const bf16x2 pv2 = pack2<F16>(p0, p1);
        pb[s][e] = pv2[0];
        pb[s][e + 1] = pv2[1];
      }
    // O^T += V^T . P^T
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8 vf =
            *reinterpret_cast<const bf16x8*>(&vt_lds[sl][(db * 32 + l32) * VROW + 16 * s + 8 * hi]);
        o_acc[db] = mfma32x32x16_t<F16>(vf, pb[s], o_acc[db]);
      }
    if (t + 1 < ntiles) store_tile(sl ^ 1);
  }

  const float l_tot = sum_halves(l);
  if (q_row >= p.M) return;
  const float inv = 1.0f / l_tot;
  uint16_t* O = p.o + b * p.o_sb + h * p.o_sh + q_row * p.o_sm;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int f0 = db * 32 + 8 * g + 4 * hi;             // features f0 .. f0+3
      if (f0 < HD) {
        const bf16x2 lo = pack2<F16>(o_acc[db][4 * g + 0] * inv, o_acc[db][4 * g + 1] * inv);
        const bf16x2 up = pack2<F16>(o_acc[db][4 * g + 2] * inv, o_acc[db][4 * g + 3] * inv);
        *reinterpret_cast<u32x2*>(O + f0) =
            u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, up)};
      }
    }
  if (p.lse && hi == 0) p.lse[b * p.lse_sb + h * p.lse_sh + q_row] = m + __log2f(l_tot);
}

template <int HD, bool F16>
hipError_t launch_hd(const AnyDimArgs& a, int bias_kind, hipStream_t s) {
  const dim3 grid((unsigned)((a.M + kAQ - 1) / kAQ), (unsigned)(a.BH)), block(kAThreads);
  switch (bias_kind) {
    case GPA_BIAS_F32:
      hipLaunchKernelGGL((attn_any_dim_kernel<HD, F16, GPA_BIAS_F32>), grid, block, 0, s, a);
      break;
    case GPA_BIAS_BF16:
      hipLaunchKernelGGL((attn_any_dim_kernel<HD, F16, GPA_BIAS_BF16>), grid, block, 0, s, a);
      break;
    case GPA_BIAS_F16:
      hipLaunchKernelGGL((attn_any_dim_kernel<HD, F16, GPA_BIAS_F16>), grid, block, 0, s, a);
      break;
    default:
      hipLaunchKernelGGL((attn_any_dim_kernel<HD, F16, GPA_BIAS_NONE>), grid, block, 0, s, a);
      break;
  }
  return hipGetLastError();
}

}  // namespace

bool attn_any_dim_supported(int64_t D) { return D == 16 || D == 32 || D == 128 || D == 256; }

template <bool F16>
hipError_t attn_any_dim_launch(const AnyDimArgs& a, int64_t D, int bias_kind, hipStream_t s) {
  switch (D) {
    case 16: return launch_hd<16, F16>(a, bias_kind, s);
    case 32: return launch_hd<32, F16>(a, bias_kind, s);
    case 128: return launch_hd<128, F16>(a, bias_kind, s);
    case 256: return launch_hd<256, F16>(a, bias_kind, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t attn_any_dim_launch<false>(const AnyDimArgs&, int64_t, int, hipStream_t);
template hipError_t attn_any_dim_launch<true>(const AnyDimArgs&, int64_t, int, hipStream_t);

}  // namespace gpa
