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

// ---------------------------------------------------------------------------
// Head dims 128 and 256: the tiled kernel.
//
// The running-max kernel above rescales every lane's HD/2 output registers
// on every tile, transposes V into LDS with 2-byte stores and computes a
// tile's scores, softmax and P.V product one after the other.  This kernel
// keeps its layout (one 32-query block per wave, scores transposed, P^T used
// in place as the B operand) and removes those three costs:
//   * A lazily moved offset: m starts at tile 0's exact row max and moves to
//     a tile's row max only when that exceeds m + kLazyUp (64 log2 units for
//     bf16 P, which has fp32's exponent range; 15 for fp16 P, below 65504),
//     in a wave-uniform branch.  Every P stays <= 2^kLazyUp and each row's
//     largest P >= 1, the row sums (fp32, of the fp32 P, as the reference)
//     and O stay far inside fp32, and the softmax is the same; after the
//     first tiles of a row the branch is rarely taken.
//   * K, V and the bias stream through a four-slot LDS ring filled by
//     buffer_load ... lds (DMA, no staging registers), three tiles ahead.
//     K rows are stored with their 16-byte chunks XOR-swizzled by key & 15
//     (a 16-lane pass of fragment reads hits 16 distinct chunks), V rows
//     row-major with chunks swizzled by (key & 3) << 2, and the V^T operand
//     is read with ds_read_b64_tr_b16 (a 32-lane pass covers all 64 banks
//     once).  The DMA lanes pick the global chunk their LDS position holds,
//     so the swizzle costs nothing; rows past N read zeros by range.
//   * Software pipelining by one tile: iteration t computes S(t+1) on the
//     matrix pipe beside the softmax of S(t) on the VALU, then O += V(t)^T .
//     P(t)^T.
// The bias comes from a pre-pass (bias_rows_kernel): per (batch, head) one
// fp32 row of bias / sm_scale over the keys rounded up to whole tiles, -inf
// past N, in the workspace.  Workgroups are renumbered XCD-aware so the query
// blocks of one (batch, head) share an XCD's L2 for their K/V stream.

template <bool F16> constexpr float kLazyUp = F16 ? 15.0f : 64.0f;
constexpr int kLSlots = 4;                    // ring slots: tiles t .. t+3

template <int KIND>
__global__ __launch_bounds__(256) void bias_rows_kernel(const void* bias, float* rows, int H,
                                                        int64_t N, int64_t npad, int64_t sb,
                                                        int64_t sh, int64_t sn, float mul) {
  const int64_t bh = blockIdx.y;
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= npad) return;
  float x = -INFINITY;
  if (n < N) {
    if constexpr (KIND == GPA_BIAS_NONE) x = 0.f;
    else x = any_bias<KIND>(bias, (bh / H) * sb + (bh % H) * sh + n * sn) * mul;
  }
  rows[bh * npad + n] = x;
}

// DMA of 4 / 16 bytes per lane into LDS at lds + 4 * lane / lds + 16 * lane.
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff,
                                         uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds, 4, voff, soff, 0, 0);
}
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff,
                                          uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}
// Wait until at most N vector-memory instructions of this wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One ring slot: a tile's K and V rows (swizzled as above) and its bias
// words (64 words: the DMA of one wave writes 4 bytes per lane).
template <int HD>
struct TiledSlot {
  uint16_t k[kAKT * HD];
  uint16_t v[kAKT * HD];
  float b[64];
};

template <int HD, bool F16>
__global__ __launch_bounds__(kAThreads, HD >= 256 ? 1 : 2) void attn_tiled_kernel(AnyDimArgs p) {
  constexpr int KS = HD / 16;                 // k-steps of the score product
  constexpr int DB = HD / 32;                 // 32-feature blocks of O
  constexpr int CH = HD / 8;                  // 16-byte chunks per key row
  constexpr int DJ = kAKT * CH / kAThreads;   // 16-byte DMAs per wave, tile and tensor
  constexpr int OPS = 2 * DJ + 1;             // DMA instructions per wave and tile
  static_assert(kAKT * CH % kAThreads == 0, "whole DMA instructions per wave");
  static_assert(kLSlots == 4, "the loop below is unrolled over four slots");
  // Four statically named slots: the compiler then knows which in-flight DMA
  // each LDS read may depend on (with one array and a runtime slot index it
  // waits for every DMA before every read).
  __shared__ __attribute__((aligned(16))) TiledSlot<HD> r0, r1, r2, r3;
  __shared__ __attribute__((aligned(16))) float b_sink[64];

  const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int qb, bhi;
  {
    const uint32_t T = gridDim.x * gridDim.y, L = blockIdx.y * gridDim.x + blockIdx.x;
    const uint32_t q8 = T / 8, r8 = T % 8, x = L % 8;
    const uint32_t item = x * q8 + (x < r8 ? x : r8) + L / 8;
    qb = (int)(item % gridDim.x);
    bhi = (int)(item / gridDim.x);
  }
  const int64_t bh = bhi, b = bh / p.H, h = bh % p.H;
  const int64_t q_row = (int64_t)qb * kAQ + wave * 32 + l32;
  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* V = p.v + b * p.v_sb + h * p.v_sh;
  const int ntiles = (int)((p.N + kAKT - 1) / kAKT);
  const float* Brow = p.ws + bh * (int64_t)ntiles * kAKT;
  const float c = p.c;

  bf16x8 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qf[ks] = q_row < p.M ? *reinterpret_cast<const bf16x8*>(Q + q_row * p.q_sm + 16 * ks + 8 * hi)
                         : bf16x8{};
  __builtin_amdgcn_sched_barrier(0);

  const uint32_t k_row = (uint32_t)p.k_sn * 2u, v_row = (uint32_t)p.v_sn * 2u;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(K, (uint32_t)((p.N - 1) * p.k_sn * 2 + HD * 2));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, (uint32_t)((p.N - 1) * p.v_sn * 2 + HD * 2));
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(Brow, (uint32_t)ntiles * kAKT * 4u);
  // LDS chunk position (wave DJ + j) 64 + lane holds key pos / CH, physical
  // chunk pos % CH, i.e. the logical chunk that the XOR swizzle maps there.
  uint32_t k_voff[DJ], v_voff[DJ];
#pragma unroll
  for (int j = 0; j < DJ; ++j) {
    const int pos = (wave * DJ + j) * 64 + lane;
    const int key = pos / CH, pch = pos % CH;
    k_voff[j] = key * k_row + (uint32_t)((pch ^ (key & 15)) * 16);
    v_voff[j] = key * v_row + (uint32_t)((pch ^ ((key & 3) << 2)) * 16);
  }
  // Wave 0's first 32 lanes fetch the tile's 32 bias words; the other lanes
  // point past the descriptor's range and land zeros (waves 1-3 into a sink,
  // so that every wave issues the same DMAs and waits).
  const uint32_t b_voff = (wave == 0 && lane < kAKT) ? (uint32_t)lane * 4u : 0x40000000u;
  auto issue = [&](int t, TiledSlot<HD>& S) {
    const uint32_t n0 = (uint32_t)t * kAKT;
#pragma unroll
    for (int j = 0; j < DJ; ++j) lds_dma16(krs, &S.k[(wave * DJ + j) * 512], k_voff[j], n0 * k_row);
#pragma unroll
    for (int j = 0; j < DJ; ++j) lds_dma16(vrs, &S.v[(wave * DJ + j) * 512], v_voff[j], n0 * v_row);
    float* dst = wave == 0 ? &S.b[0] : &b_sink[0];
    lds_dma4(brs, dst, b_voff, n0 * 4u);
  };

  int k_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) k_off[ks] = l32 * HD + (((2 * ks + hi) ^ (l32 & 15)) << 3);
  // V^T operand: lane (hi, bit 4, v = (lane & 15) >> 2, a = lane & 3) points
  // at key 4 hi + v (+ 16 s + 8 e), features 32 db + 16 bit4 + 4 a .. +3;
  // ds_read_b64_tr_b16 then hands lane l feature 32 db + l % 32 of keys
  // 16 s + 8 e + 4 hi .. +3, the key order of the score MFMA's registers.
  int v_off[DB];
  {
    const int v4 = (lane & 15) >> 2, a = lane & 3, bit4 = (lane >> 4) & 1;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int lc = 4 * db + 2 * bit4 + (a >> 1);
      v_off[db] = (4 * hi + v4) * HD + ((lc ^ (v4 << 2)) << 3) + (a & 1) * 4;
    }
  }

  auto scores = [&](const TiledSlot<HD>& S) {
    f32x16 sv;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(&S.b[8 * g + 4 * hi]);
      sv[4 * g + 0] = bv[0];
      sv[4 * g + 1] = bv[1];
      sv[4 * g + 2] = bv[2];
      sv[4 * g + 3] = bv[3];
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&S.k[k_off[ks]]);
      sv = mfma32x32x16_t<F16>(kf, qf[ks], sv);
    }
    return sv;
  };
  auto row_max = [&](const f32x16& x) {
    float mx = fmaxf(fmaxf(x[0], x[1]), x[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, x[r]), x[r + 1]);
    mx = fmaxf(mx, x[15]);
    return max_halves(mx) * c;
  };

  f32x16 o_acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o_acc[db] = f32x16{};
  float l = 0.f;

  issue(0, r0);
  issue(1, r1);
  issue(2, r2);
  wait_vmem<2 * OPS>();
  __syncthreads();
  f32x16 s_cur = scores(r0);
  float m = fmaxf(row_max(s_cur), -1.0e30f);  // finite: a tile of -inf biases scores 0

  // Iteration t: tile t in `cur`, tile t+1 in `nxt`, tile t+3 issued into
  // `dst` (the slot of tile t-1, free once every wave passed the barrier).
  auto iter = [&](int t, const TiledSlot<HD>& cur, const TiledSlot<HD>& nxt,
                  TiledSlot<HD>& dst) {
    wait_vmem<OPS>();                         // tile t+1 landed (tile t+2 in flight)
    __syncthreads();                          // ... for every wave
    issue(t + 3, dst);
    const f32x16 s_nxt = scores(nxt);
    // The V^T fragments of tile t, all read before the softmax (read after
    // it, their LDS latency sat between the softmax and the P.V product:
    // head dim 256 45.2 -> 35.6 ms, 128 32.5 -> 31.5 ms, same box).
    bf16x8 vf[DB][2];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        typedef short i16x4 __attribute__((ext_vector_type(4)));
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)&cur.v[v_off[db] + 16 * s * HD]);
        const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)&cur.v[v_off[db] + (16 * s + 8) * HD]);
        const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo), u4 = __builtin_bit_cast(bf16x4, up);
        vf[db][s] = bf16x8{l4[0], l4[1], l4[2], l4[3], u4[0], u4[1], u4[2], u4[3]};
      }
    // Softmax of S(t): move the offset only where the row max left the window.
    const float mx = row_max(s_cur);
    const bool move = mx > m + kLazyUp<F16>;
    if (__builtin_amdgcn_ballot_w64(move)) {
      const float m_new = move ? mx : m;
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o_acc[db] *= alpha;
    }
    bf16x8 pb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[8 * s + e], c, -m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[8 * s + e + 1], c, -m));
        l += p0 + p1;
        const bf16x2 pv2 = pack2<F16>(p0, p1);
        pb[s][e] = pv2[0];
        pb[s][e + 1] = pv2[1];
      }
    // O^T += V^T . P^T
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) o_acc[db] = mfma32x32x16_t<F16>(vf[db][s], pb[s], o_acc[db]);
    s_cur = s_nxt;
  };
  for (int t = 0; t < ntiles; t += 4) {
    iter(t, r0, r1, r3);
    if (t + 1 >= ntiles) break;
    iter(t + 1, r1, r2, r0);
    if (t + 2 >= ntiles) break;
    iter(t + 2, r2, r3, r1);
    if (t + 3 >= ntiles) break;
    iter(t + 3, r3, r0, r2);
  }
  wait_vmem<0>();                             // no DMA may land after the workgroup ends

  const float l_tot = sum_halves(l);
  if (q_row >= p.M) return;
  const float inv = 1.0f / l_tot;
  uint16_t* O = p.o + b * p.o_sb + h * p.o_sh + q_row * p.o_sm;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int f0 = db * 32 + 8 * g + 4 * hi;
      const bf16x2 lo = pack2<F16>(o_acc[db][4 * g + 0] * inv, o_acc[db][4 * g + 1] * inv);
      const bf16x2 up = pack2<F16>(o_acc[db][4 * g + 2] * inv, o_acc[db][4 * g + 3] * inv);
      *reinterpret_cast<u32x2*>(O + f0) =
          u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, up)};
    }
  if (p.lse && hi == 0) p.lse[b * p.lse_sb + h * p.lse_sh + q_row] = m + __log2f(l_tot);
}

template <int HD, bool F16>
hipError_t launch_tiled(const AnyDimArgs& a, int bias_kind, hipStream_t s) {
  const int64_t ntiles = (a.N + kAKT - 1) / kAKT, npad = ntiles * kAKT;
  const dim3 bgrid((unsigned)((npad + 255) / 256), (unsigned)a.BH), bblock(256);
  switch (bias_kind) {
    case GPA_BIAS_F32:
      hipLaunchKernelGGL((bias_rows_kernel<GPA_BIAS_F32>), bgrid, bblock, 0, s, a.bias, a.ws, a.H,
                         a.N, npad, a.bias_sb, a.bias_sh, a.bias_sn, a.mul);
      break;
    case GPA_BIAS_BF16:
      hipLaunchKernelGGL((bias_rows_kernel<GPA_BIAS_BF16>), bgrid, bblock, 0, s, a.bias, a.ws, a.H,
                         a.N, npad, a.bias_sb, a.bias_sh, a.bias_sn, a.mul);
      break;
    case GPA_BIAS_F16:
      hipLaunchKernelGGL((bias_rows_kernel<GPA_BIAS_F16>), bgrid, bblock, 0, s, a.bias, a.ws, a.H,
                         a.N, npad, a.bias_sb, a.bias_sh, a.bias_sn, a.mul);
      break;
    default:
      hipLaunchKernelGGL((bias_rows_kernel<GPA_BIAS_NONE>), bgrid, bblock, 0, s, a.bias, a.ws,
                         a.H, a.N, npad, a.bias_sb, a.bias_sh, a.bias_sn, a.mul);
      break;
  }
  const dim3 grid((unsigned)((a.M + kAQ - 1) / kAQ), (unsigned)(a.BH)), block(kAThreads);
  hipLaunchKernelGGL((attn_tiled_kernel<HD, F16>), grid, block, 0, s, a);
  return hipGetLastError();
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

size_t attn_any_dim_ws_bytes(int64_t BH, int64_t N, int64_t D) {
  if (D != 128 && D != 256) return 0;
  return (size_t)(BH * ((N + kAKT - 1) / kAKT) * kAKT) * sizeof(float);
}

template <bool F16>
hipError_t attn_any_dim_launch(const AnyDimArgs& a, int64_t D, int bias_kind, hipStream_t s) {
  switch (D) {
    case 16: return launch_hd<16, F16>(a, bias_kind, s);
    case 32: return launch_hd<32, F16>(a, bias_kind, s);
    case 128: return launch_tiled<128, F16>(a, bias_kind, s);
    case 256: return launch_tiled<256, F16>(a, bias_kind, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t attn_any_dim_launch<false>(const AnyDimArgs&, int64_t, int, hipStream_t);
template hipError_t attn_any_dim_launch<true>(const AnyDimArgs&, int64_t, int, hipStream_t);

}  // namespace gpa
