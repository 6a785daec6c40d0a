// Flash attention with a per-key additive bias for gfx950 (CDNA4), head_dim 64.
//
//   o[m,:]  = sum_n softmax_n(q_m.k_n * sm_scale + bias_n) v_n
//   lse[m]  = log2 sum_n 2^((q_m.k_n * sm_scale + bias_n) * log2 e)
//
// Semantics follow merging/fused_attention.py:70-127: scores in the exp2
// domain, fp32 online softmax, P rounded to bf16 for the P.V product, fp32
// accumulation, log2 log-sum-exp output.  Like the reference wrapper
// (fused_attention.py:159-160), the bias is first written to a padded
// per-key buffer -- here bias/sm_scale as bf16 (hi, lo) pairs, with the keys
// past N padded to -1e30 -- by a small pre-pass.
//
// Mapping onto CDNA4
//   * A workgroup owns 256 queries of one (batch, head): 8 waves of 32
//     queries, <= 128 VGPRs each, so four waves share a SIMD and the
//     hardware overlaps one wave's MFMAs with another's softmax.
//   * K, V and the bias pairs stream through a 4-slot LDS ring of 32-key
//     tiles filled by buffer_load ... lds (DMA into LDS, no staging
//     registers) three tiles ahead of the one being computed.  Keeping
//     three tiles (24 KB) in flight per workgroup is what hides the L2/HBM
//     latency: one tile in flight capped the kernel at the latency-bound
//     rate regardless of its arithmetic.
//   * Scores are computed transposed, S^T = K . Q^T, on
//     v_mfma_f32_32x32x16_bf16: a lane owns one query and 16 of the tile's
//     32 keys (the other 16 sit in lane^32), so the running max, the sum and
//     the rescale factor are per-lane scalars; the two halves meet through
//     v_permlane32_swap.
//   * The bias rides in a fifth k-step of the score MFMA: each key's
//     (bias_hi, bias_lo) pair times a constant (1, 1) column of Q gives
//       s = q.k + bias/sm_scale,  x = s * (sm_scale*log2 e) - m
//     at no VALU cost.  Q stays unscaled: rounding q*sm_scale*log2(e) to
//     bf16 would perturb sharp logits by ~2^-9 of their size.
//   * P^T leaves the score MFMA already in the B-operand register layout of
//     the next MFMA, O^T = V^T . P^T, when the V^T A-operand enumerates keys
//     in the same order.  V stays row-major in LDS and the V^T operand is
//     read with ds_read_b64_tr_b16: within each 16-lane group, source lane
//     4v+a loads four features of key base+v and lane i receives feature
//     c0+i of keys base..base+3.  O^T keeps one query per lane, so a
//     rescale is a per-lane multiply.
//   * The running max moves lazily: only when a tile's max exceeds it by more
//     than kTau (log2 units), so P stays <= 2^kTau and the rescale (a rare,
//     wave-uniform branch) runs on a handful of tiles per row.
//   * Row sums: with the log-sum-exp requested they accumulate the fp32
//     probabilities (before their bf16 rounding), as the reference does;
//     otherwise they sum the bf16 P the P.V product uses with
//     v_dot2_f32_bf16 (exact fp32 sums of bf16 pairs, half the VALU work),
//     normalising O by exactly the weights it was built from.
//   * LDS layouts are XOR-swizzled in 16-byte chunks so that the fragment
//     reads are free of bank conflicts under both 32- and 64-bank models;
//     the DMA lanes pick their global chunk so the swizzle costs nothing.
#include "gpa_common.h"

#include <math.h>

namespace gpa {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kQPerWG = kWaves * 32;          // 256 queries per workgroup
constexpr int kKT = 32;                       // keys per tile
constexpr int kHD = 64;                       // head dim
constexpr int kRing = 4;                      // LDS tile slots
constexpr int kAhead = kRing - 1;             // tiles in flight beyond the current one
constexpr float kTau = 8.0f;                  // lazy rescale threshold (log2)
constexpr float kPadBias = -1.0e30f;          // bias of keys past N
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint32_t* pairs;  // [rows][npad] bias pairs
  uint16_t* o;
  float* lse;
  int H;
  int64_t M, N;
  int64_t q_sb, q_sh, q_sm, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sm;
  int64_t pairs_sb, pairs_sh, lse_sb, lse_sh;
  uint32_t k_bytes, v_bytes, pair_bytes;  // extent of one (batch, head) slice
  float c;                                // sm_scale * log2(e)
};

struct PairArgs {
  const void* bias;
  uint32_t* pairs;
  int kind;
  int rows_h;  // heads with their own pair row (1 or H)
  int64_t sb, sh, sn;
  int64_t N, npad, total;
  float mul;  // 1 / sm_scale
};

// One slot of the tile ring.
struct alignas(16) Tile {
  uint16_t k[kKT * kHD];  // key rows, 16-byte chunks swizzled by k_chunk
  uint16_t v[kKT * kHD];  // value rows, 16-byte chunks swizzled by v_chunk
  uint32_t bias[kKT];     // (bias_hi | bias_lo << 16) per key
};

// K chunk swizzle: 16 consecutive keys reading one logical chunk hit 16
// distinct 16-byte bank groups (64 banks); any 8 consecutive keys hit 8
// (32 banks).
__device__ __forceinline__ int k_chunk(int key, int ch) {
  return ch ^ (key & 7) ^ ((key >> 3) & 1);
}

// V chunk swizzle for the transpose reads: the four keys of a 16-lane group
// and the two 8-byte halves of its chunks land in distinct banks.
__device__ __forceinline__ int v_chunk(int key, int ch) { return ch ^ ((key & 3) << 1); }

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

__device__ __forceinline__ uint32_t bias_pair(float x) {
  const __bf16 bhi = (__bf16)x;
  const __bf16 blo = (__bf16)(x - (float)bhi);
  return (uint32_t)__builtin_bit_cast(uint16_t, bhi) |
         ((uint32_t)__builtin_bit_cast(uint16_t, blo) << 16);
}

// DMA of 16 bytes per lane into LDS at lds + 16*lane.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff,
                                      uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// Wait until at most N vector-memory instructions of this wave are in flight
// (lgkm and export counters untouched).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__global__ __launch_bounds__(256) void bias_pairs_kernel(PairArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int64_t n = i % a.npad, row = i / a.npad;
  const int64_t hb = row % a.rows_h, bb = row / a.rows_h;
  float x = kPadBias;
  if (n < a.N) {
    const int64_t off = bb * a.sb + hb * a.sh + n * a.sn;
    if (a.kind == GPA_BIAS_F32)
      x = static_cast<const float*>(a.bias)[off] * a.mul;
    else if (a.kind == GPA_BIAS_BF16)
      x = bf16_bits_to_f32(static_cast<const uint16_t*>(a.bias)[off]) * a.mul;
    else
      x = 0.f;
  }
  a.pairs[i] = bias_pair(x);
}

// Workgroup barrier that does not drain the vector-memory counter: the
// in-flight DMAs of later tiles must stay in flight across it (the explicit
// wait_vm before it covers the tile that has to be complete).  The memory
// clobber keeps the compiler from moving LDS accesses across it, and
// lgkmcnt(0) retires this wave's LDS reads before any slot is refilled.
__device__ __forceinline__ void tile_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <bool LSE>
__global__ __launch_bounds__(kThreads, 4) void attn_keybias_kernel(AttnArgs p) {
  // Four separate LDS objects (not one array) so the compiler's LDS-DMA
  // tracking can tell which slot a DMA writes and which a read reads.
  __shared__ Tile ring0, ring1, ring2, ring3;

  const int tid = threadIdx.x;
  const int lane = tid & 63, hi = lane >> 5, l32 = lane & 31;
  // Wave index in an SGPR: the DMA's LDS base (M0) must be wave-uniform.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.y;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int64_t q_row = (int64_t)blockIdx.x * kQPerWG + wave * 32 + l32;
  const float c = p.c;

  const uint16_t* Q = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* K = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* V = p.v + b * p.v_sb + h * p.v_sh;
  const uint32_t* P = p.pairs + b * p.pairs_sb + h * p.pairs_sh;

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

  // DMA roles: waves 0-3 copy K (1 KB each), waves 4-7 copy V, lanes 0-7 of
  // wave 0 copy the 128 bytes of bias pairs.  Each lane fetches the global
  // chunk that belongs in its LDS slot under the swizzle.
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(K, p.k_bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(V, p.v_bytes);
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(P, p.pair_bytes);
  const uint32_t k_row = (uint32_t)p.k_sn * 2u, v_row = (uint32_t)p.v_sn * 2u;
  const int slot = (wave & 3) * 64 + lane;  // 16-byte slot within the K or V tile
  const int s_key = slot >> 3, s_pc = slot & 7;
  const uint32_t k_voff = s_key * k_row + k_chunk(s_key, s_pc) * 16;
  const uint32_t v_voff = s_key * v_row + v_chunk(s_key, s_pc) * 16;
  const bool k_wave = wave < 4;
  const int ntiles = (int)((p.N + kKT - 1) / kKT);

  auto issue = [&](int t, Tile& T) {
    const uint32_t n0 = (uint32_t)t * kKT;
    if (k_wave)
      dma16(krs, &T.k[(wave & 3) * 512], k_voff, n0 * k_row);
    else
      dma16(vrs, &T.v[(wave & 3) * 512], v_voff, n0 * v_row);
    if (wave == 0 && lane < 8) dma16(prs, &T.bias[0], lane * 16, n0 * 4);
  };

  // Per-lane LDS element offsets of the fragment reads (slot-independent).
  int k_off[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) k_off[ks] = l32 * kHD + (k_chunk(l32, 2 * ks + hi) << 3);
  // V^T transpose reads: block db (features 32db..), k-step s, part pp
  // (keys 16s + 8pp + 4hi + 0..3).  Within its 16-lane group this lane is
  // the source of key offset (lane&15)>>2 and feature quad lane&3.
  int v_off[2][2][2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const int key = 16 * s + 8 * pp + 4 * hi + ((lane & 15) >> 2);
        const int a = lane & 3;
        const int ch = db * 4 + ((lane >> 4) & 1) * 2 + (a >> 1);
        v_off[db][s][pp] = key * kHD + (v_chunk(key, ch) << 3) + (a & 1) * 4;
      }

  float m_run = -INFINITY;  // running max in log2 units (moved lazily)
  float l_run = 0.f;        // this lane's share of the row sum
  f32x16 o_acc[2] = {f32x16{}, f32x16{}};
  const bf16x2 ones2 = {(__bf16)1.0f, (__bf16)1.0f};

  // One tile: fetch tile t+3 into the slot tile t-1 used, compute tile t,
  // wait until tile t+1 has landed, synchronise.
  auto step = [&](const int t, const Tile& T, Tile& Tfree) {
    issue(t + kAhead, Tfree);

    // Scores s = q.k + bias/sm_scale (rows 8g + 4hi + j of the 32x32 result).
    f32x16 sv = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      sv = mfma32x32x16(*reinterpret_cast<const bf16x8*>(&T.k[k_off[ks]]), qf[ks], sv);
    {
      const uint32_t pair = T.bias[l32];
      const u32x4 kb = {hi == 0 ? pair : 0u, 0u, 0u, 0u};
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
        const bf16x2 pv = {(__bf16)p0, (__bf16)p1};
        pb[half][e] = pv[0];
        pb[half][e + 1] = pv[1];
        if (LSE)
          lsum = (half == 0 && e == 0) ? p0 + p1 : lsum + (p0 + p1);
        else
          lsum = __builtin_amdgcn_fdot2_f32_bf16(pv, ones2, lsum, false);
      }
    }
    l_run += lsum;

    // O^T += V^T . P^T; the V^T operand of k-step s covers the keys whose
    // probabilities this lane holds in its score registers 8s..8s+7.
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        typedef short i16x4 __attribute__((ext_vector_type(4)));
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)&T.v[v_off[db][s][0]]);
        const i16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)&T.v[v_off[db][s][1]]);
        const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo), u4 = __builtin_bit_cast(bf16x4, up);
        const bf16x8 vf = {l4[0], l4[1], l4[2], l4[3], u4[0], u4[1], u4[2], u4[3]};
        o_acc[db] = mfma32x32x16(vf, pb[s], o_acc[db]);
      }

    // Tile t+1 has landed once only tiles t+2 and t+3 are outstanding: two
    // DMA instructions per tile on wave 0, one on the others.
    if (wave == 0)
      wait_vm<2 * (kAhead - 1)>();
    else
      wait_vm<kAhead - 1>();
    tile_barrier();
  };

  // Prologue: tiles 0..2 in flight; wait for tile 0.
  issue(0, ring0);
  issue(1, ring1);
  issue(2, ring2);
  if (wave == 0)
    wait_vm<2 * (kAhead - 1)>();
  else
    wait_vm<kAhead - 1>();
  tile_barrier();

  // Four steps per trip so every slot is a compile-time LDS object.
  int t = 0;
  for (; t + 4 <= ntiles; t += 4) {
    step(t, ring0, ring3);
    step(t + 1, ring1, ring0);
    step(t + 2, ring2, ring1);
    step(t + 3, ring3, ring2);
  }
  if (t < ntiles) step(t++, ring0, ring3);
  if (t < ntiles) step(t++, ring1, ring0);
  if (t < ntiles) step(t++, ring2, ring1);
  // Drain the DMAs still in flight before the workgroup can exit.
  wait_vm<0>();

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

// Pair-buffer geometry: one row per (batch, head) that has its own bias.
struct PairPlan {
  int64_t rows_b, rows_h, npad;
  size_t bytes;
};

PairPlan pair_plan(int64_t B, int64_t H, int64_t N, int bias_kind, int64_t bias_sb,
                   int64_t bias_sh) {
  PairPlan pl;
  const bool none = bias_kind == GPA_BIAS_NONE;
  pl.rows_b = (none || bias_sb == 0) ? 1 : B;
  pl.rows_h = (none || bias_sh == 0) ? 1 : H;
  pl.npad = (N + kKT - 1) / kKT * kKT;
  pl.bytes = (size_t)(pl.rows_b * pl.rows_h * pl.npad) * sizeof(uint32_t);
  return pl;
}

}  // namespace
}  // namespace gpa

using namespace gpa;

extern "C" size_t gpa_attn_keybias_workspace_bytes(int64_t B, int64_t H, int64_t N, int bias_kind,
                                                   int64_t bias_sb, int64_t bias_sh) {
  if (B <= 0 || H <= 0 || N <= 0) return 0;
  return pair_plan(B, H, N, bias_kind, bias_sb, bias_sh).bytes;
}

extern "C" int gpa_attn_keybias_bf16(const void* q, const void* k, const void* v, const void* bias,
                                     int bias_kind, int64_t bias_sb, int64_t bias_sh,
                                     int64_t bias_sn, void* o, float* lse, int64_t B, int64_t H,
                                     int64_t M, int64_t N, int64_t D, int64_t q_sb, int64_t q_sh,
                                     int64_t q_sm, int64_t k_sb, int64_t k_sh, int64_t k_sn,
                                     int64_t v_sb, int64_t v_sh, int64_t v_sn, int64_t o_sb,
                                     int64_t o_sh, int64_t o_sm, int64_t lse_sb, int64_t lse_sh,
                                     void* workspace, size_t workspace_bytes, float sm_scale,
                                     void* stream) {
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
                       ((uintptr_t)v % 16 == 0) && ((uintptr_t)o % 8 == 0) && q_sm % 8 == 0 &&
                       q_sb % 8 == 0 && q_sh % 8 == 0 && k_sn % 8 == 0 && k_sb % 8 == 0 &&
                       k_sh % 8 == 0 && v_sn % 8 == 0 && v_sb % 8 == 0 && v_sh % 8 == 0 &&
                       o_sm % 4 == 0 && o_sb % 4 == 0 && o_sh % 4 == 0;
  if (!aligned || q_sm < D || k_sn < D || v_sn < D || o_sm < D) {
    gpa_set_error("gpa_attn_keybias_bf16: rows must have unit feature stride, q/k/v rows "
                  "16-byte and o rows 8-byte aligned");
    return GPA_E_INVALID;
  }
  if (B * H > 65535) {
    gpa_set_error("gpa_attn_keybias_bf16: B*H=%lld exceeds the grid limit", (long long)(B * H));
    return GPA_E_UNSUPPORTED;
  }
  const int64_t gx = (M + kQPerWG - 1) / kQPerWG;
  // Buffer offsets are 32-bit: one (batch, head) slice of K and V, plus the
  // tiles fetched past its end, must stay below 2^31 bytes.
  const int64_t span = N + (kAhead + 1) * kKT;
  if (gx > 0x7fffffff || span * k_sn * 2 >= ((int64_t)1 << 31) ||
      span * v_sn * 2 >= ((int64_t)1 << 31)) {
    gpa_set_error("gpa_attn_keybias_bf16: one head's K/V slice exceeds 2 GiB");
    return GPA_E_UNSUPPORTED;
  }
  const PairPlan pl = pair_plan(B, H, N, bias_kind, bias_sb, bias_sh);
  if (!workspace || workspace_bytes < pl.bytes || (uintptr_t)workspace % 16) {
    gpa_set_error("gpa_attn_keybias_bf16: 16-byte aligned workspace of %zu bytes required, %zu "
                  "given",
                  pl.bytes, workspace ? workspace_bytes : (size_t)0);
    return GPA_E_WORKSPACE;
  }
  hipStream_t s = (hipStream_t)stream;

  PairArgs pa{};
  pa.bias = bias;
  pa.pairs = (uint32_t*)workspace;
  pa.kind = bias_kind;
  pa.rows_h = (int)pl.rows_h;
  pa.sb = bias_sb;
  pa.sh = bias_sh;
  pa.sn = bias_sn;
  pa.N = N;
  pa.npad = pl.npad;
  pa.total = pl.rows_b * pl.rows_h * pl.npad;
  pa.mul = 1.0f / sm_scale;
  hipLaunchKernelGGL(bias_pairs_kernel, dim3((unsigned)((pa.total + 255) / 256)), dim3(256), 0, s,
                     pa);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("gpa_attn_keybias_bf16: bias pre-pass launch failed: %s", hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }

  AttnArgs p{};
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.pairs = (const uint32_t*)workspace;
  p.o = (uint16_t*)o;
  p.lse = lse;
  p.H = (int)H;
  p.M = M;
  p.N = N;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_sm = q_sm;
  p.k_sb = k_sb; p.k_sh = k_sh; p.k_sn = k_sn;
  p.v_sb = v_sb; p.v_sh = v_sh; p.v_sn = v_sn;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_sm = o_sm;
  p.pairs_sb = pl.rows_b > 1 ? pl.rows_h * pl.npad : 0;
  p.pairs_sh = pl.rows_h > 1 ? pl.npad : 0;
  p.lse_sb = lse_sb; p.lse_sh = lse_sh;
  p.k_bytes = (uint32_t)(((N - 1) * k_sn + D) * 2);
  p.v_bytes = (uint32_t)(((N - 1) * v_sn + D) * 2);
  p.pair_bytes = (uint32_t)(pl.npad * sizeof(uint32_t));
  p.c = sm_scale * kLog2e;

  const dim3 grid((unsigned)gx, (unsigned)(B * H)), block(kThreads);
  if (lse)
    hipLaunchKernelGGL(attn_keybias_kernel<true>, grid, block, 0, s, p);
  else
    hipLaunchKernelGGL(attn_keybias_kernel<false>, grid, block, 0, s, p);
  e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("gpa_attn_keybias_bf16: launch failed: %s", hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}
