// Fused similarity row max / argmax for gfx950 (CDNA4).
//
// Computes, for every source row m of a[B, M, D] against every destination
// row n of b[B, N, D]:
//     out_max[m] = max_n <a_m, b_n>        (bf16 or fp16 inputs, fp32 accumulate)
//     out_idx[m] = lowest n attaining it
// without materialising the M x N score matrix.  Semantics follow the
// reference Triton kernel merging/fused_similarity.py:33-78 (fp32 scores,
// strict `>` across tiles at :73, first index inside a tile via tl.argmax).
//
// Work decomposition
//   * A workgroup owns 256 source rows (4 waves x 4 blocks of 16; 128 rows
//     above D=128) and one contiguous destination range ("split").  Source
//     rows stay in VGPRs as MFMA B-operands for the whole kernel; destination
//     rows stream through LDS in double-buffered stages of 64 rows.
//   * Each 16x16 score tile is S^T = Dst(16xD) . Src^T(Dx16) on
//     v_mfma_f32_16x16x32_bf16 (_f16 in the fp16 instantiation), so a lane holds one source row against 4
//     destination rows and the running max/argmax is lane-local: one
//     compare and two selects per score, no cross-lane traffic until the
//     very end.  (The 16x16 shape keeps 16 tracking slots per source row,
//     half of what the 32x32 shape needs, at the same MFMA rate.)
//   * Splits are mapped onto XCDs (workgroup id mod 8 selects the XCD), so
//     all workgroups on one XCD read the same destination range and that
//     range stays resident in the XCD's L2.  Partial (max, idx) pairs per
//     split are merged by a second tiny kernel with the same tie rule.
//   * Above D = 256 (the unprojected 1024-d metric) source rows no longer fit
//     in VGPRs; sim_argmax_gemm_kernel tiles 128 x 128 with both operands in
//     LDS and loops over the features (see there).
#include "gpa_common.h"

#include <math.h>

#include <mutex>
#include <type_traits>

namespace gpa {
namespace {

constexpr int kWaves = 4;
constexpr int kTN = 64;  // destination rows per LDS stage

// 16-row source blocks held per wave (ks = D/32): four up to D=128, two
// above, which keeps the kernel within the VGPR budget of two waves/SIMD.
__host__ __device__ constexpr int src_blocks(int ks) { return ks <= 4 ? 4 : 2; }
__host__ __device__ constexpr int rows_per_wg(int ks) { return kWaves * src_blocks(ks) * 16; }

// Wait until at most N vector-memory instructions of this wave are in flight
// (lgkm and export counters untouched).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

struct SimArgs {
  const uint16_t* a;
  const uint16_t* b;
  void* out_max;       // final outputs (splits == 1 or the merge): max_dtype elements
  int max_dtype;
  int64_t* out_idx;
  uint64_t* part;      // [B][M][splits] partial keys (splits > 1), see part_key
  int64_t M, N;
  int64_t a_sb, a_sm, b_sb, b_sn, omax_sb, oidx_sb;
  int splits;          // destination splits (1, 2, 4, 8 or a multiple of 8)
  int mblocks;         // source row blocks, padded to the mapping granularity
  int64_t n_chunk;     // destination rows per split (multiple of kTN)
  int wide_tiles;      // D >= 512: destination tiles of kWN rows; split s
                       // covers tiles [s * wide_tiles / splits, (s + 1) * ...)
  // The last round's items, cut finer (D = 128, B = 1): the source blocks
  // from tail_mb0 on give each of their splits to tail_sub workgroups of
  // sub_chunk destination rows each, dispatched after the tail_item0 whole
  // items, with partials [splits][tail_sub][tail_rows].  tail_sub = 0: none.
  int tail_item0;
  int tail_sub;
  int tail_mb0;
  int64_t tail_rows;
  int64_t sub_chunk;
  uint64_t* tail;
};

// A split's (max, index) as one 64-bit key whose unsigned order is the merge
// order: a larger max wins, equal maxima go to the lower index (the split
// order of the reference's strict `>`).  High word: the max's bits mapped to
// unsigned order (-0 taken as +0, so the two compare equal); low word:
// (0x7fffffff - idx) << 1, plus the sign of a zero max in bit 0, so the
// value reported is the winning split's own.  Partials are never NaN (the
// running max starts at -inf and NaN scores never win).
__device__ __forceinline__ uint64_t part_key(float v, int idx) {
  const uint32_t b = __float_as_uint(v);
  const bool zero = (b & 0x7fffffffu) == 0;
  const uint32_t c = zero ? 0u : b;
  const uint32_t hi = (c & 0x80000000u) ? ~c : (c | 0x80000000u);
  const uint32_t lo = ((0x7fffffffu - (uint32_t)idx) << 1) | (zero ? (b >> 31) : 0u);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ void key_part(uint64_t k, float& v, int& idx) {
  const uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
  const uint32_t c = (hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi;
  v = __uint_as_float(c | ((lo & 1u) << 31));
  idx = (int)(0x7fffffffu - (lo >> 1));
}

// The row max in the caller's element type (fp32, or bf16 / fp16 rounded
// to nearest even, as torch's cast does).
__device__ __forceinline__ void store_max(const SimArgs& p, int64_t o, float v) {
  if (p.max_dtype == GPA_DTYPE_BF16)
    static_cast<__bf16*>(p.out_max)[o] = (__bf16)v;
  else if (p.max_dtype == GPA_DTYPE_F16)
    static_cast<_Float16*>(p.out_max)[o] = (_Float16)v;
  else
    static_cast<float*>(p.out_max)[o] = v;
}

// Workgroup id -> (source block, split).  Workgroups are dispatched to the
// eight XCDs round-robin, so `bid & 7` is the XCD; every XCD is given whole
// splits so that its L2 only ever holds one destination range.
__device__ __forceinline__ void map_block(const SimArgs& p, int bid, int& mblock, int& split) {
  if (p.splits == 1) {
    mblock = bid;
    split = 0;
    return;
  }
  const int x = bid & 7, y = bid >> 3;
  if (p.splits <= 8) {
    const int g = 8 / p.splits;  // XCDs sharing one split
    split = x / g;
    mblock = y * g + (x % g);
  } else {
    const int k = p.splits / 8;  // splits per XCD
    split = x * k + (y % k);
    mblock = y / k;
  }
}

// Workgroup id -> (source block, split, sub-range): sub = -1 for a whole
// split; the tail items keep the XCD of their split (bid & 7, as above).
__device__ __forceinline__ void map_item(const SimArgs& p, int bid, int& mblock, int& split,
                                         int& sub) {
  if (p.tail_sub > 0 && bid >= p.tail_item0) {
    const int t = bid - p.tail_item0, x = t & 7, y = t >> 3;
    const int k = p.splits / 8;  // splits per XCD
    sub = y % p.tail_sub;
    const int rest = y / p.tail_sub;
    split = x * k + rest % k;
    mblock = p.tail_mb0 + rest / k;
    return;
  }
  map_block(p, bid, mblock, split);
  sub = -1;
}

template <int KS, bool F16>
__global__ __launch_bounds__(256, 2) void sim_argmax_kernel(SimArgs p) {
  constexpr int kSB = src_blocks(KS);
  constexpr int kRowsPerWG = rows_per_wg(KS);
  constexpr int D = KS * 32;
  constexpr int NCH = D / 8;  // 16-byte chunks per row
  // XOR swizzle of the chunk index by the row, kept inside the row: the mask
  // is the largest power of two (<= 16) dividing the chunk count.
  constexpr int SWZ = ((NCH & -NCH) >= 16 ? 16 : (NCH & -NCH)) - 1;
  constexpr int ROW_BYTES = D * 2;
  constexpr int STAGE_BYTES = kTN * ROW_BYTES;
  constexpr int LOADS = kTN * NCH / 256;  // chunks per thread per stage
  static_assert(LOADS * 256 == kTN * NCH, "stage must split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int quad = lane >> 4, l16 = lane & 15;
  const int64_t batch = blockIdx.y;
  int mblock, split;
  map_block(p, blockIdx.x, mblock, split);
  const int64_t m_wg = (int64_t)mblock * kRowsPerWG;
  if (m_wg >= p.M) return;  // padding block: the whole workgroup leaves together

  const int64_t n_begin = (int64_t)split * p.n_chunk;
  const int64_t n_end = min(p.N, n_begin + p.n_chunk);
  const uint16_t* A = p.a + batch * p.a_sb;
  const uint16_t* Bm = p.b + batch * p.b_sb;

  // Source rows as MFMA B-operands: lane supplies row (lane%16) of its block,
  // features 8*quad .. +8 of each 32-wide k-step.
  bf16x8 sf[kSB][KS];
#pragma unroll
  for (int sb = 0; sb < kSB; ++sb) {
    const int64_t row = m_wg + wave * (kSB * 16) + sb * 16 + l16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (row < p.M) {
        sf[sb][ks] = *reinterpret_cast<const bf16x8*>(A + row * p.a_sm + ks * 32 + quad * 8);
      } else {
        sf[sb][ks] = bf16x8{};
      }
    }
  }

  // Lane-local running state: per accumulator slot, the best score and the
  // 16-row tile that first reached it.
  float best[kSB][4];
  int bt[kSB][4];
  const int tile0 = (int)(n_begin >> 4);
#pragma unroll
  for (int sb = 0; sb < kSB; ++sb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      best[sb][r] = -INFINITY;
      bt[sb][r] = tile0;
    }

  const int nstages = n_end > n_begin ? (int)((n_end - n_begin + kTN - 1) / kTN) : 0;
  u32x4 stage[LOADS];

  // Destination rows of this split through a range-checked buffer: rows past
  // the split end read as zeros (and are masked in the epilogue).
  const uint32_t b_row = (uint32_t)p.b_sn * 2u;
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(
      Bm + n_begin * p.b_sn,
      n_end > n_begin ? (uint32_t)(((n_end - n_begin - 1) * p.b_sn + D) * 2) : 0u);
  auto load_stage = [&](int st) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int id = j * 256 + tid;
      const int row = id / NCH, ch = id % NCH;
      stage[j] = buf_load16(brs, (uint32_t)(st * kTN + row) * b_row + ch * 16);
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int id = j * 256 + tid;
      const int row = id / NCH, ch = id % NCH;
      *reinterpret_cast<u32x4*>(lds + buf * STAGE_BYTES + row * ROW_BYTES +
                                ((ch ^ (row & SWZ)) << 4)) = stage[j];
    }
  };

  if (nstages > 0) {
    load_stage(0);
    store_stage(0);
  }
  __syncthreads();

  for (int st = 0; st < nstages; ++st) {
    const int cur = st & 1;
    if (st + 1 < nstages) load_stage(st + 1);
    const int64_t base = n_begin + (int64_t)st * kTN;
    const uint8_t* L = lds + cur * STAGE_BYTES;
#pragma unroll
    for (int u = 0; u < kTN / 16; ++u) {
      const int64_t tile_n = base + u * 16;
      if (tile_n >= n_end) break;
      f32x4 acc[kSB];
#pragma unroll
      for (int sb = 0; sb < kSB; ++sb) acc[sb] = f32x4{};
      const int row = u * 16 + l16;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int ch = 4 * ks + quad;
        const bf16x8 af =
            *reinterpret_cast<const bf16x8*>(L + row * ROW_BYTES + ((ch ^ (row & SWZ)) << 4));
#pragma unroll
        for (int sb = 0; sb < kSB; ++sb) acc[sb] = mfma16x16x32_t<F16>(af, sf[sb][ks], acc[sb]);
      }
      const int tile = (int)(tile_n >> 4);
      if (tile_n + 16 <= n_end) {
#pragma unroll
        for (int sb = 0; sb < kSB; ++sb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = acc[sb][r];
            const bool upd = v > best[sb][r];
            best[sb][r] = upd ? v : best[sb][r];
            bt[sb][r] = upd ? tile : bt[sb][r];
          }
      } else {
#pragma unroll
        for (int sb = 0; sb < kSB; ++sb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = acc[sb][r];
            const bool upd = (tile_n + 4 * quad + r < n_end) && v > best[sb][r];
            best[sb][r] = upd ? v : best[sb][r];
            bt[sb][r] = upd ? tile : bt[sb][r];
          }
      }
    }
    if (st + 1 < nstages) store_stage(cur ^ 1);
    __syncthreads();
  }

  // Reduce the 4 slots of each lane, then the four lanes (quads) that share a
  // source row: highest score wins, ties go to the lowest destination index.
#pragma unroll
  for (int sb = 0; sb < kSB; ++sb) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = best[sb][r];
      const int idx = bt[sb][r] * 16 + 4 * quad + r;
      const bool take = v > bv || (v == bv && idx < bi);
      bv = take ? v : bv;
      bi = take ? idx : bi;
    }
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      const float ov = __shfl_xor(bv, sh);
      const int oi = __shfl_xor(bi, sh);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    const int64_t m = m_wg + wave * (kSB * 16) + sb * 16 + l16;
    if (quad == 0 && m < p.M) {
      if (p.splits == 1) {
        store_max(p, batch * p.omax_sb + m, bv);
        p.out_idx[batch * p.oidx_sb + m] = bi;
      } else {
        p.part[(batch * p.M + m) * p.splits + split] = part_key(bv, bi);
      }
    }
  }
}


// D = 128 (the model's 128-d projected metric): the same work decomposition,
// software-pipelined.  Destination tiles of 16 rows (4 KB) arrive by
// buffer_load ... lds DMA into an 8-slot ring (each wave copies a quarter of
// a tile with one instruction; the lane picks the global chunk that lands in
// its swizzled LDS position).  Iteration i runs the 32 MFMAs of tiles
// 2i+2, 2i+3 beside the max/argmax epilogue of tiles 2i, 2i+1, whose scores
// the previous iteration produced, so the two are independent and the
// compiler's schedule interleaves them: the MFMA and the VALU unit of a wave
// overlap instead of taking turns (a forced one-MFMA-to-three-VALU pattern
// measured 4-6 % slower here).  An empty asm taking the iteration's results
// keeps each iteration's work inside it.  One barrier per iteration recycles
// the slots of the tiles just read; tiles past the split end read as zeros
// and are masked in the last epilogue.
// max(a, b, c, d) of four scores, NaN operands dropped (IEEE mode), as
// v_max3_f32 + v_max_f32.  Written as asm because the compiler's fmaxf first
// quiets every operand it cannot prove to be a computed value (an MFMA result
// is not one), which doubles the instruction count.  The operands are scores
// the MFMAs of the previous pipeline iteration (or the prologue) produced,
// more than a sched_barrier and a workgroup barrier earlier, or selects of
// them, so no MFMA-to-VALU read hazard can fall on these instructions.
__device__ __forceinline__ float max4_scores(float a, float b, float c, float d) {
  float m3, m4;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(m3) : "v"(a), "v"(b), "v"(c));
  asm("v_max_f32 %0, %1, %2" : "=v"(m4) : "v"(m3), "v"(d));
  return m4;
}

constexpr int kPipeRing = 8;                 // 16-row tile slots
constexpr int kPipePairsAhead = kPipeRing / 2 - 1;

template <bool F16>
__global__ __launch_bounds__(256, 2) void sim_argmax_d128_kernel(SimArgs p) {
  constexpr int KS = 4, kSB = 4, D = 128;
  constexpr int kRowsPerWG = rows_per_wg(KS);
  constexpr int TILE_BYTES = 16 * D * 2;
  __shared__ __attribute__((aligned(16))) uint8_t r0[TILE_BYTES], r1[TILE_BYTES], r2[TILE_BYTES],
      r3[TILE_BYTES], r4[TILE_BYTES], r5[TILE_BYTES], r6[TILE_BYTES], r7[TILE_BYTES];
  uint8_t* const ring[kPipeRing] = {r0, r1, r2, r3, r4, r5, r6, r7};

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int quad = lane >> 4, l16 = lane & 15;
  const int64_t batch = blockIdx.y;
  int mblock, split, sub;
  map_item(p, blockIdx.x, mblock, split, sub);
  // Uniform by construction; saying so keeps the DMA's buffer descriptor in
  // SGPRs (otherwise every issue runs a readfirstlane waterfall loop).
  mblock = __builtin_amdgcn_readfirstlane(mblock);
  split = __builtin_amdgcn_readfirstlane(split);
  sub = __builtin_amdgcn_readfirstlane(sub);
  const int64_t m_wg = (int64_t)mblock * kRowsPerWG;
  if (m_wg >= p.M) return;

  const int64_t s_begin = (int64_t)split * p.n_chunk;
  const int64_t n_begin = sub < 0 ? s_begin : s_begin + sub * p.sub_chunk;
  const int64_t n_end = min(p.N, sub < 0 ? s_begin + p.n_chunk
                                         : min(s_begin + p.n_chunk, n_begin + p.sub_chunk));
  const uint16_t* A = p.a + batch * p.a_sb;
  const uint16_t* Bm = p.b + batch * p.b_sb;

  bf16x8 sf[kSB][KS];
#pragma unroll
  for (int sb = 0; sb < kSB; ++sb) {
    const int64_t row = m_wg + wave * (kSB * 16) + sb * 16 + l16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      sf[sb][ks] = row < p.M ? *reinterpret_cast<const bf16x8*>(A + row * p.a_sm + ks * 32 + quad * 8)
                             : bf16x8{};
  }

  // Per source block: the running max over the lane's four destination
  // rows of every tile so far, the first tile reaching it, and that tile's
  // four scores (to find the row inside it at the end).
  float best[kSB], keep[kSB][4];
  int bt[kSB];
  const int tile0 = (int)(n_begin >> 4);
#pragma unroll
  for (int sb = 0; sb < kSB; ++sb) {
    best[sb] = -INFINITY;
    bt[sb] = tile0;
#pragma unroll
    for (int r = 0; r < 4; ++r) keep[sb][r] = -INFINITY;
  }

  const int ntiles = n_end > n_begin ? (int)((n_end - n_begin + 15) / 16) : 0;
  const int npairs = (ntiles + 1) / 2;
  const uint32_t b_row = (uint32_t)p.b_sn * 2u;
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(
      Bm + n_begin * p.b_sn,
      n_end > n_begin ? (uint32_t)(((n_end - n_begin - 1) * p.b_sn + D) * 2) : 0u);
  // DMA role: wave w fills rows 4w..4w+3 of a tile; lane l lands at LDS
  // chunk l%16 of row 4w + l/16 and fetches the global chunk the XOR
  // swizzle (chunk ^ row) puts there.
  const int d_row = 4 * wave + (lane >> 4), d_ch = (lane & 15) ^ d_row;
  const uint32_t d_voff = (uint32_t)d_row * b_row + d_ch * 16;
  auto issue = [&](int tile, uint8_t* T) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        brs, (__attribute__((address_space(3))) void*)(T + wave * 1024), 16, d_voff,
        (uint32_t)tile * 16u * b_row, 0, 0);
  };
  // A-operand reads: row l16 of the tile, logical chunk 4ks + quad.
  int a_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) a_off[ks] = l16 * (D * 2) + (((4 * ks + quad) ^ l16) << 4);

  auto mfma_tile = [&](const uint8_t* T, f32x4 (&acc)[kSB]) {
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb) acc[sb] = f32x4{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 af = *reinterpret_cast<const bf16x8*>(T + a_off[ks]);
#pragma unroll
      for (int sb = 0; sb < kSB; ++sb) acc[sb] = mfma16x16x32_t<F16>(af, sf[sb][ks], acc[sb]);
    }
  };
  // Running max / first tile reaching it (strict >: an earlier tile keeps a
  // tie), over the tile's max of the lane's four rows: v_max3 + v_max and one
  // compare and six selects per four scores instead of a compare and two
  // selects per score (296 instead of 392 VALU per 128 MFMAs).  NaN scores
  // never win: v_max3/v_max drop NaN operands, a tile whose four are all NaN
  // yields NaN, and NaN > best is false.  MASKED: rows at or past the split
  // end never win.
  auto epilogue = [&](const f32x4 (&acc)[kSB], int tile_rel, auto masked) {
    const int tile = tile0 + tile_rel;
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[r] = acc[sb][r];
        if constexpr (decltype(masked)::value)
          v[r] = n_begin + (int64_t)tile_rel * 16 + 4 * quad + r < n_end ? v[r] : -INFINITY;
      }
      const float m4 = max4_scores(v[0], v[1], v[2], v[3]);
      const bool upd = m4 > best[sb];
      best[sb] = upd ? m4 : best[sb];
      bt[sb] = upd ? tile : bt[sb];
#pragma unroll
      for (int r = 0; r < 4; ++r) keep[sb][r] = upd ? v[r] : keep[sb][r];
    }
  };

  f32x4 cur[2][kSB], nxt[2][kSB];
  auto pin = [&]() {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int sb = 0; sb < kSB; ++sb) asm volatile("" : "+v"(nxt[u][sb]));
#pragma unroll
    for (int sb = 0; sb < kSB; ++sb) {
      asm volatile("" : "+v"(best[sb]), "+v"(bt[sb]));
#pragma unroll
      for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(keep[sb][r]));
    }
  };

  if (npairs > 0) {
    // Prologue: pairs 0 .. kPipePairsAhead-1 in flight; scores of pair 0.
#pragma unroll
    for (int i = 0; i < kPipePairsAhead; ++i) {
      issue(2 * i, ring[2 * i]);
      issue(2 * i + 1, ring[2 * i + 1]);
    }
    wait_vm<2 * (kPipePairsAhead - 1)>();
    __syncthreads();
    mfma_tile(ring[0], cur[0]);
    mfma_tile(ring[1], cur[1]);
    wait_vm<2 * (kPipePairsAhead - 2)>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // Iteration i: fetch pair i+3 into the slots of pair i-1 (read by
    // iteration i-2); scores of pair i+1 beside the epilogue of pair i
    // (scored by iteration i-1); pair i+2 lands by its end.
    auto iter = [&](const int i, const uint8_t* Ta, const uint8_t* Tb, uint8_t* Ia, uint8_t* Ib) {
      __builtin_amdgcn_sched_barrier(0);
      issue(2 * (i + kPipePairsAhead), Ia);
      issue(2 * (i + kPipePairsAhead) + 1, Ib);
      mfma_tile(Ta, nxt[0]);
      mfma_tile(Tb, nxt[1]);
      epilogue(cur[0], 2 * i, std::false_type{});
      epilogue(cur[1], 2 * i + 1, std::false_type{});
      pin();
      wait_vm<2 * (kPipePairsAhead - 2)>();
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int sb = 0; sb < kSB; ++sb) {
        cur[0][sb] = nxt[0][sb];
        cur[1][sb] = nxt[1][sb];
      }
    };
    // Pair j sits in slots 2(j mod 4), 2(j mod 4)+1; iteration i reads pair
    // i+1 and fills the slots of pair i+3 = i-1 (mod 4).
    int i = 0;
    for (; i + 4 <= npairs - 1; i += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int rd = (u + 1) % 4, wr = (u + 3) % 4;
        iter(i + u, ring[2 * rd], ring[2 * rd + 1], ring[2 * wr], ring[2 * wr + 1]);
      }
    }
#pragma unroll
    for (int u = 0; u < 3; ++u)
      if (i < npairs - 1) {
        const int rd = (u + 1) % 4, wr = (u + 3) % 4;
        iter(i, ring[2 * rd], ring[2 * rd + 1], ring[2 * wr], ring[2 * wr + 1]);
        ++i;
      }
    // The last pair, masked against the split end.
    epilogue(cur[0], 2 * (npairs - 1), std::true_type{});
    epilogue(cur[1], 2 * (npairs - 1) + 1, std::true_type{});
    wait_vm<0>();
  }

#pragma unroll
  for (int sb = 0; sb < kSB; ++sb) {
    // The first of the best tile's rows holding the max (-inf rows that never
    // beat the initial -inf: the split's first row).
    // The value reported is the score at that row (so a -0 / +0 tie reports
    // the first row's sign, as a per-score running max would).
    float bv = best[sb];
    int r_best = 0;
    bool found = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool hit = !found && keep[sb][r] == bv;
      r_best = hit ? r : r_best;
      bv = hit ? keep[sb][r] : bv;
      found = found || hit;
    }
    int bi = bt[sb] * 16 + 4 * quad + r_best;
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      const float ov = __shfl_xor(bv, sh);
      const int oi = __shfl_xor(bi, sh);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    const int64_t m = m_wg + wave * (kSB * 16) + sb * 16 + l16;
    if (quad == 0 && m < p.M) {
      if (p.splits == 1) {
        store_max(p, batch * p.omax_sb + m, bv);
        p.out_idx[batch * p.oidx_sb + m] = bi;
      } else if (sub >= 0) {
        const int64_t r = m - (int64_t)p.tail_mb0 * kRowsPerWG;
        p.tail[(r * p.splits + split) * p.tail_sub + sub] = part_key(bv, bi);
      } else {
        p.part[(batch * p.M + m) * p.splits + split] = part_key(bv, bi);
      }
    }
  }
}

// D > 256 (the unprojected metric, D = 1024 for VGGT-1B): source rows no
// longer fit in VGPRs, so both operands stream through LDS, GEMM-style.
//   * A workgroup tile is 128 source x 128 destination rows; wave w owns the
//     64 x 64 quadrant (source half w & 1, destination half w >> 1) as 4 x 4
//     accumulators of v_mfma_f32_16x16x32 (S^T = Dst . Src^T, so a lane again
//     holds one source row against 4 destination rows per block).
//   * The feature dimension is walked in stages of 32 (one MFMA k-step):
//     8 KB of source and 8 KB of destination rows per stage, filled by
//     buffer_load ... lds DMA (four instructions per wave) into a ring of
//     four stages, three in flight while one is computed; one barrier per
//     stage.  Rows are 64 bytes with their four 16-byte chunks swizzled by
//     row_swz(row), so the 16 lanes reading one chunk of 16 rows hit 16
//     distinct bank groups.
//   * After the last stage of a destination tile the 64 scores per lane fold
//     into the lane's running (max, index) per source block, in increasing
//     destination order with a strict `>` (earlier index kept on ties), and
//     the accumulators restart from zero.  Destination rows past the split
//     read zeros and are masked in the fold; source rows past M read zeros
//     and are not stored.
//   * The stage sequence runs over (destination tile, feature chunk) pairs
//     without a break, so the ring keeps streaming across tile boundaries.
//   * At the end the four lanes of a source row reduce with the lowest-index
//     rule, and the two destination halves meet in LDS.
// Chunk swizzle of the 64-byte rows (four 16-byte chunks) of the GEMM-tiled
// kernels: row r keeps logical chunk c at c ^ row_swz(r), with row_swz =
// bits 1-2 of r, xor 3 when bit 3 is set.  The lanes of a fragment read take
// 16 consecutive rows at one logical chunk; any 16 of them land in 16
// distinct 16-byte bank groups of a 64-bank LDS and any 8 consecutive ones in
// 8 distinct groups of a 32-bank one.  (The earlier (r >> 2) & 3 was
// conflict-free only for the first: 4 conflict cycles per LDS instruction
// measured, SQ_LDS_BANK_CONFLICT.)
__device__ __forceinline__ int row_swz(int r) { return ((r >> 1) & 3) ^ (((r >> 3) & 1) * 3); }

constexpr int kGT = 128;                 // source and destination rows per tile
constexpr int kGStage = kGT * 32 * 2;    // bytes of one operand per 32-feature stage
constexpr int kGRing = 4;

template <bool F16>
__global__ __launch_bounds__(256, 2) void sim_argmax_gemm_kernel(SimArgs p, int D) {
  __shared__ __attribute__((aligned(16))) uint8_t a0[kGStage], a1[kGStage], a2[kGStage],
      a3[kGStage], b0[kGStage], b1[kGStage], b2[kGStage], b3[kGStage];
  __shared__ float x_best[kGT];
  __shared__ int x_idx[kGT];
  uint8_t* const ra[kGRing] = {a0, a1, a2, a3};
  uint8_t* const rb[kGRing] = {b0, b1, b2, b3};

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int quad = lane >> 4, l16 = lane & 15;
  const int64_t batch = blockIdx.y;
  int mblock, split;
  map_block(p, blockIdx.x, mblock, split);
  mblock = __builtin_amdgcn_readfirstlane(mblock);
  split = __builtin_amdgcn_readfirstlane(split);
  const int64_t m_wg = (int64_t)mblock * kGT;
  if (m_wg >= p.M) return;  // padding block: the whole workgroup leaves together

  const int64_t n_begin = (int64_t)split * p.n_chunk;
  const int64_t n_end = min(p.N, n_begin + p.n_chunk);
  const int ntiles = n_end > n_begin ? (int)((n_end - n_begin + kGT - 1) / kGT) : 0;
  const int nk = D / 32;
  const int nstages = ntiles * nk;

  // Range-checked descriptors: source rows [m_wg, M) of this workgroup and
  // destination rows [n_begin, n_end) of this split; anything past reads 0.
  const int64_t m_rows = min((int64_t)kGT, p.M - m_wg);
  const uint32_t a_row = (uint32_t)p.a_sm * 2u, b_row = (uint32_t)p.b_sn * 2u;
  const __amdgpu_buffer_rsrc_t ars = make_rsrc(p.a + batch * p.a_sb + m_wg * p.a_sm,
                                               (uint32_t)(((m_rows - 1) * p.a_sm + D) * 2));
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(
      p.b + batch * p.b_sb + n_begin * p.b_sn,
      n_end > n_begin ? (uint32_t)(((n_end - n_begin - 1) * p.b_sn + D) * 2) : 0u);
  // DMA roles: instruction j of wave w fills rows 32w + 16j .. +16 of a stage;
  // lane l lands at row +l/4, chunk l%4 and fetches the logical chunk the
  // swizzle puts there.
  uint32_t a_voff[2], b_voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = wave * 32 + j * 16 + (lane >> 2);
    const int ch = (lane & 3) ^ row_swz(row);
    a_voff[j] = (uint32_t)row * a_row + ch * 16;
    b_voff[j] = (uint32_t)row * b_row + ch * 16;
  }
  auto issue = [&](int s, uint8_t* A, uint8_t* Bd) {
    const int t = s / nk, kc = s - t * nk;
    const uint32_t ks = (uint32_t)kc * 64u;
    const uint32_t ts = (uint32_t)t * kGT * b_row + ks;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ars, (__attribute__((address_space(3))) void*)(A + (wave * 32 + j * 16) * 64), 16,
          a_voff[j], ks, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          brs, (__attribute__((address_space(3))) void*)(Bd + (wave * 32 + j * 16) * 64), 16,
          b_voff[j], ts, 0, 0);
    }
  };
  // Fragment reads: row l16 of a 16-row block, logical chunk `quad`.
  int s_off[4], d_off[4];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const int rs = wm * 64 + blk * 16 + l16, rd = wn * 64 + blk * 16 + l16;
    s_off[blk] = rs * 64 + ((quad ^ row_swz(rs)) << 4);
    d_off[blk] = rd * 64 + ((quad ^ row_swz(rd)) << 4);
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int sb = 0; sb < 4; ++sb)
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[sb][db] = f32x4{};
  float best[4];
  int bidx[4];
#pragma unroll
  for (int sb = 0; sb < 4; ++sb) {
    best[sb] = -INFINITY;
    bidx[sb] = (int)n_begin;
  }

  auto compute = [&](const uint8_t* A, const uint8_t* Bd) {
    bf16x8 sf[4], df[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      sf[blk] = *reinterpret_cast<const bf16x8*>(A + s_off[blk]);
      df[blk] = *reinterpret_cast<const bf16x8*>(Bd + d_off[blk]);
    }
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[sb][db] = mfma16x16x32_t<F16>(df[db], sf[sb], acc[sb][db]);
  };
  // Fold the finished scores of destination tile t, then restart the sums.
  auto fold = [&](int t) {
    const int64_t base = n_begin + (int64_t)t * kGT + wn * 64 + 4 * quad;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t n = base + db * 16 + r;
          const float v = acc[sb][db][r];
          const bool upd = v > best[sb] && n < n_end;
          best[sb] = upd ? v : best[sb];
          bidx[sb] = upd ? (int)n : bidx[sb];
        }
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[sb][db] = f32x4{};
  };

  // Stage s: wait until it has landed (the DMAs of the stages issued after
  // it may stay in flight), synchronise, refill the slot stage s-1 used with
  // stage s+3, compute, and fold at the end of a destination tile.
  auto step = [&](int s, const int u) {
    wait_vm<4 * (kGRing - 2)>();    // the two stages issued after s may stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // Unconditional: the last stages fetch a destination tile past the
    // split, which the descriptor turns into zeros (a branch here would make
    // the compiler drain every DMA before the next LDS read).
    issue(s + kGRing - 1, ra[(u + kGRing - 1) % kGRing], rb[(u + kGRing - 1) % kGRing]);
    compute(ra[u], rb[u]);
    const int t = s / nk;
    if (s - t * nk == nk - 1) fold(t);
  };

#pragma unroll
  for (int i = 0; i < kGRing - 1; ++i) issue(i, ra[i], rb[i]);
  int s = 0;
  for (; s + kGRing <= nstages; s += kGRing) {
#pragma unroll
    for (int u = 0; u < kGRing; ++u) step(s + u, u);
  }
#pragma unroll
  for (int u = 0; u < kGRing - 1; ++u)
    if (s < nstages) step(s++, u);
  wait_vm<0>();

  // Four lanes per source row (quads), lowest index on ties.
#pragma unroll
  for (int sb = 0; sb < 4; ++sb) {
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      const float ov = __shfl_xor(best[sb], sh);
      const int oi = __shfl_xor(bidx[sb], sh);
      if (ov > best[sb] || (ov == best[sb] && oi < bidx[sb])) {
        best[sb] = ov;
        bidx[sb] = oi;
      }
    }
  }
  // The second destination half hands its results to the first over LDS.
  if (wn == 1 && quad == 0) {
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      x_best[wm * 64 + sb * 16 + l16] = best[sb];
      x_idx[wm * 64 + sb * 16 + l16] = bidx[sb];
    }
  }
  __syncthreads();
  if (wn == 0 && quad == 0) {
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      const int r = wm * 64 + sb * 16 + l16;
      float bv = best[sb];
      int bi = bidx[sb];
      const float ov = x_best[r];
      const int oi = x_idx[r];
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
      const int64_t m = m_wg + r;
      if (m < p.M) {
        if (p.splits == 1) {
          store_max(p, batch * p.omax_sb + m, bv);
          p.out_idx[batch * p.oidx_sb + m] = bi;
        } else {
          p.part[(batch * p.M + m) * p.splits + split] = part_key(bv, bi);
        }
      }
    }
  }
}

// D a multiple of 128, >= 512 (the unprojected 1024-d metric): the GEMM
// shape at 256 x 256 workgroup tiles.  At 128 x 128 (the kernel above) a
// 64 x 64 wave tile reads 8 KB of fragments from LDS per 32-feature stage
// for 16 MFMAs (256 cycles); eight such waves per CU plus the DMA writes ask
// ~190 bytes per clock of an LDS port that delivers 128, so LDS, not the
// matrix pipe, sets the pace (23 % of peak).  Here:
//   * one workgroup per CU, four waves; wave w owns 128 source x 128
//     destination rows (source half w & 1, destination half w >> 1) as 8 x 8
//     accumulators of v_mfma_f32_16x16x32 (all 256 AGPRs), so each
//     fragment read from LDS feeds 8 MFMAs (16 KB of reads per 64 MFMAs;
//     ~95 bytes per clock with the DMA writes at full MFMA rate);
//   * 32-feature stages (16 KB of source, 16 KB of destination rows) in a
//     four-slot ring filled by buffer_load ... lds DMA (eight instructions
//     per wave per stage), three stages in flight, one barrier per stage; each
//     slot is a __shared__ array of its own and each unrolled step names
//     its slots statically: with one array and a runtime slot index the
//     compiler cannot tell a fragment read from an in-flight DMA and waits
//     for every DMA before each read (a six-slot ring built that way ran
//     29 % slower);
//   * the fragments of stage s+1 are read from LDS while the 32 MFMAs of
//     stage s run on the ones read the iteration before (two register sets),
//     since one wave per SIMD has no second wave to hide the LDS latency;
//   * rows keep the 64-byte layout and row_swz chunk swizzle of the
//     kernel above (conflict-free), so a wave's fragments sit at one base
//     address plus 1 KB steps (immediate offsets);
//   * the fold after a destination tile's last stage (one source block at a
//     time) takes the max of each group of four destination rows first, as
//     the D = 128 kernel does, and the final reductions are those of the
//     kernel above (strict `>` in destination order per lane, lowest index
//     across lanes and halves);
//   * up to 64 destination splits (8 per XCD), so the workgroups an XCD
//     runs together share source blocks as well as destination tiles in L2
//     (the plan below).
// What bounds it: each 32-feature stage moves 32 KB from L2 into a CU's LDS
// for 4.2 MFLOP (131 FLOP per byte, ~30 bytes per clock per CU at the MFMA
// peak).  With 256 x 128 tiles (24 KB per 2.1 MFLOP, ~45 bytes per clock)
// the L2 did not keep up on all 256 CUs at once: 39 % of peak at D = 1024.
constexpr int kWM = 256;                  // source rows per workgroup tile
constexpr int kWN = 256;                  // destination rows per workgroup tile
constexpr int kWRing = 4;

// NK: the stages per destination tile (D / 32) as a constant, so that a
// tile's stages unroll completely and no accumulator is carried around a
// loop (a loop over the stages left the register allocator copying the sums
// at every back edge, and with a runtime count it spills).
template <bool F16, int NK>
__global__ __launch_bounds__(256, 1) void sim_argmax_wide_kernel(SimArgs p, int D) {
  constexpr int kSA = kWM * 64, kSB_ = kWN * 64;   // stage bytes per operand
  __shared__ __attribute__((aligned(16))) uint8_t a0[kSA], a1[kSA], a2[kSA], a3[kSA],
      b0[kSB_], b1[kSB_], b2[kSB_], b3[kSB_];
  __shared__ float x_best[kWM];
  __shared__ int x_idx[kWM];
  uint8_t* const ra[kWRing] = {a0, a1, a2, a3};
  uint8_t* const rb[kWRing] = {b0, b1, b2, b3};

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int quad = lane >> 4, l16 = lane & 15;
  const int64_t batch = blockIdx.y;
  int mblock, split;
  map_block(p, blockIdx.x, mblock, split);
  mblock = __builtin_amdgcn_readfirstlane(mblock);
  split = __builtin_amdgcn_readfirstlane(split);
  const int64_t m_wg = (int64_t)mblock * kWM;
  if (m_wg >= p.M) return;  // padding block: the whole workgroup leaves together

  // Split `split` covers whole tiles [t0, t1): the splits differ by at most
  // one tile, so no XCD is left with empty ones.
  const int t0 = (int)((int64_t)split * p.wide_tiles / p.splits);
  const int t1 = (int)((int64_t)(split + 1) * p.wide_tiles / p.splits);
  const int64_t n_begin = (int64_t)t0 * kWN;
  const int64_t n_end = min(p.N, (int64_t)t1 * kWN);
  const int ntiles = n_end > n_begin ? t1 - t0 : 0;
  // First row of tile t (relative to n_begin): a split holds at least kWN
  // rows, and its last tile, when the split ends inside it, starts kWN rows
  // before the end instead, so no tile reaches past n_end.  Rows scored
  // twice carry the same value and index: the max and the lowest index
  // attaining it do not change.  (Past the last tile, the prefetch fetches
  // that tile again.)
  const int lim_rows = (int)(n_end - n_begin);
  auto tile_row = [&](int t) __attribute__((always_inline)) {
    return __builtin_amdgcn_readfirstlane(min(t * kWN, lim_rows - kWN));
  };
  constexpr int nk = NK;                   // a multiple of kWRing
  static_assert(NK % kWRing == 0 && NK >= kWRing, "whole groups of ring slots");
  const int nstages = ntiles * nk;

  const int64_t m_rows = min((int64_t)kWM, p.M - m_wg);
  const uint32_t a_row = (uint32_t)p.a_sm * 2u, b_row = (uint32_t)p.b_sn * 2u;
  const __amdgpu_buffer_rsrc_t ars = make_rsrc(p.a + batch * p.a_sb + m_wg * p.a_sm,
                                               (uint32_t)(((m_rows - 1) * p.a_sm + D) * 2));
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(
      p.b + batch * p.b_sb + n_begin * p.b_sn,
      n_end > n_begin ? (uint32_t)(((n_end - n_begin - 1) * p.b_sn + D) * 2) : 0u);
  // DMA roles: instruction j of wave w fills rows 64w + 16j .. +16 of a
  // stage's source and destination rows; lane l lands at row +l/4, chunk
  // l%4 and fetches the logical chunk the swizzle puts there.
  uint32_t a_voff[4], b_voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = wave * 64 + j * 16 + (lane >> 2);
    a_voff[j] = (uint32_t)row * a_row + (((lane & 3) ^ row_swz(row)) * 16);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = wave * 64 + j * 16 + (lane >> 2);
    b_voff[j] = (uint32_t)row * b_row + (((lane & 3) ^ row_swz(row)) * 16);
  }
  auto issue = [&](int t, int kc, uint8_t* A, uint8_t* Bd) __attribute__((always_inline)) {
    // Wave-uniform offsets (the compiler cannot prove the tile counter
    // uniform and would otherwise loop over lanes around each load).
    const uint32_t ks = __builtin_amdgcn_readfirstlane((uint32_t)kc * 64u);
    const uint32_t ts = __builtin_amdgcn_readfirstlane((uint32_t)tile_row(t) * b_row + ks);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ars, (__attribute__((address_space(3))) void*)(A + (wave * 64 + j * 16) * 64), 16,
          a_voff[j], ks, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          brs, (__attribute__((address_space(3))) void*)(Bd + (wave * 64 + j * 16) * 64), 16,
          b_voff[j], ts, 0, 0);
  };
  // Fragment blk of a wave: rows 128 wm + 16 blk + l16 (source), 128 wn +
  // 16 blk + l16 (destination), logical chunk quad; the swizzle term depends
  // on l16 only.
  const int swz = (quad ^ row_swz(l16)) << 4;
  const int s_base = (wm * 128 + l16) * 64 + swz;
  const int d_base = (wn * 128 + l16) * 64 + swz;

  f32x4 acc[8][8];                         // a tile's first stage starts them
  // Per source block: the running max, the first row of the first group of
  // four destination rows reaching it, and that group's four scores.
  float best[8];
  int bidx[8];
  float keep[8][4];
#pragma unroll
  for (int sb = 0; sb < 8; ++sb) {
    best[sb] = -INFINITY;
    bidx[sb] = 0;                          // relative to n_begin until the end
#pragma unroll
    for (int r = 0; r < 4; ++r) keep[sb][r] = -INFINITY;
  }

  bf16x8 fs0[8], fd0[8], fs1[8], fd1[8];
  auto read = [&](const uint8_t* A, const uint8_t* Bd, bf16x8 (&fs)[8], bf16x8 (&fd)[8])
      __attribute__((always_inline)) {
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      fs[blk] = *reinterpret_cast<const bf16x8*>(A + s_base + blk * 1024);
      fd[blk] = *reinterpret_cast<const bf16x8*>(Bd + d_base + blk * 1024);
    }
  };
  // The 64 MFMAs of a stage; a destination tile's first stage takes a zero
  // C operand instead of clearing the sums in the fold (with the clearing
  // there, the register allocator moved the 128 sums between registers at
  // every loop back edge).
  auto mma = [&](const bf16x8 (&fs)[8], const bf16x8 (&fd)[8], auto first)
      __attribute__((always_inline)) {
    constexpr bool Z = decltype(first)::value;
#pragma unroll
    for (int sb = 0; sb < 8; ++sb)
#pragma unroll
      for (int db = 0; db < 8; ++db)
        acc[sb][db] = mfma16x16x32_t<F16>(fd[db], fs[sb], Z ? f32x4{} : acc[sb][db]);
  };
  // Fold the finished scores of destination tile t: one source block at a
  // time (a scheduling barrier between them), so that at most one block's
  // 32 scores leave the accumulator registers at once.
  // Destination rows past the split end (rel >= lim) never win.  (Every
  // lambda here is forced inline: a call would put the accumulators it
  // reaches by reference into scratch memory.)
  // Each block's fold is a chain of dependent compares and selects, so two
  // blocks go together (their chains interleave).  No row is masked: tiles
  // hold no rows past the split end (tile_row).  Per accumulator (four
  // consecutive destination rows of one source row) v_max3 + v_max, one
  // compare and six selects keep the first group reaching the running max
  // and its four scores (strict `>`: an earlier group keeps a tie); the row
  // inside the group is picked once at the end.  9 instead of 12 VALU
  // instructions per four scores: 0.7-1.1 % faster at D = 512-1024 (same
  // box, outputs bit-identical).  The accumulators live in AGPRs, so the
  // asm operands are VGPR copies (v_accvgpr_read), never MFMA results.
  auto fold = [&](int t) __attribute__((always_inline)) {
    const int base = tile_row(t) + wn * 128 + 4 * quad;    // relative to n_begin
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
      if (sb % 2 == 0) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const float m4 = max4_scores(acc[sb][db][0], acc[sb][db][1], acc[sb][db][2], acc[sb][db][3]);
        const bool upd = m4 > best[sb];
        best[sb] = upd ? m4 : best[sb];
        bidx[sb] = upd ? base + db * 16 : bidx[sb];
#pragma unroll
        for (int r = 0; r < 4; ++r) keep[sb][r] = upd ? acc[sb][db][r] : keep[sb][r];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Stage kc of destination tile t (ring slot u = kc % kWRing): wait for
  // stage kc+1 (stages kc+2, kc+3 stay in flight); barrier, after which
  // every wave has read stage kc's fragments, so its slot takes the DMA of
  // stage kc+4 at once (in the next tile past nk: three steps for a stage
  // to land); read stage kc+1's fragments into the other register set while
  // the 64 MFMAs of stage kc run, the reads and DMA issues spread over the
  // whole stage (left to itself the scheduler read each fragment just before
  // its first MFMA and waited for it there; all 24 issued within the first
  // 24 MFMAs measured 7 % slower than spread, same box).  A tile's stages are whole groups of
  // kWRing (nk is a multiple of it), so u is a constant in each unrolled
  // step.  (The stages past the end fetch a destination tile past the
  // split: zeros.)
  auto step = [&](const int t, const int kc, const int u, auto cur, auto first)
      __attribute__((always_inline)) {
    constexpr bool C0 = decltype(cur)::value;
    __builtin_amdgcn_sched_barrier(0);
    wait_vm<8 * (kWRing - 2)>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    int kn = kc + kWRing, tn = t;
    if (kn >= nk) {
      kn -= nk;
      ++tn;
    }
    issue(tn, kn, ra[u], rb[u]);
    if constexpr (C0) {
      read(ra[(u + 1) % kWRing], rb[(u + 1) % kWRing], fs1, fd1);
      mma(fs0, fd0, first);
    } else {
      read(ra[(u + 1) % kWRing], rb[(u + 1) % kWRing], fs0, fd0);
      mma(fs1, fd1, first);
    }
    // MFMA (0x008), DS read (0x100), VMEM (0x010): eight groups of eight
    // MFMAs, each carrying two of the 16 reads and one of the 8 DMA issues.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 5, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  if (nstages > 0) {
#pragma unroll
    for (int i = 0; i < kWRing; ++i) issue(0, i, ra[i], rb[i]);
    wait_vm<8 * (kWRing - 1)>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    read(ra[0], rb[0], fs0, fd0);
    // A loop per destination tile around the stage loop: with one loop and
    // an `if` for the fold, the compiler predicated the fold into every
    // group (accumulators read, selected and written back each time).
    using T_ = std::true_type;
    using F_ = std::false_type;
    for (int t = 0; t < ntiles; ++t) {
      step(t, 0, 0, T_{}, T_{});
      step(t, 1, 1, F_{}, F_{});
      step(t, 2, 2, T_{}, F_{});
      step(t, 3, 3, F_{}, F_{});
#pragma unroll
      for (int g = kWRing; g < nk; g += kWRing) {
        step(t, g + 0, 0, T_{}, F_{});
        step(t, g + 1, 1, F_{}, F_{});
        step(t, g + 2, 2, T_{}, F_{});
        step(t, g + 3, 3, F_{}, F_{});
      }
      fold(t);
    }
  }
  wait_vm<0>();
  // The first row of the best group holding the max, and its score (so a
  // -0 / +0 tie reports the first row's sign, as a per-score running max
  // would); a lane whose scores never beat -inf keeps row 0 of the split.
#pragma unroll
  for (int sb = 0; sb < 8; ++sb) {
    float bv = best[sb];
    int r_best = 0;
    bool found = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool hit = !found && keep[sb][r] == bv;
      r_best = hit ? r : r_best;
      bv = hit ? keep[sb][r] : bv;
      found = found || hit;
    }
    best[sb] = bv;
    bidx[sb] += r_best + (int)n_begin;
  }

  // Four lanes per source row (quads), lowest index on ties.
#pragma unroll
  for (int sb = 0; sb < 8; ++sb) {
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
      const float ov = __shfl_xor(best[sb], sh);
      const int oi = __shfl_xor(bidx[sb], sh);
      if (ov > best[sb] || (ov == best[sb] && oi < bidx[sb])) {
        best[sb] = ov;
        bidx[sb] = oi;
      }
    }
  }
  // The second destination half hands its results to the first over LDS.
  if (wn == 1 && quad == 0) {
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
      x_best[wm * 128 + sb * 16 + l16] = best[sb];
      x_idx[wm * 128 + sb * 16 + l16] = bidx[sb];
    }
  }
  __syncthreads();
  if (wn == 0 && quad == 0) {
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
      const int r = wm * 128 + sb * 16 + l16;
      float bv = best[sb];
      int bi = bidx[sb];
      const float ov = x_best[r];
      const int oi = x_idx[r];
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
      const int64_t m = m_wg + r;
      if (m < p.M) {
        if (p.splits == 1) {
          store_max(p, batch * p.omax_sb + m, bv);
          p.out_idx[batch * p.oidx_sb + m] = bi;
        } else {
          p.part[(batch * p.M + m) * p.splits + split] = part_key(bv, bi);
        }
      }
    }
  }
}

// Merge a row's partial keys: the largest key, i.e. the largest max and,
// among equal maxima, the lowest index -- what the reference's strict `>`
// across destination tiles keeps.  A row's keys are contiguous, so a wave
// reads whole lines, 16 bytes per load, all before any compare (a
// compare-then-load loop over [split][row] planes took 31 us for 75,000
// rows x 16 splits, 8 % of that call).
__global__ __launch_bounds__(256) void sim_argmax_merge_kernel(SimArgs p, int64_t B) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= B * p.M) return;
  const int64_t batch = t / p.M, m = t % p.M;
  const int64_t r = m - (int64_t)p.tail_mb0 * rows_per_wg(4);
  const bool in_tail = p.tail_sub > 0 && r >= 0;
  const int parts = in_tail ? p.splits * p.tail_sub : p.splits;
  const uint64_t* k = in_tail ? p.tail + r * parts : p.part + t * p.splits;
  uint64_t best = 0;
  constexpr int kBatch = 16;
  for (int s0 = 0; s0 < parts; s0 += kBatch) {
    uint64_t v[kBatch];
    if (parts % 2 == 0) {                  // 16-byte aligned pairs (also a short batch)
      const int n = min(kBatch, parts - s0);
#pragma unroll
      for (int u = 0; u < kBatch; u += 2) {
        u32x4 w = {0u, 0u, 0u, 0u};
        if (u < n) w = *reinterpret_cast<const u32x4*>(k + s0 + u);
        v[u] = ((uint64_t)w[1] << 32) | w[0];
        v[u + 1] = ((uint64_t)w[3] << 32) | w[2];
      }
    } else {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) v[u] = s0 + u < parts ? k[s0 + u] : 0;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) best = v[u] > best ? v[u] : best;
  }
  float bv;
  int bi;
  key_part(best, bv, bi);
  store_max(p, batch * p.omax_sb + m, bv);
  p.out_idx[batch * p.oidx_sb + m] = bi;
}

struct SimPlan {
  int splits;
  int mblocks;       // padded source blocks
  int64_t n_chunk;   // destination rows per split (the largest split when wide)
  int wide_tiles;    // see SimArgs
  int tail_sub;      // 0: no tail (see SimArgs)
  int tail_mb0;
  int64_t tail_rows;
  int64_t sub_chunk;
  size_t part_bytes;  // [B][M][splits] partial keys
  size_t ws_bytes;
};

// Workgroups the current device holds at two per CU (the similarity
// kernels' occupancy): the round size the tail is cut for.
int device_slots() {
  static std::mutex mu;
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 512;
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = 2 * cus;
  }
  return cache[dev];
}

// Largest feature dim of the GEMM-tiled kernel (D > 256).
constexpr int64_t kMaxD = 4096;

// Which kernel serves a feature dim: register-resident source rows up to
// 256, the 256 x 256-tile kernel for multiples of 128 from 512, the
// 128 x 128-tile kernel for the rest.
// D served by sim_argmax_wide_kernel (one instantiation per D; wider D
// goes to the GEMM-tiled kernel, where a runtime stage count spills).
__host__ __device__ constexpr bool wide_dim(int64_t D) {
  return D >= 512 && D <= 1024 && D % 128 == 0;
}
// ... and at least one whole destination tile (every split then holds >= kWN
// rows: one split, or >= 1,024 rows each).
__host__ __device__ constexpr bool use_wide(int64_t D, int64_t N) { return wide_dim(D) && N >= kWN; }

SimPlan make_plan(int64_t B, int64_t M, int64_t N, int64_t D) {
  SimPlan pl{};
  const bool gemm = D > 256;
  const bool wide = use_wide(D, N);
  const int rows = wide ? kWM : gemm ? kGT : rows_per_wg((int)(D / 32));
  const int64_t mb = (M + rows - 1) / rows;
  // Split the destination range until the grid holds >= 2048 workgroups
  // (8 per CU on 256 CUs) or a split would drop below 512 rows.  Once there
  // are several splits, use at least 8 so that each XCD owns one range.
  // (75,000 x 25,000 with the last round cut as below: 8 splits 350 us,
  // 16 splits 366 us; 32 splits without a cut 397 us: below ~1,000 rows a
  // workgroup's start-up costs more than its work.)
  int splits = 1;
  while (splits < 16 && mb * B * splits < 2048 && N / (splits * 2) >= 512) splits *= 2;
  if (splits > 1 && splits < 8 && N / 8 >= 512) splits = 8;
  // Wide D: a workgroup re-reads its 256 source rows (512 KB at D = 1024)
  // for every destination tile, which no L2 holds for 32 different blocks.
  // With k = splits / 8 splits per XCD the 32 workgroups an XCD runs at
  // once are 32 / k source blocks x k destination ranges, stepping through
  // their tiles together, so one round fetches 32 / k blocks and k tiles
  // into L2 instead of 32 blocks and one tile: k = 8 fetches a quarter.
  // Keep >= 3 tiles per split.
  const int64_t wtiles = (N + kWN - 1) / kWN;
  if (wide && splits >= 8)
    while (splits < 64 && wtiles / (splits * 2) >= 3) splits *= 2;
  pl.splits = splits;
  int64_t mbp = mb;
  if (splits > 1 && splits < 8) {
    const int g = 8 / splits;
    mbp = (mb + g - 1) / g * g;
  }
  pl.mblocks = (int)mbp;
  const int64_t per = (N + splits - 1) / splits;
  const int gran = wide ? kWN : gemm ? kGT : kTN;   // whole destination tiles per split
  pl.n_chunk = (per + gran - 1) / gran * gran;
  if (wide) {
    // Near-equal whole-tile ranges (see SimArgs::wide_tiles); n_chunk is
    // the largest.
    pl.wide_tiles = (int)wtiles;
    pl.n_chunk = (wtiles + splits - 1) / splits * kWN;
  }
  pl.part_bytes = splits > 1 ? (size_t)(B * splits * M) * (sizeof(float) + sizeof(int32_t)) : 0;
  pl.ws_bytes = pl.part_bytes;
  // The last round (D = 128, one batch, whole XCD-mapped splits): when the
  // (block, split) items leave a partial last round of `rem` items, the last
  // T = ceil(rem / splits) source blocks give each split to P workgroups of
  // a P-th of its destination rows, P = 2 slots / (T * splits), so the end
  // of the call is up to two rounds of short items instead of a partial
  // round of long ones.  (75,000 x 25,000: 2,344 items = 4 rounds of 512 +
  // 296; the last 37 blocks' 296 items become 888 of 1,056 rows: 364 ->
  // 350 us.  200 frames: 6,504 = 12 rounds + 360; the last 45 blocks' items
  // halved: 2,453 -> 2,415 us.)
  if (D == 128 && B == 1 && splits >= 8 && splits % 8 == 0) {
    const int64_t slots = device_slots();
    const int64_t items = mb * splits;
    const int64_t rem = items % slots;
    if (items > slots && rem != 0) {
      const int64_t T = (rem + splits - 1) / splits;
      const int64_t P = 2 * slots / (T * splits);
      if (P >= 2 && T < mb) {
        pl.tail_sub = (int)P;
        pl.tail_mb0 = (int)(mb - T);
        pl.tail_rows = M - (mb - T) * rows;
        pl.sub_chunk = ((pl.n_chunk + P - 1) / P + 31) / 32 * 32;
        pl.ws_bytes += (size_t)(splits * P * pl.tail_rows) * (sizeof(float) + sizeof(int32_t));
      }
    }
  }
  return pl;
}

}  // namespace
}  // namespace gpa

using namespace gpa;

extern "C" size_t gpa_sim_argmax_workspace_bytes(int64_t B, int64_t M, int64_t N, int64_t D) {
  if (B <= 0 || M <= 0 || N <= 0) return 0;
  return make_plan(B, M, N, D).ws_bytes;
}

namespace {

// Shared by the bf16 and fp16 entry points: the kernels differ only in the
// MFMA instruction; `fn` names the entry point in error messages.
template <bool F16>
int sim_argmax_run(const char* fn, const void* a, const void* b, void* out_max, int max_dtype,
                   int64_t* out_idx,
                   int64_t B, int64_t M, int64_t N, int64_t D, int64_t a_sb, int64_t a_sm,
                   int64_t b_sb, int64_t b_sn, int64_t omax_sb, int64_t oidx_sb, void* workspace,
                   size_t workspace_bytes, void* stream) {
  gpa_clear_error();
  if (B < 0 || M < 0 || N < 0 || D < 0) {
    gpa_set_error("%s: negative size (B=%lld M=%lld N=%lld D=%lld)", fn,
                  (long long)B, (long long)M, (long long)N, (long long)D);
    return GPA_E_INVALID;
  }
  if (B == 0 || M == 0) return GPA_OK;
  if (N == 0) {
    gpa_set_error("%s: empty destination set (N=0)", fn);
    return GPA_E_INVALID;
  }
  if (max_dtype != GPA_DTYPE_F32 && max_dtype != GPA_DTYPE_BF16 && max_dtype != GPA_DTYPE_F16) {
    gpa_set_error("%s: unknown max_dtype %d", fn, max_dtype);
    return GPA_E_INVALID;
  }
  if (!a || !b || !out_max || !out_idx) {
    gpa_set_error("%s: null tensor pointer", fn);
    return GPA_E_INVALID;
  }
  if (D % 32 != 0 || D < 32 || D > kMaxD) {
    gpa_set_error("%s: feature dim D=%lld unsupported (multiple of 32, 32..%lld)", fn,
                  (long long)D, (long long)kMaxD);
    return GPA_E_UNSUPPORTED;
  }
  if (N > (int64_t)0x7fffff00 || M > ((int64_t)1 << 40)) {
    gpa_set_error("%s: N=%lld exceeds the int32 index range", fn, (long long)N);
    return GPA_E_UNSUPPORTED;
  }
  const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
  if ((pa % 16) || (pb % 16) || (a_sm % 8) || (b_sn % 8) || (a_sb % 8) || (b_sb % 8) ||
      a_sm < D || b_sn < D) {
    gpa_set_error("%s: rows must be 16-byte aligned with unit feature stride "
                  "(a_sm=%lld b_sn=%lld a_sb=%lld b_sb=%lld)", fn,
                  (long long)a_sm, (long long)b_sn, (long long)a_sb, (long long)b_sb);
    return GPA_E_INVALID;
  }
  if (B > 65535) {
    gpa_set_error("%s: batch %lld exceeds the grid limit", fn, (long long)B);
    return GPA_E_UNSUPPORTED;
  }

  const SimPlan pl = make_plan(B, M, N, D);
  // Buffer offsets are 32-bit: one split of destination rows, plus the
  // tiles fetched past its end (two stages, eight 16-row tiles, or one
  // 256-row tile), and one source block must stay below 2^31 bytes.
  const int64_t past = use_wide(D, N) ? kWN : 2 * kTN, src_rows = use_wide(D, N) ? kWM : kGT;
  if ((pl.n_chunk + past) * b_sn * 2 >= ((int64_t)1 << 31) ||
      src_rows * a_sm * 2 >= ((int64_t)1 << 31)) {
    gpa_set_error("%s: destination split or source block exceeds 2 GiB (N=%lld, row strides "
                  "%lld / %lld)", fn, (long long)N, (long long)a_sm, (long long)b_sn);
    return GPA_E_UNSUPPORTED;
  }
  SimArgs p{};
  p.a = (const uint16_t*)a;
  p.b = (const uint16_t*)b;
  p.out_max = out_max;
  p.max_dtype = max_dtype;
  p.out_idx = out_idx;
  p.M = M;
  p.N = N;
  p.a_sb = a_sb;
  p.a_sm = a_sm;
  p.b_sb = b_sb;
  p.b_sn = b_sn;
  p.omax_sb = omax_sb;
  p.oidx_sb = oidx_sb;
  p.splits = pl.splits;
  p.mblocks = pl.mblocks;
  p.n_chunk = pl.n_chunk;
  p.wide_tiles = pl.wide_tiles;
  p.tail_sub = pl.tail_sub;
  p.tail_mb0 = pl.tail_mb0;
  p.tail_rows = pl.tail_rows;
  p.sub_chunk = pl.sub_chunk;
  p.tail_item0 = pl.tail_mb0 * pl.splits;
  if (pl.splits > 1) {
    // The partial-key merge reads the workspace 16 bytes at a time.
    if (!workspace || workspace_bytes < pl.ws_bytes || (uintptr_t)workspace % 16) {
      gpa_set_error("%s: 16-byte aligned workspace of %zu bytes required, %zu given", fn,
                    pl.ws_bytes, workspace ? workspace_bytes : (size_t)0);
      return GPA_E_WORKSPACE;
    }
    p.part = (uint64_t*)workspace;
    if (pl.tail_sub > 0) p.tail = (uint64_t*)((char*)workspace + pl.part_bytes);
  }
  // Whole (block, split) items, then the tail's sub-range items.
  const int64_t grid_x =
      pl.tail_sub > 0 ? (int64_t)pl.tail_mb0 * pl.splits +
                            (int64_t)(pl.mblocks - pl.tail_mb0) * pl.splits * pl.tail_sub
                      : (int64_t)pl.mblocks * pl.splits;
  if (grid_x > 0x7fffffff) {
    gpa_set_error("%s: grid too large", fn);
    return GPA_E_UNSUPPORTED;
  }
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)grid_x, (unsigned)B), block(256);
  switch (D / 32) {
#define GPA_SIM_CASE(ks) \
  case ks: hipLaunchKernelGGL((sim_argmax_kernel<ks, F16>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL(sim_argmax_d128_kernel<F16>, grid, block, 0, s, p); break;
    GPA_SIM_CASE(1) GPA_SIM_CASE(2) GPA_SIM_CASE(3)
    GPA_SIM_CASE(5) GPA_SIM_CASE(6) GPA_SIM_CASE(7) GPA_SIM_CASE(8)
#undef GPA_SIM_CASE
    default:
      switch (use_wide(D, N) ? D / 32 : 0) {
#define GPA_SIM_WIDE(nk) \
  case nk: hipLaunchKernelGGL((sim_argmax_wide_kernel<F16, nk>), grid, block, 0, s, p, (int)D); break;
        GPA_SIM_WIDE(16) GPA_SIM_WIDE(20) GPA_SIM_WIDE(24) GPA_SIM_WIDE(28) GPA_SIM_WIDE(32)
#undef GPA_SIM_WIDE
        default:
          hipLaunchKernelGGL(sim_argmax_gemm_kernel<F16>, grid, block, 0, s, p, (int)D);
      }
      break;
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && pl.splits > 1) {
    const int64_t total = B * M;
    hipLaunchKernelGGL(sim_argmax_merge_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, s, p, B);
    e = hipGetLastError();
  }
  if (e != hipSuccess) {
    gpa_set_error("%s: launch failed: %s", fn, hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}

}  // namespace

extern "C" int gpa_sim_argmax_bf16(const void* a, const void* b, void* out_max, int max_dtype,
                                   int64_t* out_idx, int64_t B, int64_t M, int64_t N, int64_t D, int64_t a_sb,
                                   int64_t a_sm, int64_t b_sb, int64_t b_sn, int64_t omax_sb,
                                   int64_t oidx_sb, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  return sim_argmax_run<false>("gpa_sim_argmax_bf16", a, b, out_max, max_dtype, out_idx, B, M, N,
                               D, a_sb, a_sm, b_sb, b_sn, omax_sb, oidx_sb, workspace,
                               workspace_bytes, stream);
}

extern "C" int gpa_sim_argmax_f16(const void* a, const void* b, void* out_max, int max_dtype,
                                  int64_t* out_idx, int64_t B, int64_t M, int64_t N, int64_t D, int64_t a_sb,
                                  int64_t a_sm, int64_t b_sb, int64_t b_sn, int64_t omax_sb,
                                  int64_t oidx_sb, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  return sim_argmax_run<true>("gpa_sim_argmax_f16", a, b, out_max, max_dtype, out_idx, B, M, N,
                              D, a_sb, a_sm, b_sb, b_sn, omax_sb, oidx_sb, workspace,
                              workspace_bytes, stream);
}
