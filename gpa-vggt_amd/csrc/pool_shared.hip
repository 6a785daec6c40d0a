// Content-adaptive pooled summaries of the frame-special shared K/V set.
//
// For every (batch b, head h, frame s) group of the frame's patch keys
// x_p = k[b, h, s*P + pts + p, :] (p < gh*gw on a gh x gw patch grid, head
// dim 64):
//   seeds   y_g = x at the stride-kp lattice patches (gy*kp, gx*kp),
//           g = gy*nw + gx, nh = ceil(gh/kp), nw = ceil(gw/kp)
//   assign  a_p = argmax_g bf16( bf16(x_p / max(|x_p|, 1e-6)) . bf16(y_g / max(|y_g|, 1e-6)) )
//           (fp32 dot products rounded to bf16, lowest g on ties)
//   size    n_g = #{p : a_p = g}
//   pooled  K_g = sum_{a_p = g} k_p / max(n_g, 1),  V_g likewise from v
// written as pk, pv [B, H, S*npool, 64] bf16 and size [B, H, S, npool] fp32.
//
// This is the `_pool` of vggt/layers/attention.py:113-140 under bf16
// autocast: the normalised keys and seeds enter the einsum (:130) in bf16,
// its scores come back in bf16, argmax takes the first maximum, and the
// sums run in fp32 (scatter_add_, :132-139) before the cast back.  The fp16
// instantiation is the same under fp16 autocast on fp16 keys and values
// (fp16 normalised rows, fp16 MFMA, scores rounded to fp16).  The
// reference sums with atomics in a run-dependent order; here every sum has
// a fixed order, so the means are deterministic.
//
// One workgroup (4 waves) per group; wave w takes the 32-row tiles
// t = w, w+4, ... of the frame, first of K (assignment and K sums), then of
// V (V sums), so each K and V row is read from memory once.
//   Assignment: the normalised seeds are the A operands of
//   v_mfma_f32_32x32x16_bf16 (one or two blocks of 32 seeds, held in
//   registers), the tile's normalised keys the B operand; a lane's 16 scores
//   of a row are rounded to bf16 and reduced with the partner lane (lowest
//   seed on ties).  The assignment bytes go to LDS, the counts to LDS
//   counters.
//   Sums, in the same iteration: a one-hot GEMM per feature half,
//   D[seed][feature] += sum_rows [a_row == seed] x[row][feature], exact bf16
//   products summed in fp32.  The tile's raw rows (already in registers for
//   the assignment) are staged in the wave's LDS tile and read back
//   transposed as the B operand (rows along k); the A operand is built from
//   the assignment bytes.
//   Each wave ends a sweep with partial sums over its tiles; the four
//   partials meet in LDS and are added in wave order (fixed), then divided
//   by the counts.
// HBM-bound: every K and V row read once.
#include "gpa_common.h"

#include <math.h>

namespace gpa {
namespace {

constexpr int kPoolThreads = 256;
constexpr int kPoolWaves = kPoolThreads / 64;
constexpr int kPoolD = 64;
constexpr int kMaxPool = 64;      // seeds per frame (kp >= 5 at grid 37)
constexpr int kMaxPatches = 4096;

struct PoolArgs {
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* pk;
  uint16_t* pv;
  float* size;
  int32_t* assign;   // nullable
  int64_t k_sb, k_sh, k_sn, v_sb, v_sh, v_sn;
  int H, S, P, pts, gh, gw, kp, nw, npool;
};

// Row stride of a wave's staged tile (32 rows x 32 features), in bf16: 8 of
// padding, so the transposed reads (lanes = features, the two lane halves 8
// rows apart) fall in different banks.
constexpr int kStage = 32 + 8;
// Row stride of the partial-sum buffer (32 features + 1 of padding).
constexpr int kRed = 33;

// A score rounded to the 16-bit format, as the autocast einsum returns it.
template <bool F16>
__device__ __forceinline__ float round16(float x) { return half_to_f32<F16>(f32_to_half<F16>(x)); }
// 1.0 in the 16-bit format: the one-hot A operand.
template <bool F16>
constexpr uint32_t kOne16 = F16 ? 0x3c00u : 0x3f80u;

// NSB: blocks of 32 seeds (1 or 2), so the accumulators of an absent block
// take no registers.  One block fits three waves per SIMD without spills
// (158 VGPRs), 8 % faster than two; two blocks stay at two (spills at three).
template <int NSB, bool F16>
__global__ __launch_bounds__(kPoolThreads) __attribute__((amdgpu_waves_per_eu(NSB == 1 ? 3 : 1)))
void pool_shared_kernel(PoolArgs a) {
  __shared__ int count[kMaxPool];
  __shared__ __attribute__((aligned(16))) uint8_t asg[kMaxPatches];
  __shared__ __attribute__((aligned(16))) uint16_t stage[kPoolWaves][32][kStage];
  __shared__ float red[kPoolWaves][kMaxPool][kRed];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int grp = blockIdx.x;                  // (b*H + h)*S + s
  const int s = grp % a.S;
  const int bh = grp / a.S;
  const int h = bh % a.H, b = bh / a.H;
  const int npatch = a.gh * a.gw;
  const uint16_t* K = a.k + b * a.k_sb + h * a.k_sh + ((int64_t)s * a.P + a.pts) * a.k_sn;
  const uint16_t* Vp = a.v + b * a.v_sb + h * a.v_sh + ((int64_t)s * a.P + a.pts) * a.v_sn;
  // The bases and output pointers, formed here so that the argument block's
  // strides need not stay live in SGPRs (they spilled to VGPR lanes).
  uint16_t* PK = a.pk;
  uint16_t* PV = a.pv;
  float* SZ = a.size;
  int32_t* AS = a.assign;
  asm volatile("" : "+s"(K), "+s"(Vp), "+s"(PK), "+s"(PV), "+s"(SZ), "+s"(AS));

  for (int g = tid; g < a.npool; g += kPoolThreads) count[g] = 0;

  // Features 16ks + 8hi .. +8 (ks < 4) of a row: the MFMA operand layout of
  // a 16-feature k-step.  Lanes l and l^32 share a row.
  auto load_half = [&](const uint16_t* base, int64_t stride, int p, bf16x8 (&r)[4]) {
    const uint16_t* row = base + (int64_t)p * stride + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) r[ks] = *reinterpret_cast<const bf16x8*>(row + 16 * ks);
  };
  // x / max(|x|, 1e-6) in fp32, rounded to bf16; both lanes of a row take part.
  auto normalise = [&](const bf16x8 (&r)[4], bf16x8 (&nb)[4]) {
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = half_to_f32<F16>(r[ks][e]);
        ss = __builtin_fmaf(f, f, ss);
      }
    const float inv = 1.0f / fmaxf(__builtin_sqrtf(sum_halves(ss)), 1e-6f);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) nb[ks][e] = f32_to_half<F16>(half_to_f32<F16>(r[ks][e]) * inv);
  };

  // Seed blocks: block sb holds seeds 32sb .. 32sb+31 in lane rows l32 (zero
  // past npool; their scores are masked anyway).
  bf16x8 seed[NSB][4];
#pragma unroll
  for (int sb = 0; sb < NSB; ++sb) {
    const int g = sb * 32 + l32;
    const int gc = g < a.npool ? g : a.npool - 1;
    const int gy = gc / a.nw, gx = gc % a.nw;
    bf16x8 r[4];
    load_half(K, a.k_sn, gy * a.kp * a.gw + gx * a.kp, r);
    normalise(r, seed[sb]);
    if (g >= a.npool)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) seed[sb][ks] = bf16x8{};
  }
  __syncthreads();                             // counts cleared

  uint16_t(&st)[32][kStage] = stage[wave];
  const int ntile = (npatch + 31) / 32;        // ntile * 32 <= kMaxPatches
  const int64_t out_row0 = ((int64_t)bh * a.S + s) * a.npool;   // row of [B, H, S*npool]

  // Score a tile's normalised rows against the seeds; the row's seed (lowest
  // on ties) goes to asg, the count and the optional assignment output.
  auto assign_tile = [&](int t, bool valid, const bf16x8 (&rk)[4]) {
    bf16x8 xb[4];
    normalise(rk, xb);
    float best = -INFINITY;
    int bi = 0;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      f32x16 sc = {};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) sc = mfma32x32x16_t<F16>(seed[sb][ks], xb[ks], sc);
#pragma unroll
      for (int r = 0; r < 16; ++r) {           // seeds in increasing order
        const int g = sb * 32 + mfma_row(r, hi);
        const float v = round16<F16>(sc[r]);
        if (g < a.npool && v > best) {
          best = v;
          bi = g;
        }
      }
    }
    const float pb = __shfl_xor(best, 32);
    const int pi = __shfl_xor(bi, 32);
    if (pb > best || (pb == best && pi < bi)) bi = pi;
    if (hi == 0) {
      const int p = t * 32 + l32;
      asg[p] = valid ? (uint8_t)bi : (uint8_t)0xff;   // 0xff matches no seed
      if (valid) {
        atomicAdd(&count[bi], 1);
        if (AS) AS[(int64_t)grp * npatch + p] = bi;
      }
    }
  };

  // One-hot sums of a tile into acc[feature half][seed block].  The rows are
  // staged in the wave's LDS tile and read back transposed (rows along k);
  // the wave's own LDS writes and reads execute in order, so no barrier is
  // needed between the staging and the reads, nor before the next staging.
  auto sum_tile = [&](int t, bool valid, const bf16x8 (&rx)[4], f32x16 (&acc)[2][NSB]) {
#pragma unroll
    for (int fh = 0; fh < 2; ++fh) {
      // Features 32fh .. 32fh+31: this lane holds 16ks + 8hi .. +8 of
      // ks = 2fh and 2fh+1.
#pragma unroll
      for (int c = 0; c < 2; ++c)
        *reinterpret_cast<bf16x8*>(&st[l32][16 * c + 8 * hi]) = valid ? rx[2 * fh + c] : bf16x8{};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int r0 = 16 * kk + 8 * hi;       // rows r0 .. r0+7 of the tile
        const uint2 ab = *reinterpret_cast<const uint2*>(&asg[t * 32 + r0]);
        u32x4 bx;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          bx[q] = (uint32_t)st[r0 + 2 * q][l32] | ((uint32_t)st[r0 + 2 * q + 1][l32] << 16);
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          const uint32_t id = (uint32_t)(sb * 32 + l32);
          u32x4 oh;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t w = q < 2 ? ab.x : ab.y;
            const uint32_t b0 = (w >> (16 * (q & 1))) & 0xffu, b1 = (w >> (16 * (q & 1) + 8)) & 0xffu;
            oh[q] = (b0 == id ? kOne16<F16> : 0u) | (b1 == id ? kOne16<F16> << 16 : 0u);
          }
          acc[fh][sb] = mfma32x32x16_t<F16>(__builtin_bit_cast(bf16x8, oh),
                                            __builtin_bit_cast(bf16x8, bx), acc[fh][sb]);
        }
      }
    }
  };

  // The four waves' partial sums meet in LDS, one feature half at a time,
  // and are added in wave order; the means go straight to the output.
  auto reduce_store = [&](f32x16 (&acc)[2][NSB], uint16_t* out) {
#pragma unroll
    for (int fh = 0; fh < 2; ++fh) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave][sb * 32 + mfma_row(r, hi)][l32] = acc[fh][sb][r];
      __syncthreads();
      for (int e = tid; e < a.npool * 32; e += kPoolThreads) {
        const int g = e >> 5, f = e & 31;
        const float sum = ((red[0][g][f] + red[1][g][f]) + red[2][g][f]) + red[3][g][f];
        const float inv = 1.0f / fmaxf((float)count[g], 1.0f);
        out[(out_row0 + g) * kPoolD + 32 * fh + f] =
            __builtin_bit_cast(uint16_t, f32_to_half<F16>(sum * inv));
      }
      __syncthreads();
    }
  };

  // Wave w takes tiles w, w+4, ...; the next tile's rows load while this
  // one is processed.  Sweep 1 over K: assignment and K sums; sweep 2 over
  // V: V sums with the assignment of the same wave's tiles.  Each row of K
  // and V is read once.
  auto sweep = [&](const uint16_t* X, int64_t x_sn, bool with_assign, uint16_t* out) {
    f32x16 acc[2][NSB] = {};
    bf16x8 nx[4];
    const int p0 = wave * 32 + l32;
    load_half(X, x_sn, p0 < npatch ? p0 : npatch - 1, nx);
    for (int t = wave; t < ntile; t += kPoolWaves) {
      const int p = t * 32 + l32;
      const bool valid = p < npatch;
      bf16x8 rx[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) rx[ks] = nx[ks];
      const int pn = p + 32 * kPoolWaves;
      load_half(X, x_sn, pn < npatch ? pn : npatch - 1, nx);
      if (with_assign) assign_tile(t, valid, rx);
      sum_tile(t, valid, rx, acc);
    }
    reduce_store(acc, out);                    // the first barrier completes the counts
  };
  sweep(K, a.k_sn, true, PK);
  sweep(Vp, a.v_sn, false, PV);
  for (int g = tid; g < a.npool; g += kPoolThreads) SZ[out_row0 + g] = (float)count[g];
}

// More than 64 seeds per frame (pool stride <= 4 at grid 37, down to every
// patch a seed at stride 1): the seeds no longer fit in registers, so they
// are taken in super-chunks of 64 (two blocks of 32, as above).
//   Assignment: for each super-chunk every wave sweeps its tiles of K
//   (tiles w, w+4, ...), scores them against the chunk's 64 normalised
//   seeds exactly as above (16-bit rounded scores, lowest seed on ties) and
//   keeps, per patch, the best score so far and its seed in LDS, replaced
//   only by a strictly larger score of a later chunk: the same first maximum
//   as one scan over all seeds in increasing order.  A patch whose scores
//   are all NaN keeps seed 0, as above.
//   Counts once the assignment is final, then the sums: per super-chunk, a
//   sweep of K and one of V with the one-hot GEMM of the 64-seed kernel
//   (seed ids now 16-bit), partial sums per wave over its tiles, the four
//   waves added in wave order: every group mean is summed in the same order
//   as in pool_shared_kernel.  K is read 2 * ceil(npool / 64) times and V
//   ceil(npool / 64) times per frame (from L2 after the first sweep); one
//   workgroup per (batch, head, frame) group as above.
constexpr uint16_t kNoSeed = 0xffff;
// Tiles per wave in flight in the many-seed sweeps (each sweep is a chain of
// short per-tile steps; with one tile ahead it waited out most of each
// tile's load).
constexpr int kManyAhead = 2;

// The per-patch best scores (assignment), then either the partial sums of
// the one-hot path or the sort keys and seed offsets share one LDS area.
constexpr int kManyArea = kPoolWaves * kMaxPool * kRed > 2 * kMaxPatches + 1
                              ? kPoolWaves * kMaxPool * kRed : 2 * kMaxPatches + 1;
// Up to this many 64-seed chunks the sums run as one-hot MFMA products over
// tiles (the 64-seed kernel's scheme, once per chunk); above, the sorted
// member lists, whose cost does not grow with the seed count (100 seeds:
// 0.625 vs 0.69 ms; 169 seeds: 0.91 vs 0.80 ms; 1,369: 6.35 vs 3.10 ms).
constexpr int kOneHotChunks = 2;

template <bool F16>
__global__ __launch_bounds__(kPoolThreads, 2) void pool_many_kernel(PoolArgs a) {
  __shared__ int count[kMaxPatches];
  __shared__ __attribute__((aligned(16))) uint16_t asg[kMaxPatches];
  __shared__ __attribute__((aligned(16))) float area[kManyArea];
  __shared__ __attribute__((aligned(16))) uint16_t stage[kPoolWaves][32][kStage];
  float* const best = area;                                              // assignment
  float (*const red)[kMaxPool][kRed] = reinterpret_cast<float (*)[kMaxPool][kRed]>(area);  // sums

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int grp = blockIdx.x;                  // (b*H + h)*S + s
  const int s = grp % a.S;
  const int bh = grp / a.S;
  const int h = bh % a.H, b = bh / a.H;
  const int npatch = a.gh * a.gw;
  const int ntile = (npatch + 31) / 32;        // ntile * 32 <= kMaxPatches
  const int nsc = (a.npool + kMaxPool - 1) / kMaxPool;
  const uint16_t* K = a.k + b * a.k_sb + h * a.k_sh + ((int64_t)s * a.P + a.pts) * a.k_sn;
  const uint16_t* Vp = a.v + b * a.v_sb + h * a.v_sh + ((int64_t)s * a.P + a.pts) * a.v_sn;
  const int64_t out_row0 = ((int64_t)bh * a.S + s) * a.npool;
  uint16_t* PK = a.pk;
  uint16_t* PV = a.pv;
  float* SZ = a.size;
  int32_t* AS = a.assign;
  asm volatile("" : "+s"(K), "+s"(Vp), "+s"(PK), "+s"(PV), "+s"(SZ), "+s"(AS));

  for (int g = tid; g < a.npool; g += kPoolThreads) count[g] = 0;
  for (int p = tid; p < ntile * 32; p += kPoolThreads) {
    asg[p] = kNoSeed;
    best[p] = -INFINITY;
  }

  auto load_half = [&](const uint16_t* base, int64_t stride, int p, bf16x8 (&r)[4]) {
    const uint16_t* row = base + (int64_t)p * stride + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) r[ks] = *reinterpret_cast<const bf16x8*>(row + 16 * ks);
  };
  auto normalise = [&](const bf16x8 (&r)[4], bf16x8 (&nb)[4]) {
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = half_to_f32<F16>(r[ks][e]);
        ss = __builtin_fmaf(f, f, ss);
      }
    const float inv = 1.0f / fmaxf(__builtin_sqrtf(sum_halves(ss)), 1e-6f);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) nb[ks][e] = f32_to_half<F16>(half_to_f32<F16>(r[ks][e]) * inv);
  };
  __syncthreads();                             // counts and patch state cleared

  // Assignment, one super-chunk of 64 seeds at a time.
  for (int sc = 0; sc < nsc; ++sc) {
    const int g0 = sc * kMaxPool;
    bf16x8 seed[2][4];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int g = g0 + sb * 32 + l32;
      const int gc = g < a.npool ? g : a.npool - 1;
      const int gy = gc / a.nw, gx = gc % a.nw;
      bf16x8 r[4];
      load_half(K, a.k_sn, gy * a.kp * a.gw + gx * a.kp, r);
      normalise(r, seed[sb]);
      if (g >= a.npool)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) seed[sb][ks] = bf16x8{};
    }
    // This wave's next two tiles in registers (one slot per unrolled step),
    // so two tiles' loads are in flight while one is scored.
    bf16x8 ring[kManyAhead][4];
#pragma unroll
    for (int j = 0; j < kManyAhead; ++j) {
      const int pj = (wave + kPoolWaves * j) * 32 + l32;
      load_half(K, a.k_sn, pj < npatch ? pj : npatch - 1, ring[j]);
    }
    auto assign_tile = [&](const int t, bf16x8 (&slot)[4]) {
      const int p = t * 32 + l32;
      const bool valid = p < npatch;
      bf16x8 rx[4], xb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) rx[ks] = slot[ks];
      const int pn = p + 32 * kPoolWaves * kManyAhead;
      load_half(K, a.k_sn, pn < npatch ? pn : npatch - 1, slot);
      normalise(rx, xb);
      float bv = -INFINITY;
      int bi = g0;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        f32x16 sc16 = {};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) sc16 = mfma32x32x16_t<F16>(seed[sb][ks], xb[ks], sc16);
#pragma unroll
        for (int r = 0; r < 16; ++r) {         // seeds in increasing order
          const int g = g0 + sb * 32 + mfma_row(r, hi);
          const float v = round16<F16>(sc16[r]);
          if (g < a.npool && v > bv) {
            bv = v;
            bi = g;
          }
        }
      }
      const float pb = __shfl_xor(bv, 32);
      const int pi = __shfl_xor(bi, 32);
      if (pb > bv || (pb == bv && pi < bi)) {
        bv = pb;
        bi = pi;
      }
      // This wave owns tile t in every chunk, so its LDS updates are ordered.
      if (hi == 0 && valid && bv > best[p]) {
        best[p] = bv;
        asg[p] = (uint16_t)bi;
      }
    };
    static_assert(kManyAhead == 2, "the loop below is unrolled over two slots");
    for (int t = wave; t < ntile; t += kPoolWaves * kManyAhead) {
      assign_tile(t, ring[0]);
      if (t + kPoolWaves >= ntile) break;
      assign_tile(t + kPoolWaves, ring[1]);
    }
  }
  __syncthreads();                             // assignment final; `best` is dead from here
  for (int p = tid; p < npatch; p += kPoolThreads) {
    uint16_t g = asg[p];
    if (g == kNoSeed) {                        // every score NaN: seed 0
      g = 0;
      asg[p] = 0;
    }
    atomicAdd(&count[g], 1);
    if (AS) AS[(int64_t)grp * npatch + p] = g;
  }
  __syncthreads();

  if (nsc <= kOneHotChunks) {
    uint16_t(&st)[32][kStage] = stage[wave];
    // One-hot sums of a tile for the seeds g0 .. g0+63 (see sum_tile above).
    auto sum_tile = [&](int t, int g0, bool valid, const bf16x8 (&rx)[4], f32x16 (&acc)[2][2]) {
#pragma unroll
      for (int fh = 0; fh < 2; ++fh) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
          *reinterpret_cast<bf16x8*>(&st[l32][16 * c + 8 * hi]) = valid ? rx[2 * fh + c] : bf16x8{};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int r0 = 16 * kk + 8 * hi;       // rows r0 .. r0+7 of the tile
          const u32x4 ab = *reinterpret_cast<const u32x4*>(&asg[t * 32 + r0]);
          u32x4 bx;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            bx[q] = (uint32_t)st[r0 + 2 * q][l32] | ((uint32_t)st[r0 + 2 * q + 1][l32] << 16);
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) {
            const uint32_t id = (uint32_t)(g0 + sb * 32 + l32);
            u32x4 oh;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t b0 = ab[q] & 0xffffu, b1 = ab[q] >> 16;
              oh[q] = (b0 == id ? kOne16<F16> : 0u) | (b1 == id ? kOne16<F16> << 16 : 0u);
            }
            acc[fh][sb] = mfma32x32x16_t<F16>(__builtin_bit_cast(bf16x8, oh),
                                              __builtin_bit_cast(bf16x8, bx), acc[fh][sb]);
          }
        }
      }
    };
    auto reduce_store = [&](f32x16 (&acc)[2][2], int g0, uint16_t* out) {
      const int ng = min(kMaxPool, a.npool - g0);
#pragma unroll
      for (int fh = 0; fh < 2; ++fh) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int r = 0; r < 16; ++r) red[wave][sb * 32 + mfma_row(r, hi)][l32] = acc[fh][sb][r];
        __syncthreads();
        for (int e = tid; e < ng * 32; e += kPoolThreads) {
          const int g = e >> 5, f = e & 31;
          const float sum = ((red[0][g][f] + red[1][g][f]) + red[2][g][f]) + red[3][g][f];
          const float inv = 1.0f / fmaxf((float)count[g0 + g], 1.0f);
          out[(out_row0 + g0 + g) * kPoolD + 32 * fh + f] =
              __builtin_bit_cast(uint16_t, f32_to_half<F16>(sum * inv));
        }
        __syncthreads();
      }
    };
    auto sweep = [&](const uint16_t* X, int64_t x_sn, int g0, uint16_t* out) {
      f32x16 acc[2][2] = {};
      bf16x8 ring[kManyAhead][4];
#pragma unroll
      for (int j = 0; j < kManyAhead; ++j) {
        const int pj = (wave + kPoolWaves * j) * 32 + l32;
        load_half(X, x_sn, pj < npatch ? pj : npatch - 1, ring[j]);
      }
      auto step = [&](const int t, bf16x8 (&slot)[4]) {
        const int p = t * 32 + l32;
        const bool valid = p < npatch;
        bf16x8 rx[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) rx[ks] = slot[ks];
        const int pn = p + 32 * kPoolWaves * kManyAhead;
        load_half(X, x_sn, pn < npatch ? pn : npatch - 1, slot);
        sum_tile(t, g0, valid, rx, acc);
      };
      for (int t = wave; t < ntile; t += kPoolWaves * kManyAhead) {
        step(t, ring[0]);
        if (t + kPoolWaves >= ntile) break;
        step(t + kPoolWaves, ring[1]);
      }
      reduce_store(acc, g0, out);
    };
    for (int sc = 0; sc < nsc; ++sc) {
      sweep(K, a.k_sn, sc * kMaxPool, PK);
      sweep(Vp, a.v_sn, sc * kMaxPool, PV);
    }
  } else {
    // Members of every seed in increasing patch order: the offsets are the
    // exclusive scan of the counts (wave 0), the member list a bitonic sort of
    // the keys (seed << 12 | patch) of all patches (unique keys, so the order
    // is fixed).  Both live in `area`, free now that the assignment is final.
    uint32_t* const keys = reinterpret_cast<uint32_t*>(area);            // [n2 <= 4096]
    int* const off = reinterpret_cast<int*>(area) + kMaxPatches;          // [npool + 1]
    int n2 = 32;
    while (n2 < npatch) n2 <<= 1;
    for (int i = tid; i < n2; i += kPoolThreads)
      keys[i] = i < npatch ? ((uint32_t)asg[i] << 12) | (uint32_t)i : 0xffffffffu;
    if (wave == 0) {
      const int per = (a.npool + 63) / 64, g_lo = lane * per;
      const int g_hi = min(g_lo + per, a.npool);
      int run = 0;
      for (int g = g_lo; g < g_hi; ++g) run += count[g];
      int incl = run;                            // inclusive scan over the lanes' totals
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
      }
      run = incl - run;
      for (int g = g_lo; g < g_hi; ++g) {
        off[g] = run;
        run += count[g];
      }
      if (lane == 63) off[a.npool] = incl;
    }
    // Each thread owns pairs tid, tid + 256, ... of a stage (at most eight) and
    // loads all of them before it writes any.
    const int npair = n2 >> 1;
    for (int k2 = 2; k2 <= n2; k2 <<= 1)
      for (int j2 = k2 >> 1; j2 > 0; j2 >>= 1) {
        __syncthreads();
        uint32_t x[kMaxPatches / 2 / kPoolThreads], y[kMaxPatches / 2 / kPoolThreads];
#pragma unroll
        for (int u = 0; u < kMaxPatches / 2 / kPoolThreads; ++u) {
          const int q = tid + u * kPoolThreads;
          const int i = ((q & ~(j2 - 1)) << 1) | (q & (j2 - 1));
          if (q < npair) {
            x[u] = keys[i];
            y[u] = keys[i + j2];
          }
        }
#pragma unroll
        for (int u = 0; u < kMaxPatches / 2 / kPoolThreads; ++u) {
          const int q = tid + u * kPoolThreads;
          const int i = ((q & ~(j2 - 1)) << 1) | (q & (j2 - 1));
          if (q < npair && (x[u] > y[u]) == ((i & k2) == 0)) {
            keys[i] = y[u];
            keys[i + j2] = x[u];
          }
        }
      }
    __syncthreads();
  
    // Group sums.  The 16 lane groups (16 lanes, four features per lane) each
    // take a contiguous range of seeds, i.e. of sorted positions, and stream
    // it eight rows at a time (all loads of a batch issued before any add),
    // adding each seed's member rows in increasing patch order (fp32): every
    // mean has one fixed summation order, and each K and V row is read once.
    // A seed is written when its run of positions ends; seeds without
    // members in between get zeros (mean of nothing, as the count clamp of
    // the smaller-seed kernels gives).
    {
      const int sub = lane >> 4, f4 = (lane & 15) * 4;
      const int G = wave * 4 + sub;
      const int gs = (int)((int64_t)a.npool * G / 16), ge = (int)((int64_t)a.npool * (G + 1) / 16);
      const int q0 = off[gs], q1 = off[ge];
      int g = gs;
      float sk[4] = {0.f, 0.f, 0.f, 0.f}, sv[4] = {0.f, 0.f, 0.f, 0.f};
      auto put = [&](int gg, const float (&xk)[4], const float (&xv)[4], float inv) {
        const bf16x2 k01 = pack2<F16>(xk[0] * inv, xk[1] * inv), k23 = pack2<F16>(xk[2] * inv, xk[3] * inv);
        const bf16x2 v01 = pack2<F16>(xv[0] * inv, xv[1] * inv), v23 = pack2<F16>(xv[2] * inv, xv[3] * inv);
        *reinterpret_cast<u32x2*>(PK + (out_row0 + gg) * kPoolD + f4) =
            u32x2{__builtin_bit_cast(uint32_t, k01), __builtin_bit_cast(uint32_t, k23)};
        *reinterpret_cast<u32x2*>(PV + (out_row0 + gg) * kPoolD + f4) =
            u32x2{__builtin_bit_cast(uint32_t, v01), __builtin_bit_cast(uint32_t, v23)};
      };
      // Finish seed g, zero the seeds up to `upto` (exclusive), start `upto`.
      auto flush = [&](int upto) {
        put(g, sk, sv, 1.0f / fmaxf((float)(off[g + 1] - off[g]), 1.0f));
        const float z[4] = {0.f, 0.f, 0.f, 0.f};
        for (int e = g + 1; e < upto; ++e) put(e, z, z, 1.0f);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          sk[c] = 0.f;
          sv[c] = 0.f;
        }
        g = upto;
      };
      // Two batches of eight rows: the loads of the next batch are in flight
      // while the current one is added.
      constexpr int kBatch = 8;
      struct Batch {
        uint32_t kk[kBatch];
        u32x2 kr[kBatch], vr[kBatch];
      };
      auto load = [&](int q, Batch& bt) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          bt.kk[u] = q + u < q1 ? keys[q + u] : 0u;
          const int p = (int)(bt.kk[u] & 0xfffu);
          bt.kr[u] = q + u < q1 ? *reinterpret_cast<const u32x2*>(K + (int64_t)p * a.k_sn + f4) : u32x2{};
          bt.vr[u] = q + u < q1 ? *reinterpret_cast<const u32x2*>(Vp + (int64_t)p * a.v_sn + f4) : u32x2{};
        }
      };
      auto add = [&](int q, const Batch& bt) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          if (q + u < q1) {
            const int gg = (int)(bt.kk[u] >> 12);
            if (gg != g) flush(gg);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              sk[2 * e] += half_to_f32<F16>(__builtin_bit_cast(__bf16, (uint16_t)(bt.kr[u][e] & 0xffffu)));
              sk[2 * e + 1] += half_to_f32<F16>(__builtin_bit_cast(__bf16, (uint16_t)(bt.kr[u][e] >> 16)));
              sv[2 * e] += half_to_f32<F16>(__builtin_bit_cast(__bf16, (uint16_t)(bt.vr[u][e] & 0xffffu)));
              sv[2 * e + 1] += half_to_f32<F16>(__builtin_bit_cast(__bf16, (uint16_t)(bt.vr[u][e] >> 16)));
            }
          }
        }
      };
      Batch b0, b1;
      if (q0 < q1) load(q0, b0);
      for (int q = q0; q < q1; q += 2 * kBatch) {
        if (q + kBatch < q1) load(q + kBatch, b1);
        add(q, b0);
        if (q + kBatch >= q1) break;
        if (q + 2 * kBatch < q1) load(q + 2 * kBatch, b0);
        add(q + kBatch, b1);
      }
      if (gs < ge) flush(ge);
    }
  }
  for (int g = tid; g < a.npool; g += kPoolThreads) SZ[out_row0 + g] = (float)count[g];
}

}  // namespace
}  // namespace gpa

using namespace gpa;

namespace {

// Shared by the bf16 and fp16 entry points; `fn` names the entry point in
// error messages.
template <bool F16>
int pool_run(const char* fn, const void* k, const void* v, void* pooled_k, void* pooled_v,
             float* size, int32_t* assign, int64_t B, int64_t H, int64_t S, int64_t P,
             int64_t pts, int64_t grid_h, int64_t grid_w, int64_t kp, int64_t D, int64_t k_sb,
             int64_t k_sh, int64_t k_sn, int64_t v_sb, int64_t v_sh, int64_t v_sn,
             void* stream) {
  gpa_clear_error();
  if (B < 0 || H < 0 || S < 0 || P < 0 || pts < 0 || grid_h < 0 || grid_w < 0 || kp <= 0) {
    gpa_set_error("%s: negative size or kp <= 0", fn);
    return GPA_E_INVALID;
  }
  if (D != kPoolD) {
    gpa_set_error("%s: head dim %lld unsupported (64 only)", fn, (long long)D);
    return GPA_E_UNSUPPORTED;
  }
  if (B == 0 || H == 0 || S == 0 || grid_h == 0 || grid_w == 0) return GPA_OK;
  if (!k || !v || !pooled_k || !pooled_v || !size) {
    gpa_set_error("%s: null pointer", fn);
    return GPA_E_INVALID;
  }
  if (P < pts + grid_h * grid_w) {
    gpa_set_error("%s: frame of %lld tokens cannot hold %lld specials and a "
                  "%lldx%lld patch grid", fn, (long long)P, (long long)pts, (long long)grid_h,
                  (long long)grid_w);
    return GPA_E_INVALID;
  }
  const int64_t nh = (grid_h + kp - 1) / kp, nw = (grid_w + kp - 1) / kp;
  if (grid_h * grid_w > kMaxPatches) {
    gpa_set_error("%s: %lld patches exceed the kernel's 4096", fn,
                  (long long)(grid_h * grid_w));
    return GPA_E_UNSUPPORTED;
  }
  const bool aligned = (uintptr_t)k % 16 == 0 && (uintptr_t)v % 16 == 0 &&
                       (B == 1 || (k_sb % 8 == 0 && v_sb % 8 == 0)) &&
                       (H == 1 || (k_sh % 8 == 0 && v_sh % 8 == 0)) && k_sn % 8 == 0 &&
                       v_sn % 8 == 0 && k_sn >= D && v_sn >= D;
  if (!aligned) {
    gpa_set_error("%s: k and v rows must be 16-byte aligned, unit feature "
                  "stride", fn);
    return GPA_E_INVALID;
  }
  const int64_t groups = B * H * S;
  if (groups > 0x7fffffff) {
    gpa_set_error("%s: too many groups", fn);
    return GPA_E_UNSUPPORTED;
  }
  PoolArgs a{};
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.pk = (uint16_t*)pooled_k;
  a.pv = (uint16_t*)pooled_v;
  a.size = size;
  a.assign = assign;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_sn = k_sn;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_sn = v_sn;
  a.H = (int)H; a.S = (int)S; a.P = (int)P; a.pts = (int)pts;
  a.gh = (int)grid_h; a.gw = (int)grid_w;
  a.kp = (int)kp; a.nw = (int)nw; a.npool = (int)(nh * nw);
  if (a.npool > kMaxPool)
    hipLaunchKernelGGL((pool_many_kernel<F16>), dim3((unsigned)groups), dim3(kPoolThreads), 0,
                       (hipStream_t)stream, a);
  else if (a.npool > 32)
    hipLaunchKernelGGL((pool_shared_kernel<2, F16>), dim3((unsigned)groups), dim3(kPoolThreads), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((pool_shared_kernel<1, F16>), dim3((unsigned)groups), dim3(kPoolThreads), 0,
                       (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("%s: launch failed: %s", fn, hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}

}  // namespace

#define GPA_POOL_ARGS                                                                         \
  const void *k, const void *v, void *pooled_k, void *pooled_v, float *size, int32_t *assign, \
      int64_t B, int64_t H, int64_t S, int64_t P, int64_t pts, int64_t grid_h, int64_t grid_w, \
      int64_t kp, int64_t D, int64_t k_sb, int64_t k_sh, int64_t k_sn, int64_t v_sb,          \
      int64_t v_sh, int64_t v_sn, void *stream
#define GPA_POOL_PASS                                                                         \
  k, v, pooled_k, pooled_v, size, assign, B, H, S, P, pts, grid_h, grid_w, kp, D, k_sb, k_sh, \
      k_sn, v_sb, v_sh, v_sn, stream

extern "C" int gpa_pool_shared_bf16(GPA_POOL_ARGS) {
  return pool_run<false>("gpa_pool_shared_bf16", GPA_POOL_PASS);
}

extern "C" int gpa_pool_shared_f16(GPA_POOL_ARGS) {
  return pool_run<true>("gpa_pool_shared_f16", GPA_POOL_PASS);
}
