// Merge front end: the metric projection, L2 normalisation, dst/src split
// and bf16 cast of the bipartite merge in one pass over the metric.
//
// For every batch b and output row j (token t = order[j], or t = j):
//   y = bf16( bf16(x[b, t, :]) @ proj )          C -> 128, fp32 accumulation
//   n = sqrt(sum_c y_c^2)                         fp32 (rounded to bf16 in mode 1)
//   out[b, j, :] = bf16( y / n )
//
// This is merging/merge.py:180-187 as it runs inside the model, under bf16
// autocast: `metric @ proj` casts both operands to bf16 and returns bf16,
// `metric.norm` runs in fp32, the division promotes to fp32, and the split
// gathers `a = metric[..., a_idx, :]`, `b = metric[..., b_idx, :]` feed
// fused_similarity_argmax, which rounds them to bf16 (fused_similarity.py:
// 90-95).  With `order` = [dst positions | src positions] the output holds b
// followed by a, in the layout the similarity kernel reads.  Mode 1 is the
// same chain without autocast on a bf16 metric: there the norm comes back in
// bf16 before the division.  Mode 2 is the chain under fp16 autocast: the
// metric and the projection are rounded to fp16, the product runs on the
// fp16 MFMA and y is rounded to fp16 (the norm, the division and the final
// bf16 cast as in mode 0).  There is no epsilon: a zero row gives NaN, as
// in the reference.
//
// Design: HBM-bound (one read of the metric, 4 KB per token in fp32, and a
// 256-byte write), so the 1024 x 128 bf16 projection (256 KB) must not be
// re-read per tile.  A persistent grid of one 512-thread workgroup per CU
// keeps it in registers: wave w holds the B operands of output columns
// [16w, 16w+16) for all of C (C/32 MFMA k-steps, 4 VGPRs each).  16-row
// blocks of the metric stream through LDS: 32 threads load one row with
// 16-byte loads (two blocks in flight), convert to bf16 and
// store it chunk-swizzled, so the MFMA A-operand reads are conflict-free;
// each wave then runs its 16x16 output tile over the whole of C.  The row
// sums of squares meet in LDS in a fixed wave order, so the result is
// deterministic.
#include "gpa_common.h"

#include <math.h>
#include <type_traits>

namespace gpa {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = 16;   // rows per block step
constexpr int kOut = 128;   // projected width, 16 columns per wave

struct MetricArgs {
  const void* x;
  int64_t sb, sn;          // metric batch / token strides (elements)
  const uint16_t* proj;    // [C][128] bf16 bits
  const int64_t* order;    // [N] or null
  uint16_t* out;           // [rows][128] bf16 bits
  int64_t N, rows;         // rows = B * N
  int nblocks;
  int norm_bf16;
};

__device__ __forceinline__ float bf16r(float x) { return (float)(__bf16)x; }

// The projection's rounding: bf16, or fp16 under fp16 autocast.  The empty
// asm keeps the fp16 round trip a real rounding step.
template <bool P16>
__device__ __forceinline__ float proj_round(float x) {
  if constexpr (P16) {
    uint32_t u = __builtin_bit_cast(uint16_t, (_Float16)x);
    asm volatile("" : "+v"(u));
    return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
  } else {
    return bf16r(x);
  }
}

template <int C, bool F32, bool P16>
__global__ __launch_bounds__(kThreads, 1) void merge_metric_kernel(MetricArgs a) {
  static_assert(F32 || !P16, "the fp16 projection takes an fp32 metric");
  constexpr int kSteps = C / 32;                         // MFMA k-steps
  constexpr int kSpan = F32 ? 4 : 8;                     // elements per 16-byte load
  constexpr int kLoads = C / (32 * kSpan);               // loads per thread per row
  using Raw = std::conditional_t<F32, f32x4, bf16x8>;
  __shared__ __attribute__((aligned(16))) __bf16 A[kRows][C];   // chunk c of row r at c ^ r
  __shared__ __attribute__((aligned(16))) float ssq[kWaves][kRows];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int lr = tid >> 5, lc = tid & 31;                // loader: row lr, 32 threads per row
  const int col = wave * 16 + r16;

  // B operands, packed two bf16 per VGPR; the empty asm keeps them packed
  // (left alone, the compiler holds one bf16 per VGPR and repacks per use).
  u32x4 bfrag[kSteps];
#pragma unroll
  for (int ks = 0; ks < kSteps; ++ks) {
    const uint16_t* p = a.proj + (int64_t)(ks * 32 + g * 8) * kOut + col;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      bfrag[ks][q] = (uint32_t)p[2 * q * kOut] | ((uint32_t)p[(2 * q + 1) * kOut] << 16);
    asm volatile("" : "+v"(bfrag[ks]));
  }

  auto load = [&](Raw (&raw)[kLoads], int blk) {
    int64_t i = (int64_t)blk * kRows + lr;
    if (i >= a.rows) i = a.rows - 1;                     // tail rows: any valid row
    const int64_t b = i / a.N, j = i - b * a.N;
    const int64_t t = a.order ? a.order[j] : j;
    const Raw* row = reinterpret_cast<const Raw*>(
        static_cast<const char*>(a.x) + (b * a.sb + t * a.sn) * (F32 ? 4 : 2));
#pragma unroll
    for (int l = 0; l < kLoads; ++l) raw[l] = row[l * 32 + lc];
  };
  // The swizzle only permutes chunks within aligned groups of 16 (256 B), so
  // every LDS address is a per-lane base plus a compile-time offset.
  __bf16* const st_base = F32 ? &A[lr][(((lc >> 1) ^ lr) << 3) + (lc & 1) * 4]
                              : &A[lr][((lc & 15) ^ lr) << 3] + (lc >> 4) * 128;
  const __bf16* rd_base[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) rd_base[q] = &A[r16][((q * 4 + g) ^ r16) << 3];
  auto stage = [&](const Raw (&raw)[kLoads]) {
#pragma unroll
    for (int l = 0; l < kLoads; ++l) {
      if constexpr (F32) {                                 // chunk l*16 + (lc >> 1)
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f32_to_half<P16>(raw[l][e]);
        *reinterpret_cast<bf16x4*>(st_base + l * 128) = v;
      } else {                                             // chunk l*32 + lc
        *reinterpret_cast<bf16x8*>(st_base + l * 256) = raw[l];
      }
    }
  };
  auto finish = [&](int blk) {
    __syncthreads();                                     // A staged
    f32x4 acc[4] = {};
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      const bf16x8 af = *reinterpret_cast<const bf16x8*>(rd_base[ks & 3] + (ks >> 2) * 128);
      acc[ks & 3] = mfma16x16x32_t<P16>(af, __builtin_bit_cast(bf16x8, bfrag[ks]), acc[ks & 3]);
    }
    // At most four A fragments in flight: the resident projection leaves no
    // room for the compiler's habit of issuing every LDS read up front.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int ks = 4; ks < kSteps; ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    float y[4], s[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      y[r] = proj_round<P16>((acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]));   // row 4g + r
      s[r] = y[r] * y[r];
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) s[r] += __shfl_xor(s[r], m);
    }
    if (r16 == 0) *reinterpret_cast<f32x4*>(&ssq[wave][4 * g]) = f32x4{s[0], s[1], s[2], s[3]};
    __syncthreads();                                     // sums of squares in; A free
    f32x4 tot = *reinterpret_cast<const f32x4*>(&ssq[0][4 * g]);
#pragma unroll
    for (int w = 1; w < kWaves; ++w) tot += *reinterpret_cast<const f32x4*>(&ssq[w][4 * g]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t i = (int64_t)blk * kRows + 4 * g + r;
      float n = sqrtf(tot[r]);
      if (a.norm_bf16) n = bf16r(n);
      if (i < a.rows) a.out[i * kOut + col] = __builtin_bit_cast(uint16_t, (__bf16)(y[r] / n));
    }
  };

  const int G = gridDim.x;
  int blk = blockIdx.x;
  Raw raw0[kLoads], raw1[kLoads];
  load(raw0, blk);
  load(raw1, blk + G);
  for (; blk < a.nblocks; blk += 2 * G) {
    stage(raw0);
    load(raw0, blk + 2 * G);
    finish(blk);
    if (blk + G >= a.nblocks) break;                     // workgroup-uniform
    stage(raw1);
    load(raw1, blk + 3 * G);
    finish(blk + G);
  }
}

int cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int C>
void launch(bool f32, bool p16, dim3 grid, hipStream_t s, const MetricArgs& a) {
  if (p16)
    hipLaunchKernelGGL((merge_metric_kernel<C, true, true>), grid, dim3(kThreads), 0, s, a);
  else if (f32)
    hipLaunchKernelGGL((merge_metric_kernel<C, true, false>), grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((merge_metric_kernel<C, false, false>), grid, dim3(kThreads), 0, s, a);
}

}  // namespace
}  // namespace gpa

using namespace gpa;

extern "C" int gpa_merge_metric_bf16(const void* metric, int metric_dtype, int64_t B, int64_t N,
                                     int64_t C, int64_t m_sb, int64_t m_sn, const void* proj,
                                     int64_t P, const int64_t* order, int norm_mode, void* out,
                                     void* stream) {
  gpa_clear_error();
  if (B < 0 || N < 0 || C < 0) {
    gpa_set_error("gpa_merge_metric_bf16: negative size");
    return GPA_E_INVALID;
  }
  if (metric_dtype != GPA_DTYPE_F32 && metric_dtype != GPA_DTYPE_BF16) {
    gpa_set_error("gpa_merge_metric_bf16: metric dtype %d is not fp32 or bf16", metric_dtype);
    return GPA_E_UNSUPPORTED;
  }
  if (norm_mode < 0 || norm_mode > 2) {
    gpa_set_error("gpa_merge_metric_bf16: norm_mode %d is not 0, 1 or 2", norm_mode);
    return GPA_E_INVALID;
  }
  if (norm_mode == 2 && metric_dtype != GPA_DTYPE_F32) {
    gpa_set_error("gpa_merge_metric_bf16: the fp16 projection (norm_mode 2) takes an fp32 metric");
    return GPA_E_UNSUPPORTED;
  }
  if (P != kOut || (C != 256 && C != 512 && C != 768 && C != 1024)) {
    gpa_set_error("gpa_merge_metric_bf16: projection %lld -> %lld unsupported (C in "
                  "{256, 512, 768, 1024}, 128 outputs)", (long long)C, (long long)P);
    return GPA_E_UNSUPPORTED;
  }
  if (B == 0 || N == 0) return GPA_OK;
  if (!metric || !proj || !out) {
    gpa_set_error("gpa_merge_metric_bf16: null pointer");
    return GPA_E_INVALID;
  }
  const bool aligned = (uintptr_t)metric % 16 == 0 && (uintptr_t)proj % 2 == 0 &&
                       (uintptr_t)out % 2 == 0 && (B == 1 || m_sb % 8 == 0) &&
                       (N == 1 || m_sn % 8 == 0);
  if (!aligned) {
    gpa_set_error("gpa_merge_metric_bf16: metric rows must be 16-byte aligned, unit feature "
                  "stride");
    return GPA_E_INVALID;
  }
  const int64_t nblocks = (B * N + kRows - 1) / kRows;
  if (nblocks > 0x3fffffff) {
    gpa_set_error("gpa_merge_metric_bf16: too many rows");
    return GPA_E_UNSUPPORTED;
  }
  MetricArgs a{};
  a.x = metric;
  a.sb = m_sb;
  a.sn = m_sn;
  a.proj = (const uint16_t*)proj;
  a.order = order;
  a.out = (uint16_t*)out;
  a.N = N;
  a.rows = B * N;
  a.nblocks = (int)nblocks;
  a.norm_bf16 = norm_mode == 1;
  const int64_t g = nblocks < cu_count() ? nblocks : cu_count();
  const bool f32 = metric_dtype == GPA_DTYPE_F32;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)g);
  switch (C) {
    case 256: launch<256>(f32, norm_mode == 2, grid, s, a); break;
    case 512: launch<512>(f32, norm_mode == 2, grid, s, a); break;
    case 768: launch<768>(f32, norm_mode == 2, grid, s, a); break;
    default: launch<1024>(f32, norm_mode == 2, grid, s, a); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("gpa_merge_metric_bf16: launch failed: %s", hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}
