// Register-only probes of what the power limit leaves for an instruction mix.
//
// Not part of the product library (it is built into libgpa_probe.so, which
// only the benchmark loads).  Each wave runs `iters` steps of one of these
// mixes on fragments it loaded once from `src`, with no memory traffic in
// the loop, and writes one float per lane at the end so nothing is dead:
//
//   mode 0  8 x v_mfma_f32_32x32x16_bf16 per step
//   mode 1  16 x v_mfma_f32_16x16x32_bf16 per step (the same FLOPs)
//   mode 2  one key tile of the attention main loop for a wave's two
//           32-query blocks: S of the next tile (8 x 32x32x16, the C operand
//           starting from a bias row), the softmax of the current scores
//           (32 FMA + 32 exp2 + 16 bf16 packs per lane, in the
//           exponent domain with a fixed offset), their row sums (8 x
//           4x4x4 with a ones operand) and O += V^T P (8 x 32x32x16), one
//           MFMA to three VALU instructions as the kernel interleaves them.
//
// Modes 0 and 1 count 262,144 FLOP per wave and step, mode 2 the tile's
// 16 x 32x32x16 = 524,288 (the attention's algorithmic work; the row sums
// are not counted, as the attention does not count them).  With random
// operands the multipliers toggle as on real data, so the time these take
// is the ceiling the power limit sets for the mix; with all-zero operands
// the clock stays high.  K and V fragments stay fixed across steps (the
// kernel reads new ones from LDS each tile).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGrid = 512;   // two workgroups of four waves per CU on 256 CUs

__device__ __forceinline__ bf16x8 frag(const bf16x8* src, int64_t n, int64_t i) {
  return src[i % n];
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void mix_probe(const bf16x8* __restrict__ src, int64_t nsrc,
                                                   float* __restrict__ out, int iters) {
  // 64 KB of LDS per workgroup caps every mode at two workgroups per CU,
  // two waves per SIMD, as the attention runs.
  __shared__ float pad[16384];
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int64_t base = (int64_t)gid * 32;
  pad[threadIdx.x * 64] = 0.f;
  __syncthreads();
  float acc_sum = pad[(threadIdx.x * 64 + 64) & 16383];
  if constexpr (MODE == 0) {
    bf16x8 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = frag(src, nsrc, base + i);
      b[i] = frag(src, nsrc, base + 8 + i);
    }
    f32x16 acc[4] = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[7 - i], acc[i & 3], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_sum += acc[j][r];
  } else if constexpr (MODE == 1) {
    bf16x8 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = frag(src, nsrc, base + i);
      b[i] = frag(src, nsrc, base + 8 + i);
    }
    f32x4 acc[8] = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc[i & 7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i & 7], b[7 - (i & 7)], acc[i & 7],
                                                             0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc_sum += acc[j][r];
  } else {
    bf16x8 qf[2][4], kf[4], vf[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qf[j][ks] = frag(src, nsrc, base + 4 * j + ks);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kf[ks] = frag(src, nsrc, base + 8 + ks);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) vf[db][s] = frag(src, nsrc, base + 12 + 2 * db + s);
    f32x16 bias16;
#pragma unroll
    for (int r = 0; r < 16; ++r) bias16[r] = 0.25f * (float)((threadIdx.x + r) & 7);
    const float c = 0.125f * 1.4426950408889634f, neg_m = -4.0f;
    const __bf16 one = (__bf16)1.0f;
    const bf16x4 ones4 = {one, one, one, one};
    f32x16 sa[2] = {}, sb[2] = {}, o[2][2] = {};
    f32x4 l[2] = {};
    // One tile: S of the next tile into s_nxt beside the softmax of s_cur,
    // its row sums and its P.V product.  Two tiles per loop trip with the
    // score buffers swapping roles, so no register copy joins the mix.
    auto tile = [&](f32x16 (&s_cur)[2], f32x16 (&s_nxt)[2]) __attribute__((always_inline)) {
      __builtin_amdgcn_sched_barrier(0);
      // The operands stand for a new tile's fragments: opaque to the
      // compiler, so no product is hoisted out of the loop.
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) asm volatile("" : "+v"(kf[ks]));
#pragma unroll
      for (int db = 0; db < 2; ++db) asm volatile("" : "+v"(vf[db][0]), "+v"(vf[db][1]));
      asm volatile("" : "+v"(bias16));
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          s_nxt[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[j][ks],
                                                            ks == 0 ? bias16 : s_nxt[j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bf16x8 pb[2];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[j][8 * half + e], c, neg_m));
            const float p1 =
                __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[j][8 * half + e + 1], c, neg_m));
            const bf16x2 pv = {(__bf16)p0, (__bf16)p1};
            pb[half][e] = pv[0];
            pb[half][e + 1] = pv[1];
          }
          const bf16x4 lo = {pb[half][0], pb[half][1], pb[half][2], pb[half][3]};
          const bf16x4 up = {pb[half][4], pb[half][5], pb[half][6], pb[half][7]};
          l[j] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(ones4, lo, l[j], 0, 0, 0);
          l[j] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(ones4, up, l[j], 0, 0, 0);
        }
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int s = 0; s < 2; ++s)
            o[j][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][s], pb[s], o[j][db], 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 24; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // three VALU
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        asm volatile("" : "+v"(s_nxt[j]), "+v"(l[j]));
        asm volatile("" : "+v"(o[j][0]), "+v"(o[j][1]));
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int it = 0; it < iters; it += 2) {
      tile(sa, sb);
      tile(sb, sa);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc_sum += l[j][0];
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_sum += o[j][db][r];
    }
  }
  out[gid] = acc_sum;
}

}  // namespace

// Launches mode `mode` (0, 1, 2) on `stream`: kGrid workgroups of 256
// threads, fragments read from src[0 .. nsrc) (16-byte elements, wrapped),
// one float per thread into out[0 .. gpa_probe_threads()).  Returns 0, or -1
// for invalid arguments, -4 if the launch failed.
extern "C" int gpa_probe_threads(void) { return kGrid * 256; }

extern "C" double gpa_probe_flops(int mode, int iters) {
  const double per_step = (mode == 2 ? 16.0 : 8.0) * 32768.0;
  const int steps = mode == 2 ? (iters + 1) / 2 * 2 : iters;   // mode 2 runs pairs of tiles
  return (double)kGrid * 4 * steps * per_step;
}

extern "C" int gpa_probe_mfma_mix(int mode, const void* src, int64_t nsrc, float* out, int iters,
                                  void* stream) {
  if (mode < 0 || mode > 2 || !src || nsrc <= 0 || !out || iters <= 0) return -1;
  const bf16x8* s = static_cast<const bf16x8*>(src);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (mode == 0) hipLaunchKernelGGL(mix_probe<0>, dim3(kGrid), dim3(256), 0, st, s, nsrc, out, iters);
  else if (mode == 1) hipLaunchKernelGGL(mix_probe<1>, dim3(kGrid), dim3(256), 0, st, s, nsrc, out, iters);
  else hipLaunchKernelGGL(mix_probe<2>, dim3(kGrid), dim3(256), 0, st, s, nsrc, out, iters);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
