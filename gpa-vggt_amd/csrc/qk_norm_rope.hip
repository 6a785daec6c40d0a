// Fused qk LayerNorm + 2D rotary embedding + cast: the attention operands of
// a VGGT block straight from its QKV projection.
//
// For every token n and head h of the projection rows qkv[b, n, :]
// (q at column h*64, k at column k_offset + h*64), with x the 64 bf16
// features:
//
//   y = (x - mean(x)) / sqrt(var(x) + eps) * w + beta          (fp32)
//   out[j]      = y[j] cos(p a_j) - y[j+16] sin(p a_j)   j in [0,16) of each 32-half
//   out[j + 16] = y[j+16] cos(p a_j) + y[j] sin(p a_j)
//
// where the first 32 features rotate with the token's row coordinate and the
// last 32 with its column coordinate (p from pos[n mod period]), and the
// (cos, sin) of p * a_j come from a host-built table.  Output is written
// head-major [B, H, N, 64], the layout of the attention kernel and of the
// K/V merge, once, in bf16 or fp32.
//
// This replaces the torch op sequence of vggt/layers/attention.py:210-220
// (q_norm / k_norm LayerNorm, then vggt/layers/rope.py:167-209 on q and k,
// then the bf16 cast of merging/fused_attention.py:139-144): about ten
// passes over fp32 [B, H, N, 64] tensors become one read of the bf16
// projection and one write.
//
// Work split: eight lanes own one (token, head, q|k) row, 16 bytes each;
// the LayerNorm moments and the rotation partner (feature j <-> j+16 is lane
// c <-> c^2 within the eight) are cross-lane exchanges, done with DPP
// operand modifiers (quad permutes and the half-row mirror) rather than
// ds_bpermute.  The 32 lane groups of a workgroup own 32 consecutive
// (q|k, head) slices -- all of them at 16 heads -- of eight consecutive
// tokens, so each pass reads 4 KB of consecutive projection columns (one
// token's q and k), all eight loads issued before any arithmetic.  The
// projection is read and the outputs written with nontemporal hints (each
// byte is touched once).  Measured on the 200-frame shape: 4.4 TB/s (bf16
// out) and 4.7 TB/s (fp32 k) of read + write traffic, against 5.2 TB/s for
// a plain device copy; four tokens per workgroup with ds_bpermute exchanges
// and cached accesses ran 0.54 / 0.65 ms against 0.51 / 0.60 ms now.
// Reading 128-byte pieces of 6 KB-strided rows instead (one head, many
// tokens per workgroup) ran 11 % slower; one 16-byte load per lane in
// flight held the kernel to ~3 TB/s.  HBM-bound.
#include "gpa_common.h"

namespace gpa {
namespace {

constexpr int kThreads = 256;
constexpr int kLanesPerRow = 8;
constexpr int kSlicesPerBlock = kThreads / kLanesPerRow;   // 32 (q|k, head) slices
constexpr int kTokens = 8;                                 // tokens per workgroup
constexpr int kHeadDim = 64;

struct QkArgs {
  const uint16_t* qkv;
  int64_t sb, sn, k_offset;
  const float* w;      // [2][64]: q then k
  const float* beta;   // [2][64]
  float eps;
  const int32_t* pos;  // [period][2] or null (no rotation)
  int64_t period;
  const float* cs;     // [npos][16][2] (cos, sin)
  int32_t npos;
  void* q_out;
  void* k_out;
  int q_f32, k_f32;
  int64_t B, N, H;
  int64_t rows;        // B * N
};

// Lane exchanges inside eight-lane groups through DPP (a VALU operand
// modifier) rather than ds_bpermute round trips through the LDS unit.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kHalfMirror = 0x141; // row_half_mirror: lane i <-> 7 - i within 8

// Sum over the eight lanes of a group: quad sums, then the other quad's sum
// (whose lanes the half-row mirror pairs with this quad's).
__device__ __forceinline__ float group_sum8(float v) {
  v += dpp<kQuadSwap1>(v);
  v += dpp<kQuadSwap2>(v);
  v += dpp<kHalfMirror>(v);
  return v;
}

// F16: the projection and the 16-bit outputs are fp16 (the fp16-autocast
// stack) instead of bf16; the arithmetic is the same fp32.
template <bool F16>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(QkArgs a) {
  // Lane group g owns slice 32*blockIdx.y + g (q heads, then k heads) for
  // the kTokens tokens of blockIdx.x; groups past 2H load the last slice
  // and store nothing.  Token numbers fit 32 bits (checked on the host),
  // which keeps the index arithmetic off the 64-bit division path.
  const int c = threadIdx.x % kLanesPerRow;    // features 8c .. 8c+7
  const uint32_t g = threadIdx.x / kLanesPerRow;
  const uint32_t H = (uint32_t)a.H, N = (uint32_t)a.N;
  const uint32_t slice = blockIdx.y * (uint32_t)kSlicesPerBlock + g;
  const bool slice_ok = slice < 2 * H;
  const uint32_t sl = slice_ok ? slice : 2 * H - 1;
  const int which = sl < H ? 0 : 1;            // 0: q, 1: k
  const uint32_t h = which ? sl - H : sl;
  const int64_t col = (which ? a.k_offset : 0) + (int64_t)h * kHeadDim + c * 8;
  const uint32_t tok0 = blockIdx.x * (uint32_t)kTokens;
  const uint32_t last = (uint32_t)(a.rows - 1);

  bf16x8 xv[kTokens];
#pragma unroll
  for (int r = 0; r < kTokens; ++r) {
    const uint32_t row = min(tok0 + r, last);   // every lane joins the exchanges
    const uint32_t b = row / N, n = row - b * N;
    const u32x4* src =
        reinterpret_cast<const u32x4*>(a.qkv + (int64_t)b * a.sb + (int64_t)n * a.sn + col);
    xv[r] = __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(src));
  }
  const float* w = a.w + which * kHeadDim + c * 8;
  const float* be = a.beta + which * kHeadDim + c * 8;
  void* out = which ? a.k_out : a.q_out;
  const bool out_f32 = which ? a.k_f32 : a.q_f32;

#pragma unroll
  for (int r = 0; r < kTokens; ++r) {
    const bool valid = slice_ok && tok0 + r <= last;
    const uint32_t row = min(tok0 + r, last);
    const uint32_t b = row / N, n = row - b * N;
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = half_to_f32<F16>(xv[r][i]);

    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += x[i];
    const float mean = group_sum8(s) * (1.0f / kHeadDim);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] -= mean;
      ss += x[i] * x[i];
    }
    const float rstd = rsqrtf(group_sum8(ss) * (1.0f / kHeadDim) + a.eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = x[i] * rstd * w[i] + be[i];

    if (a.pos != nullptr) {
      int p = a.pos[(n % (uint32_t)a.period) * 2 + (c >= 4 ? 1 : 0)];
      p = p < 0 ? 0 : (p >= a.npos ? a.npos - 1 : p);
      const float sgn = (c & 2) ? 1.0f : -1.0f;   // second quarter of a half: +, first: -
      const float2* cs = reinterpret_cast<const float2*>(a.cs) + (int64_t)p * 16 + (c & 1) * 8;
      float partner[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) partner[i] = dpp<kQuadSwap2>(x[i]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float2 t = cs[i];
        x[i] = __builtin_fmaf(x[i], t.x, sgn * partner[i] * t.y);
      }
    }
    if (!valid) continue;

    const int64_t o = (((int64_t)b * H + h) * N + n) * kHeadDim + c * 8;
    if (out_f32) {
      f32x4* dst = reinterpret_cast<f32x4*>(static_cast<float*>(out) + o);
      __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, dst);
      __builtin_nontemporal_store(f32x4{x[4], x[5], x[6], x[7]}, dst + 1);
    } else {
      bf16x8 yv;
#pragma unroll
      for (int i = 0; i < 8; ++i) yv[i] = f32_to_half<F16>(x[i]);
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, yv),
                                  reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + o));
    }
  }
}

}  // namespace
}  // namespace gpa

using namespace gpa;

namespace {

// Shared by the bf16 and fp16 entry points (F16 selects the 16-bit format of
// the projection and of 16-bit outputs); `fn` names the entry point in error
// messages.
template <bool F16>
int qk_run(const char* fn, const void* qkv, int64_t B, int64_t N, int64_t H, int64_t D,
           int64_t qkv_sb, int64_t qkv_sn, int64_t k_offset, const float* ln_weight,
           const float* ln_bias, float eps, const int32_t* pos, int64_t period,
           const float* rope_cs, int64_t npos, void* q_out, int q_dtype, void* k_out,
           int k_dtype, void* stream) {
  gpa_clear_error();
  if (B < 0 || N < 0 || H < 0) {
    gpa_set_error("%s: negative size", fn);
    return GPA_E_INVALID;
  }
  if (D != kHeadDim) {
    gpa_set_error("%s: head dim %lld is not implemented (64 only)", fn, (long long)D);
    return GPA_E_UNSUPPORTED;
  }
  if (B == 0 || N == 0 || H == 0) return GPA_OK;
  if (!qkv || !ln_weight || !ln_bias || !q_out || !k_out) {
    gpa_set_error("%s: null pointer", fn);
    return GPA_E_INVALID;
  }
  if (pos != nullptr && (period <= 0 || rope_cs == nullptr || npos <= 0 || npos > (1 << 20))) {
    gpa_set_error("%s: rotation needs period > 0, a table and 0 < npos <= 2^20", fn);
    return GPA_E_INVALID;
  }
  const int half = F16 ? GPA_DTYPE_F16 : GPA_DTYPE_BF16;
  for (int dt : {q_dtype, k_dtype}) {
    if (dt != GPA_DTYPE_F32 && dt != half) {
      gpa_set_error("%s: output dtype %d is not fp32 or %s", fn, dt, F16 ? "fp16" : "bf16");
      return GPA_E_UNSUPPORTED;
    }
  }
  const bool aligned = (uintptr_t)qkv % 16 == 0 && (uintptr_t)q_out % 16 == 0 &&
                       (uintptr_t)k_out % 16 == 0 && (B == 1 || qkv_sb % 8 == 0) &&
                       (N == 1 || qkv_sn % 8 == 0) && k_offset % 8 == 0 && k_offset >= H * D;
  if (!aligned) {
    gpa_set_error("%s: rows must be 16-byte aligned and k must follow q (k_offset >= H*64, "
                  "multiple of 8)", fn);
    return GPA_E_INVALID;
  }
  if (2 * H > 65535) {
    gpa_set_error("%s: too many heads", fn);
    return GPA_E_UNSUPPORTED;
  }
  QkArgs a{};
  a.qkv = (const uint16_t*)qkv;
  a.sb = qkv_sb; a.sn = qkv_sn; a.k_offset = k_offset;
  a.w = ln_weight; a.beta = ln_bias; a.eps = eps;
  a.pos = pos; a.period = period; a.cs = rope_cs; a.npos = (int32_t)npos;
  a.q_out = q_out; a.k_out = k_out;
  a.q_f32 = q_dtype == GPA_DTYPE_F32; a.k_f32 = k_dtype == GPA_DTYPE_F32;
  a.B = B; a.N = N; a.H = H; a.rows = B * N;
  const int64_t blocks = (a.rows + kTokens - 1) / kTokens;
  const int64_t sblocks = (2 * H + kSlicesPerBlock - 1) / kSlicesPerBlock;
  if (a.rows > 0xffffffffLL - kTokens || blocks > 0x7fffffff || period > 0x7fffffff) {
    gpa_set_error("%s: problem exceeds the grid limit", fn);
    return GPA_E_UNSUPPORTED;
  }
  hipLaunchKernelGGL(qk_norm_rope_kernel<F16>, dim3((unsigned)blocks, (unsigned)sblocks),
                     dim3(kThreads), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("%s: launch failed: %s", fn, hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}

}  // namespace

#define GPA_QK_ARGS                                                                          \
  const void *qkv, int64_t B, int64_t N, int64_t H, int64_t D, int64_t qkv_sb, int64_t qkv_sn, \
      int64_t k_offset, const float *ln_weight, const float *ln_bias, float eps,              \
      const int32_t *pos, int64_t period, const float *rope_cs, int64_t npos, void *q_out,    \
      int q_dtype, void *k_out, int k_dtype, void *stream
#define GPA_QK_PASS                                                                          \
  qkv, B, N, H, D, qkv_sb, qkv_sn, k_offset, ln_weight, ln_bias, eps, pos, period, rope_cs,  \
      npos, q_out, q_dtype, k_out, k_dtype, stream

extern "C" int gpa_qk_norm_rope_bf16(GPA_QK_ARGS) {
  return qk_run<false>("gpa_qk_norm_rope_bf16", GPA_QK_PASS);
}

extern "C" int gpa_qk_norm_rope_f16(GPA_QK_ARGS) {
  return qk_run<true>("gpa_qk_norm_rope_f16", GPA_QK_PASS);
}
