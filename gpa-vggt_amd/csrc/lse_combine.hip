// Exact merge of two attentions over a partition of the keys, by their
// log2 log-sum-exp, written straight into the token-major projection input.
//
//   m = max(la, lb),  wa = 2^(la - m),  wb = 2^(lb - m)
//   y[b, n, h*D + d] = (oa[b,h,n,d] * wa + ob[b,h,n,d] * wb) / (wa + wb)
//
// This is the combine of the frame-special split path
// (vggt/layers/attention.py:166-176): `oa`/`la` come from the own-frame
// attention, laid out frame-major ([B*S, H, P, D] and [B*S, H, P]), `ob`/`lb`
// from the shared-set attention ([B, H, N, D], [B, H, N]), N = S*P.  The
// reference permutes `oa` back to [B, H, N, D], rounds the two weights to the
// activation dtype and combines in that dtype before transposing to
// [B, N, C]; here the weights and the sum stay in fp32, one rounding to
// the output format, and the output is written once in its final layout.
// Instantiated for bf16 and for fp16 operands (the fp16-autocast evaluation
// stack); y has the operands' format.
//
// Operands are addressed per (b, h, s, p) with token n = s*P + p, so both the
// frame-major and the token-major layouts (and views of them) are plain
// strides.  HBM-bound: 16-byte loads of eight bf16 per thread.
#include "gpa_common.h"

namespace gpa {
namespace {

constexpr int kThreads = 256;

struct CombineArgs {
  const uint16_t* oa;
  const float* la;
  const uint16_t* ob;
  const float* lb;
  uint16_t* y;
  int64_t B, H, N, P, D;
  int64_t oa_b, oa_h, oa_s, oa_p;
  int64_t la_b, la_h, la_s, la_p;
  int64_t ob_b, ob_h, ob_s, ob_p;
  int64_t lb_b, lb_h, lb_s, lb_p;
  int64_t y_b, y_n, y_h;
  int64_t total;  // B * N * H * D / 8
};

template <bool F16>
__global__ __launch_bounds__(kThreads) void lse_combine_kernel(CombineArgs a) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= a.total) return;
  const int64_t dch = a.D / 8;
  const int64_t dc = i % dch;
  int64_t r = i / dch;
  const int64_t h = r % a.H;
  r /= a.H;
  const int64_t n = r % a.N, b = r / a.N;
  const int64_t s = n / a.P, p = n % a.P;

  const float la = a.la[b * a.la_b + h * a.la_h + s * a.la_s + p * a.la_p];
  const float lb = a.lb[b * a.lb_b + h * a.lb_h + s * a.lb_s + p * a.lb_p];
  const float m = fmaxf(la, lb);
  const float wa = __builtin_amdgcn_exp2f(la - m), wb = __builtin_amdgcn_exp2f(lb - m);
  const float inv = 1.0f / (wa + wb);
  const float ca = wa * inv, cb = wb * inv;

  const bf16x8 xa = *reinterpret_cast<const bf16x8*>(
      a.oa + b * a.oa_b + h * a.oa_h + s * a.oa_s + p * a.oa_p + dc * 8);
  const bf16x8 xb = *reinterpret_cast<const bf16x8*>(
      a.ob + b * a.ob_b + h * a.ob_h + s * a.ob_s + p * a.ob_p + dc * 8);
  bf16x8 yv;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    yv[j] = f32_to_half<F16>(
        __builtin_fmaf(half_to_f32<F16>(xa[j]), ca, half_to_f32<F16>(xb[j]) * cb));
  *reinterpret_cast<bf16x8*>(a.y + b * a.y_b + n * a.y_n + h * a.y_h + dc * 8) = yv;
}

}  // namespace
}  // namespace gpa

using namespace gpa;

namespace {

template <bool F16>
int lse_combine_run(const char* fn, const void* oa, const float* la, const void* ob,
                    const float* lb, void* y, int64_t B, int64_t H, int64_t N, int64_t P,
                    int64_t D, int64_t oa_b, int64_t oa_h, int64_t oa_s, int64_t oa_p,
                    int64_t la_b, int64_t la_h, int64_t la_s, int64_t la_p, int64_t ob_b,
                    int64_t ob_h, int64_t ob_s, int64_t ob_p, int64_t lb_b, int64_t lb_h,
                    int64_t lb_s, int64_t lb_p, int64_t y_b, int64_t y_n, int64_t y_h,
                    void* stream) {
  gpa_clear_error();
  if (B < 0 || H < 0 || N < 0 || P <= 0 || D < 0) {
    gpa_set_error("%s: negative size or P <= 0", fn);
    return GPA_E_INVALID;
  }
  if (B == 0 || H == 0 || N == 0 || D == 0) return GPA_OK;
  if (!oa || !la || !ob || !lb || !y) {
    gpa_set_error("%s: null pointer", fn);
    return GPA_E_INVALID;
  }
  if (N % P != 0) {
    gpa_set_error("%s: N=%lld is not a multiple of P=%lld", fn, (long long)N, (long long)P);
    return GPA_E_INVALID;
  }
  const bool aligned = D % 8 == 0 && (uintptr_t)oa % 16 == 0 && (uintptr_t)ob % 16 == 0 &&
                       (uintptr_t)y % 16 == 0 && oa_b % 8 == 0 && oa_h % 8 == 0 &&
                       oa_s % 8 == 0 && oa_p % 8 == 0 && ob_b % 8 == 0 && ob_h % 8 == 0 &&
                       ob_s % 8 == 0 && ob_p % 8 == 0 && y_b % 8 == 0 && y_n % 8 == 0 &&
                       y_h % 8 == 0;
  if (!aligned) {
    gpa_set_error("%s: D must be a multiple of 8 and rows 16-byte aligned", fn);
    return GPA_E_INVALID;
  }
  CombineArgs a{};
  a.oa = (const uint16_t*)oa;
  a.la = la;
  a.ob = (const uint16_t*)ob;
  a.lb = lb;
  a.y = (uint16_t*)y;
  a.B = B; a.H = H; a.N = N; a.P = P; a.D = D;
  a.oa_b = oa_b; a.oa_h = oa_h; a.oa_s = oa_s; a.oa_p = oa_p;
  a.la_b = la_b; a.la_h = la_h; a.la_s = la_s; a.la_p = la_p;
  a.ob_b = ob_b; a.ob_h = ob_h; a.ob_s = ob_s; a.ob_p = ob_p;
  a.lb_b = lb_b; a.lb_h = lb_h; a.lb_s = lb_s; a.lb_p = lb_p;
  a.y_b = y_b; a.y_n = y_n; a.y_h = y_h;
  a.total = B * N * H * (D / 8);
  const int64_t blocks = (a.total + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) {
    gpa_set_error("%s: problem exceeds the grid limit", fn);
    return GPA_E_UNSUPPORTED;
  }
  hipLaunchKernelGGL(lse_combine_kernel<F16>, dim3((unsigned)blocks), dim3(kThreads), 0,
                     (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    gpa_set_error("%s: launch failed: %s", fn, hipGetErrorString(e));
    return GPA_E_LAUNCH;
  }
  return GPA_OK;
}

}  // namespace

#define GPA_COMBINE_ARGS                                                                   \
  const void *oa, const float *la, const void *ob, const float *lb, void *y, int64_t B,    \
      int64_t H, int64_t N, int64_t P, int64_t D, int64_t oa_b, int64_t oa_h, int64_t oa_s, \
      int64_t oa_p, int64_t la_b, int64_t la_h, int64_t la_s, int64_t la_p, int64_t ob_b,  \
      int64_t ob_h, int64_t ob_s, int64_t ob_p, int64_t lb_b, int64_t lb_h, int64_t lb_s,  \
      int64_t lb_p, int64_t y_b, int64_t y_n, int64_t y_h, void *stream
#define GPA_COMBINE_PASS                                                                   \
  oa, la, ob, lb, y, B, H, N, P, D, oa_b, oa_h, oa_s, oa_p, la_b, la_h, la_s, la_p, ob_b,  \
      ob_h, ob_s, ob_p, lb_b, lb_h, lb_s, lb_p, y_b, y_n, y_h, stream

extern "C" int gpa_lse_combine_bf16(GPA_COMBINE_ARGS) {
  return lse_combine_run<false>("gpa_lse_combine_bf16", GPA_COMBINE_PASS);
}

extern "C" int gpa_lse_combine_f16(GPA_COMBINE_ARGS) {
  return lse_combine_run<true>("gpa_lse_combine_f16", GPA_COMBINE_PASS);
}
