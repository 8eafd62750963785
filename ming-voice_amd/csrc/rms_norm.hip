// RMSNorm over the last dim, one workgroup per row (fused_ops.py:16-37).
//   var = mean(x_f32^2); y = bf16(x * rsqrt(var + eps)); out = (w_f32 * y) cast to the output dtype.
#include "mm_common.h"
#include "mm_select.h"

namespace {

using namespace mmd;

constexpr int kThreads = 256;

template <class TX, class TW, class TY>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const typename TX::T* __restrict__ x, int64_t n, int64_t xs,
                                                            const typename TW::T* __restrict__ w, float eps,
                                                            typename TY::T* __restrict__ y, int64_t ys) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const typename TX::T* xr = x + row * xs;
  const float rstd = row_rstd256<TX>(xr, n, eps, red);
  typename TY::T* yr = y + row * ys;
  for (int64_t i = threadIdx.x; i < n; i += kThreads) {
    const float v = round_bf16(TX::ld(xr, i) * rstd);
    TY::st(yr, i, TW::ld(w, i) * v);
  }
}

template <class TX, class TW, class TY>
int launch(const void* x, int64_t rows, int64_t n, int64_t xs, const void* w, float eps, void* y, int64_t ys, hipStream_t s) {
  hipLaunchKernelGGL((rms_norm_kernel<TX, TW, TY>), dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s,
                     static_cast<const typename TX::T*>(x), n, xs, static_cast<const typename TW::T*>(w), eps,
                     static_cast<typename TY::T*>(y), ys);
  return mm::check_launch("rms_norm");
}

template <class TX, class TW>
int dispatch_y(int y_dtype, const void* x, int64_t rows, int64_t n, int64_t xs, const void* w, float eps, void* y,
               int64_t ys, hipStream_t s) {
  switch (y_dtype) {
    case MM_BF16: return launch<TX, TW, BF16>(x, rows, n, xs, w, eps, y, ys, s);
    case MM_FP16: return launch<TX, TW, FP16>(x, rows, n, xs, w, eps, y, ys, s);
    case MM_FP32: return launch<TX, TW, FP32>(x, rows, n, xs, w, eps, y, ys, s);
  }
  return mm::set_error(MM_ERR_ARG, "rms_norm: unsupported output dtype %d", y_dtype);
}

template <class TX>
int dispatch_w(int w_dtype, int y_dtype, const void* x, int64_t rows, int64_t n, int64_t xs, const void* w, float eps,
               void* y, int64_t ys, hipStream_t s) {
  switch (w_dtype) {
    case MM_BF16: return dispatch_y<TX, BF16>(y_dtype, x, rows, n, xs, w, eps, y, ys, s);
    case MM_FP16: return dispatch_y<TX, FP16>(y_dtype, x, rows, n, xs, w, eps, y, ys, s);
    case MM_FP32: return dispatch_y<TX, FP32>(y_dtype, x, rows, n, xs, w, eps, y, ys, s);
  }
  return mm::set_error(MM_ERR_ARG, "rms_norm: unsupported weight dtype %d", w_dtype);
}

}  // namespace

extern "C" int mm_rms_norm(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t x_row_stride, const void* w,
                           int w_dtype, float eps, void* y, int y_dtype, int64_t y_row_stride, void* stream) {
  MM_REQUIRE(rows >= 0 && n > 0, "rms_norm: bad shape rows=%lld n=%lld", (long long)rows, (long long)n);
  MM_REQUIRE(rows <= 0x7fffffffLL, "rms_norm: too many rows (%lld)", (long long)rows);
  MM_REQUIRE(x && w && y, "rms_norm: null pointer");
  MM_REQUIRE(x_row_stride >= n && y_row_stride >= n, "rms_norm: row stride smaller than the row");
  if (rows == 0) return MM_OK;
  hipStream_t s = MM_STREAM(stream);
  switch (x_dtype) {
    case MM_BF16: return dispatch_w<BF16>(w_dtype, y_dtype, x, rows, n, x_row_stride, w, eps, y, y_row_stride, s);
    case MM_FP16: return dispatch_w<FP16>(w_dtype, y_dtype, x, rows, n, x_row_stride, w, eps, y, y_row_stride, s);
    case MM_FP32: return dispatch_w<FP32>(w_dtype, y_dtype, x, rows, n, x_row_stride, w, eps, y, y_row_stride, s);
  }
  return mm::set_error(MM_ERR_ARG, "rms_norm: unsupported input dtype %d", x_dtype);
}
