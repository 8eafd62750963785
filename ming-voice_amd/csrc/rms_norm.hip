// RMSNorm over the last dim, one workgroup per row (fused_ops.py:16-37).
//   var = mean(x_f32^2); y = bf16(x * rsqrt(var + eps)); out = (w_f32 * y) cast to the output dtype.
#include "mm_common.h"
#include "mm_select.h"

#include <type_traits>

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

// bf16 rows, weight and output, 16-byte aligned with n a multiple of 8 and at most 2048 * NCH: thread i holds the row's
// 8-element chunks i + 256 j (j < NCH) from the sum of squares to the output, its weight chunks loaded with them, so
// the workgroup waits for memory once (the element loop above waits once per pass of 256 elements). The sums run
// as row_rstd256's (a thread's chunks in j order, then the waves), so the output is bit-identical.
template <int NCH>
__global__ __launch_bounds__(kThreads) void rms_norm_bf16_kernel(const uint16_t* __restrict__ x, int64_t n, int64_t xs,
                                                                 const uint16_t* __restrict__ w, float eps,
                                                                 uint16_t* __restrict__ y, int64_t ys) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const int nch = static_cast<int>(n / 8);
  const rsrc_t xr = make_rsrc(x + row * xs, n * 2), wr = make_rsrc(w, n * 2);
  uint4 xv[NCH], wv[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = threadIdx.x + kThreads * j;
    const uint32_t off = c < nch ? static_cast<uint32_t>(c) * 16u : kPast;
    xv[j] = buf16(xr, off);
    wv[j] = buf16(wr, off);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j)
    if (threadIdx.x + kThreads * j < nch) ss = chunk_ss_bf16x8(xv[j], ss);
  ss = wave_sum(ss);
  if (lane_id() == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float rstd = rsqrtf((((red[0] + red[1]) + red[2]) + red[3]) / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = threadIdx.x + kThreads * j;
    if (c >= nch) continue;
    const uint32_t xq[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w}, wq[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = round_bf16(__uint_as_float(xq[i] << 16) * rstd), hi = round_bf16(__uint_as_float(xq[i] & 0xffff0000u) * rstd);
      o[i] = static_cast<uint32_t>(f32_to_bf16(__uint_as_float(wq[i] << 16) * lo)) |
             (static_cast<uint32_t>(f32_to_bf16(__uint_as_float(wq[i] & 0xffff0000u) * hi)) << 16);
    }
    reinterpret_cast<uint4*>(y + row * ys)[c] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <class TX, class TW, class TY>
int launch(const void* x, int64_t rows, int64_t n, int64_t xs, const void* w, float eps, void* y, int64_t ys, hipStream_t s) {
  if constexpr (std::is_same<TX, BF16>::value && std::is_same<TW, BF16>::value && std::is_same<TY, BF16>::value) {
    const bool fast = n % 8 == 0 && n <= 8192 && xs % 8 == 0 && ys % 8 == 0 && mm::aligned16(x) && mm::aligned16(w) &&
                      mm::aligned16(y);
    if (fast) {
      const auto* xp = static_cast<const uint16_t*>(x);
      const auto* wp = static_cast<const uint16_t*>(w);
      auto* yp = static_cast<uint16_t*>(y);
      const dim3 grid(static_cast<unsigned>(rows));
      if (n <= 2048) hipLaunchKernelGGL(rms_norm_bf16_kernel<1>, grid, dim3(kThreads), 0, s, xp, n, xs, wp, eps, yp, ys);
      else hipLaunchKernelGGL(rms_norm_bf16_kernel<4>, grid, dim3(kThreads), 0, s, xp, n, xs, wp, eps, yp, ys);
      return mm::check_launch("rms_norm");
    }
  }
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
