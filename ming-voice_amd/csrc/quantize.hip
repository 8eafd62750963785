// Symmetric per-row int8 weight quantisation (fused_moe.py:199-204), one workgroup per row:
//   amax = max(max_k |w|, 1e-8); scale = amax / 127; q = clamp(round_half_even(w / scale), -127, 127).
// With a bf16 scale output the scale is rounded to bf16 first and q divides by the rounded value.
#include "mm_common.h"

namespace {

using namespace mmd;

template <class TW>
__global__ __launch_bounds__(256) void quantize_kernel(const typename TW::T* __restrict__ w, int64_t K, int64_t ws,
                                                       int8_t* __restrict__ q, int64_t qs, void* __restrict__ scale,
                                                       int scale_dtype) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const typename TW::T* wr = w + row * ws;
  float m = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += 256) m = fmaxf(m, fabsf(TW::ld(wr, k)));
  m = wave_max(m);
  if (lane_id() == 0) red[threadIdx.x / kWave] = m;
  __syncthreads();
  const float amax = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), 1e-8f);
  float s = amax / 127.0f;
  if (scale_dtype == MM_BF16) s = round_bf16(s);
  if (threadIdx.x == 0) {
    if (scale_dtype == MM_BF16) static_cast<uint16_t*>(scale)[row] = f32_to_bf16(s);
    else static_cast<float*>(scale)[row] = s;
  }
  int8_t* qr = q + row * qs;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const float v = rintf(TW::ld(wr, k) / s);
    qr[k] = static_cast<int8_t>(fminf(fmaxf(v, -127.f), 127.f));
  }
}

template <class TW>
int launch(const void* w, int64_t rows, int64_t K, int64_t ws, int8_t* q, int64_t qs, void* scale, int sd, hipStream_t st) {
  hipLaunchKernelGGL(quantize_kernel<TW>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, st,
                     static_cast<const typename TW::T*>(w), K, ws, q, qs, scale, sd);
  return mm::check_launch("quantize_rows_int8");
}

}  // namespace

extern "C" int mm_quantize_rows_int8(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t w_row_stride, int8_t* q,
                                     int64_t q_row_stride, void* scale, int scale_dtype, void* stream) {
  MM_REQUIRE(rows >= 0 && rows <= 0x7fffffffLL && K > 0, "quantize_rows_int8: bad shape rows=%lld K=%lld",
             (long long)rows, (long long)K);
  MM_REQUIRE(w && q && scale, "quantize_rows_int8: null pointer");
  MM_REQUIRE(w_row_stride >= K && q_row_stride >= K, "quantize_rows_int8: row stride smaller than K");
  MM_REQUIRE(scale_dtype == MM_FP32 || scale_dtype == MM_BF16, "quantize_rows_int8: scale dtype must be fp32 or bf16");
  if (rows == 0) return MM_OK;
  hipStream_t st = MM_STREAM(stream);
  switch (w_dtype) {
    case MM_BF16: return launch<BF16>(w, rows, K, w_row_stride, q, q_row_stride, scale, scale_dtype, st);
    case MM_FP16: return launch<FP16>(w, rows, K, w_row_stride, q, q_row_stride, scale, scale_dtype, st);
    case MM_FP32: return launch<FP32>(w, rows, K, w_row_stride, q, q_row_stride, scale, scale_dtype, st);
  }
  return mm::set_error(MM_ERR_ARG, "quantize_rows_int8: unsupported weight dtype %d", w_dtype);
}
