// Small-M linear, M <= 16 (fastlinear.py:123-174): y = act(norm?(x) . W^T + b) [+ residual].
// HBM-bound GEMV: each wave streams weight rows with 16-byte loads, the activation rows are re-read from
// the L1/L2 caches. The optional RMSNorm prologue runs first as its own pass into a bf16 scratch buffer,
// with the rounding points of the reference (x -> bf16(x * rstd) -> * g -> bf16, rstd = 1/sqrt(ss/K + eps)).
#include "mm_common.h"

namespace {

using namespace mmd;

constexpr int kMaxM = 16;

struct LinArgs {
  const uint16_t* x;
  int64_t xs;
  int M;
  int64_t K;
  const uint16_t* w;
  int64_t N, ws;
  const uint16_t* b;
  int act;
  const uint16_t* res;
  int64_t rs;
  uint16_t* y;
  int64_t ys;
};

__global__ __launch_bounds__(256) void small_norm_kernel(const uint16_t* __restrict__ x, int64_t xs, int64_t K,
                                                         const uint16_t* __restrict__ g, float eps,
                                                         uint16_t* __restrict__ xn) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  const uint16_t* xr = x + m * xs;
  float ss = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const float v = bf16_to_f32(xr[k]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if (lane_id() == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rstd = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    const float v = round_bf16(bf16_to_f32(xr[k]) * rstd);
    xn[m * K + k] = f32_to_bf16(v * bf16_to_f32(g[k]));
  }
}

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == MM_ACT_GELU_TANH) {
    v = round_bf16(v);
    const float c = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    const float t = 2.0f / (1.0f + __expf(-2.0f * c)) - 1.0f;
    return 0.5f * v * (1.0f + t);
  }
  if (act == MM_ACT_SILU) {
    v = round_bf16(v);
    return v / (1.0f + __expf(-v));
  }
  return v;
}

// Each wave computes GPW = 64/LPR rows at a time, R times; LPR lanes share one row, NC chunks per lane.
template <int LPR, int NC, int R>
__global__ __launch_bounds__(256) void small_linear_kernel(LinArgs a) {
  constexpr int GPW = kWave / LPR;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int g = lane / LPR, s = lane % LPR;
  const int64_t nch = a.K / 8;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * (GPW * R);
  for (int i = 0; i < R; ++i) {
    const int64_t n = row0 + static_cast<int64_t>(GPW) * i + g;
    const bool nok = n < a.N;
    float acc[kMaxM];
#pragma unroll
    for (int m = 0; m < kMaxM; ++m) acc[m] = 0.f;
    for (int64_t c0 = 0; c0 < nch; c0 += static_cast<int64_t>(LPR) * NC) {  // one pass unless K is very long
      uint4 w[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
        w[j] = (nok && c < nch) ? *reinterpret_cast<const uint4*>(a.w + n * a.ws + c * 8) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int m = 0; m < kMaxM; ++m) {
        if (m < a.M) {
          const uint16_t* xr = a.x + m * a.xs;
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
            const uint4 xv = c < nch ? *reinterpret_cast<const uint4*>(xr + c * 8) : make_uint4(0, 0, 0, 0);
            acc[m] = dot8_bf16(w[j], xv, acc[m]);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kMaxM; ++m)
      if (m < a.M) acc[m] = group_sum<LPR>(acc[m]);
#pragma unroll
    for (int m = 0; m < kMaxM; ++m) {
      if (m < a.M && s == 0 && nok) {
        float v = acc[m];
        if (a.b) v += bf16_to_f32(a.b[n]);
        v = apply_act(v, a.act);
        if (a.res) v = round_bf16(v) + bf16_to_f32(a.res[m * a.rs + n]);
        a.y[m * a.ys + n] = f32_to_bf16(v);
      }
    }
  }
}

template <int LPR, int NC>
int launch(const LinArgs& a, hipStream_t st) {
  constexpr int R = 2;
  constexpr int rows_per_wg = 4 * (kWave / LPR) * R;
  hipLaunchKernelGGL((small_linear_kernel<LPR, NC, R>), dim3(static_cast<unsigned>((a.N + rows_per_wg - 1) / rows_per_wg)),
                     dim3(256), 0, st, a);
  return mm::check_launch("small_linear");
}

}  // namespace

extern "C" int mm_small_linear(const void* x, int64_t M, int64_t K, int64_t x_row_stride, const void* w, int64_t N,
                               int64_t w_row_stride, const void* b, int act, const void* residual,
                               int64_t res_row_stride, const void* norm_g, float norm_eps, void* xn_buf, void* y,
                               int64_t y_row_stride, void* stream) {
  MM_REQUIRE(M >= 1 && M <= kMaxM, "small_linear: M=%lld must be in [1, %d]", (long long)M, kMaxM);
  MM_REQUIRE(K > 0 && N > 0 && K % 8 == 0, "small_linear: K=%lld must be a positive multiple of 8, N=%lld > 0",
             (long long)K, (long long)N);
  MM_REQUIRE(N <= 0x7fffffffLL * 8, "small_linear: N too large");
  MM_REQUIRE(x && w && y, "small_linear: null pointer");
  MM_REQUIRE(act == MM_ACT_NONE || act == MM_ACT_GELU_TANH || act == MM_ACT_SILU, "small_linear: unknown act %d", act);
  MM_REQUIRE(x_row_stride >= K && w_row_stride >= K && y_row_stride >= N, "small_linear: row stride too small");
  MM_REQUIRE(!residual || res_row_stride >= N, "small_linear: residual row stride too small");
  MM_REQUIRE(mm::aligned16(w) && (w_row_stride * 2) % 16 == 0, "small_linear: weight rows must be 16-byte aligned");
  hipStream_t st = MM_STREAM(stream);
  const uint16_t* xin = static_cast<const uint16_t*>(x);
  int64_t xs = x_row_stride;
  if (norm_g) {
    MM_REQUIRE(xn_buf && mm::aligned16(xn_buf), "small_linear: norm prologue needs a 16-byte aligned xn_buf [M, K]");
    hipLaunchKernelGGL(small_norm_kernel, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, xin, xs, K,
                       static_cast<const uint16_t*>(norm_g), norm_eps, static_cast<uint16_t*>(xn_buf));
    int rc = mm::check_launch("small_linear norm");
    if (rc) return rc;
    xin = static_cast<const uint16_t*>(xn_buf);
    xs = K;
  } else {
    MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0, "small_linear: x rows must be 16-byte aligned");
  }
  LinArgs a{xin, xs, static_cast<int>(M), K, static_cast<const uint16_t*>(w), N, w_row_stride,
            static_cast<const uint16_t*>(b), act, static_cast<const uint16_t*>(residual), res_row_stride,
            static_cast<uint16_t*>(y), y_row_stride};
  // rows of nch 16-byte chunks; rows longer than LPR * NC chunks take several passes
  const int64_t nch = K / 8;
  if (nch >= 128) return launch<64, 4>(a, st);
  return launch<16, 4>(a, st);
}
