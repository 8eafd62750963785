// Small-M linear, M <= 16 (fastlinear.py:123-174): y = act(norm?(x) . W^T + b) [+ residual].
// HBM-bound GEMV, latency-bound at decode sizes (a few MB per call). For rows of up to 1024 16-byte chunks
// (K <= 8192) one pass covers the row: a wave shares each of its rows across its 64 lanes and issues all
// weight loads of its rows at once, so it waits for memory once; the activation chunks come from the L1/L2
// caches. The optional RMSNorm prologue is fused there: the lanes of a wave hold the whole activation row,
// so they sum its squares themselves, with the rounding points of the reference (x -> bf16(x * rstd) -> * g
// -> bf16, rstd = 1/sqrt(ss/K + eps)). Longer rows take several passes and run the norm as its own kernel.
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
  bool norm_once;  // the norm prologue rounds once, bf16(x * rstd * g) (F.rms_norm), instead of twice
  const uint16_t* res;
  int64_t rs;
  uint16_t* y;
  int64_t ys;
};

__global__ __launch_bounds__(256) void small_norm_kernel(const uint16_t* __restrict__ x, int64_t xs, int64_t K,
                                                         const uint16_t* __restrict__ g, float eps, bool once,
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
    const float v = bf16_to_f32(xr[k]) * rstd;
    xn[m * K + k] = f32_to_bf16((once ? v : round_bf16(v)) * bf16_to_f32(g[k]));
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

__device__ __forceinline__ void epilogue(const LinArgs& a, int m, int64_t n, float v) {
  if (a.b) v += bf16_to_f32(a.b[n]);
  v = apply_act(v, a.act);
  if (a.res) v = round_bf16(v) + bf16_to_f32(a.res[m * a.rs + n]);
  a.y[m * a.ys + n] = f32_to_bf16(v);
}

// Elementwise bf16(bf16(x * rstd) * g) of one 8-element chunk (the norm prologue's rounding points), or with
// `once` bf16(x * rstd * g) (F.rms_norm's single rounding, the reference's path for more than 16 rows).
__device__ __forceinline__ uint4 norm_chunk(uint4 xv, uint4 gv, float rstd, bool once) {
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
  uint32_t r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x0 = __uint_as_float(xw[i] << 16) * rstd, x1 = __uint_as_float(xw[i] & 0xffff0000u) * rstd;
    const float y0 = (once ? x0 : round_bf16(x0)) * __uint_as_float(gw[i] << 16);
    const float y1 = (once ? x1 : round_bf16(x1)) * __uint_as_float(gw[i] & 0xffff0000u);
    r[i] = static_cast<uint32_t>(f32_to_bf16(y0)) | (static_cast<uint32_t>(f32_to_bf16(y1)) << 16);
  }
  return make_uint4(r[0], r[1], r[2], r[3]);
}

__device__ __forceinline__ float sumsq8(uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a0 = __uint_as_float(w[i] << 16), a1 = __uint_as_float(w[i] & 0xffff0000u);
    s = fmaf(a0, a0, s);
    s = fmaf(a1, a1, s);
  }
  return s;
}

// Token rows whose activation chunks are held at once (1 when there is a single row).
constexpr int row_group(int NC) { return NC <= 2 ? 8 : NC <= 4 ? 4 : NC <= 8 ? 2 : 1; }

// One pass per row (64 * NC >= K / 8): the 64 lanes of a wave share a row, lane s holding chunks
// s + 64 j (j < NC), and a wave computes R rows whose R * NC weight loads per lane are all issued at once,
// so it waits for memory once. Chunk indices past the row are clamped to its last chunk (a valid address)
// and their products dropped by a select. Token rows go in groups of MG: the activation chunks of a whole
// group are loaded before any of its math. NORM: the whole activation row passes through the wave's lanes,
// so the wave sums its squares itself; with several rows the 4 waves of the workgroup split the group's
// rows, normalise them into LDS, and all read them back. The bias, GELU / SiLU and residual run once per
// group in parallel, lane = (token row, output row), with the bias and residuals read before any store.
// GLU (R = 2): the wave's two rows are gate row p and up row p + N of a [2N, K] weight, and the output is
// y[:, p] = bf16(bf16(silu(g)) * u) with g, u the bf16-rounded projections: small_linear followed by
// silu_mul (fast_talker.py:258-260), bit for bit, without the [M, 2N] intermediate.
// SPLIT: each workgroup takes the one token group blockIdx.y of a grid with a y row per group; otherwise it
// takes every group in turn.
template <int NC, int R, bool NORM, bool GLU, int MG, bool SPLIT = false>
__global__ __launch_bounds__(256) void small_linear_1pass_kernel(LinArgs a, const uint16_t* __restrict__ norm_g,
                                                                 float norm_eps) {
  static_assert(!GLU || R == 2, "GLU pairs a gate row with an up row");
  static_assert(MG * R <= kWave, "one epilogue lane per (token row, output row)");
  constexpr bool kShareNorm = NORM && MG > 1;
  constexpr int OUTS = GLU ? 1 : R;  // output rows per wave
  __shared__ uint4 lx[kShareNorm ? MG * NC * kWave : 1];
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int64_t nch = a.K / 8;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * OUTS;
  // weight row of the wave's i-th row, clamped into the matrix
  auto wrow = [&](int i) -> int64_t {
    const int64_t n = GLU ? n0 + i * a.N : n0 + i;
    return (GLU ? n0 < a.N : n < a.N) ? n : (GLU ? i * a.N + a.N - 1 : a.N - 1);
  };
  int64_t cc[NC];
  bool cin[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int64_t c = lane + static_cast<int64_t>(kWave) * j;
    cin[j] = c < nch;
    cc[j] = cin[j] ? c : nch - 1;
  }
  uint4 w[R][NC];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t nl = wrow(i);
#pragma unroll
    for (int j = 0; j < NC; ++j) w[i][j] = *reinterpret_cast<const uint4*>(a.w + nl * a.ws + cc[j] * 8);
  }
  uint4 gv[NC];
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < NC; ++j) gv[j] = *reinterpret_cast<const uint4*>(norm_g + cc[j] * 8);
  }
  // this lane's epilogue slot: token row m0 + e_mm, output row e_n
  const int e_mm = lane / OUTS, e_i = lane % OUTS;
  const int64_t e_n = n0 + e_i;
  const bool e_on = e_mm < MG && e_n < a.N;
  const int64_t e_nc = e_n < a.N ? e_n : a.N - 1;
  // A single token row (decode): bias and residual through buffer resources (empty when absent: the load
  // returns 0, no branch) and the row's activation chunks, all issued with the weights, so the wave waits
  // for memory once instead of once per conditional load. Several rows keep the plain loads (prefetching
  // them costs more registers than it saves).
  constexpr bool kPrefetch = MG == 1;
  const rsrc_t brs = make_rsrc(a.b, (kPrefetch && !GLU && a.b) ? a.N * 2 : 0);
  const rsrc_t rrs = make_rsrc(a.res, (kPrefetch && !GLU && a.res) ? static_cast<int64_t>(a.M) * a.rs * 2 : 0);
  const float bias = kPrefetch ? bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(brs, static_cast<int>(e_nc * 2), 0, 0))
                               : ((!GLU && a.b) ? bf16_to_f32(a.b[e_nc]) : 0.f);
  uint4 xfirst[NC];
  if constexpr (kPrefetch) {
#pragma unroll
    for (int j = 0; j < NC; ++j)
      xfirst[j] = *reinterpret_cast<const uint4*>(a.x + (SPLIT ? static_cast<int64_t>(blockIdx.y) * MG * a.xs : 0) +
                                                  cc[j] * 8);
  }
  const int mfirst = SPLIT ? static_cast<int>(blockIdx.y) * MG : 0;
  for (int m0 = mfirst; m0 < kMaxM; m0 += MG) {
    if (m0 >= a.M) break;  // uniform
    const int e_m = min(m0 + e_mm, a.M - 1);
    const float res =
        kPrefetch ? bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(rrs, static_cast<int>((e_m * a.rs + e_nc) * 2), 0, 0))
                  : ((!GLU && a.res) ? bf16_to_f32(a.res[e_m * a.rs + e_nc]) : 0.f);
    uint4 xg[MG][NC];
    if constexpr (kShareNorm) {
      for (int mm = wave; mm < MG; mm += 4) {
        const uint16_t* xr = a.x + min(m0 + mm, a.M - 1) * a.xs;  // rows past M re-read the last one, unused
        uint4 xv[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) xv[j] = *reinterpret_cast<const uint4*>(xr + cc[j] * 8);
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j) ss += cin[j] ? sumsq8(xv[j]) : 0.f;
        const float rstd = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(a.K) + norm_eps);
#pragma unroll
        for (int j = 0; j < NC; ++j) lx[(mm * NC + j) * kWave + lane] = norm_chunk(xv[j], gv[j], rstd, a.norm_once);
      }
      __syncthreads();
#pragma unroll
      for (int mm = 0; mm < MG; ++mm)
#pragma unroll
        for (int j = 0; j < NC; ++j) xg[mm][j] = lx[(mm * NC + j) * kWave + lane];
      __syncthreads();  // the next group overwrites lx
    } else {
#pragma unroll
      for (int mm = 0; mm < MG; ++mm) {
        const uint16_t* xr = a.x + min(m0 + mm, a.M - 1) * a.xs;
#pragma unroll
        for (int j = 0; j < NC; ++j)
          xg[mm][j] = (kPrefetch && m0 == mfirst) ? xfirst[j] : *reinterpret_cast<const uint4*>(xr + cc[j] * 8);
      }
    }
    float keep = 0.f, keep_up = 0.f;
#pragma unroll
    for (int mm = 0; mm < MG; ++mm) {
      if (m0 + mm < a.M) {  // uniform
        uint4* xv = xg[mm];
        if constexpr (NORM && !kShareNorm) {
          float ss = 0.f;
#pragma unroll
          for (int j = 0; j < NC; ++j) ss += cin[j] ? sumsq8(xv[j]) : 0.f;
          const float rstd = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(a.K) + norm_eps);
#pragma unroll
          for (int j = 0; j < NC; ++j) xv[j] = norm_chunk(xv[j], gv[j], rstd, a.norm_once);
        }
#pragma unroll
        for (int i = 0; i < R; ++i) {
          float t = 0.f;
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            const float d = dot8_bf16(w[i][j], xv[j], 0.f);
            t += cin[j] ? d : 0.f;
          }
          t = wave_sum(t);  // every lane holds the sum; the lane of its epilogue slot keeps it
          if constexpr (GLU) {
            if (e_mm == mm) (i == 0 ? keep : keep_up) = t;
          } else {
            if (e_mm == mm && e_i == i) keep = t;
          }
        }
      }
    }
    const int m = m0 + e_mm;
    if (e_on && m < a.M) {
      if constexpr (GLU) {
        a.y[m * a.ys + n0] = f32_to_bf16(round_bf16(silu(round_bf16(keep))) * round_bf16(keep_up));
      } else {
        float v = apply_act(a.b ? keep + bias : keep, a.act);
        if (a.res) v = round_bf16(v) + res;
        a.y[m * a.ys + e_n] = f32_to_bf16(v);
      }
    }
    if constexpr (SPLIT) break;  // this workgroup's one group
  }
}

// Rows longer than one pass: each wave computes GPW = 64/LPR rows at a time, R times; LPR lanes share one
// row, NC chunks per lane per pass.
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
    for (int m = 0; m < kMaxM; ++m)
      if (m < a.M && s == 0 && nok) epilogue(a, m, n, acc[m]);
  }
}

template <int NC, int R, bool GLU, int MG>
void launch_1pass_mg(const LinArgs& a, const uint16_t* g, float eps, hipStream_t st) {
  // Several token groups run in parallel workgroups (grid y) when the whole grid fits on the GPU at once: the
  // workgroups of one row block then read its weights together (one HBM read), where one workgroup taking the
  // groups in turn leaves a single wave per SIMD working through them serially. Larger grids keep one y row,
  // since workgroups of the same rows that are not resident together would each stream the weights.
  const unsigned gx = static_cast<unsigned>(GLU ? (a.N + 3) / 4 : (a.N + 4 * R - 1) / (4 * R));
  const unsigned ng = static_cast<unsigned>((a.M + MG - 1) / MG);
  const bool split = ng > 1 && static_cast<int64_t>(gx) * ng <= static_cast<int64_t>(4) * mm::cu_count();
  if (split) {
    const dim3 grid(gx, ng);
    if (g) hipLaunchKernelGGL((small_linear_1pass_kernel<NC, R, true, GLU, MG, true>), grid, dim3(256), 0, st, a, g, eps);
    else hipLaunchKernelGGL((small_linear_1pass_kernel<NC, R, false, GLU, MG, true>), grid, dim3(256), 0, st, a, g, eps);
    return;
  }
  const dim3 grid(gx);
  if (g) hipLaunchKernelGGL((small_linear_1pass_kernel<NC, R, true, GLU, MG>), grid, dim3(256), 0, st, a, g, eps);
  else hipLaunchKernelGGL((small_linear_1pass_kernel<NC, R, false, GLU, MG>), grid, dim3(256), 0, st, a, g, eps);
}

template <int NC, int R, bool GLU = false>
int launch_1pass(const LinArgs& a, const uint16_t* g, float eps, hipStream_t st) {
  if (a.M == 1) launch_1pass_mg<NC, R, GLU, 1>(a, g, eps, st);
  else launch_1pass_mg<NC, R, GLU, row_group(NC)>(a, g, eps, st);
  return mm::check_launch(GLU ? "small_linear_glu" : "small_linear");
}

// R rows per wave when that still gives every CU a workgroup; one row per wave otherwise.
template <int NC, int RMAX>
int launch_1pass_r(const LinArgs& a, const uint16_t* g, float eps, hipStream_t st) {
  if (RMAX > 1 && a.N >= static_cast<int64_t>(4) * RMAX * mm::cu_count()) return launch_1pass<NC, RMAX>(a, g, eps, st);
  return launch_1pass<NC, 1>(a, g, eps, st);
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
  const bool once = (act & MM_NORM_ROUND_ONCE) != 0;
  act &= ~MM_NORM_ROUND_ONCE;
  MM_REQUIRE(act == MM_ACT_NONE || act == MM_ACT_GELU_TANH || act == MM_ACT_SILU, "small_linear: unknown act %d", act);
  MM_REQUIRE((x_row_stride >= K || x_row_stride == 0) && w_row_stride >= K && y_row_stride >= N,
             "small_linear: row stride too small (x rows may also repeat one row, stride 0)");
  MM_REQUIRE(!residual || res_row_stride >= N, "small_linear: residual row stride too small");
  MM_REQUIRE(mm::rsrc_fits(N * 2) && (!residual || mm::rsrc_fits(M * res_row_stride * 2)),
             "small_linear: bias or residual spans 2^31 bytes or more");
  MM_REQUIRE(mm::aligned16(w) && (w_row_stride * 2) % 16 == 0, "small_linear: weight rows must be 16-byte aligned");
  hipStream_t st = MM_STREAM(stream);
  const uint16_t* xin = static_cast<const uint16_t*>(x);
  int64_t xs = x_row_stride;
  const int64_t nch = K / 8;
  if (nch <= 64 * 16) {  // one pass per row, norm fused
    MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0, "small_linear: x rows must be 16-byte aligned");
    MM_REQUIRE(!norm_g || mm::aligned16(norm_g), "small_linear: norm_g must be 16-byte aligned");
    LinArgs a{xin, xs, static_cast<int>(M), K, static_cast<const uint16_t*>(w), N, w_row_stride,
              static_cast<const uint16_t*>(b), act, once, static_cast<const uint16_t*>(residual), res_row_stride,
              static_cast<uint16_t*>(y), y_row_stride};
    auto g = static_cast<const uint16_t*>(norm_g);
    // chunks per lane NC = ceil(nch / 64), rounded up to an instantiated size; at most 16 loads per lane
    // (rows per wave measured on MI355X: 2 at K = 896; at K = 2048 1 up to N = 2048, 2 from N = 16 per CU on,
    // where each wave's activation row (and norm weights) from L2 then serves two weight rows: one token,
    // 6416 / 8192 / 126464 rows with the norm fused 9.3 / 10.8 / 120.5 -> 8.6 / 9.5 / 88.5 us)
    if (nch <= 64) return launch_1pass_r<1, 4>(a, g, norm_eps, st);
    if (nch <= 128) return launch_1pass_r<2, 2>(a, g, norm_eps, st);
    if (nch <= 256) {
      if (N >= static_cast<int64_t>(16) * mm::cu_count()) return launch_1pass<4, 2>(a, g, norm_eps, st);
      return launch_1pass<4, 1>(a, g, norm_eps, st);
    }
    if (nch <= 512) return launch_1pass_r<8, 2>(a, g, norm_eps, st);
    if (nch <= 768) return launch_1pass_r<12, 1>(a, g, norm_eps, st);
    return launch_1pass_r<16, 1>(a, g, norm_eps, st);
  }
  if (norm_g) {
    MM_REQUIRE(xn_buf && mm::aligned16(xn_buf), "small_linear: norm prologue needs a 16-byte aligned xn_buf [M, K]");
    hipLaunchKernelGGL(small_norm_kernel, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, xin, xs, K,
                       static_cast<const uint16_t*>(norm_g), norm_eps, once, static_cast<uint16_t*>(xn_buf));
    int rc = mm::check_launch("small_linear norm");
    if (rc) return rc;
    xin = static_cast<const uint16_t*>(xn_buf);
    xs = K;
  } else {
    MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0, "small_linear: x rows must be 16-byte aligned");
  }
  LinArgs a{xin, xs, static_cast<int>(M), K, static_cast<const uint16_t*>(w), N, w_row_stride,
            static_cast<const uint16_t*>(b), act, false, static_cast<const uint16_t*>(residual), res_row_stride,
            static_cast<uint16_t*>(y), y_row_stride};
  return launch<64, 4>(a, st);  // several passes of 256 chunks per row
}

namespace {

template <int NC>
int launch_glu(const LinArgs& a, const uint16_t* g, float eps, hipStream_t st) {
  return launch_1pass<NC, 2, true>(a, g, eps, st);
}

}  // namespace

extern "C" int mm_small_linear_glu(const void* x, int64_t M, int64_t K, int64_t x_row_stride, const void* w,
                                   int64_t inter, int64_t w_row_stride, const void* norm_g, float norm_eps, void* y,
                                   int64_t y_row_stride, void* stream) {
  MM_REQUIRE(M >= 1 && M <= kMaxM, "small_linear_glu: M=%lld must be in [1, %d]", (long long)M, kMaxM);
  MM_REQUIRE(K > 0 && inter > 0 && K % 8 == 0 && K <= 8192,
             "small_linear_glu: K=%lld must be a positive multiple of 8 up to 8192, inter=%lld > 0", (long long)K,
             (long long)inter);
  MM_REQUIRE(x && w && y, "small_linear_glu: null pointer");
  MM_REQUIRE(x_row_stride >= K && w_row_stride >= K && y_row_stride >= inter, "small_linear_glu: row stride too small");
  MM_REQUIRE(mm::aligned16(w) && (w_row_stride * 2) % 16 == 0 && mm::aligned16(x) && (x_row_stride * 2) % 16 == 0,
             "small_linear_glu: x and weight rows must be 16-byte aligned");
  MM_REQUIRE(!norm_g || mm::aligned16(norm_g), "small_linear_glu: norm_g must be 16-byte aligned");
  LinArgs a{static_cast<const uint16_t*>(x), x_row_stride, static_cast<int>(M), K, static_cast<const uint16_t*>(w),
            inter, w_row_stride, nullptr, MM_ACT_NONE, false, nullptr, 0, static_cast<uint16_t*>(y), y_row_stride};
  auto g = static_cast<const uint16_t*>(norm_g);
  hipStream_t st = MM_STREAM(stream);
  const int64_t nch = K / 8;
  if (nch <= 64) return launch_glu<1>(a, g, norm_eps, st);
  if (nch <= 128) return launch_glu<2>(a, g, norm_eps, st);
  if (nch <= 256) return launch_glu<4>(a, g, norm_eps, st);
  if (nch <= 512) return launch_glu<8>(a, g, norm_eps, st);
  if (nch <= 768) return launch_glu<12>(a, g, norm_eps, st);
  return launch_glu<16>(a, g, norm_eps, st);
}
