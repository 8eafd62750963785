// The thinker's attention mixers for decode and short prefills on gfx950:
//
//   kda_recurrent_kernel   Kimi delta attention, the recurrent form fla's fused_recurrent_kda computes (called at
//                          engine.py:258 and inside the model's KDA layers): per head a [K, V] fp32 state, per token
//                          q, k l2-normalised (q scaled), a per-key-channel decay exp(g) from the gate, the delta
//                          rule update and the readout. One workgroup per head holds the state in registers for
//                          all T tokens: thread (kg, c) keeps rows kg*K/4 .. of column c; the sums over k go
//                          through LDS in a fixed order.
//   short_conv_kernel      the depthwise causal convolution of ShortConvolution's step form (a cache of the last W
//                          inputs per channel), SiLU, T tokens in order.
//   rms_norm_gated_kernel  FusedRMSNormGated with a sigmoid gate: bf16(x * rsqrt(mean(x^2) + eps) * w * sigmoid(g)).
//   mla_split_kernel / mla_merge_kernel
//                          single-token attention of an MLA layer over its static cache (engine.py:523-548: k, v
//                          [heads, max_len, d], rows written at the position with index_copy_): the new k, v rows
//                          are stored at pos, then softmax(scale q . K[0..pos]^T) . V[0..pos] in two passes
//                          (64-position chunks, then a merge of the chunks' softmax states), all in fp32.
#include "mm_common.h"

namespace {

using namespace mmd;

// ------------------------------------------------------------------------------------------------- KDA

struct KdaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const void* g;
  const void* beta;
  int g_dtype, beta_dtype;
  int64_t q_ts, k_ts, v_ts, g_ts, b_ts;  // token strides (elements); head h at h * K (q, k, g), h * V (v), h (beta)
  const float* A_log;                      // [H]
  const float* dt_bias;                    // [H * K]
  float lower_bound;                       // NaN: the softplus gate
  int use_l2norm, use_gate;
  float scale;
  float* state;                            // [H, K, V] fp32, updated in place
  uint16_t* o;                             // [T, H, V] bf16
  int64_t o_ts;
  int T, H;
};

__device__ __forceinline__ float ld_any(const void* p, int dt, int64_t i) {
  return dt == MM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// softplus with the usual threshold: x above 20 returns x
__device__ __forceinline__ float softplus20(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

// One workgroup of 4 * V threads per head; thread (kg = tid / V, c = tid % V) holds state rows kg * RK .. + RK - 1
// of column c, RK = K / 4.
template <int K, int V>
__global__ __launch_bounds__(4 * V) void kda_recurrent_kernel(KdaArgs a) {
  constexpr int RK = K / 4;
  constexpr int NT = 4 * V;
  __shared__ float red_q[4], red_k[4];
  __shared__ float part_u[4][V], part_o[4][V];
  const int h = blockIdx.x;
  const int tid = threadIdx.x, c = tid % V, kg = tid / V;
  const int r0 = kg * RK;
  float* st = a.state + static_cast<int64_t>(h) * K * V;
  float S[RK];
#pragma unroll
  for (int i = 0; i < RK; ++i) S[i] = st[static_cast<int64_t>(r0 + i) * V + c];
  float nA = 0.f, dtb[RK];
  if (a.use_gate) {
    nA = __expf(a.A_log[h]);
#pragma unroll
    for (int i = 0; i < RK; ++i) dtb[i] = a.dt_bias[static_cast<int64_t>(h) * K + r0 + i];
  }
  for (int t = 0; t < a.T; ++t) {
    float qv[RK], kv[RK], gv[RK];
    const uint16_t* qp = a.q + t * a.q_ts + static_cast<int64_t>(h) * K + r0;
    const uint16_t* kp = a.k + t * a.k_ts + static_cast<int64_t>(h) * K + r0;
#pragma unroll
    for (int i = 0; i < RK; ++i) {
      qv[i] = bf16_to_f32(qp[i]);
      kv[i] = bf16_to_f32(kp[i]);
      gv[i] = ld_any(a.g, a.g_dtype, t * a.g_ts + static_cast<int64_t>(h) * K + r0 + i);
    }
    const float vc = bf16_to_f32(a.v[t * a.v_ts + static_cast<int64_t>(h) * V + c]);
    const float beta = ld_any(a.beta, a.beta_dtype, t * a.b_ts + h);
    float sq = 0.f, sk = 0.f;
    if (a.use_l2norm) {
#pragma unroll
      for (int i = 0; i < RK; ++i) {
        sq = fmaf(qv[i], qv[i], sq);
        sk = fmaf(kv[i], kv[i], sk);
      }
      if (c == 0) {
        red_q[kg] = sq;
        red_k[kg] = sk;
      }
    }
    __syncthreads();
    float qs = a.scale, ks = 1.f;
    if (a.use_l2norm) {
      qs = a.scale / sqrtf(((red_q[0] + red_q[1]) + red_q[2]) + red_q[3] + 1e-6f);
      ks = 1.f / sqrtf(((red_k[0] + red_k[1]) + red_k[2]) + red_k[3] + 1e-6f);
    }
    // decay, then the part of v the state already predicts from k
    float pu = 0.f;
#pragma unroll
    for (int i = 0; i < RK; ++i) {
      float gl = gv[i];
      if (a.use_gate) {
        const float x = gl + dtb[i];
        gl = isnan(a.lower_bound) ? -nA * softplus20(x) : a.lower_bound / (1.f + __expf(-nA * x));
      }
      S[i] *= __expf(gl);
      kv[i] *= ks;
      pu = fmaf(kv[i], S[i], pu);
    }
    part_u[kg][c] = pu;
    __syncthreads();
    const float u = (vc - (((part_u[0][c] + part_u[1][c]) + part_u[2][c]) + part_u[3][c])) * beta;
    float po = 0.f;
#pragma unroll
    for (int i = 0; i < RK; ++i) {
      S[i] = fmaf(kv[i], u, S[i]);
      po = fmaf(qv[i] * qs, S[i], po);
    }
    part_o[kg][c] = po;
    __syncthreads();
    if (kg == 0) {
      const float o = ((part_o[0][c] + part_o[1][c]) + part_o[2][c]) + part_o[3][c];
      a.o[t * a.o_ts + static_cast<int64_t>(h) * V + c] = f32_to_bf16(o);
    }
    // the next token's partials reuse red_* / part_*: every thread has read them before this barrier's end
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < RK; ++i) st[static_cast<int64_t>(r0 + i) * V + c] = S[i];
  static_assert(NT <= 1024 && K % 4 == 0, "kda shape");
}

// ----------------------------------------------------------------------------------------- short conv

// y[t, ch] = silu(sum_j w[ch, j] * win[j] + b[ch]), win = the last W inputs of the channel (cache[ch, 1..W-1] then
// x[t, ch]); the cache keeps the window. fp32 math, one rounding of y.
template <int W>
__global__ __launch_bounds__(256) void short_conv_kernel(const uint16_t* __restrict__ x, int64_t xs, int T, int64_t C,
                                                         uint16_t* __restrict__ cache, const uint16_t* __restrict__ w,
                                                         const uint16_t* __restrict__ b, int act,
                                                         uint16_t* __restrict__ y, int64_t ys) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (ch >= C) return;
  float win[W], wt[W];
#pragma unroll
  for (int j = 0; j < W; ++j) {
    win[j] = bf16_to_f32(cache[ch * W + j]);
    wt[j] = bf16_to_f32(w[ch * W + j]);
  }
  const float bias = b ? bf16_to_f32(b[ch]) : 0.f;
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int j = 0; j + 1 < W; ++j) win[j] = win[j + 1];
    win[W - 1] = bf16_to_f32(x[t * xs + ch]);
    float acc = bias;
#pragma unroll
    for (int j = 0; j < W; ++j) acc = fmaf(wt[j], win[j], acc);
    if (act) acc = silu(acc);
    y[t * ys + ch] = f32_to_bf16(acc);
  }
#pragma unroll
  for (int j = 0; j < W; ++j) cache[ch * W + j] = f32_to_bf16(win[j]);  // inputs are bf16: exact
}

// --------------------------------------------------------------------------------------- gated RMSNorm

// One wave per row of n (<= 512) elements: y = bf16(x * rsqrt(mean(x^2) + eps) * w * sigmoid(g)), fp32 math.
__global__ __launch_bounds__(256) void rms_norm_gated_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                             const uint16_t* __restrict__ g, int64_t gs,
                                                             const uint16_t* __restrict__ w, int64_t rows, int n,
                                                             float eps, uint16_t* __restrict__ y, int64_t ys) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (row >= rows) return;
  const int lane = lane_id();
  float xv[8], ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = lane + kWave * j;
    xv[j] = i < n ? bf16_to_f32(x[row * xs + i]) : 0.f;
    ss = fmaf(xv[j], xv[j], ss);
  }
  const float rstd = rsqrtf(wave_sum(ss) / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = lane + kWave * j;
    if (i < n) {
      const float gv = bf16_to_f32(g[row * gs + i]);
      y[row * ys + i] = f32_to_bf16(xv[j] * rstd * bf16_to_f32(w[i]) / (1.f + __expf(-gv)));
    }
  }
}

// ------------------------------------------------------------------------------------ MLA decode attention

constexpr int kMlaChunk = 64;  // positions per workgroup: 4 waves of 16

struct MlaArgs {
  const uint16_t* q;      // [nh, dqk]
  const uint16_t* k_new;  // [nh, dqk]
  const uint16_t* v_new;  // [nh, dv]
  uint16_t* kc;           // [nh, max_len, dqk]
  uint16_t* vc;           // [nh, max_len, dv]
  const void* pos;
  int pos_dtype;
  int nh, dqk, dv;
  int64_t max_len;
  float scale;
  float* ws;  // [nh, nc, dv + 2]: a chunk's unnormalised sum of p * v, then its max and sum of p
  int nc;
  uint16_t* out;  // [nh, dv]
};

__device__ __forceinline__ int64_t load_pos64(const void* p, int dt) {
  return dt == MM_INT64 ? *static_cast<const int64_t*>(p) : static_cast<int64_t>(*static_cast<const int32_t*>(p));
}

// Grid (chunks, heads) x 4 waves. Wave w scores positions t0 .. t0+15 (t0 = chunk * 64 + 16 w): 4 lanes per
// position, each a quarter of the q . k dot (dqk / 4 elements, 16-byte loads), reduced over the 4 lanes; the new
// row stands in for row pos (it is also stored there, by the wave that holds pos). Softmax over the chunk, then
// lane = value dimension for p . V.
template <int DQ4, int NDV>
__global__ __launch_bounds__(256) void mla_split_kernel(MlaArgs a) {
  __shared__ float sp[4][16];
  __shared__ float sm[4], sl[4];
  __shared__ float sacc[4][64 * NDV];
  const int tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int h = blockIdx.y, chunk = blockIdx.x;
  const int64_t pos = load_pos64(a.pos, a.pos_dtype);
  const int64_t c0 = static_cast<int64_t>(chunk) * kMlaChunk;
  if (pos < 0 || pos >= a.max_len || c0 > pos) return;  // uniform over the workgroup
  const int64_t t0 = c0 + wave * 16;
  const int tl = lane / 4, qd = lane % 4;  // position t0 + tl, quarter qd of the dims
  const int64_t t = t0 + tl;
  const int dq4 = a.dqk / 4;               // elements per quarter (a multiple of 8)
  const uint16_t* qrow = a.q + static_cast<int64_t>(h) * a.dqk + qd * dq4;
  const bool is_new = t == pos;
  const uint16_t* krow = is_new ? a.k_new + static_cast<int64_t>(h) * a.dqk + qd * dq4
                                : a.kc + (static_cast<int64_t>(h) * a.max_len + min(t, a.max_len - 1)) * a.dqk + qd * dq4;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < DQ4; ++j) {
    if (j * 8 < dq4) {
      const uint4 qa = *reinterpret_cast<const uint4*>(qrow + j * 8);
      const uint4 kb = *reinterpret_cast<const uint4*>(krow + j * 8);
      s = dot8_bf16(kb, qa, s);
    }
  }
  s += __shfl_xor(s, 1, kWave);
  s += __shfl_xor(s, 2, kWave);
  const bool valid = t <= pos;
  const float sc = valid ? s * a.scale : -INFINITY;
  if (qd == 0) sp[wave][tl] = sc;
  // the wave holding pos stores the new rows into the cache
  if (pos >= t0 && pos < t0 + 16) {
    uint16_t* kd = a.kc + (static_cast<int64_t>(h) * a.max_len + pos) * a.dqk;
    uint16_t* vd = a.vc + (static_cast<int64_t>(h) * a.max_len + pos) * a.dv;
    for (int i = lane; i < a.dqk; i += kWave) kd[i] = a.k_new[static_cast<int64_t>(h) * a.dqk + i];
    for (int i = lane; i < a.dv; i += kWave) vd[i] = a.v_new[static_cast<int64_t>(h) * a.dv + i];
  }
  __syncthreads();
  // chunk softmax state (every wave computes the same max and sum from LDS)
  float m = -INFINITY;
  for (int i = 0; i < 64; ++i) m = fmaxf(m, sp[i / 16][i % 16]);  // finite: position c0 <= pos is valid
  // p . V over the wave's 16 positions, lane = value dimension
  float acc[NDV], lsum = 0.f;
#pragma unroll
  for (int j = 0; j < NDV; ++j) acc[j] = 0.f;
  for (int i = 0; i < 16; ++i) {
    const int64_t tt = t0 + i;
    const float p = tt <= pos ? __expf(sp[wave][i] - m) : 0.f;
    lsum += p;
    const uint16_t* vrow = tt == pos ? a.v_new + static_cast<int64_t>(h) * a.dv
                                     : a.vc + (static_cast<int64_t>(h) * a.max_len + min(tt, a.max_len - 1)) * a.dv;
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      const int d = lane + kWave * j;
      if (d < a.dv && p != 0.f) acc[j] = fmaf(p, bf16_to_f32(vrow[d]), acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NDV; ++j) sacc[wave][lane + kWave * j] = acc[j];
  if (lane == 0) sl[wave] = lsum;
  if (lane == 0) sm[wave] = m;
  __syncthreads();
  if (wave != 0) return;
  float* dst = a.ws + (static_cast<int64_t>(h) * a.nc + chunk) * (a.dv + 2);
#pragma unroll
  for (int j = 0; j < NDV; ++j) {
    const int d = lane + kWave * j;
    if (d < a.dv) dst[d] = ((sacc[0][d] + sacc[1][d]) + sacc[2][d]) + sacc[3][d];
  }
  if (lane == 0) {
    dst[a.dv] = m;
    dst[a.dv + 1] = ((sl[0] + sl[1]) + sl[2]) + sl[3];
  }
}

// One wave per head: merges the chunks 0 .. pos / 64 (max of the maxima, rescaled sums) and writes bf16.
// A position outside [0, max_len) writes NaN (and the split kernel wrote nothing).
template <int NDV>
__global__ __launch_bounds__(64) void mla_merge_kernel(MlaArgs a) {
  const int h = blockIdx.x, lane = lane_id();
  const int64_t pos = load_pos64(a.pos, a.pos_dtype);
  if (pos < 0 || pos >= a.max_len) {
    for (int d = lane; d < a.dv; d += kWave) a.out[static_cast<int64_t>(h) * a.dv + d] = 0x7fc0;  // NaN
    return;
  }
  const int n = static_cast<int>(pos / kMlaChunk) + 1;
  const float* base = a.ws + static_cast<int64_t>(h) * a.nc * (a.dv + 2);
  float m = -INFINITY;
  for (int c = 0; c < n; ++c) m = fmaxf(m, base[static_cast<int64_t>(c) * (a.dv + 2) + a.dv]);
  float acc[NDV], l = 0.f;
#pragma unroll
  for (int j = 0; j < NDV; ++j) acc[j] = 0.f;
  for (int c = 0; c < n; ++c) {
    const float* p = base + static_cast<int64_t>(c) * (a.dv + 2);
    const float w = __expf(p[a.dv] - m);
    l = fmaf(p[a.dv + 1], w, l);
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      const int d = lane + kWave * j;
      if (d < a.dv) acc[j] = fmaf(p[d], w, acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NDV; ++j) {
    const int d = lane + kWave * j;
    if (d < a.dv) a.out[static_cast<int64_t>(h) * a.dv + d] = f32_to_bf16(acc[j] / l);
  }
}

template <int K, int V>
int launch_kda(const KdaArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((kda_recurrent_kernel<K, V>), dim3(static_cast<unsigned>(a.H)), dim3(4 * V), 0, st, a);
  return mm::check_launch("kda_recurrent");
}

}  // namespace

extern "C" int mm_kda_recurrent(const void* q, int64_t q_ts, const void* k, int64_t k_ts, const void* v, int64_t v_ts,
                                const void* g, int g_dtype, int64_t g_ts, const void* beta, int beta_dtype,
                                int64_t beta_ts, const float* A_log, const float* dt_bias, float lower_bound,
                                int use_qk_l2norm, int use_gate, float scale, int64_t T, int64_t H, int64_t K,
                                int64_t V, float* state, void* o, int64_t o_ts, void* stream) {
  MM_REQUIRE(T >= 0 && T <= (1 << 20) && H >= 1 && H <= 65535, "kda_recurrent: bad T=%lld or H=%lld", (long long)T,
             (long long)H);
  // a thread holds K / 4 floats each of state, q, k, g and dt_bias; 4 V threads per workgroup
  MM_REQUIRE((K == 64 || K == 128) && (V == 64 || V == 128), "kda_recurrent: head dims K=%lld, V=%lld must be 64 or 128",
             (long long)K, (long long)V);
  MM_REQUIRE(g_dtype == MM_BF16 || g_dtype == MM_FP32, "kda_recurrent: g must be bf16 or fp32");
  MM_REQUIRE(beta_dtype == MM_BF16 || beta_dtype == MM_FP32, "kda_recurrent: beta must be bf16 or fp32");
  MM_REQUIRE(q && k && v && g && beta && state && o, "kda_recurrent: null pointer");
  MM_REQUIRE(!use_gate || (A_log && dt_bias), "kda_recurrent: the gate needs A_log and dt_bias");
  MM_REQUIRE(q_ts >= H * K && k_ts >= H * K && g_ts >= H * K && v_ts >= H * V && beta_ts >= H && o_ts >= H * V,
             "kda_recurrent: token strides smaller than a token's heads");
  if (T == 0) return MM_OK;
  KdaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.g = g;
  a.beta = beta;
  a.g_dtype = g_dtype;
  a.beta_dtype = beta_dtype;
  a.q_ts = q_ts;
  a.k_ts = k_ts;
  a.v_ts = v_ts;
  a.g_ts = g_ts;
  a.b_ts = beta_ts;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.lower_bound = lower_bound;
  a.use_l2norm = use_qk_l2norm;
  a.use_gate = use_gate;
  a.scale = scale;
  a.state = state;
  a.o = static_cast<uint16_t*>(o);
  a.o_ts = o_ts;
  a.T = static_cast<int>(T);
  a.H = static_cast<int>(H);
  hipStream_t st = MM_STREAM(stream);
  if (K == 64 && V == 64) return launch_kda<64, 64>(a, st);
  if (K == 64 && V == 128) return launch_kda<64, 128>(a, st);
  if (K == 128 && V == 64) return launch_kda<128, 64>(a, st);
  if (K == 128 && V == 128) return launch_kda<128, 128>(a, st);
  return mm::set_error(MM_ERR_ARG, "kda_recurrent: K=%lld, V=%lld not instantiated", (long long)K, (long long)V);
}

extern "C" int mm_short_conv(const void* x, int64_t x_ts, int64_t T, int64_t C, void* cache, int64_t W, const void* w,
                             const void* b, int act, void* y, int64_t y_ts, void* stream) {
  MM_REQUIRE(T >= 0 && C >= 1 && C <= (1LL << 31) / 8, "short_conv: bad T=%lld or C=%lld", (long long)T, (long long)C);
  MM_REQUIRE(W >= 2 && W <= 8, "short_conv: kernel width %lld must be in [2, 8]", (long long)W);
  MM_REQUIRE(x && cache && w && y, "short_conv: null pointer");
  MM_REQUIRE(x_ts >= C && y_ts >= C, "short_conv: token strides smaller than the channels");
  if (T == 0) return MM_OK;
  const auto* xp = static_cast<const uint16_t*>(x);
  auto* cp = static_cast<uint16_t*>(cache);
  const auto* wp = static_cast<const uint16_t*>(w);
  const auto* bp = static_cast<const uint16_t*>(b);
  auto* yp = static_cast<uint16_t*>(y);
  dim3 grid(static_cast<unsigned>((C + 255) / 256));
  hipStream_t st = MM_STREAM(stream);
  switch (W) {
    case 2: hipLaunchKernelGGL(short_conv_kernel<2>, grid, dim3(256), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts); break;
    case 3: hipLaunchKernelGGL(short_conv_kernel<3>, grid, dim3(256), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts); break;
    case 4: hipLaunchKernelGGL(short_conv_kernel<4>, grid, dim3(256), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts); break;
    case 5: hipLaunchKernelGGL(short_conv_kernel<5>, grid, dim3(256), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts); break;
    case 6: hipLaunchKernelGGL(short_conv_kernel<6>, grid, dim3(256), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts); break;
    case 7: hipLaunchKernelGGL(short_conv_kernel<7>, grid, dim3(256), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts); break;
    default: hipLaunchKernelGGL(short_conv_kernel<8>, grid, dim3(256), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts); break;
  }
  return mm::check_launch("short_conv");
}

extern "C" int mm_rms_norm_gated(const void* x, int64_t x_rs, const void* g, int64_t g_rs, const void* w, int64_t rows,
                                 int64_t n, float eps, void* y, int64_t y_rs, void* stream) {
  MM_REQUIRE(rows >= 0 && n >= 1 && n <= 512, "rms_norm_gated: row length %lld must be in [1, 512]", (long long)n);
  MM_REQUIRE(x && g && w && y, "rms_norm_gated: null pointer");
  MM_REQUIRE(x_rs >= n && g_rs >= n && y_rs >= n, "rms_norm_gated: row strides smaller than the row");
  if (rows == 0) return MM_OK;
  hipLaunchKernelGGL(rms_norm_gated_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, MM_STREAM(stream),
                     static_cast<const uint16_t*>(x), x_rs, static_cast<const uint16_t*>(g), g_rs,
                     static_cast<const uint16_t*>(w), rows, static_cast<int>(n), eps, static_cast<uint16_t*>(y), y_rs);
  return mm::check_launch("rms_norm_gated");
}

extern "C" int64_t mm_mla_attn_workspace(int nh, int dv, int64_t max_len) {
  if (nh < 1 || dv < 1 || max_len < 1) return 0;
  return static_cast<int64_t>(nh) * ((max_len + kMlaChunk - 1) / kMlaChunk) * (dv + 2) * 4;
}

extern "C" int mm_mla_decode_attn(const void* q, const void* k_new, const void* v_new, int nh, int dqk, int dv,
                                  void* k_cache, void* v_cache, int64_t max_len, const void* pos, int pos_dtype,
                                  float scale, void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  MM_REQUIRE(nh >= 1 && nh <= 65535 && max_len >= 1 && max_len <= (1LL << 24), "mla_decode_attn: bad nh or max_len");
  MM_REQUIRE(dqk % 32 == 0 && dqk >= 32 && dqk <= 512, "mla_decode_attn: dqk=%d must be a multiple of 32 in [32, 512]",
             dqk);
  MM_REQUIRE(dv >= 1 && dv <= 256, "mla_decode_attn: dv=%d must be in [1, 256]", dv);
  MM_REQUIRE(pos_dtype == MM_INT64 || pos_dtype == MM_INT32, "mla_decode_attn: pos must be int64 or int32");
  MM_REQUIRE(q && k_new && v_new && k_cache && v_cache && pos && out && workspace, "mla_decode_attn: null pointer");
  MM_REQUIRE(mm::aligned16(q) && mm::aligned16(k_new) && mm::aligned16(k_cache) && mm::aligned16(workspace),
             "mla_decode_attn: q, k_new, k_cache and the workspace must be 16-byte aligned");
  MM_REQUIRE(workspace_bytes >= mm_mla_attn_workspace(nh, dv, max_len), "mla_decode_attn: workspace too small");
  MlaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.pos = pos;
  a.pos_dtype = pos_dtype;
  a.nh = nh;
  a.dqk = dqk;
  a.dv = dv;
  a.max_len = max_len;
  a.scale = scale;
  a.ws = static_cast<float*>(workspace);
  a.nc = static_cast<int>((max_len + kMlaChunk - 1) / kMlaChunk);
  a.out = static_cast<uint16_t*>(out);
  hipStream_t st = MM_STREAM(stream);
  dim3 grid(static_cast<unsigned>(a.nc), static_cast<unsigned>(nh));
  const int dq4 = dqk / 4;  // 16-byte pieces per quarter: dq4 / 8
  if (dq4 <= 8 * 2 && dv <= 64) hipLaunchKernelGGL((mla_split_kernel<2, 1>), grid, dim3(256), 0, st, a);
  else if (dq4 <= 8 * 2) hipLaunchKernelGGL((mla_split_kernel<2, 4>), grid, dim3(256), 0, st, a);
  else if (dv <= 128) hipLaunchKernelGGL((mla_split_kernel<16, 2>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((mla_split_kernel<16, 4>), grid, dim3(256), 0, st, a);
  int rc = mm::check_launch("mla_decode_attn split");
  if (rc) return rc;
  if (dv <= 64) hipLaunchKernelGGL(mla_merge_kernel<1>, dim3(static_cast<unsigned>(nh)), dim3(64), 0, st, a);
  else if (dv <= 128) hipLaunchKernelGGL(mla_merge_kernel<2>, dim3(static_cast<unsigned>(nh)), dim3(64), 0, st, a);
  else hipLaunchKernelGGL(mla_merge_kernel<4>, dim3(static_cast<unsigned>(nh)), dim3(64), 0, st, a);
  return mm::check_launch("mla_decode_attn merge");
}
