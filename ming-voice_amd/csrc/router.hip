// MoE router: fp32 logits GEMV/GEMM and top-k selection (fused_ops.py:40-103, engine.py:326-333).
#include "mm_common.h"
#include "mm_select.h"

namespace {

using namespace mmd;

constexpr int kMaxExperts = 1024;      // per-lane slots = kMaxExperts / 64
constexpr int kSlots = kMaxExperts / kWave;

template <class TX>
__device__ __forceinline__ float4 load4(const typename TX::T* p, int64_t i) {
  return make_float4(TX::ld(p, i), TX::ld(p, i + 1), TX::ld(p, i + 2), TX::ld(p, i + 3));
}

__device__ __attribute__((aligned(16))) float g_zero4[4];  // zero source for masked vector loads

// 4 consecutive elements from an address aligned to 4 elements, in one load.
template <class TX>
__device__ __forceinline__ float4 load4v(const typename TX::T* p) {
  if constexpr (sizeof(typename TX::T) == 4) {
    return *reinterpret_cast<const float4*>(p);
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    const typename TX::T h[4] = {static_cast<typename TX::T>(v.x & 0xffff), static_cast<typename TX::T>(v.x >> 16),
                                 static_cast<typename TX::T>(v.y & 0xffff), static_cast<typename TX::T>(v.y >> 16)};
    return make_float4(TX::ld(h, 0), TX::ld(h, 1), TX::ld(h, 2), TX::ld(h, 3));
  }
}

// logits for up to 8 tokens: one workgroup per expert, its 4 waves split the hidden dim (float4 loads of
// the fp32 router row), partial sums reduced through LDS in wave order. (A router row is 4-8 KB: spread
// over E workgroups the rows stream at full-chip bandwidth; one CU alone keeps too few misses in flight.)
// With norm_w (bf16) the rows are RMS-normalised on the fly exactly as mm_rms_norm writes them,
// xn = bf16(w * bf16(x * rstd)); workgroup 0 then stores xn to xn_out ([n_tokens, H], bf16) when given.
template <class TX>
__global__ __launch_bounds__(256) void router_gemv_kernel(const typename TX::T* __restrict__ x, int n_tokens, int64_t H,
                                                          int64_t xs, const float* __restrict__ w32, int E,
                                                          float* __restrict__ logits,
                                                          const uint16_t* __restrict__ norm_w, float eps,
                                                          uint16_t* __restrict__ xn_out) {
  __shared__ float red[4][8];
  __shared__ float red4[4];
  const int e = blockIdx.x;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const float* wr = w32 + static_cast<int64_t>(e) * H;
  float rstd[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) rstd[t] = 1.f;
  if (norm_w) {
    for (int t = 0; t < n_tokens; ++t) {
      const float r = row_rstd256<TX>(x + t * xs, H, eps, red4);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (q == t) rstd[q] = r;
    }
  }
  const bool store_xn = xn_out && blockIdx.x == 0;
  float acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = 0.f;
  if ((H & 3) == 0) {
    for (int64_t h = 4 * static_cast<int64_t>(threadIdx.x); h < H; h += 4 * 256) {
      const float4 wv = *reinterpret_cast<const float4*>(wr + h);
      float4 nw = make_float4(1.f, 1.f, 1.f, 1.f);
      if (norm_w) nw = make_float4(bf16_to_f32(norm_w[h]), bf16_to_f32(norm_w[h + 1]), bf16_to_f32(norm_w[h + 2]),
                                   bf16_to_f32(norm_w[h + 3]));
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if (t < n_tokens) {
          float4 xv = load4<TX>(x + t * xs, h);
          if (norm_w) {
            xv.x = round_bf16(nw.x * round_bf16(xv.x * rstd[t]));
            xv.y = round_bf16(nw.y * round_bf16(xv.y * rstd[t]));
            xv.z = round_bf16(nw.z * round_bf16(xv.z * rstd[t]));
            xv.w = round_bf16(nw.w * round_bf16(xv.w * rstd[t]));
            if (store_xn) {
              uint16_t* o = xn_out + t * H + h;
              o[0] = f32_to_bf16(xv.x);
              o[1] = f32_to_bf16(xv.y);
              o[2] = f32_to_bf16(xv.z);
              o[3] = f32_to_bf16(xv.w);
            }
          }
          acc[t] = fmaf(xv.x, wv.x, acc[t]);
          acc[t] = fmaf(xv.y, wv.y, acc[t]);
          acc[t] = fmaf(xv.z, wv.z, acc[t]);
          acc[t] = fmaf(xv.w, wv.w, acc[t]);
        }
      }
    }
  } else {
    for (int64_t h = threadIdx.x; h < H; h += 256) {
      const float wv = wr[h];
      const float nw = norm_w ? bf16_to_f32(norm_w[h]) : 1.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if (t < n_tokens) {
          float xv = TX::ld(x + t * xs, h);
          if (norm_w) {
            xv = round_bf16(nw * round_bf16(xv * rstd[t]));
            if (store_xn) xn_out[t * H + h] = f32_to_bf16(xv);
          }
          acc[t] = fmaf(xv, wv, acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t < n_tokens) {
      const float v = wave_sum(acc[t]);
      if (lane == 0) red[wave][t] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < n_tokens)
    logits[static_cast<int64_t>(threadIdx.x) * E + e] =
        ((red[0][threadIdx.x] + red[1][threadIdx.x]) + red[2][threadIdx.x]) + red[3][threadIdx.x];
}

// The same for bf16 rows of at most 2048 * J elements (H a multiple of 8, 16-byte aligned rows), in one
// memory round trip: thread i owns the 8-element chunks i + 256 j, and every load of the workgroup (its
// router row, the RMSNorm weight, the token rows) is issued at kernel start through buffer resources.
// The sum of squares runs over the chunks exactly as row_rstd256 does, so xn matches mm_rms_norm bit for
// bit; a chunk's logit terms are added in element order, chunks in j order, then the waves in order.
template <int J, int NT>
__global__ __launch_bounds__(256) void router_gemv_bf16_kernel(const uint16_t* __restrict__ x, int n_tokens, int64_t H,
                                                               int64_t xs, const float* __restrict__ w32, int E,
                                                               float* __restrict__ logits,
                                                               const uint16_t* __restrict__ norm_w, float eps,
                                                               uint16_t* __restrict__ xn_out) {
  __shared__ float red_ss[NT][4];
  __shared__ float red[4][NT];
  const int e = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int nch = static_cast<int>(H / 8);
  const rsrc_t wr = make_rsrc(w32 + static_cast<int64_t>(e) * H, H * 4);
  const rsrc_t xr = make_rsrc(x, static_cast<int64_t>(n_tokens) * xs * 2);
  const rsrc_t nr = make_rsrc(norm_w, norm_w ? H * 2 : 0);
  uint4 wv[J][2], nv[J], xv[J][NT];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = tid + 256 * j;
    const bool ok = c < nch;
    wv[j][0] = buf16(wr, ok ? static_cast<uint32_t>(c) * 32u : kPast);
    wv[j][1] = buf16(wr, ok ? static_cast<uint32_t>(c) * 32u + 16u : kPast);
    nv[j] = buf16(nr, ok ? static_cast<uint32_t>(c) * 16u : kPast);
#pragma unroll
    for (int t = 0; t < NT; ++t)  // a token past n_tokens reads zero (no branch: a load behind one is waited on)
      xv[j][t] = buf16(xr, ok && t < n_tokens ? static_cast<uint32_t>(t * xs * 2 + c * 16) : kPast);
  }
  float rstd[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) rstd[t] = 1.f;
  if (norm_w) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < n_tokens) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < J; ++j) ss = chunk_ss_bf16x8(xv[j][t], ss);
        ss = wave_sum(ss);
        if (lane == 0) red_ss[t][wave] = ss;
      }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (t < n_tokens)
        rstd[t] = rsqrtf((((red_ss[t][0] + red_ss[t][1]) + red_ss[t][2]) + red_ss[t][3]) / static_cast<float>(H) + eps);
  }
  const bool store_xn = xn_out && e == 0;
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = tid + 256 * j;
    const uint32_t wq[8] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w, wv[j][1].x, wv[j][1].y, wv[j][1].z, wv[j][1].w};
    const uint32_t nq[4] = {nv[j].x, nv[j].y, nv[j].z, nv[j].w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < n_tokens) {
        const uint32_t xq[4] = {xv[j][t].x, xv[j][t].y, xv[j][t].z, xv[j][t].w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float lo = __uint_as_float(xq[i] << 16), hi = __uint_as_float(xq[i] & 0xffff0000u);
          if (norm_w) {
            lo = round_bf16(__uint_as_float(nq[i] << 16) * round_bf16(lo * rstd[t]));
            hi = round_bf16(__uint_as_float(nq[i] & 0xffff0000u) * round_bf16(hi * rstd[t]));
          }
          o[i] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
          acc[t] = fmaf(lo, __uint_as_float(wq[2 * i]), acc[t]);
          acc[t] = fmaf(hi, __uint_as_float(wq[2 * i + 1]), acc[t]);
        }
        if (store_xn && c < nch) reinterpret_cast<uint4*>(xn_out + t * H)[c] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t < n_tokens) {
      const float v = wave_sum(acc[t]);
      if (lane == 0) red[wave][t] = v;
    }
  }
  __syncthreads();
  if (tid < n_tokens)
    logits[static_cast<int64_t>(tid) * E + e] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
}

// logits for many tokens on fp32 MFMA (v_mfma_f32_16x16x4_f32): a workgroup of 16 waves computes 16
// tokens x 16 experts, each wave a contiguous run of the hidden dim. In a wave the lane (row r = lane % 16,
// quarter q = lane / 16) takes k = run + 16j + 4q + i of token row r and router row r, so the 4 quarters
// of a row read adjacent 16-byte pieces; MFMA step i of group j takes element i (any k order is valid
// while the token and expert operands of a lane agree). Each lane fetches its groups in batches of 8 before
// issuing their MFMAs; the 16 wave partials are summed through LDS in wave order.
constexpr int kRouterWaves = 16;

template <class TX>
__global__ __launch_bounds__(kRouterWaves * 64) void router_mfma_kernel(const typename TX::T* __restrict__ x,
                                                                        int n_tokens, int64_t H, int64_t xs,
                                                                        const float* __restrict__ w32, int E,
                                                                        float* __restrict__ logits) {
  constexpr int U = 8;  // 16-k groups in flight per lane
  __shared__ float red[kRouterWaves][16][17];
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int t0 = blockIdx.y * 16, e0 = blockIdx.x * 16;
  const int row = lane % 16, q = lane / 16;
  const int t = t0 + row, e = e0 + row;
  const bool tok = t < n_tokens, exp_ok = e < E;
  // this wave's run of the hidden dim: KW consecutive k, KW a multiple of 16
  const int64_t KW = (H + kRouterWaves * 16 - 1) / (kRouterWaves * 16) * 16;
  const int64_t kw0 = static_cast<int64_t>(wave) * KW;
  const typename TX::T* xr = x + static_cast<int64_t>(tok ? t : 0) * xs;
  const float* wr = w32 + static_cast<int64_t>(exp_ok ? e : 0) * H;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  // vector path: whole 4-element pieces at aligned addresses, loads made unconditional (masked pieces read
  // zeros) so that no load sits in a divergent branch
  const bool vec = (H & 3) == 0 && (xs & 3) == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & (4 * sizeof(typename TX::T) - 1)) == 0 &&
                   (reinterpret_cast<uintptr_t>(w32) & 15) == 0;
  if (vec) {
    const typename TX::T* xz = reinterpret_cast<const typename TX::T*>(g_zero4);
    for (int64_t j0 = 0; j0 < KW; j0 += 16 * U) {
      float4 av[U], bv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t k = kw0 + j0 + 16 * u + 4 * q;
        const bool in = j0 + 16 * u < KW && k < H;  // H % 4 == 0: a piece is whole or out
        bv[u] = *reinterpret_cast<const float4*>(in && exp_ok ? wr + k : g_zero4);
        av[u] = load4v<TX>(in && tok ? xr + k : xz);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].x, bv[u].x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].y, bv[u].y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].z, bv[u].z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u].w, bv[u].w, acc, 0, 0, 0);
      }
    }
  } else {
    for (int64_t j = 0; j < KW; j += 16) {
      const int64_t k = kw0 + j + 4 * q;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool in = k + i < H;
        const float a1 = (tok && in) ? TX::ld(xr, k + i) : 0.f;
        const float b1 = (exp_ok && in) ? wr[k + i] : 0.f;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc, 0, 0, 0);
      }
    }
  }
  // D[token = 4*(lane/16) + v][expert = lane % 16]
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave][4 * q + v][row] = acc[v];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int i = threadIdx.x / 16, jj = threadIdx.x % 16;
    if (t0 + i < n_tokens && e0 + jj < E) {
      float sum = red[0][i][jj];
#pragma unroll
      for (int w = 1; w < kRouterWaves; ++w) sum += red[w][i][jj];
      logits[static_cast<int64_t>(t0 + i) * E + e0 + jj] = sum;
    }
  }
}

// router_mfma_kernel with the RMSNorm fused, for the prefill block (bf16 rows of at most 512 * NC
// elements, H a multiple of 8, 16-byte aligned): wave w first normalises token row t0 + w in one pass
// (norm_row_chunks64: the bits of mm_rms_norm) into LDS, and the workgroups of the first expert group store
// those rows to xn_out; the MFMA loop is router_mfma_kernel's, with the token operand read from LDS, so
// the logits are those of mm_rms_norm + router_mfma_kernel bit for bit. Saves the norm's launch.
template <int NC>
__global__ __launch_bounds__(kRouterWaves * 64) void router_norm_mfma_kernel(const uint16_t* __restrict__ x,
                                                                             int n_tokens, int64_t H, int64_t xs,
                                                                             const uint16_t* __restrict__ norm_w,
                                                                             float eps, const float* __restrict__ w32,
                                                                             int E, float* __restrict__ logits,
                                                                             uint16_t* __restrict__ xn_out) {
  constexpr int U = 8;  // 16-k groups in flight per lane
  extern __shared__ uint4 rows_lds[];
  __shared__ float red[kRouterWaves][16][17];
  uint16_t* xl = reinterpret_cast<uint16_t*>(rows_lds);
  const int64_t P = H + 16;  // LDS row pitch (elements): the 16 rows an operand load reads hit distinct banks
  const int lane = lane_id(), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int t0 = blockIdx.y * 16, e0 = blockIdx.x * 16;
  {
    const int t = t0 + wave;
    const int64_t nch = H / 8;
    const rsrc_t xr = make_rsrc(x, static_cast<int64_t>(n_tokens) * xs * 2);
    const rsrc_t nr = make_rsrc(norm_w, H * 2);
    uint4 xv[NC], nv[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t c = lane + 64 * j;
      xv[j] = buf16(xr, c < nch && t < n_tokens ? static_cast<uint32_t>(t * xs * 2 + c * 16) : kPast);
      nv[j] = buf16(nr, c < nch ? static_cast<uint32_t>(c * 16) : kPast);
    }
    norm_row_chunks64<NC>(xv, nv, H, eps);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t c = lane + 64 * j;
      if (c < nch) {
        *reinterpret_cast<uint4*>(xl + wave * P + c * 8) = xv[j];
        if (blockIdx.x == 0 && t < n_tokens) *reinterpret_cast<uint4*>(xn_out + static_cast<int64_t>(t) * H + c * 8) = xv[j];
      }
    }
  }
  __syncthreads();
  const int row = lane % 16, q = lane / 16;
  const int e = e0 + row;
  const bool exp_ok = e < E;
  const int64_t KW = (H + kRouterWaves * 16 - 1) / (kRouterWaves * 16) * 16;
  const int64_t kw0 = static_cast<int64_t>(wave) * KW;
  const float* wr = w32 + static_cast<int64_t>(exp_ok ? e : 0) * H;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t j0 = 0; j0 < KW; j0 += 16 * U) {
    float4 bv[U];
    uint2 araw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = kw0 + j0 + 16 * u + 4 * q;
      const bool in = j0 + 16 * u < KW && k < H;
      bv[u] = *reinterpret_cast<const float4*>(in && exp_ok ? wr + k : g_zero4);
      araw[u] = in ? *reinterpret_cast<const uint2*>(xl + row * P + k) : make_uint2(0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(araw[u].x << 16), bv[u].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(araw[u].x & 0xffff0000u), bv[u].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(araw[u].y << 16), bv[u].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(araw[u].y & 0xffff0000u), bv[u].w, acc, 0, 0, 0);
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave][4 * q + v][row] = acc[v];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int i = threadIdx.x / 16, jj = threadIdx.x % 16;
    if (t0 + i < n_tokens && e0 + jj < E) {
      float sum = red[0][i][jj];
#pragma unroll
      for (int w = 1; w < kRouterWaves; ++w) sum += red[w][i][jj];
      logits[static_cast<int64_t>(t0 + i) * E + e0 + jj] = sum;
    }
  }
}

struct SelectArgs {
  const float* logits;
  int n_tokens, E;
  const float* bias;
  int scoring, n_group, topk_group, top_k;
  float scale;
  int append_shared;
  void* ids;
  int ids_dtype;
  float* wts;
  int64_t out_stride;
};

// One wave per token: selection, weights and the optional shared-expert slot.
template <int NS>
__global__ __launch_bounds__(256) void router_select_kernel(SelectArgs a) {
  __shared__ float rbuf[4][NS * kWave];
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform: the logit row's address too
  const int t = blockIdx.x * 4 + wv;
  if (t >= a.n_tokens) return;
  const int lane = lane_id();
  const SelectParams sp{a.bias, a.E, a.scoring, a.n_group, a.topk_group, a.top_k, a.scale, a.append_shared};
  int id;
  float w;
  bool has;
  select_any<NS>(sp, a.logits + static_cast<int64_t>(t) * a.E, rbuf[wv], id, w, has);
  if (has) {
    const int64_t o = static_cast<int64_t>(t) * a.out_stride + lane;
    a.wts[o] = w;
    if (a.ids_dtype == MM_INT64) static_cast<int64_t*>(a.ids)[o] = id;
    else static_cast<int32_t*>(a.ids)[o] = id;
  }
}

int check_select(int64_t n_tokens, int64_t E, int scoring, int n_group, int topk_group, int top_k, int append_shared,
                 const void* ids, int ids_dtype, const float* wts, int64_t out_row_stride) {
  MM_REQUIRE(n_tokens >= 0 && n_tokens <= 0x7fffffffLL, "router: bad token count %lld", (long long)n_tokens);
  MM_REQUIRE(E >= 1 && E <= kMaxExperts, "router: n_experts must be in [1, %d], got %lld", kMaxExperts, (long long)E);
  MM_REQUIRE(top_k >= 1 && top_k <= E && top_k + (append_shared ? 1 : 0) <= kWave,
             "router: top_k=%d out of range for %lld experts", top_k, (long long)E);
  MM_REQUIRE(scoring == MM_SCORE_SIGMOID_GROUP || scoring == MM_SCORE_SOFTMAX, "router: unknown scoring mode %d", scoring);
  MM_REQUIRE(n_group >= 1 && E % n_group == 0 && n_group <= kMaxExperts, "router: n_group=%d must divide n_experts=%lld",
             n_group, (long long)E);
  MM_REQUIRE(scoring == MM_SCORE_SIGMOID_GROUP || n_group == 1, "router: softmax scoring takes n_group=1 (got %d)", n_group);
  MM_REQUIRE(topk_group >= 1 && topk_group <= n_group, "router: topk_group=%d must be in [1, n_group=%d]", topk_group, n_group);
  MM_REQUIRE(static_cast<int64_t>(topk_group) * (E / n_group) >= top_k,
             "router: top_k=%d exceeds the experts of the kept groups (%lld)", top_k,
             (long long)(static_cast<int64_t>(topk_group) * (E / n_group)));
  MM_REQUIRE(ids_dtype == MM_INT32 || ids_dtype == MM_INT64, "router: ids dtype must be int32 or int64");
  MM_REQUIRE(ids && wts, "router: null output pointer");
  MM_REQUIRE(out_row_stride >= top_k + (append_shared ? 1 : 0), "router: output row stride %lld too small",
             (long long)out_row_stride);
  return MM_OK;
}

int launch_select(const float* logits, int64_t n_tokens, int64_t E, const float* bias, int scoring, int n_group,
                  int topk_group, int top_k, float scale, int append_shared, void* ids, int ids_dtype, float* wts,
                  int64_t out_row_stride, hipStream_t s) {
  SelectArgs a{logits, static_cast<int>(n_tokens), static_cast<int>(E), bias, scoring, n_group, topk_group, top_k,
               scale, append_shared, ids, ids_dtype, wts, out_row_stride};
  const unsigned blocks = static_cast<unsigned>((n_tokens + 3) / 4);
  switch (select_slots(E, n_group)) {  // lane-held slots: enough for the experts and the groups
    case 1: hipLaunchKernelGGL(router_select_kernel<1>, dim3(blocks), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(router_select_kernel<2>, dim3(blocks), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(router_select_kernel<4>, dim3(blocks), dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(router_select_kernel<kSlots>, dim3(blocks), dim3(256), 0, s, a); break;
  }
  return mm::check_launch("router_select");
}

template <class TX>
int launch_logits(const void* x, int64_t n_tokens, int64_t H, int64_t xs, const float* w32, int64_t E, float* logits,
                  hipStream_t s, const void* norm_w = nullptr, float eps = 0.f, void* xn_out = nullptr) {
  const auto* xp = static_cast<const typename TX::T*>(x);
  const auto* nw = static_cast<const uint16_t*>(norm_w);
  auto* xo = static_cast<uint16_t*>(xn_out);
  const bool fast = TX::kBf16 && (H & 7) == 0 && H <= 4096 && (xs & 7) == 0 && mm::aligned16(x) && mm::aligned16(w32) &&
                    (!norm_w || mm::aligned16(norm_w)) && (!xn_out || mm::aligned16(xn_out)) &&
                    n_tokens * xs * 2 < (1LL << 31);
  if (n_tokens <= 8 && fast) {  // the RMSNorm is fused only for up to 8 tokens; larger batches take normalised rows
    const auto* xb = static_cast<const uint16_t*>(x);
    const dim3 grid(static_cast<unsigned>(E));
    const int nt = static_cast<int>(n_tokens), e = static_cast<int>(E);
    if (H <= 2048 && n_tokens == 1)
      hipLaunchKernelGGL((router_gemv_bf16_kernel<1, 1>), grid, dim3(256), 0, s, xb, nt, H, xs, w32, e, logits, nw, eps, xo);
    else if (H <= 2048)
      hipLaunchKernelGGL((router_gemv_bf16_kernel<1, 8>), grid, dim3(256), 0, s, xb, nt, H, xs, w32, e, logits, nw, eps, xo);
    else if (n_tokens == 1)
      hipLaunchKernelGGL((router_gemv_bf16_kernel<2, 1>), grid, dim3(256), 0, s, xb, nt, H, xs, w32, e, logits, nw, eps, xo);
    else
      hipLaunchKernelGGL((router_gemv_bf16_kernel<2, 8>), grid, dim3(256), 0, s, xb, nt, H, xs, w32, e, logits, nw, eps, xo);
  } else if (n_tokens <= 8) {
    hipLaunchKernelGGL(router_gemv_kernel<TX>, dim3(static_cast<unsigned>(E)), dim3(256), 0, s, xp,
                       static_cast<int>(n_tokens), H, xs, w32, static_cast<int>(E), logits, nw, eps, xo);
  } else {
    dim3 grid(static_cast<unsigned>((E + 15) / 16), static_cast<unsigned>((n_tokens + 15) / 16));
    hipLaunchKernelGGL(router_mfma_kernel<TX>, grid, dim3(kRouterWaves * 64), 0, s, xp, static_cast<int>(n_tokens), H,
                       xs, w32, static_cast<int>(E), logits);
  }
  return mm::check_launch("router_logits");
}

}  // namespace

namespace mm {

// Router of the MoE block front for bf16 tokens: RMSNorm (norm_w bf16, eps) into xn_out ([n_tokens, H]
// bf16), logits of the normalised rows, then the selection with the shared expert appended. The norm runs
// inside the logits kernel (router_gemv_bf16_kernel up to 8 tokens, router_norm_mfma_kernel above, each
// workgroup normalising its 16 token rows); rows too long or misaligned for those normalise first
// (mm_rms_norm). Either way xn is bit-identical. with_select false stops after the logits (a caller that
// selects inside its next kernel).
int router_front(const void* x, int64_t n_tokens, int64_t H, int64_t xs, const void* norm_w, float eps,
                 const float* w32, const SelectParams& sp, float* logits, void* ids, int ids_dtype, float* wts,
                 int64_t out_row_stride, void* xn_out, hipStream_t s, bool with_select) {
  MM_REQUIRE(n_tokens >= 1 && n_tokens <= 0x7fffffffLL, "router: bad token count");
  int rc;
  const bool fused = n_tokens > 8 && H % 8 == 0 && H <= 4096 && xs % 8 == 0 && xn_out && aligned16(x) &&
                     aligned16(norm_w) && aligned16(xn_out) && aligned16(w32) && n_tokens * xs * 2 < (1LL << 31);
  if (n_tokens <= 8) {
    rc = launch_logits<BF16>(x, n_tokens, H, xs, w32, sp.E, logits, s, norm_w, eps, xn_out);
  } else if (fused) {  // the norm inside the logits kernel: one launch fewer
    dim3 grid(static_cast<unsigned>((sp.E + 15) / 16), static_cast<unsigned>((n_tokens + 15) / 16));
    const size_t lds = static_cast<size_t>(16) * (H + 16) * 2;
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* nw = static_cast<const uint16_t*>(norm_w);
    auto* xo = static_cast<uint16_t*>(xn_out);
    if (H <= 2048) {
      if ((rc = allow_lds(router_norm_mfma_kernel<4>, lds, "router_norm"))) return rc;
      hipLaunchKernelGGL(router_norm_mfma_kernel<4>, grid, dim3(kRouterWaves * 64), lds, s, xp,
                         static_cast<int>(n_tokens), H, xs, nw, eps, w32, static_cast<int>(sp.E), logits, xo);
    } else {
      if ((rc = allow_lds(router_norm_mfma_kernel<8>, lds, "router_norm"))) return rc;
      hipLaunchKernelGGL(router_norm_mfma_kernel<8>, grid, dim3(kRouterWaves * 64), lds, s, xp,
                         static_cast<int>(n_tokens), H, xs, nw, eps, w32, static_cast<int>(sp.E), logits, xo);
    }
    if ((rc = check_launch("router_norm"))) return rc;
  } else {
    rc = mm_rms_norm(x, MM_BF16, n_tokens, H, xs, norm_w, MM_BF16, eps, xn_out, MM_BF16, H, s);
    if (rc) return rc;
    rc = launch_logits<BF16>(xn_out, n_tokens, H, H, w32, sp.E, logits, s);
  }
  if (rc || !with_select) return rc;
  return launch_select(logits, n_tokens, sp.E, sp.bias, sp.scoring, sp.n_group, sp.topk_group, sp.top_k, sp.scale,
                       sp.append_shared, ids, ids_dtype, wts, out_row_stride, s);
}

int check_router_args(int64_t n_tokens, int64_t E, int scoring, int n_group, int topk_group, int top_k,
                      int append_shared, const void* ids, int ids_dtype, const float* wts, int64_t out_row_stride) {
  return check_select(n_tokens, E, scoring, n_group, topk_group, top_k, append_shared, ids, ids_dtype, wts,
                      out_row_stride);
}


}  // namespace mm

extern "C" int mm_router_select(const float* logits, int64_t n_tokens, int64_t n_experts, const float* bias, int scoring,
                                int n_group, int topk_group, int top_k, float scale, int append_shared, void* ids,
                                int ids_dtype, float* wts, int64_t out_row_stride, void* stream) {
  int rc = check_select(n_tokens, n_experts, scoring, n_group, topk_group, top_k, append_shared, ids, ids_dtype, wts,
                        out_row_stride);
  if (rc) return rc;
  MM_REQUIRE(logits, "router_select: null logits");
  if (n_tokens == 0) return MM_OK;
  return launch_select(logits, n_tokens, n_experts, bias, scoring, n_group, topk_group, top_k, scale, append_shared,
                       ids, ids_dtype, wts, out_row_stride, MM_STREAM(stream));
}

extern "C" int mm_router(const void* x, int x_dtype, int64_t n_tokens, int64_t hidden, int64_t x_row_stride,
                         const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                         int topk_group, int top_k, float scale, int append_shared, float* logits, void* ids,
                         int ids_dtype, float* wts, int64_t out_row_stride, void* stream) {
  int rc = check_select(n_tokens, n_experts, scoring, n_group, topk_group, top_k, append_shared, ids, ids_dtype, wts,
                        out_row_stride);
  if (rc) return rc;
  MM_REQUIRE(x && w32 && logits, "router: null pointer");
  MM_REQUIRE(hidden > 0 && x_row_stride >= hidden, "router: bad hidden size %lld / stride %lld", (long long)hidden,
             (long long)x_row_stride);
  if (n_tokens == 0) return MM_OK;
  hipStream_t s = MM_STREAM(stream);
  switch (x_dtype) {
    case MM_BF16: rc = launch_logits<BF16>(x, n_tokens, hidden, x_row_stride, w32, n_experts, logits, s); break;
    case MM_FP16: rc = launch_logits<FP16>(x, n_tokens, hidden, x_row_stride, w32, n_experts, logits, s); break;
    case MM_FP32: rc = launch_logits<FP32>(x, n_tokens, hidden, x_row_stride, w32, n_experts, logits, s); break;
    default: return mm::set_error(MM_ERR_ARG, "router: unsupported x dtype %d", x_dtype);
  }
  if (rc) return rc;
  return launch_select(logits, n_tokens, n_experts, bias, scoring, n_group, topk_group, top_k, scale, append_shared, ids,
                       ids_dtype, wts, out_row_stride, s);
}
