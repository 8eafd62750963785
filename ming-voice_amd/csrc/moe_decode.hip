// Decode MoE for 1..8 tokens (fused_moe.py:13-83): expert-gathered GEMV pair, HBM-bound.
//
// Kernel A (gate/up): grid (row tiles of I, distinct experts). Each workgroup finds the distinct experts of
// the batch from the ids (in first-appearance order), takes the one given by blockIdx.y, and streams its
// gate and up rows once with 16-byte loads, dotting them with every token routed to that expert.
//   a[p, r] = bf16(bf16(silu(bf16(g))) * bf16(u)),  g/u = x_t . row (* row scale for int8)
// Kernel B (down + combine): grid (row tiles of H). Each wave streams the down rows of one distinct
// expert for the tile, dots them with a[p] of every pair routed there, rounds to bf16 (after the row
// scale for int8) and parks the result in LDS; the workgroup then sums over slots in order per token:
//   y[t, h] = bf16(sum_k wts[t,k] * part[t*nk+k, h]) (+ residual, rounded again)
#include "mm_common.h"
#include "mm_select.h"

namespace {

using namespace mmd;

constexpr int kMaxPairs = 64;

struct DecodeArgs {
  const uint16_t* x;
  int64_t xs;
  int n_tokens, nk, P;
  const void* ids;
  int ids_dtype;
  int64_t ids_rs;
  const float* wts;
  int64_t wts_rs;
  const void* w_gu;
  const void* w_d;
  const void* s_gu;
  const void* s_d;
  int s_dtype;
  int E1;
  int64_t H, I;
  int64_t gu_se, gu_sn, d_se, d_sn, sgu_se, sd_se;
  const uint16_t* res;
  int64_t res_rs;
  uint16_t* a_buf;
  uint16_t* y;
  int64_t ys;
};

// Distinct experts of the batch. Lane p < P holds pair p's expert; returns the expert of distinct slot u
// (or -1 when the batch has fewer distinct experts) and the mask of pairs routed to it. Distinct experts
// are enumerated in first-appearance order: the lowest remaining lane leads, and one ballot takes every
// pair of its expert (one readlane + one ballot per distinct expert, no per-pair shuffles).
__device__ __forceinline__ int distinct_expert(const DecodeArgs& a, int u, unsigned long long& pairs) {
  const int lane = lane_id();
  int64_t id = -1;
  if (lane < a.P) {
    const int t = lane / a.nk, k = lane - t * a.nk;
    id = load_id(a.ids, a.ids_dtype, t * a.ids_rs + k);
    if (id < 0 || id >= a.E1) id = -1;
  }
  const int my = static_cast<int>(id);
  unsigned long long remaining = __ballot(my >= 0);
  for (int i = 0; remaining; ++i) {
    const int leader = __ffsll(static_cast<long long>(remaining)) - 1;
    const int e = __builtin_amdgcn_readlane(my, leader);
    const unsigned long long same = __ballot(my == e);
    if (i == u) {
      pairs = same;
      return e;
    }
    remaining &= ~same;
  }
  pairs = 0ull;
  return -1;
}

// 16-byte chunk c of a weight row holds CE elements; the matching activation chunk is CE bf16 values.
template <bool Q>
struct Act {
  uint4 v[Q ? 2 : 1];
};

template <bool Q>
__device__ __forceinline__ void load_act(Act<Q>& o, const uint16_t* row, int64_t c, bool ok) {
  if (!ok) {
    o.v[0] = make_uint4(0, 0, 0, 0);
    if (Q) o.v[Q ? 1 : 0] = make_uint4(0, 0, 0, 0);
    return;
  }
  const uint4* p = reinterpret_cast<const uint4*>(row + c * (Q ? 16 : 8));
  o.v[0] = p[0];
  if (Q) o.v[Q ? 1 : 0] = p[1];
}

template <bool Q>
__device__ __forceinline__ float dot_chunk(const uint4& w, const Act<Q>& x, float acc) {
  if constexpr (Q) return dot16_i8_bf16(w, x.v[0], x.v[Q ? 1 : 0], acc);
  else return dot8_bf16(w, x.v[0], acc);
}

__device__ __forceinline__ uint4 load_w(const void* base, int64_t byte_off, bool ok) {
  if (!ok) return make_uint4(0, 0, 0, 0);
  return *reinterpret_cast<const uint4*>(static_cast<const char*>(base) + byte_off);
}

// ------------------------------------------------------------------------------------------- kernel A

// Epilogue of one gate/up row pair for one pair p: scales (int8), bf16 rounding points, SiLU, product.
template <bool Q>
__device__ __forceinline__ void gate_up_store(const DecodeArgs& a, int e, int64_t r, int p, float ag, float au) {
  if (Q) {
    ag *= load_scale(a.s_gu, a.s_dtype, static_cast<int64_t>(e) * a.sgu_se + r);
    au *= load_scale(a.s_gu, a.s_dtype, static_cast<int64_t>(e) * a.sgu_se + a.I + r);
  }
  const float gg = round_bf16(ag), uu = round_bf16(au);
  const float act = round_bf16(silu(gg));
  a.a_buf[static_cast<int64_t>(p) * a.I + r] = f32_to_bf16(act * uu);
}

// One token per expert (batch 1, or a batch whose tokens chose distinct experts): the token's activation
// chunks stay in registers for all rows of the wave.
template <bool Q, int LPR, int NC, int R>
__device__ __forceinline__ void gate_up_one(const DecodeArgs& a, int e, int p, const char* wbase, int64_t row0) {
  constexpr int ES = Q ? 1 : 2;
  constexpr int GPW = kWave / LPR;
  const int lane = lane_id();
  const int g = lane / LPR, s = lane % LPR;
  const int64_t nch = a.H * ES / 16;
  const int tok = p / a.nk;
  float accg[R], accu[R];
#pragma unroll
  for (int i = 0; i < R; ++i) accg[i] = accu[i] = 0.f;
  for (int64_t c0 = 0; c0 < nch; c0 += static_cast<int64_t>(LPR) * NC) {  // one pass unless H is long
    Act<Q> xa[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
      load_act<Q>(xa[j], a.x + tok * a.xs, c, c < nch);
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t r = row0 + static_cast<int64_t>(GPW) * i + g;
      const bool rok = r < a.I;
      uint4 wg[NC], wu[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
        const bool ok = rok && c < nch;
        wg[j] = load_w(wbase, r * a.gu_sn * ES + c * 16, ok);
        wu[j] = load_w(wbase, (r + a.I) * a.gu_sn * ES + c * 16, ok);
      }
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        accg[i] = dot_chunk<Q>(wg[j], xa[j], accg[i]);
        accu[i] = dot_chunk<Q>(wu[j], xa[j], accu[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = row0 + static_cast<int64_t>(GPW) * i + g;
    const float ag = group_sum<LPR>(accg[i]), au = group_sum<LPR>(accu[i]);
    if (s == 0 && r < a.I) gate_up_store<Q>(a, e, r, p, ag, au);
  }
}

// Several tokens per expert: their activation rows are staged in LDS (bf16). Each weight row pair is loaded
// once into registers and dotted with every staged row in turn, so registers hold only the weight chunks.
// Needs the row in one pass (nch <= LPR * NC); the caller takes gate_up_one per token otherwise.
template <bool Q, int LPR, int NC, int R, int MAXT>
__device__ __forceinline__ void gate_up_many(const DecodeArgs& a, int e, int cntp, const int* spid, const char* wbase,
                                             int64_t row0, uint16_t* xs) {
  constexpr int ES = Q ? 1 : 2;
  constexpr int GPW = kWave / LPR;
  const int lane = lane_id();
  const int g = lane / LPR, s = lane % LPR;
  const int64_t nch = a.H * ES / 16;
  // stage the rows of this group's tokens (whole workgroup; the group is uniform across it)
  const int64_t row_chunks = a.H / 8;  // 16-byte chunks of one bf16 row
  for (int64_t i = threadIdx.x; i < cntp * row_chunks; i += blockDim.x) {
    const int t = static_cast<int>(i / row_chunks);
    const int64_t c = i % row_chunks;
    const int tok = spid[t] / a.nk;
    reinterpret_cast<uint4*>(xs + t * a.H)[c] = reinterpret_cast<const uint4*>(a.x + static_cast<int64_t>(tok) * a.xs)[c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = row0 + static_cast<int64_t>(GPW) * i + g;
    const bool rok = r < a.I;
    uint4 wg[NC], wu[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t c = s + static_cast<int64_t>(LPR) * j;
      const bool ok = rok && c < nch;
      wg[j] = load_w(wbase, r * a.gu_sn * ES + c * 16, ok);
      wu[j] = load_w(wbase, (r + a.I) * a.gu_sn * ES + c * 16, ok);
    }
    for (int t = 0; t < cntp; ++t) {
      float ag = 0.f, au = 0.f;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t c = s + static_cast<int64_t>(LPR) * j;
        Act<Q> xv;
        load_act<Q>(xv, xs + t * a.H, c, c < nch);
        ag = dot_chunk<Q>(wg[j], xv, ag);
        au = dot_chunk<Q>(wu[j], xv, au);
      }
      ag = group_sum<LPR>(ag);
      au = group_sum<LPR>(au);
      if (s == 0 && rok) gate_up_store<Q>(a, e, r, spid[t], ag, au);
    }
  }
  __syncthreads();  // the staging buffer is reused by the next group
}

constexpr int kMaxTokens = 8;

template <bool Q, int LPR, int NC, int R, int MAXT>
__global__ __launch_bounds__(256) void decode_gate_up_kernel(DecodeArgs a) {
  extern __shared__ uint4 xs_raw[];  // MAXT bf16 rows of the hidden dim (MAXT > 1 only)
  __shared__ int spid[MAXT];
  unsigned long long pairs;
  const int e = distinct_expert(a, blockIdx.y, pairs);
  if (e < 0) return;
  constexpr int ES = Q ? 1 : 2;
  constexpr int GPW = kWave / LPR;  // row pairs per wave per step
  const int wave = threadIdx.x / kWave;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * (GPW * R);
  const char* wbase = static_cast<const char*>(a.w_gu) + static_cast<int64_t>(e) * a.gu_se * ES;
  if constexpr (MAXT == 1) {
    while (pairs) {
      const int p = __ffsll(static_cast<long long>(pairs)) - 1;
      pairs &= pairs - 1ull;
      gate_up_one<Q, LPR, NC, R>(a, e, p, wbase, row0);
    }
  } else {
    const bool one_pass = a.H * ES / 16 <= static_cast<int64_t>(LPR) * NC;
    while (pairs) {
      if (!one_pass || __popcll(pairs) == 1) {
        const int p = __ffsll(static_cast<long long>(pairs)) - 1;
        pairs &= pairs - 1ull;
        gate_up_one<Q, LPR, NC, R>(a, e, p, wbase, row0);
        continue;
      }
      int cntp = 0;
      while (pairs && cntp < MAXT) {  // the next MAXT pairs of this expert, in pair order
        const int p = __ffsll(static_cast<long long>(pairs)) - 1;
        pairs &= pairs - 1ull;
        if (threadIdx.x == 0) spid[cntp] = p;
        ++cntp;
      }
      __syncthreads();
      gate_up_many<Q, LPR, NC, R, MAXT>(a, e, cntp, spid, wbase, row0, reinterpret_cast<uint16_t*>(xs_raw));
    }
  }
}

// ------------------------------------------------------------------------------------------- kernel B

constexpr int kDownWaves = 8;

template <bool Q, int LPR, int NC>
__global__ __launch_bounds__(kDownWaves * 64) void decode_down_kernel(DecodeArgs a) {
  constexpr int ES = Q ? 1 : 2;
  constexpr int RW = kWave / LPR;  // output rows per workgroup
  __shared__ float part[kMaxPairs][RW];
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int g = lane / LPR, s = lane % LPR;
  const int64_t h = static_cast<int64_t>(blockIdx.x) * RW + g;
  const bool hok = h < a.H;
  const int64_t nch = a.I * ES / 16;

  for (int i = threadIdx.x; i < kMaxPairs * RW; i += blockDim.x) (&part[0][0])[i] = 0.f;
  __syncthreads();

  for (int u = wave;; u += kDownWaves) {
    unsigned long long pairs;
    const int e = distinct_expert(a, u, pairs);
    if (e < 0) break;
    const char* wbase = static_cast<const char*>(a.w_d) + static_cast<int64_t>(e) * a.d_se * ES;
    float sc = 1.f;
    if (Q && hok) sc = load_scale(a.s_d, a.s_dtype, static_cast<int64_t>(e) * a.sd_se + h);
    if (nch <= static_cast<int64_t>(LPR) * NC) {
      // the whole row fits one pass: load the weights once for every pair of the expert
      uint4 w[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t c = s + static_cast<int64_t>(LPR) * j;
        w[j] = load_w(wbase, h * a.d_sn * ES + c * 16, hok && c < nch);
      }
      while (pairs) {
        const int p = __ffsll(static_cast<long long>(pairs)) - 1;
        pairs &= pairs - 1ull;
        const uint16_t* ar = a.a_buf + static_cast<int64_t>(p) * a.I;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          const int64_t c = s + static_cast<int64_t>(LPR) * j;
          Act<Q> av;
          load_act<Q>(av, ar, c, c < nch);
          acc = dot_chunk<Q>(w[j], av, acc);
        }
        acc = group_sum<LPR>(acc);
        if (s == 0 && hok) part[p][g] = round_bf16(Q ? acc * sc : acc);
      }
    } else {
      // long rows: passes of LPR * NC chunks per pair (weights re-read from cache for later pairs)
      while (pairs) {
        const int p = __ffsll(static_cast<long long>(pairs)) - 1;
        pairs &= pairs - 1ull;
        const uint16_t* ar = a.a_buf + static_cast<int64_t>(p) * a.I;
        float acc = 0.f;
        for (int64_t c0 = 0; c0 < nch; c0 += static_cast<int64_t>(LPR) * NC) {
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
            const uint4 w = load_w(wbase, h * a.d_sn * ES + c * 16, hok && c < nch);
            Act<Q> av;
            load_act<Q>(av, ar, c, c < nch);
            acc = dot_chunk<Q>(w, av, acc);
          }
        }
        acc = group_sum<LPR>(acc);
        if (s == 0 && hok) part[p][g] = round_bf16(Q ? acc * sc : acc);
      }
    }
  }
  __syncthreads();

  // combine: one thread per (token, row), slots summed in order
  const int tid = threadIdx.x;
  if (tid < a.n_tokens * RW) {
    const int t = tid / RW, r = tid % RW;
    const int64_t hh = static_cast<int64_t>(blockIdx.x) * RW + r;
    if (hh < a.H) {
      float acc = 0.f;
      for (int k = 0; k < a.nk; ++k) acc = fmaf(a.wts[t * a.wts_rs + k], part[t * a.nk + k][r], acc);
      float out = round_bf16(acc);
      if (a.res) out = out + bf16_to_f32(a.res[t * a.res_rs + hh]);
      a.y[t * a.ys + hh] = f32_to_bf16(out);
    }
  }
}

// --------------------------------------------------------------------------------------------- launch

template <bool Q, int LPR, int NC, int R, int MAXT>
int launch_a(const DecodeArgs& a, hipStream_t st) {
  constexpr int rows_per_wg = 4 * (kWave / LPR) * R;
  dim3 grid(static_cast<unsigned>((a.I + rows_per_wg - 1) / rows_per_wg), static_cast<unsigned>(min(a.P, a.E1)));
  const size_t lds = MAXT > 1 ? static_cast<size_t>(MAXT) * a.H * 2 : 0;
  hipLaunchKernelGGL((decode_gate_up_kernel<Q, LPR, NC, R, MAXT>), grid, dim3(256), lds, st, a);
  return mm::check_launch("moe_decode gate_up");
}

template <bool Q, int LPR, int NC>
int launch_b(const DecodeArgs& a, hipStream_t st) {
  constexpr int RW = kWave / LPR;
  dim3 grid(static_cast<unsigned>((a.H + RW - 1) / RW));
  hipLaunchKernelGGL((decode_down_kernel<Q, LPR, NC>), grid, dim3(kDownWaves * 64), 0, st, a);
  return mm::check_launch("moe_decode down");
}

// Template choice. A row of nch 16-byte chunks is split over LPR lanes with NC chunks per lane per
// pass; rows longer than LPR * NC chunks take several passes, so a few instances cover every shape.
// Row pairs per wave of the single-token gate/up kernel: one (more, smaller workgroups) measured best over
// 28 distinct layers against two to four.
#ifndef MM_GU_R_BF16
#define MM_GU_R_BF16 1
#endif
#ifndef MM_GU_R_I8
#define MM_GU_R_I8 1
#endif

template <bool Q, int LPR, int NC>
int dispatch_a_t(const DecodeArgs& a, hipStream_t st) {
  // tokens staged per group: one per token of the batch (a token naming an expert twice adds groups),
  // bounded so that the staged rows fit 64 KB of LDS
  int maxt = a.n_tokens;
  while (maxt > 1 && static_cast<int64_t>(maxt) * a.H * 2 > 65536) maxt /= 2;
  constexpr int R = Q ? MM_GU_R_I8 : MM_GU_R_BF16;  // row pairs per wave
  if (maxt <= 1) return launch_a<Q, LPR, NC, R, 1>(a, st);
  if (maxt <= 2) return launch_a<Q, LPR, NC, 2, 2>(a, st);
  if (maxt <= 4) return launch_a<Q, LPR, NC, 2, 4>(a, st);
  return launch_a<Q, LPR, NC, 2, 8>(a, st);
}

template <bool Q>
int dispatch_a(const DecodeArgs& a, hipStream_t st) {
  const int64_t nch = a.H * (Q ? 1 : 2) / 16;  // gate/up rows run over the hidden dim
  if (nch < 64) return dispatch_a_t<Q, 16, 4>(a, st);
  if (nch <= 128) return dispatch_a_t<Q, 64, 2>(a, st);
  if (nch <= 192) return dispatch_a_t<Q, 64, 3>(a, st);
  return dispatch_a_t<Q, 64, 4>(a, st);
}

// Lanes per row and chunks per lane of the down kernel for rows of the benchmarked size (1408 inter):
// 32 lanes read 512 contiguous bytes of a row per instruction; measured over 28 distinct layers, 32 lanes
// beat 16 (256-byte pieces) and 64 (one row per wave step, too little work per wave).
#ifndef MM_DOWN_BF16_LPR
#define MM_DOWN_BF16_LPR 32
#define MM_DOWN_BF16_NC 6
#endif
#ifndef MM_DOWN_I8_LPR
#define MM_DOWN_I8_LPR 32
#define MM_DOWN_I8_NC 3
#endif

template <bool Q>
int dispatch_b(const DecodeArgs& a, hipStream_t st) {
  const int64_t nch = a.I * (Q ? 1 : 2) / 16;  // down rows run over the intermediate dim
  if constexpr (Q) {  // int8 chunks carry 32-byte activation chunks: fewer chunks per lane
    if (nch > 48) return launch_b<Q, MM_DOWN_I8_LPR, MM_DOWN_I8_NC>(a, st);
    return launch_b<Q, 8, 6>(a, st);
  } else {
    if (nch >= 128) return launch_b<Q, MM_DOWN_BF16_LPR, MM_DOWN_BF16_NC>(a, st);
    if (nch > 32) return launch_b<Q, 8, 12>(a, st);
    return launch_b<Q, 8, 4>(a, st);
  }
}

}  // namespace

namespace mm {

// Validates the stacked expert descriptor for the 16-byte-chunk kernels.
int check_experts(const char* who, const mm_experts* ex) {
  MM_REQUIRE(ex, "%s: null expert descriptor", who);
  MM_REQUIRE(ex->w_dtype == MM_BF16 || ex->w_dtype == MM_INT8, "%s: expert weights must be bf16 or int8", who);
  const int64_t es = ex->w_dtype == MM_INT8 ? 1 : 2;
  MM_REQUIRE(ex->w_gu && ex->w_d, "%s: null expert weights", who);
  MM_REQUIRE(ex->n_slots >= 1 && ex->hidden > 0 && ex->inter > 0, "%s: bad expert shape", who);
  MM_REQUIRE((ex->hidden * es) % 16 == 0 && (ex->inter * es) % 16 == 0,
             "%s: hidden=%lld and inter=%lld must be multiples of %lld elements (16-byte rows)", who,
             (long long)ex->hidden, (long long)ex->inter, (long long)(16 / es));
  MM_REQUIRE(ex->gu_stride_n >= ex->hidden && ex->gu_stride_e >= 2 * ex->inter * ex->gu_stride_n,
             "%s: w_gu strides do not describe [E, 2I, H] with a contiguous last dim", who);
  MM_REQUIRE(ex->d_stride_n >= ex->inter && ex->d_stride_e >= ex->hidden * ex->d_stride_n,
             "%s: w_d strides do not describe [E, H, I] with a contiguous last dim", who);
  MM_REQUIRE(aligned16(ex->w_gu) && aligned16(ex->w_d) && (ex->gu_stride_n * es) % 16 == 0 &&
                 (ex->gu_stride_e * es) % 16 == 0 && (ex->d_stride_n * es) % 16 == 0 && (ex->d_stride_e * es) % 16 == 0,
             "%s: expert weight rows must be 16-byte aligned", who);
  if (ex->w_dtype == MM_INT8) {
    MM_REQUIRE(ex->s_gu && ex->s_d, "%s: int8 experts need s_gu and s_d", who);
    MM_REQUIRE(ex->s_dtype == MM_FP32 || ex->s_dtype == MM_BF16, "%s: scales must be fp32 or bf16", who);
    MM_REQUIRE(ex->sgu_stride_e >= 2 * ex->inter && ex->sd_stride_e >= ex->hidden, "%s: bad scale strides", who);
  }
  return MM_OK;
}

}  // namespace mm

extern "C" int mm_moe_decode(const void* x, int64_t n_tokens, int64_t x_row_stride, const mm_experts* ex,
                             const void* ids, int ids_dtype, int64_t nk, int64_t ids_row_stride, const float* wts,
                             int64_t wts_row_stride, const void* residual, int64_t res_row_stride, void* a_buf, void* y,
                             int64_t y_row_stride, int phases, void* stream) {
  int rc = mm::check_experts("moe_decode", ex);
  if (rc) return rc;
  MM_REQUIRE(n_tokens >= 1 && nk >= 1 && n_tokens * nk <= kMaxPairs,
             "moe_decode: n_tokens * nk must be in [1, %d] (got %lld x %lld)", kMaxPairs, (long long)n_tokens,
             (long long)nk);
  MM_REQUIRE(x && ids && wts && a_buf && y, "moe_decode: null pointer");
  MM_REQUIRE(ids_dtype == MM_INT32 || ids_dtype == MM_INT64, "moe_decode: ids must be int32 or int64");
  MM_REQUIRE(x_row_stride >= ex->hidden && y_row_stride >= ex->hidden, "moe_decode: row stride smaller than hidden");
  MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0, "moe_decode: x rows must be 16-byte aligned");
  MM_REQUIRE(mm::aligned16(a_buf), "moe_decode: a_buf must be 16-byte aligned");
  MM_REQUIRE(ids_row_stride >= nk && wts_row_stride >= nk, "moe_decode: ids/wts row stride smaller than nk");
  MM_REQUIRE(!residual || res_row_stride >= ex->hidden, "moe_decode: residual row stride smaller than hidden");
  MM_REQUIRE(ex->n_slots <= 0x7fffffff && ex->hidden <= 0x7fffffff && ex->inter <= 0x7fffffff, "moe_decode: shape too large");
  DecodeArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.xs = x_row_stride;
  a.n_tokens = static_cast<int>(n_tokens);
  a.nk = static_cast<int>(nk);
  a.P = static_cast<int>(n_tokens * nk);
  a.ids = ids;
  a.ids_dtype = ids_dtype;
  a.ids_rs = ids_row_stride;
  a.wts = wts;
  a.wts_rs = wts_row_stride;
  a.w_gu = ex->w_gu;
  a.w_d = ex->w_d;
  a.s_gu = ex->s_gu;
  a.s_d = ex->s_d;
  a.s_dtype = ex->s_dtype;
  a.E1 = static_cast<int>(ex->n_slots);
  a.H = ex->hidden;
  a.I = ex->inter;
  a.gu_se = ex->gu_stride_e;
  a.gu_sn = ex->gu_stride_n;
  a.d_se = ex->d_stride_e;
  a.d_sn = ex->d_stride_n;
  a.sgu_se = ex->sgu_stride_e;
  a.sd_se = ex->sd_stride_e;
  a.res = static_cast<const uint16_t*>(residual);
  a.res_rs = res_row_stride;
  a.a_buf = static_cast<uint16_t*>(a_buf);
  a.y = static_cast<uint16_t*>(y);
  a.ys = y_row_stride;
  hipStream_t st = MM_STREAM(stream);
  const bool q = ex->w_dtype == MM_INT8;
  if (phases == MM_PHASE_ALL) phases = MM_PHASE_GATE_UP | MM_PHASE_DOWN;
  if (phases & MM_PHASE_GATE_UP) {
    rc = q ? dispatch_a<true>(a, st) : dispatch_a<false>(a, st);
    if (rc) return rc;
  }
  if (phases & MM_PHASE_DOWN) return q ? dispatch_b<true>(a, st) : dispatch_b<false>(a, st);
  return MM_OK;
}

namespace mm {
int check_router_args(int64_t n_tokens, int64_t E, int scoring, int n_group, int topk_group, int top_k,
                      int append_shared, const void* ids, int ids_dtype, const float* wts, int64_t out_row_stride);
int router_front(const void* x, int64_t n_tokens, int64_t H, int64_t xs, const void* norm_w, float eps,
                 const float* w32, const mmd::SelectParams& sp, float* logits, void* ids, int ids_dtype, float* wts,
                 int64_t out_row_stride, void* xn_out, hipStream_t s);
}  // namespace mm

// Whole MoE block for 1..8 tokens in four launches: router logits (RMSNorm fused; the normalised rows go
// to the workspace), selection, gate/up on the normalised rows, down + combine with the raw rows as
// residual. (Selecting in the router's last-finishing workgroup instead costs more in device-wide fences
// than the launch it saves.) The ids / weights it writes are the ones the unfused chain produces.
extern "C" int mm_moe_block_decode(const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w, float eps,
                                   const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                                   int topk_group, int top_k, float scale, const mm_experts* ex, float* logits,
                                   void* ids, int ids_dtype, float* wts, void* a_buf, void* workspace,
                                   int add_residual, void* y, int64_t y_row_stride, void* stream) {
  int rc = mm::check_experts("moe_block_decode", ex);
  if (rc) return rc;
  const int64_t nk = static_cast<int64_t>(top_k) + 1;
  rc = mm::check_router_args(n_tokens, n_experts, scoring, n_group, topk_group, top_k, 1, ids, ids_dtype, wts, nk);
  if (rc) return rc;
  MM_REQUIRE(n_tokens >= 1 && n_tokens <= kMaxTokens && n_tokens * nk <= kMaxPairs,
             "moe_block_decode: 1..%d tokens with (top_k + 1) * tokens <= %d", kMaxTokens, kMaxPairs);
  MM_REQUIRE(ex->n_slots == n_experts + 1, "moe_block_decode: expert slots (%lld) must be n_experts + 1 (shared last)",
             (long long)ex->n_slots);
  MM_REQUIRE(x && norm_w && w32 && logits && a_buf && workspace && y, "moe_block_decode: null pointer");
  MM_REQUIRE(x_row_stride >= ex->hidden && y_row_stride >= ex->hidden, "moe_block_decode: row stride smaller than hidden");
  MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0 && mm::aligned16(a_buf) && mm::aligned16(workspace),
             "moe_block_decode: x, a_buf and workspace must be 16-byte aligned");
  MM_REQUIRE(ex->hidden <= 0x7fffffff && ex->inter <= 0x7fffffff, "moe_block_decode: shape too large");
  hipStream_t st = MM_STREAM(stream);
  const mmd::SelectParams sp{bias, static_cast<int>(n_experts), scoring, n_group, topk_group, top_k, scale, 1};
  void* xn = workspace;
  rc = mm::router_front(x, n_tokens, ex->hidden, x_row_stride, norm_w, eps, w32, sp, logits, ids, ids_dtype, wts, nk,
                        xn, st);
  if (rc) return rc;
  DecodeArgs a;
  a.x = static_cast<const uint16_t*>(xn);
  a.xs = ex->hidden;
  a.n_tokens = static_cast<int>(n_tokens);
  a.nk = static_cast<int>(nk);
  a.P = static_cast<int>(n_tokens * nk);
  a.ids = ids;
  a.ids_dtype = ids_dtype;
  a.ids_rs = nk;
  a.wts = wts;
  a.wts_rs = nk;
  a.w_gu = ex->w_gu;
  a.w_d = ex->w_d;
  a.s_gu = ex->s_gu;
  a.s_d = ex->s_d;
  a.s_dtype = ex->s_dtype;
  a.E1 = static_cast<int>(ex->n_slots);
  a.H = ex->hidden;
  a.I = ex->inter;
  a.gu_se = ex->gu_stride_e;
  a.gu_sn = ex->gu_stride_n;
  a.d_se = ex->d_stride_e;
  a.d_sn = ex->d_stride_n;
  a.sgu_se = ex->sgu_stride_e;
  a.sd_se = ex->sd_stride_e;
  a.res = add_residual ? static_cast<const uint16_t*>(x) : nullptr;
  a.res_rs = x_row_stride;
  a.a_buf = static_cast<uint16_t*>(a_buf);
  a.y = static_cast<uint16_t*>(y);
  a.ys = y_row_stride;
  const bool q = ex->w_dtype == MM_INT8;
  rc = q ? dispatch_a<true>(a, st) : dispatch_a<false>(a, st);
  if (rc) return rc;
  return q ? dispatch_b<true>(a, st) : dispatch_b<false>(a, st);
}
