// Grouped prefill MoE on bf16 MFMA (fused_moe.py:92-196).
//
// Pairs are grouped by expert into blocks of 64 rows by mm_align_blocks. Kernel GU computes, for one block
// and 64 columns of I, the gate and up projections of the 64 gathered token rows with
// v_mfma_f32_16x16x32_bf16 over LDS-staged k-slabs and writes a = bf16(bf16(silu(bf16(g))) * bf16(u)) per
// pair. Kernel DOWN computes o[pair] = f32(bf16(a . Wd^T [* s])) * w_pair for 128 columns of H. Kernel
// COMBINE sums the slots of each token in order (fp32) and rounds to bf16, adding the residual if given.
// int8 weights are widened to bf16 (exact for |q| <= 127) on their way into LDS; the row scale multiplies
// the fp32 accumulator before the bf16 rounding, as in the reference.
#include "mm_common.h"

namespace {

using namespace mmd;

constexpr int kBM = 64;        // rows (pairs) per block, = align block_m
constexpr int kBK = 64;        // k-slab
constexpr int kLdsK = kBK + 8; // padded LDS row (elements) against bank conflicts
constexpr int kThreads = 256;

struct PrefillArgs {
  const uint16_t* x;
  int64_t xs;
  int n_tokens, nk, P, E1;
  const void* ids;
  int ids_dtype;
  const float* wts;
  const int32_t* sorted_ids;
  const int32_t* bexp;
  int nb;
  const void* w_gu;
  const void* w_d;
  const void* s_gu;
  const void* s_d;
  int s_dtype;
  int64_t H, I;
  int64_t gu_se, gu_sn, d_se, d_sn, sgu_se, sd_se;
  const uint16_t* res;
  int64_t res_rs;
  uint16_t* a_buf;
  float* o_buf;
  uint16_t* y;
  int64_t ys;
};

// 16 int8 -> 16 bf16 (exact), as two uint4 of packed bf16 pairs.
__device__ __forceinline__ void widen_i8(const uint4& q, uint4& lo, uint4& hi) {
  uint32_t in[4] = {q.x, q.y, q.z, q.w};
  uint32_t out[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = in[i];
    const uint32_t b0 = f32_to_bf16(sbyte(v, 0)), b1 = f32_to_bf16(sbyte(v, 1));
    const uint32_t b2 = f32_to_bf16(sbyte(v, 2)), b3 = f32_to_bf16(sbyte(v, 3));
    out[2 * i] = b0 | (b1 << 16);
    out[2 * i + 1] = b2 | (b3 << 16);
  }
  lo = make_uint4(out[0], out[1], out[2], out[3]);
  hi = make_uint4(out[4], out[5], out[6], out[7]);
}

// Stage `rows` weight rows x kBK k-values (bf16 in LDS) starting at k0. Row r of the tile is weight row
// row_of(r); rows past `nrows` or k past K are zero.
template <bool Q, int ROWS, class RowFn>
__device__ __forceinline__ void stage_w(uint16_t (*lds)[kLdsK], const char* wbase, int64_t row_stride_el, int64_t K,
                                        int64_t k0, RowFn row_of) {
  constexpr int ES = Q ? 1 : 2;
  constexpr int CPR = kBK * ES / 16;  // 16-byte chunks per row of the slab
  constexpr int TOTAL = ROWS * CPR;
  for (int i = threadIdx.x; i < TOTAL; i += kThreads) {
    const int r = i / CPR, c = i % CPR;
    const int64_t wr = row_of(r);
    const int64_t k = k0 + static_cast<int64_t>(c) * (16 / ES);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (wr >= 0 && k < K) v = *reinterpret_cast<const uint4*>(wbase + (wr * row_stride_el + k) * ES);
    if constexpr (Q) {
      uint4 lo, hi;
      widen_i8(v, lo, hi);
      *reinterpret_cast<uint4*>(&lds[r][c * 16]) = lo;
      *reinterpret_cast<uint4*>(&lds[r][c * 16 + 8]) = hi;
    } else {
      *reinterpret_cast<uint4*>(&lds[r][c * 8]) = v;
    }
  }
}

// Stage kBM activation rows x kBK (bf16) from rows given by src_row(r) (nullptr = zero row).
template <class SrcFn>
__device__ __forceinline__ void stage_a(uint16_t (*lds)[kLdsK], int64_t K, int64_t k0, SrcFn src_row) {
  constexpr int CPR = kBK / 8;
  for (int i = threadIdx.x; i < kBM * CPR; i += kThreads) {
    const int r = i / CPR, c = i % CPR;
    const uint16_t* src = src_row(r);
    const int64_t k = k0 + c * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (src && k < K) v = *reinterpret_cast<const uint4*>(src + k);
    *reinterpret_cast<uint4*>(&lds[r][c * 8]) = v;
  }
}

__device__ __forceinline__ bf16x8_t lds_frag(const uint16_t (*lds)[kLdsK], int row, int k) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(&lds[row][k]));
}

// ------------------------------------------------------------------------------------------- gate / up

template <bool Q>
__global__ __launch_bounds__(kThreads) void prefill_gate_up_kernel(PrefillArgs a) {
  constexpr int ES = Q ? 1 : 2;
  const int blk = blockIdx.x;
  const int e = a.bexp[blk];
  if (e < 0) return;
  __shared__ uint16_t sa[kBM][kLdsK];
  __shared__ uint16_t sb[128][kLdsK];  // rows 0..63 gate, 64..127 up
  __shared__ int spair[kBM];
  const int64_t n0 = static_cast<int64_t>(blockIdx.y) * 64;
  if (threadIdx.x < kBM) spair[threadIdx.x] = a.sorted_ids[static_cast<int64_t>(blk) * kBM + threadIdx.x];
  __syncthreads();
  const char* wbase = static_cast<const char*>(a.w_gu) + static_cast<int64_t>(e) * a.gu_se * ES;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int wm = wave / 2, wn = wave % 2;
  floatx4 accg[2][2], accu[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      accg[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
      accu[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  const int64_t I = a.I;
  for (int64_t k0 = 0; k0 < a.H; k0 += kBK) {
    stage_a(sa, a.H, k0, [&](int r) -> const uint16_t* {
      const int p = spair[r];
      return p < a.P ? a.x + static_cast<int64_t>(p / a.nk) * a.xs : nullptr;
    });
    stage_w<Q, 128>(sb, wbase, a.gu_sn, a.H, k0, [&](int r) -> int64_t {
      const int64_t col = n0 + (r & 63);
      if (col >= I) return -1;
      return r < 64 ? col : I + col;
    });
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 32) {
      const int kk = ks + 8 * (lane / 16);
      bf16x8_t fa[2], fg[2], fu[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = lds_frag(sa, 32 * wm + 16 * i + (lane % 16), kk);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        fg[j] = lds_frag(sb, 32 * wn + 16 * j + (lane % 16), kk);
        fu[j] = lds_frag(sb, 64 + 32 * wn + 16 * j + (lane % 16), kk);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          accg[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fg[j], accg[i][j], 0, 0, 0);
          accu[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fu[j], accu[i][j], 0, 0, 0);
        }
    }
    __syncthreads();
  }
  // epilogue: D[row = 4*(lane/16) + v][col = lane%16] of each 16x16 tile
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = n0 + 32 * wn + 16 * j + (lane % 16);
    if (col >= I) continue;
    float sg = 1.f, su = 1.f;
    if (Q) {
      sg = load_scale(a.s_gu, a.s_dtype, static_cast<int64_t>(e) * a.sgu_se + col);
      su = load_scale(a.s_gu, a.s_dtype, static_cast<int64_t>(e) * a.sgu_se + I + col);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 32 * wm + 16 * i + 4 * (lane / 16) + v;
        const int p = spair[row];
        if (p >= a.P) continue;
        float g = accg[i][j][v], u = accu[i][j][v];
        if (Q) { g *= sg; u *= su; }
        const float gg = round_bf16(g), uu = round_bf16(u);
        a.a_buf[static_cast<int64_t>(p) * I + col] = f32_to_bf16(round_bf16(silu(gg)) * uu);
      }
  }
}

// ----------------------------------------------------------------------------------------------- down

template <bool Q>
__global__ __launch_bounds__(kThreads) void prefill_down_kernel(PrefillArgs a) {
  constexpr int ES = Q ? 1 : 2;
  const int blk = blockIdx.x;
  const int e = a.bexp[blk];
  if (e < 0) return;
  __shared__ uint16_t sa[kBM][kLdsK];
  __shared__ uint16_t sb[128][kLdsK];
  __shared__ int spair[kBM];
  const int64_t n0 = static_cast<int64_t>(blockIdx.y) * 128;
  if (threadIdx.x < kBM) spair[threadIdx.x] = a.sorted_ids[static_cast<int64_t>(blk) * kBM + threadIdx.x];
  __syncthreads();
  const char* wbase = static_cast<const char*>(a.w_d) + static_cast<int64_t>(e) * a.d_se * ES;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int wm = wave / 2, wn = wave % 2;  // wave tile: 32 rows x 64 cols
  floatx4 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int64_t H = a.H, I = a.I;
  for (int64_t k0 = 0; k0 < I; k0 += kBK) {
    stage_a(sa, I, k0, [&](int r) -> const uint16_t* {
      const int p = spair[r];
      return p < a.P ? a.a_buf + static_cast<int64_t>(p) * I : nullptr;
    });
    stage_w<Q, 128>(sb, wbase, a.d_sn, I, k0, [&](int r) -> int64_t {
      const int64_t h = n0 + r;
      return h < H ? h : -1;
    });
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 32) {
      const int kk = ks + 8 * (lane / 16);
      bf16x8_t fa[2], fb[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = lds_frag(sa, 32 * wm + 16 * i + (lane % 16), kk);
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = lds_frag(sb, 64 * wn + 16 * j + (lane % 16), kk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t h = n0 + 64 * wn + 16 * j + (lane % 16);
    if (h >= H) continue;
    float sc = 1.f;
    if (Q) sc = load_scale(a.s_d, a.s_dtype, static_cast<int64_t>(e) * a.sd_se + h);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 32 * wm + 16 * i + 4 * (lane / 16) + v;
        const int p = spair[row];
        if (p >= a.P) continue;
        float val = acc[i][j][v];
        if (Q) val *= sc;
        a.o_buf[static_cast<int64_t>(p) * H + h] = round_bf16(val) * a.wts[p];
      }
  }
}

// -------------------------------------------------------------------------------------------- combine

__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillArgs a) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(a.n_tokens) * a.H;
  if (idx >= total) return;
  const int64_t t = idx / a.H, h = idx % a.H;
  const float* o = a.o_buf + t * a.nk * a.H + h;
  float acc = 0.f;
  for (int k = 0; k < a.nk; ++k) {
    const int64_t id = load_id(a.ids, a.ids_dtype, t * a.nk + k);
    if (id >= 0 && id < a.E1) acc += o[static_cast<int64_t>(k) * a.H];  // dropped pairs have no row
  }
  float out = round_bf16(acc);
  if (a.res) out += bf16_to_f32(a.res[t * a.res_rs + h]);
  a.y[t * a.ys + h] = f32_to_bf16(out);
}

}  // namespace

namespace mm {
int check_experts(const char* who, const mm_experts* ex);
}

extern "C" int mm_moe_prefill(const void* x, int64_t n_tokens, int64_t x_row_stride, const mm_experts* ex, int64_t nk,
                              const void* ids, int ids_dtype, const float* wts, const int32_t* sorted_ids, const int32_t* bexp, int64_t nb,
                              int32_t block_m, const void* residual, int64_t res_row_stride, void* a_buf, float* o_buf,
                              void* y, int64_t y_row_stride, int phases, void* stream) {
  int rc = mm::check_experts("moe_prefill", ex);
  if (rc) return rc;
  MM_REQUIRE(block_m == kBM, "moe_prefill: block_m must be %d (got %d)", kBM, block_m);
  MM_REQUIRE(n_tokens >= 0 && nk >= 1 && n_tokens * nk <= (1LL << 30), "moe_prefill: bad token/slot counts");
  MM_REQUIRE(nb >= 0 && nb <= 0x7fffffffLL / kBM, "moe_prefill: bad block count");
  if (n_tokens == 0) return MM_OK;
  MM_REQUIRE(ids_dtype == MM_INT32 || ids_dtype == MM_INT64, "moe_prefill: ids must be int32 or int64");
  MM_REQUIRE(x && ids && wts && sorted_ids && bexp && a_buf && o_buf && y, "moe_prefill: null pointer");
  MM_REQUIRE(x_row_stride >= ex->hidden && y_row_stride >= ex->hidden, "moe_prefill: row stride smaller than hidden");
  MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0, "moe_prefill: x rows must be 16-byte aligned");
  MM_REQUIRE(mm::aligned16(a_buf), "moe_prefill: a_buf must be 16-byte aligned");
  MM_REQUIRE(!residual || res_row_stride >= ex->hidden, "moe_prefill: residual row stride smaller than hidden");
  PrefillArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.xs = x_row_stride;
  a.n_tokens = static_cast<int>(n_tokens);
  a.nk = static_cast<int>(nk);
  a.P = static_cast<int>(n_tokens * nk);
  a.E1 = static_cast<int>(ex->n_slots);
  a.ids = ids;
  a.ids_dtype = ids_dtype;
  a.wts = wts;
  a.sorted_ids = sorted_ids;
  a.bexp = bexp;
  a.nb = static_cast<int>(nb);
  a.w_gu = ex->w_gu;
  a.w_d = ex->w_d;
  a.s_gu = ex->s_gu;
  a.s_d = ex->s_d;
  a.s_dtype = ex->s_dtype;
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
  a.o_buf = o_buf;
  a.y = static_cast<uint16_t*>(y);
  a.ys = y_row_stride;
  hipStream_t st = MM_STREAM(stream);
  const bool q = ex->w_dtype == MM_INT8;
  if (phases == MM_PHASE_ALL) phases = MM_PHASE_GATE_UP | MM_PHASE_DOWN | MM_PHASE_COMBINE;
  if (nb > 0 && (phases & MM_PHASE_GATE_UP)) {
    dim3 g1(static_cast<unsigned>(nb), static_cast<unsigned>((a.I + 63) / 64));
    if (q) hipLaunchKernelGGL(prefill_gate_up_kernel<true>, g1, dim3(kThreads), 0, st, a);
    else hipLaunchKernelGGL(prefill_gate_up_kernel<false>, g1, dim3(kThreads), 0, st, a);
    rc = mm::check_launch("moe_prefill gate_up");
    if (rc) return rc;
  }
  if (nb > 0 && (phases & MM_PHASE_DOWN)) {
    dim3 g2(static_cast<unsigned>(nb), static_cast<unsigned>((a.H + 127) / 128));
    if (q) hipLaunchKernelGGL(prefill_down_kernel<true>, g2, dim3(kThreads), 0, st, a);
    else hipLaunchKernelGGL(prefill_down_kernel<false>, g2, dim3(kThreads), 0, st, a);
    rc = mm::check_launch("moe_prefill down");
    if (rc) return rc;
  }
  if (!(phases & MM_PHASE_COMBINE)) return MM_OK;
  const int64_t total = n_tokens * a.H;
  hipLaunchKernelGGL(prefill_combine_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, st, a);
  return mm::check_launch("moe_prefill combine");
}
