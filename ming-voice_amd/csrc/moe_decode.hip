// Decode MoE for 1..8 tokens (fused_moe.py:13-83): expert-gathered GEMV pair, HBM-bound.
//
// Kernel A (gate/up): grid (row tiles of I, slots of the batch). The workgroup of slot u reads the slot's
// expert with one scalar load and streams its gate and up rows once with 16-byte buffer loads, dotting them
// with the token (one token: per slot; a batch: the first slot of each distinct expert takes every token
// routed there, staged in LDS).
//   a[p, r] = bf16(bf16(silu(bf16(g))) * bf16(u)),  g/u = x_t . row (* row scale for int8)
// Kernel B (down + combine): grid (row tiles of H). Each wave streams the tile's down rows of one slot's
// expert, dots them with a[p] of the pairs routed there, rounds to bf16 (after the row scale for int8)
// and parks the result in LDS; the workgroup then sums over slots in order per token:
//   y[t, h] = bf16(sum_k wts[t,k] * part[t*nk+k, h]) (+ residual, rounded again)
// Both kernels keep each lane's loads back to back: buffer loads return zero past a row's end (no branch
// or mask per load), the combine's operands are fetched at kernel start without a wait, and the one-token
// instances fit 64 VGPRs, so a whole grid is resident at once (8 waves per SIMD).
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
  // one token with the selection fused into the gate/up kernel (sel_logits non-null): the router's logits, the
  // selection parameters, and the ids / weights buffers it writes (the same ones `ids` / `wts` point at)
  const float* sel_logits;
  SelectParams sp;
  void* ids_w;
  float* wts_w;
};

// ------------------------------------------------------------------------------------------- pairs
//
// Slot u = t * nk + k is pair u of the batch. With one token every slot is computed on its own (a
// repeated expert is streamed once per slot: exact, and free of any cross-lane bookkeeping before the
// weight loads). With several tokens a slot is handled only when it is the first of its expert, together
// with every later pair routed there, so each distinct expert is streamed once.

// Slot u's expert, read at a wave-uniform address (a scalar load), or -1 for an id outside [0, E1).
__device__ __forceinline__ int slot_expert(const DecodeArgs& a, int u) {
  const int t = u / a.nk, k = u - t * a.nk;
  const int64_t id = load_id(a.ids, a.ids_dtype, t * a.ids_rs + k);
  return (id < 0 || id >= a.E1) ? -1 : static_cast<int>(id);
}

// Lane p < P holds pair p's expert; other lanes hold -1.
__device__ __forceinline__ int lane_pair_expert(const DecodeArgs& a) {
  const int lane = lane_id();
  return lane < a.P ? slot_expert(a, lane) : -1;
}

// 16-byte chunk c of a weight row holds CE elements; the matching activation chunk is CE bf16 values.
template <bool Q>
struct Act {
  uint4 v[Q ? 2 : 1];
};

// Activation chunk c (CE bf16 values) of the row starting at byte `row` of resource r; kPast when !ok.
template <bool Q>
__device__ __forceinline__ void buf_act(Act<Q>& o, rsrc_t r, uint32_t row, int64_t c, bool ok) {
  const uint32_t off = ok ? row + static_cast<uint32_t>(c) * (Q ? 32u : 16u) : kPast;
  o.v[0] = buf16(r, off);
  if (Q) o.v[Q ? 1 : 0] = buf16(r, off + 16u);
}

template <bool Q>
__device__ __forceinline__ float dot_chunk(const uint4& w, const Act<Q>& x, float acc) {
  if constexpr (Q) return dot16_i8_bf16(w, x.v[0], x.v[Q ? 1 : 0], acc);
  else return dot8_bf16(w, x.v[0], acc);
}

// Makes the compiler treat the int8 weight chunks as changed, so that their widening to float is redone
// next to each dot instead of hoisted out of a loop over the pairs of one expert: hoisted, the 16 widened
// floats per chunk stay live across the loop (122 instead of 63 VGPRs for the multi-token down kernel),
// which halves the waves a SIMD holds (down at 2 / 4 / 8 int8 tokens: 11.6 / 18.2 / 28.3 -> 9.2 / 15.5 /
// 25.3 us). Widening again costs a few VALU operations per byte.
template <int N>
__device__ __forceinline__ void keep_raw(uint4 (&w)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("" : "+v"(w[j].x), "+v"(w[j].y), "+v"(w[j].z), "+v"(w[j].w));
}

// ------------------------------------------------------------------------------------------- kernel A

// Epilogue of one gate/up row pair for one pair p: scales (int8, fetched with the weights), bf16 rounding
// points, SiLU, product.
template <bool Q>
__device__ __forceinline__ void gate_up_store(const DecodeArgs& a, int64_t r, int p, float ag, float au, float sg,
                                              float su) {
  if (Q) {
    ag *= sg;
    au *= su;
  }
  const float gg = round_bf16(ag), uu = round_bf16(au);
  const float act = round_bf16(silu(gg));
  a.a_buf[static_cast<int64_t>(p) * a.I + r] = f32_to_bf16(act * uu);
}

// The int8 row scales of gate row r and up row r + I of expert e (1 for bf16 weights), loaded without a branch on the
// scale type (scale_row), so nothing waits for them before the epilogue uses them.
template <bool Q>
__device__ __forceinline__ void gate_up_scales(const DecodeArgs& a, int e, int64_t r, bool rok, float& sg, float& su) {
  sg = su = 1.f;
  if (Q) {
    const ScaleRow sr = scale_row(a.s_gu, a.s_dtype, static_cast<int64_t>(e) * a.sgu_se, 2 * a.I);
    const uint32_t i = static_cast<uint32_t>(rok ? r : 0);
    sg = scale_at(sr, i);
    su = scale_at(sr, i + static_cast<uint32_t>(a.I));
  }
}

// One token for one expert: the token's activation chunks stay in registers for all rows of the wave.
template <bool Q, int LPR, int NC, int R>
__device__ __forceinline__ void gate_up_one(const DecodeArgs& a, int e, int p, const char* wbase, int64_t row0) {
  constexpr int ES = Q ? 1 : 2;
  constexpr int GPW = kWave / LPR;
  const int lane = lane_id();
  const int g = lane / LPR, s = lane % LPR;
  const int64_t nch = a.H * ES / 16;
  const int tok = p / a.nk;
  float accg[R], accu[R], sg[R], su[R];
#pragma unroll
  for (int i = 0; i < R; ++i) accg[i] = accu[i] = 0.f;
  const uint32_t rowb = static_cast<uint32_t>(a.gu_sn * ES);
  const rsrc_t wr = make_rsrc(wbase, 2 * a.I * a.gu_sn * ES);
  const rsrc_t xr = make_rsrc(a.x, static_cast<int64_t>(a.n_tokens) * a.xs * 2);
  const uint32_t xrow = static_cast<uint32_t>(tok * a.xs * 2);
  for (int64_t c0 = 0; c0 < nch; c0 += static_cast<int64_t>(LPR) * NC) {  // one pass unless H is long
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t r = row0 + static_cast<int64_t>(GPW) * i + g;
      const bool rok = r < a.I;
      const uint32_t goff = static_cast<uint32_t>(r) * rowb, uoff = static_cast<uint32_t>(r + a.I) * rowb;
      uint4 wg[NC], wu[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
        const bool ok = rok && c < nch;
        wg[j] = buf16(wr, ok ? goff + static_cast<uint32_t>(c) * 16u : kPast);
        wu[j] = buf16(wr, ok ? uoff + static_cast<uint32_t>(c) * 16u : kPast);
      }
      Act<Q> xa[NC];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
        buf_act<Q>(xa[j], xr, xrow, c, c < nch);
      }
      if (c0 == 0) gate_up_scales<Q>(a, e, r, rok, sg[i], su[i]);  // issued behind the weights
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
    if (s == 0 && r < a.I) gate_up_store<Q>(a, r, p, ag, au, sg[i], su[i]);
  }
}

// Several tokens per expert: their activation rows are staged in LDS (bf16), each padded with zeros to the LPR * NC
// chunks that the lanes of a row cover, so the reads need no mask (a chunk past the row's end adds 0 * 0 products, as
// the masked reads of the one-token kernel do). The staging issues all of a thread's loads before its stores (one
// trip to memory; issued one by one behind their range tests, the loads had waited for each other). Each weight row
// pair is loaded once into registers and dotted with every staged row in turn. int8 chunks are widened once per row
// pair to packed bf16 (exact) and dotted with v_dot2_f32_bf16: two products per operation and 8 VGPRs per chunk,
// where widening to fp32 per token or once and keeping the floats (16 VGPRs per chunk, 111 VGPRs at 8 tokens) took
// longer; the next row pair's int8 weights are requested into the raw registers once these are widened, so they
// stream during this pair's dots. The gate and up sums of G tokens are reduced over the row's lanes together
// (group_sums: group_sum's totals, bit for bit) and the lanes then run the epilogue of one token each, where a sum
// and an epilogue per token and row were three quarters of the wave's instructions.
// Needs the row in one pass (nch <= LPR * NC); the caller takes gate_up_one per token otherwise.
template <bool Q, int LPR, int NC>
constexpr int staged_row_elems() {
  return LPR * NC * (Q ? 16 : 8);  // bf16 activations per staged row
}

// Tokens per group: 2 measured best (int8 gate/up over 28 cold layers at 2 / 4 / 8 tokens 17.4 / 30.5 / 45.8 us,
// against 17.4 / 30.8 / 46.9 with 4 and 17.4 / 30.7 / 49.3 with 8).
#ifndef MM_GU_MANY_G
#define MM_GU_MANY_G 2
#endif

// The R row pairs of one wave for the cntp staged tokens, G tokens at a time: the 2 G sums of a group are reduced
// together and stored by one lane each.
template <bool Q, int LPR, int NC, int R, int G>
__device__ __forceinline__ void gate_up_many_rows(const DecodeArgs& a, int e, int cntp, const int* spid,
                                                  const uint16_t* xs, rsrc_t wr, uint32_t rowb, int64_t row0,
                                                  uint4 (&wg)[NC], uint4 (&wu)[NC]) {
  constexpr int GPW = kWave / LPR;
  constexpr int ROW = staged_row_elems<Q, LPR, NC>();
  constexpr int LOGN = G == 1 ? 1 : G == 2 ? 2 : G == 4 ? 3 : 4;  // log2 of the 2 G sums of a group
  static_assert(2 * G <= LPR && (G & (G - 1)) == 0 && G <= 8, "token group");
  const int lane = lane_id();
  const int g = lane / LPR, s = lane % LPR;
  const int64_t nch = a.H * (Q ? 1 : 2) / 16;
  auto load_w = [&](int64_t r) {
    const bool rok = r < a.I;
    const uint32_t goff = static_cast<uint32_t>(r) * rowb, uoff = static_cast<uint32_t>(r + a.I) * rowb;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t c = s + static_cast<int64_t>(LPR) * j;
      const bool ok = rok && c < nch;
      wg[j] = buf16(wr, ok ? goff + static_cast<uint32_t>(c) * 16u : kPast);
      wu[j] = buf16(wr, ok ? uoff + static_cast<uint32_t>(c) * 16u : kPast);
    }
  };
  // after group_sums a lane holds the gate total of the group's token vi < G (its up total, value G + vi, is at
  // lane ^ 1) or an up total; the G gate lanes among the first 2 G of the row store
  const int vi = sums_index<LPR, 2 * G>(lane);
  const bool storer = vi < G && (s >> LOGN) == 0;
  float sg = 1.f, su = 1.f;
  gate_up_scales<Q>(a, e, row0 + g, row0 + g < a.I, sg, su);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = row0 + static_cast<int64_t>(GPW) * i + g;
    const bool rok = r < a.I;
    uint4 gl[NC], gh[NC], ul[NC], uh[NC];  // int8: the chunks widened to bf16 (elements 0-7, 8-15)
    float sgn = 1.f, sun = 1.f;
    if constexpr (Q) {
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        widen_i8(wg[j], gl[j], gh[j]);
        widen_i8(wu[j], ul[j], uh[j]);
      }
      if (i + 1 < R) {  // the next row pair streams during this one's dots
        const int64_t rn = r + GPW;
        load_w(rn);
        gate_up_scales<Q>(a, e, rn, rn < a.I, sgn, sun);
      }
    }
    // x[t]: gate sum of token t0 + t, x[G + t]: its up sum. A row past cntp (the last group) holds stale values:
    // its sums stay in their own lanes through group_sums and are not stored.
    for (int t0 = 0; t0 < cntp; t0 += G) {
      float x[2 * G];
#pragma unroll
      for (int t = 0; t < G; ++t) {
        const uint4* row = reinterpret_cast<const uint4*>(xs + (t0 + t) * ROW);
        float ag = 0.f, au = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          const int c = s + LPR * j;
          if constexpr (Q) {
            const uint4 x0 = row[2 * c], x1 = row[2 * c + 1];
            ag = dot8_bf16(gh[j], x1, dot8_bf16(gl[j], x0, ag));
            au = dot8_bf16(uh[j], x1, dot8_bf16(ul[j], x0, au));
          } else {
            const uint4 x0 = row[c];
            ag = dot8_bf16(wg[j], x0, ag);
            au = dot8_bf16(wu[j], x0, au);
          }
        }
        x[t] = ag;
        x[G + t] = au;
      }
      group_sums<LPR, 2 * G>(x);
      const float up = dpp_f32<kDppXor1>(x[0]);
      if (storer && t0 + vi < cntp && rok) gate_up_store<Q>(a, r, spid[t0 + vi], x[0], up, sg, su);
    }
    if constexpr (Q) {
      sg = sgn;
      su = sun;
    } else if (i + 1 < R) {
      const int64_t rn = r + GPW;
      load_w(rn);
      gate_up_scales<Q>(a, e, rn, rn < a.I, sg, su);
    }
  }
}

template <bool Q, int LPR, int NC, int R, int MAXT>
__device__ __forceinline__ void gate_up_many(const DecodeArgs& a, int e, int cntp, const int* spid, const char* wbase,
                                             int64_t row0, uint16_t* xs) {
  constexpr int ES = Q ? 1 : 2;
  constexpr int GPW = kWave / LPR;
  constexpr int ROW = staged_row_elems<Q, LPR, NC>();
  const int lane = lane_id();
  const int g = lane / LPR, s = lane % LPR;
  const int64_t nch = a.H * ES / 16;
  const uint32_t rowb = static_cast<uint32_t>(a.gu_sn * ES);
  const rsrc_t wr = make_rsrc(wbase, 2 * a.I * a.gu_sn * ES);
  // the first row pair's weights, in flight during the staging below
  uint4 wg[NC], wu[NC];
  {
    const int64_t r = row0 + g;
    const bool rok = r < a.I;
    const uint32_t goff = static_cast<uint32_t>(r) * rowb, uoff = static_cast<uint32_t>(r + a.I) * rowb;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t c = s + static_cast<int64_t>(LPR) * j;
      const bool ok = rok && c < nch;
      wg[j] = buf16(wr, ok ? goff + static_cast<uint32_t>(c) * 16u : kPast);
      wu[j] = buf16(wr, ok ? uoff + static_cast<uint32_t>(c) * 16u : kPast);
    }
  }
  // stage the rows of this group's tokens and their zero padding (whole workgroup; the group is uniform across it),
  // every load of a batch issued before its stores, so the staging waits for memory once (up to 8 pieces per thread
  // and batch)
  {
    const int row_chunks = static_cast<int>(a.H / 8);  // 16-byte pieces of one bf16 row
    constexpr int PAD_CHUNKS = ROW / 8;               // ... of one staged row
    const int total = cntp * PAD_CHUNKS;
    constexpr int SB = 8;
    for (int b0 = threadIdx.x; b0 < total; b0 += SB * static_cast<int>(blockDim.x)) {
      uint4 v[SB];
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const int i = b0 + j * static_cast<int>(blockDim.x);
        const int ic = i < total ? i : total - 1;  // clamped: the value is not stored past the end
        const int t = ic / PAD_CHUNKS, c = ic % PAD_CHUNKS;
        const int tok = spid[t] / a.nk;
        v[j] = reinterpret_cast<const uint4*>(a.x + static_cast<int64_t>(tok) * a.xs)[c < row_chunks ? c : 0];
        v[j] = c < row_chunks ? v[j] : make_uint4(0u, 0u, 0u, 0u);
      }
      keep_raw(v);  // all loads here, not each sunk into its store's branch
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const int i = b0 + j * static_cast<int>(blockDim.x);
        if (i < total) reinterpret_cast<uint4*>(xs)[i] = v[j];
      }
    }
  }
  __syncthreads();
  constexpr int G = MM_GU_MANY_G < MAXT ? MM_GU_MANY_G : MAXT;  // groups never reach past the MAXT staged rows
  gate_up_many_rows<Q, LPR, NC, R, G>(a, e, cntp, spid, xs, wr, rowb, row0, wg, wu);
  __syncthreads();  // the staging buffer is reused by the next group
}

constexpr int kMaxTokens = 8;

// Grid (row tiles of I, slots). ONE (one token): the workgroup computes its slot's pair. Otherwise the
// workgroup of the first slot of each distinct expert takes every pair routed there.
// SEL (one token): the experts are selected here from the router's logits instead of read from ids. Row y = 0
// of the grid is the shared expert's slot (last, no selection needed), so its workgroups are dispatched
// first and stream while the others select: each wave of a routed workgroup ranks the 64 logits itself (no
// LDS, no barrier) and takes its slot's pick; workgroup (0, 1) writes ids and weights for the down kernel.
template <bool Q, int LPR, int NC, int R, int MAXT, bool ONE, bool SEL = false>
__global__ __launch_bounds__(256) void decode_gate_up_kernel(DecodeArgs a) {
  extern __shared__ uint4 xs_raw[];  // MAXT bf16 rows of the hidden dim (MAXT > 1 only)
  __shared__ int spid[MAXT];
  int u = blockIdx.y;
  int e;
  if constexpr (SEL) {
    const int shared_slot = a.nk - 1;
    u = blockIdx.y == 0 ? shared_slot : static_cast<int>(blockIdx.y) - 1;
    if (u == shared_slot) {
      e = a.sp.E;
    } else {
      int id;
      float w;
      bool has;
      select_token64(a.sp, a.sel_logits, id, w, has);
      e = __builtin_amdgcn_readlane(id, u);
      if (blockIdx.x == 0 && blockIdx.y == 1 && threadIdx.x < kWave && has) {
        a.wts_w[lane_id()] = w;
        if (a.ids_dtype == MM_INT64) static_cast<int64_t*>(a.ids_w)[lane_id()] = id;
        else static_cast<int32_t*>(a.ids_w)[lane_id()] = id;
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the selection's registers out of the streaming code
  } else {
    e = slot_expert(a, u);
  }
  if (e < 0) return;
  constexpr int ES = Q ? 1 : 2;
  constexpr int GPW = kWave / LPR;  // row pairs per wave per step
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * (GPW * R);
  const char* wbase = static_cast<const char*>(a.w_gu) + static_cast<int64_t>(e) * a.gu_se * ES;
  if constexpr (ONE) {
    gate_up_one<Q, LPR, NC, R>(a, e, u, wbase, row0);
  } else {
    unsigned long long pairs = __ballot(lane_pair_expert(a) == e);
    if (__ffsll(static_cast<long long>(pairs)) - 1 != u) return;  // an earlier slot streams this expert
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
}

// ------------------------------------------------------------------------------------------- kernel B

constexpr int kDownWaves = 8;
// Largest batch whose down kernel reads each expert row again for every pair (RELOAD below), per weight type:
// int8 down over 28 cold layers at 2 / 4 / 8 tokens 11.3 / 19.2 / 33.8 us reloading, 11.8 / 18.9 / 31.2 holding the
// row; bf16 15.4 / 26.5 / 46.5 reloading, 15.2 / 25.0 / 41.3 holding it.
#ifndef MM_DOWN_RELOAD_I8
#define MM_DOWN_RELOAD_I8 4
#endif
#ifndef MM_DOWN_RELOAD_BF16
#define MM_DOWN_RELOAD_BF16 1
#endif
// Rows per lane group of the down kernel: one token (RL1), batches that reload the rows per pair (RLR) and
// batches that hold them (RLH). Two rows dot every activation chunk a lane loads twice, halving the grid's
// activation reads; over 28 cold layers, down at int8 2 / 4 tokens 11.3 / 19.3 -> 10.5 / 18.1 us, bf16 4 / 8
// tokens 25.0 / 41.3 -> 24.0 / 37.7. Holding two int8 rows takes 87 instead of 59 VGPRs (8 tokens 31.3 -> 35.4).
#ifndef MM_DOWN_RL1_I8
#define MM_DOWN_RL1_I8 2
#endif
#ifndef MM_DOWN_RLR_I8
#define MM_DOWN_RLR_I8 2
#endif
#ifndef MM_DOWN_RLH_I8
#define MM_DOWN_RLH_I8 1
#endif
#ifndef MM_DOWN_RL1_BF16
#define MM_DOWN_RL1_BF16 1
#endif
#ifndef MM_DOWN_RLH_BF16
#define MM_DOWN_RLH_BF16 2
#endif

// Grid: row tiles of H (RW = 64 / LPR * RL rows: lane group g holds rows g * RL ... g * RL + RL - 1). Wave w takes slots w, w + 8, ... (ONE: each; otherwise the
// first slot of each distinct expert, with all its pairs), streams the tile's rows of the slot's expert
// (LPR lanes per row) once, dots them with a[p] of the pairs, rounds to bf16 (after the row scale for int8)
// into LDS; the workgroup then sums over slots in order per token and adds the residual.
template <bool Q, int LPR, int NC, int RL, bool ONEPASS, bool ONE, bool RELOAD>
__global__ __launch_bounds__(kDownWaves * 64) void decode_down_kernel(DecodeArgs a) {
  static_assert(RL == 1 || ONEPASS, "several rows per lane group need one-pass rows");
  constexpr int RW = kWave / LPR * RL;  // output rows per workgroup
  constexpr int CE = Q ? 16 : 8;   // weights per 16-byte chunk
  __shared__ float part[kMaxPairs][RW];
  __shared__ float swts[kMaxPairs];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane / LPR, s = lane % LPR;
  const int h = static_cast<int>(blockIdx.x) * RW + g * RL;  // the lane group's first row (of RL)
  const bool hok = h < a.H;
  const int64_t nch = a.I / CE;

  // Lane p holds pair p's expert: one load per lane for every slot the wave takes (read back by readlane), issued
  // first so that waiting for it does not wait for the loads below. One bf16 token (SCALAR_ID): each slot's expert
  // by a scalar load, as no scale load needs the barrier below (which turns these into vector loads: a scalar load
  // is used only where no store can reach it, and the barrier counts as one).
  constexpr bool SCALAR_ID = ONE && !Q;
  const int myid = SCALAR_ID ? -1 : lane_pair_expert(a);
  // The combine's operands are fetched now, into registers, so their loads overlap the weight stream: the
  // slot weight of pair tid and the residual of this thread's (token, row) output. Nothing waits here.
  const int tid = threadIdx.x;
  const int ct = tid / RW, cr = tid % RW;
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * RW + cr;
  const bool combiner = tid < a.n_tokens * RW && ch < a.H;
  // (buffer loads: no branch on a null residual or on the thread's role sits before them)
  const rsrc_t rr = make_rsrc(a.res, a.res ? (static_cast<int64_t>(a.n_tokens - 1) * a.res_rs + a.H) * 2 : 0);
  const uint16_t res_raw =
      static_cast<uint16_t>(buf2(rr, combiner ? static_cast<uint32_t>((ct * a.res_rs + ch) * 2) : kPast));
  const rsrc_t wtr = make_rsrc(a.wts, (static_cast<int64_t>(a.n_tokens - 1) * a.wts_rs + a.nk) * 4);
  const int wt_t = tid / a.nk;
  const float wt = __uint_as_float(
      buf4(wtr, tid < a.P ? static_cast<uint32_t>((wt_t * a.wts_rs + tid - wt_t * a.nk) * 4) : kPast));

  const rsrc_t ar = make_rsrc(a.a_buf, static_cast<int64_t>(a.P) * a.I * 2);
  for (int u = wave; u < a.P; u += kDownWaves) {
    const int e = SCALAR_ID ? slot_expert(a, u) : __builtin_amdgcn_readlane(myid, u);
    if (e < 0) {  // a dropped pair contributes nothing
      if (s < RL) part[u][g * RL + s] = 0.f;
      continue;
    }
    unsigned long long pairs = 1ull << u;
    if (!ONE) {
      pairs = __ballot(myid == e);
      if (__ffsll(static_cast<long long>(pairs)) - 1 != u) continue;  // an earlier slot has this expert
    }
    // the expert's down matrix as one resource; this lane group's row starts at byte wrow
    const rsrc_t wr = make_rsrc(static_cast<const char*>(a.w_d) + static_cast<int64_t>(e) * a.d_se * (Q ? 1 : 2),
                                a.H * a.d_sn * (Q ? 1 : 2));
    if constexpr (ONEPASS) {
      // the whole row in registers. RELOAD (one token, int8 batches of up to 4 tokens): loaded with each pair's
      // activations, the later pairs reading it again from cache, so that every load of a pass is in flight at
      // once. Otherwise loaded once before the loop over pairs: the wave then waits for it (and the scale) on
      // entering the loop, before the first pair's activations are requested, but reads it once (8 int8 tokens:
      // the shared expert's 8 pairs re-reading it cost 1.2 us more than the wait; at 2 / 4 tokens the reload
      // saved 0.5 / 0.3 us). Held across the loop, int8 chunks are kept raw (keep_raw) so that their widening (16
      // floats each, halving the waves per SIMD) is not hoisted out of it.
      // RL > 1: a lane group holds RL adjacent rows, each activation chunk dotted with all of them
      uint4 w[RL][NC];
      float sc[RL];
      auto load_w = [&] {
#pragma unroll
        for (int r = 0; r < RL; ++r) {
          const uint32_t wrow = static_cast<uint32_t>((h + r < a.H ? h + r : 0) * a.d_sn * (Q ? 1 : 2));
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            const int64_t c = s + static_cast<int64_t>(LPR) * j;
            w[r][j] = buf16(wr, c < nch ? wrow + static_cast<uint32_t>(c) * 16u : kPast);
          }
        }
#pragma unroll
        for (int r = 0; r < RL; ++r) sc[r] = 1.f;
        if (Q) {
          const ScaleRow sr = scale_row(a.s_d, a.s_dtype, static_cast<int64_t>(e) * a.sd_se, a.H);
#pragma unroll
          for (int r = 0; r < RL; ++r) sc[r] = scale_at(sr, static_cast<uint32_t>(h + r < a.H ? h + r : 0));
        }
      };
      if (!RELOAD) load_w();
      do {
        const int p = __ffsll(static_cast<long long>(pairs)) - 1;
        pairs &= pairs - 1ull;
        if (RELOAD) load_w();
        const uint32_t arow = static_cast<uint32_t>(p * a.I * 2);
        Act<Q> av[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          const int64_t c = s + static_cast<int64_t>(LPR) * j;
          buf_act<Q>(av[j], ar, arow, c, c < nch);
        }
        // every load above is issued before the first wait: a compiler barrier keeps the scheduler from moving the
        // activation or scale loads past the dots or into the storing lane's branch (a round trip each)
        if (!SCALAR_ID) asm volatile("" ::: "memory");
        float acc[RL];
#pragma unroll
        for (int r = 0; r < RL; ++r) acc[r] = 0.f;
        if constexpr (RL == 1) {
#pragma unroll
          for (int j = 0; j < NC; ++j) acc[0] = dot_chunk<Q>(w[0][j], av[j], acc[0]);
        } else {
#pragma unroll
          for (int j = 0; j < NC; ++j) {  // chunk by chunk: one chunk's widened activations live at a time
#pragma unroll
            for (int r = 0; r < RL; ++r) acc[r] = dot_chunk<Q>(w[r][j], av[j], acc[r]);
          }
        }
        if constexpr (RL == 1) {
          const float t = group_sum<LPR>(acc[0]);
          if (s == 0 && hok) part[p][g] = round_bf16(Q ? t * sc[0] : t);
        } else {
          // transposed sums (group_sum's totals, bit for bit): lane s < RL of the group ends with row vi's total
          group_sums<LPR, RL>(acc);
          const int vi = sums_index<LPR, RL>(lane);
          float scv = sc[0];
#pragma unroll
          for (int r = 1; r < RL; ++r) scv = vi == r ? sc[r] : scv;
          if (s < RL && h + vi < a.H) part[p][g * RL + vi] = round_bf16(Q ? acc[0] * scv : acc[0]);
        }
        if (Q && !RELOAD) {
#pragma unroll
          for (int r = 0; r < RL; ++r) keep_raw(w[r]);
        }
      } while (!ONE && pairs);
    } else {
      // long rows: passes of LPR * NC chunks per pair (weights re-read from cache for later pairs)
      const uint32_t wrow = static_cast<uint32_t>((hok ? h : 0) * a.d_sn * (Q ? 1 : 2));
      float sc = 1.f;
      if (Q) sc = scale_at(scale_row(a.s_d, a.s_dtype, static_cast<int64_t>(e) * a.sd_se, a.H), hok ? h : 0);
      while (pairs) {
        const int p = __ffsll(static_cast<long long>(pairs)) - 1;
        pairs &= pairs - 1ull;
        const uint32_t arow = static_cast<uint32_t>(p * a.I * 2);
        float acc = 0.f;
        for (int64_t c0 = 0; c0 < nch; c0 += static_cast<int64_t>(LPR) * NC) {
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            const int64_t c = c0 + s + static_cast<int64_t>(LPR) * j;
            const uint4 w = buf16(wr, c < nch ? wrow + static_cast<uint32_t>(c) * 16u : kPast);
            Act<Q> av;
            buf_act<Q>(av, ar, arow, c, c < nch);
            acc = dot_chunk<Q>(w, av, acc);
          }
        }
        acc = group_sum<LPR>(acc);
        if (s == 0 && hok) part[p][g] = round_bf16(Q ? acc * sc : acc);
      }
    }
  }
  if (tid < a.P) swts[tid] = wt;
  __syncthreads();

  // combine: one thread per (token, row), slots summed in order
  if (combiner) {
    float acc = 0.f;
    for (int k = 0; k < a.nk; ++k) acc = fmaf(swts[ct * a.nk + k], part[ct * a.nk + k][cr], acc);
    float out = round_bf16(acc);
    if (a.res) out = out + bf16_to_f32(res_raw);
    a.y[ct * a.ys + ch] = f32_to_bf16(out);
  }
}

// --------------------------------------------------------------------------------------------- launch

template <bool Q, int LPR, int NC, int R, int MAXT>
int launch_a(const DecodeArgs& a, hipStream_t st) {
  constexpr int rows_per_wg = 4 * (kWave / LPR) * R;
  dim3 grid(static_cast<unsigned>((a.I + rows_per_wg - 1) / rows_per_wg), static_cast<unsigned>(a.P));
  const size_t lds = MAXT > 1 ? static_cast<size_t>(MAXT) * staged_row_elems<Q, LPR, NC>() * 2 : 0;
  if (a.n_tokens == 1 && a.sel_logits)
    hipLaunchKernelGGL((decode_gate_up_kernel<Q, LPR, NC, R, MAXT, true, true>), grid, dim3(256), lds, st, a);
  else if (a.n_tokens == 1)
    hipLaunchKernelGGL((decode_gate_up_kernel<Q, LPR, NC, R, MAXT, true>), grid, dim3(256), lds, st, a);
  else
    hipLaunchKernelGGL((decode_gate_up_kernel<Q, LPR, NC, R, MAXT, false>), grid, dim3(256), lds, st, a);
  return mm::check_launch("moe_decode gate_up");
}

template <bool Q, int LPR, int NC, int RL1 = 1, int RLR = 1, int RLH = 1>
int launch_b(const DecodeArgs& a, hipStream_t st) {
  const auto grid = [&](int rw) { return dim3(static_cast<unsigned>((a.H + rw - 1) / rw)); };
  constexpr int RW = kWave / LPR;
  const bool onepass = a.I * (Q ? 1 : 2) / 16 <= static_cast<int64_t>(LPR) * NC;
  const dim3 block(kDownWaves * 64);
  if (onepass && a.n_tokens == 1)
    hipLaunchKernelGGL((decode_down_kernel<Q, LPR, NC, RL1, true, true, true>), grid(RW * RL1), block, 0, st, a);
  else if (onepass && a.n_tokens <= (Q ? MM_DOWN_RELOAD_I8 : MM_DOWN_RELOAD_BF16))
    hipLaunchKernelGGL((decode_down_kernel<Q, LPR, NC, RLR, true, false, true>), grid(RW * RLR), block, 0, st, a);
  else if (onepass)
    hipLaunchKernelGGL((decode_down_kernel<Q, LPR, NC, RLH, true, false, false>), grid(RW * RLH), block, 0, st, a);
  else
    hipLaunchKernelGGL((decode_down_kernel<Q, LPR, NC, 1, false, false, false>), grid(RW), block, 0, st, a);
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
  while (maxt > 1 && static_cast<int64_t>(maxt) * staged_row_elems<Q, LPR, NC>() * 2 > 65536) maxt /= 2;
  constexpr int R = Q ? MM_GU_R_I8 : MM_GU_R_BF16;  // row pairs per wave, one token
  // several tokens: two row pairs per wave, except int8 batches of up to 4 tokens (one row pair, 64 VGPRs, 8 waves
  // per SIMD: 3-4 % faster at 2 and 4 tokens); at 8 tokens one row pair (also 8 waves per SIMD) took 64.2 us
  // against 53.7
  constexpr int RS = Q ? 1 : 2;
  if (maxt <= 1) return launch_a<Q, LPR, NC, R, 1>(a, st);
  if (maxt <= 2) return launch_a<Q, LPR, NC, RS, 2>(a, st);
  if (maxt <= 4) return launch_a<Q, LPR, NC, RS, 4>(a, st);
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
    if (nch > 48) return launch_b<Q, MM_DOWN_I8_LPR, MM_DOWN_I8_NC, MM_DOWN_RL1_I8, MM_DOWN_RLR_I8, MM_DOWN_RLH_I8>(a, st);
    return launch_b<Q, 8, 6>(a, st);
  } else {
    if (nch >= 128) return launch_b<Q, MM_DOWN_BF16_LPR, MM_DOWN_BF16_NC, MM_DOWN_RL1_BF16, 1, MM_DOWN_RLH_BF16>(a, st);
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
  if (ex->w_gu_slabs) {
    MM_REQUIRE(mm_gate_up_slabs_bytes(ex) > 0,
               "%s: a prefill copy of w_gu needs hidden a multiple of 64 and inter a multiple of 4 (bf16) or 8 (int8)",
               who);
    MM_REQUIRE(aligned16(ex->w_gu_slabs), "%s: the prefill copy of w_gu must be 16-byte aligned", who);
  }
  if (ex->w_d_slabs) {
    MM_REQUIRE(mm_down_slabs_bytes(ex) > 0,
               "%s: a prefill copy of w_d needs inter a multiple of 64 and hidden a multiple of 8 (bf16) or 16 (int8)",
               who);
    MM_REQUIRE(aligned16(ex->w_d_slabs), "%s: the prefill copy of w_d must be 16-byte aligned", who);
  }
  return MM_OK;
}

// The decode kernels address one expert's gate/up rows and its down rows through one buffer resource each.
int check_decode_spans(const char* who, const mm_experts* ex) {
  const int64_t es = ex->w_dtype == MM_INT8 ? 1 : 2;
  const int64_t gu = 2 * ex->inter * ex->gu_stride_n * es, d = ex->hidden * ex->d_stride_n * es;
  MM_REQUIRE(rsrc_fits(gu) && rsrc_fits(d),
             "%s: one expert's weights span %lld (gate/up) and %lld (down) bytes; each must stay below 2^31", who,
             (long long)gu, (long long)d);
  return MM_OK;
}

}  // namespace mm

extern "C" int mm_moe_decode(const void* x, int64_t n_tokens, int64_t x_row_stride, const mm_experts* ex,
                             const void* ids, int ids_dtype, int64_t nk, int64_t ids_row_stride, const float* wts,
                             int64_t wts_row_stride, const void* residual, int64_t res_row_stride, void* a_buf, void* y,
                             int64_t y_row_stride, int phases, void* stream) {
  int rc = mm::check_experts("moe_decode", ex);
  if (!rc) rc = mm::check_decode_spans("moe_decode", ex);
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
  MM_REQUIRE(mm::rsrc_fits(n_tokens * x_row_stride * 2) && mm::rsrc_fits(n_tokens * nk * ex->inter * 2),
             "moe_decode: x rows or a_buf span 2^31 bytes or more");
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
  a.sel_logits = nullptr;
  a.sp = mmd::SelectParams{nullptr, 0, 0, 1, 1, 1, 1.f, 0};
  a.ids_w = nullptr;
  a.wts_w = nullptr;
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
                 int64_t out_row_stride, void* xn_out, hipStream_t s, bool with_select = true);
}  // namespace mm

// Whole MoE block for 1..8 tokens in four launches: router logits (RMSNorm fused; the normalised rows go
// to the workspace), selection, gate/up on the normalised rows, down + combine with the raw rows as
// residual. (Selecting in the router's last-finishing workgroup instead costs more in device-wide fences
// than the launch it saves.) The ids / weights it writes are the ones the unfused chain produces.
static int block_decode(const char* who, const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w,
                        float eps, const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                        int topk_group, int top_k, float scale, const mm_experts* ex, float* logits, void* ids,
                        int ids_dtype, float* wts, void* a_buf, void* workspace, int add_residual, void* y,
                        int64_t y_row_stride, void* stream) {
  int rc = mm::check_experts(who, ex);
  if (!rc) rc = mm::check_decode_spans(who, ex);
  if (rc) return rc;
  const int64_t nk = static_cast<int64_t>(top_k) + 1;
  rc = mm::check_router_args(n_tokens, n_experts, scoring, n_group, topk_group, top_k, 1, ids, ids_dtype, wts, nk);
  if (rc) return rc;
  MM_REQUIRE(n_tokens >= 1 && n_tokens <= kMaxTokens && n_tokens * nk <= kMaxPairs,
             "%s: 1..%d tokens with (top_k + 1) * tokens <= %d", who, kMaxTokens, kMaxPairs);
  MM_REQUIRE(ex->n_slots == n_experts + 1, "%s: expert slots (%lld) must be n_experts + 1 (shared last)", who,
             (long long)ex->n_slots);
  MM_REQUIRE(x && norm_w && w32 && logits && a_buf && workspace && y, "%s: null pointer", who);
  MM_REQUIRE(x_row_stride >= ex->hidden && y_row_stride >= ex->hidden, "%s: row stride smaller than hidden", who);
  MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0 && mm::aligned16(a_buf) && mm::aligned16(workspace),
             "%s: x, a_buf and workspace must be 16-byte aligned", who);
  MM_REQUIRE(ex->hidden <= 0x7fffffff && ex->inter <= 0x7fffffff, "%s: shape too large", who);
  hipStream_t st = MM_STREAM(stream);
  const mmd::SelectParams sp{bias, static_cast<int>(n_experts), scoring, n_group, topk_group, top_k, scale, 1};
  void* xn = workspace;
  // one token, bf16 experts, at most 64 experts without groups: the gate/up kernel selects (one launch fewer;
  // 31.4 -> 29.0 us per cold layer). int8 keeps the separate selection: its selecting instance holds 105
  // VGPRs (4 waves per SIMD) and the layer ran slower (25.1 -> 28.1 us); held to 8 waves per SIMD
  // (amdgpu_waves_per_eu, 47 VGPRs, no spills) it only tied (25.12 against 25.10 us), and tied again after the
  // branch-free scale loads (23.9 against 23.4-24.2 us).
  const bool fuse_select = n_tokens == 1 && n_experts <= 64 && n_group <= 1 && ex->w_dtype == MM_BF16;
  rc = mm::router_front(x, n_tokens, ex->hidden, x_row_stride, norm_w, eps, w32, sp, logits, ids, ids_dtype, wts, nk,
                        xn, st, !fuse_select);
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
  a.sel_logits = fuse_select ? logits : nullptr;
  a.sp = sp;
  a.ids_w = ids;
  a.wts_w = wts;
  const bool q = ex->w_dtype == MM_INT8;
  rc = q ? dispatch_a<true>(a, st) : dispatch_a<false>(a, st);
  if (rc) return rc;
  return q ? dispatch_b<true>(a, st) : dispatch_b<false>(a, st);
}

extern "C" int mm_moe_block_decode(const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w, float eps,
                                   const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                                   int topk_group, int top_k, float scale, const mm_experts* ex, float* logits,
                                   void* ids, int ids_dtype, float* wts, void* a_buf, void* workspace,
                                   int add_residual, void* y, int64_t y_row_stride, void* stream) {
  return block_decode("moe_block_decode", x, n_tokens, x_row_stride, norm_w, eps, w32, n_experts, bias, scoring,
                      n_group, topk_group, top_k, scale, ex, logits, ids, ids_dtype, wts, a_buf, workspace,
                      add_residual, y, y_row_stride, stream);
}

// ------------------------------------------------------------------------------- allocation-free variant
//
// The scratch of mm_moe_block_decode (the normalised rows and the gated activations) in a file-scope device
// array instead of caller buffers. Each device holds its own copy at its own address, found once per device
// with hipGetSymbolAddress; the host never passes the array's name itself (a host-side stand-in) to a kernel.
// Every byte the kernels read from it is written earlier in the same call (the router writes all normalised
// rows, gate/up every activation row of a kept pair, and down never reads the row of a dropped pair), so
// nothing needs clearing between calls. Calls that overlap on one device share the array and race.

static __device__ __align__(256) unsigned char scratch[MM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// The current device's address of `scratch` (looked up on the first call on each device).
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mm::set_error(MM_ERR_HIP, "HIP error in hipGetDevice: %s", hipGetErrorString(e));
  MM_REQUIRE(dev >= 0 && dev < kMaxDevices, "moe_block_decode_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return mm::set_error(MM_ERR_HIP, "HIP error in hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MM_OK;
}

}  // namespace

extern "C" int64_t mm_moe_block_decode_noalloc_bytes(int64_t n_tokens, int64_t top_k, int64_t hidden, int64_t inter) {
  if (n_tokens < 1 || top_k < 0 || hidden < 1 || inter < 1 || n_tokens > kMaxTokens || hidden > (1 << 20) ||
      inter > (1 << 20))
    return -1;
  const int64_t xn = (n_tokens * hidden * 2 + 255) / 256 * 256;
  return xn + n_tokens * (top_k + 1) * inter * 2;
}

extern "C" int mm_moe_block_decode_noalloc(const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w,
                                           float eps, const float* w32, int64_t n_experts, const float* bias,
                                           int scoring, int n_group, int topk_group, int top_k, float scale,
                                           const mm_experts* ex, float* logits, void* ids, int ids_dtype, float* wts,
                                           int add_residual, void* y, int64_t y_row_stride, void* stream) {
  MM_REQUIRE(ex, "moe_block_decode_noalloc: null expert descriptor");
  const int64_t need = mm_moe_block_decode_noalloc_bytes(n_tokens, top_k, ex->hidden, ex->inter);
  MM_REQUIRE(need > 0, "moe_block_decode_noalloc: bad shape (%lld tokens, top_k %d, hidden %lld, inter %lld)",
             (long long)n_tokens, top_k, (long long)ex->hidden, (long long)ex->inter);
  MM_REQUIRE(need <= MM_NOALLOC_SCRATCH_BYTES,
             "moe_block_decode_noalloc: %lld tokens x %d slots at hidden %lld / inter %lld need %lld bytes of "
             "scratch, above the %d-byte maximum",
             (long long)n_tokens, top_k + 1, (long long)ex->hidden, (long long)ex->inter, (long long)need,
             MM_NOALLOC_SCRATCH_BYTES);
  void* base = nullptr;
  int rc = scratch_on_current_device(&base);
  if (rc) return rc;
  char* xn = static_cast<char*>(base);
  char* a_buf = xn + (n_tokens * ex->hidden * 2 + 255) / 256 * 256;
  return block_decode("moe_block_decode_noalloc", x, n_tokens, x_row_stride, norm_w, eps, w32, n_experts, bias,
                      scoring, n_group, topk_group, top_k, scale, ex, logits, ids, ids_dtype, wts, a_buf, xn,
                      add_residual, y, y_row_stride, stream);
}
