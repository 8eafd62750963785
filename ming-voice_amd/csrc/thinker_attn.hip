// The thinker's attention mixers for decode and short prefills on gfx950:
//
//   kda_prep_kernel / kda_recurrent_kernel
//                          Kimi delta attention, the recurrent form fla's fused_recurrent_kda computes (called at
//                          engine.py:258 and inside the model's KDA layers): per head a [K, V] fp32 state, per token
//                          q, k l2-normalised (q scaled), a per-key-channel decay exp(g) from the gate, the delta
//                          rule update and the readout. The per-token inputs are prepared for all tokens at once
//                          into a workspace; then a wave holds 4 value columns of one head's state in registers
//                          for all T tokens (the columns are independent), the sums over k go through lanes in a
//                          fixed order and the inputs through LDS 16 tokens at a time.
//   kda_short_kernel       the same recurrence for up to 2 tokens (a decode step) in one launch: a workgroup holds
//                          16 value columns, the sums over k go through lanes, then LDS.
//   short_conv_kernel      the depthwise causal convolution of ShortConvolution's step form (a cache of the last W
//                          inputs per channel), SiLU, T tokens in parallel.
//   rms_norm_gated_kernel  FusedRMSNormGated with a sigmoid gate: bf16(x * rsqrt(mean(x^2) + eps) * w * sigmoid(g)).
//   kda_token_kernel       one decode token of a KDA layer's core (the three above plus the gate's LoRA
//                          up-projections) in one launch, one workgroup per head.
//   mla_split_kernel / mla_merge_kernel
//                          single-token attention of an MLA layer over its static cache (engine.py:523-548: k, v
//                          [heads, max_len, d], rows written at the position with index_copy_): the new k, v rows
//                          are stored at pos, then softmax(scale q . K[0..pos]^T) . V[0..pos] in two passes
//                          (32-position chunks, then a merge of the chunks' softmax states), all in fp32.
#include "mm_common.h"

namespace {

using namespace mmd;

__device__ __forceinline__ float bf_lo(uint32_t x) { return __uint_as_float(x << 16); }
// v, or zero when !ok (a select per dword, no branch)
__device__ __forceinline__ uint4 and_mask16(const uint4& v, bool ok) {
  const uint32_t m = ok ? ~0u : 0u;
  return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
}
__device__ __forceinline__ float bf_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

// Orders a wave's LDS stores before its later loads (and loads before later stores) without a workgroup barrier:
// a wave's LDS instructions execute in program order, so only the compiler's reordering has to be fenced.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

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
  int use_l2norm, use_gate, beta_logits;
  float scale;
  float* state;                            // [H, K, V] fp32, updated in place
  uint16_t* o;                             // [T, H, V] bf16
  int64_t o_ts;
  int T, H, V;
  const int64_t* n_valid;                  // device scalar or null: tokens from n_valid on are padding
};

// The prompt's real tokens: the first n_valid (clamped to [0, T]) when given, else all T. A padding token leaves the
// state exactly as it is: its decay is 1 and its write strength 0 (engine.py:252-253, the padded prefill).
__device__ __forceinline__ int kda_valid(const KdaArgs& a) {
  if (!a.n_valid) return a.T;
  const int64_t n = *a.n_valid;
  return static_cast<int>(n < 0 ? 0 : n > a.T ? a.T : n);
}

__device__ __forceinline__ float ld_any(const void* p, int dt, int64_t i) {
  return dt == MM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// softplus with the usual threshold: x above 20 returns x
__device__ __forceinline__ float softplus20(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

constexpr int kKdaCols = 16;   // value columns per workgroup of kda_short_kernel and kda_token_kernel
constexpr int kKdaChunk = 16;  // tokens kda_recurrent_kernel stages in LDS at a time
constexpr int kKdaShortT = 2;  // prompts up to this long take kda_short_kernel (one launch, no workspace)
// kda_recurrent_kernel's shape: 4 state rows per lane, 4 waves per workgroup. At 16 heads of 128 x 128 that is 256
// workgroups of 4 waves, one per CU and one wave per SIMD (graph-timed over 21 states, 512 / 128 / 16 tokens:
// 114 / 36 / 11 us per call, against 146 / 44 / 13 with 8 rows per lane and one wave per workgroup, 125-133 / 38-41
// with 8 rows and 2 or 4 waves or 4 rows and 2 waves).
constexpr int kKdaRpl = 4, kKdaNwb = 4;

// Prompts of up to kKdaShortT tokens (a decode step) in one launch, without the workspace: grid (V / 16, H) x 256
// threads; each value column of the recurrence is independent (u and o of column v read
// only column v of S), so a head's columns spread over V / 16 workgroups. Wave w, lane (rg = lane / 16,
// c = lane % 16) holds state rows r = 16 i + 4 w + rg (i < K / 16) of column 16 * blockIdx.x + c: one load of a
// wave reads 4 rows x 64 bytes. Per token the first K threads (whole waves) put each key channel's q, k and decay
// into LDS, once for the workgroup, with the sums of q^2 and k^2. Sums over rows: lane-internal, then over the
// 4 row groups of a wave (xor 16, then 32), then over the 4 waves through LDS, in a fixed order.
template <int K>
__global__ __launch_bounds__(256) void kda_short_kernel(KdaArgs a) {
  constexpr int CB = kKdaCols, RPT = K / 16;
  static_assert(K % kWave == 0 && K <= 256, "kda key dim");
  __shared__ float s_q[K], s_k[K], s_dec[K];
  __shared__ float s_red[K / kWave][2];
  __shared__ float part_u[4][CB], part_o[4][CB];
  const int h = blockIdx.y;
  const int tid = threadIdx.x, w = tid / kWave, lane = lane_id();
  const int c = lane % CB, rg = lane / CB;
  const int64_t V = a.V;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * CB + c;
  float* st = a.state + static_cast<int64_t>(h) * K * V + col;
  float S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = st[static_cast<int64_t>(16 * i + 4 * w + rg) * V];
  const bool chan = tid < K;  // whole waves
  float nA = 0.f, dtb = 0.f;
  if (a.use_gate) {
    nA = __expf(a.A_log[h]);
    if (chan) dtb = a.dt_bias[static_cast<int64_t>(h) * K + tid];
  }
  const int nv = kda_valid(a);
  for (int t = 0; t < a.T; ++t) {
    if (chan) {
      const int64_t i = static_cast<int64_t>(h) * K + tid;
      const float qv = bf16_to_f32(a.q[t * a.q_ts + i]);
      const float kv = bf16_to_f32(a.k[t * a.k_ts + i]);
      float gl = ld_any(a.g, a.g_dtype, t * a.g_ts + i);
      if (a.use_gate) {
        const float x = gl + dtb;
        gl = isnan(a.lower_bound) ? -nA * softplus20(x) : a.lower_bound / (1.f + __expf(-nA * x));
      }
      s_q[tid] = qv;
      s_k[tid] = kv;
      s_dec[tid] = t < nv ? __expf(gl) : 1.f;
      if (a.use_l2norm) {
        const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
        if (lane == 0) {
          s_red[w][0] = sq;
          s_red[w][1] = sk;
        }
      }
    }
    const float vc = bf16_to_f32(a.v[t * a.v_ts + static_cast<int64_t>(h) * V + col]);
    float beta = ld_any(a.beta, a.beta_dtype, t * a.b_ts + h);
    if (a.beta_logits) beta = 1.f / (1.f + __expf(-beta));
    if (t >= nv) beta = 0.f;
    __syncthreads();
    float qs = a.scale, ks = 1.f;
    if (a.use_l2norm) {
      float sq = s_red[0][0], sk = s_red[0][1];
#pragma unroll
      for (int j = 1; j < K / kWave; ++j) {
        sq += s_red[j][0];
        sk += s_red[j][1];
      }
      qs = a.scale / sqrtf(sq + 1e-6f);
      ks = 1.f / sqrtf(sk + 1e-6f);
    }
    // decay, then the part of v the state already predicts from k
    float pu = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = 16 * i + 4 * w + rg;
      S[i] *= s_dec[r];
      pu = fmaf(s_k[r] * ks, S[i], pu);
    }
    pu += __shfl_xor(pu, 16, kWave);
    pu += __shfl_xor(pu, 32, kWave);
    if (rg == 0) part_u[w][c] = pu;
    __syncthreads();
    const float u = (vc - (((part_u[0][c] + part_u[1][c]) + part_u[2][c]) + part_u[3][c])) * beta;
    float po = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = 16 * i + 4 * w + rg;
      S[i] = fmaf(s_k[r] * ks, u, S[i]);
      po = fmaf(s_q[r] * qs, S[i], po);
    }
    po += __shfl_xor(po, 16, kWave);
    po += __shfl_xor(po, 32, kWave);
    if (rg == 0) part_o[w][c] = po;
    // the next token rewrites s_* after this barrier, when every thread has read them; part_u / part_o are
    // rewritten after the next token's first and second barriers, when wave 0 has read them
    __syncthreads();
    if (w == 0 && rg == 0) {
      const float o = ((part_o[0][c] + part_o[1][c]) + part_o[2][c]) + part_o[3][c];
      a.o[t * a.o_ts + static_cast<int64_t>(h) * V + col] = f32_to_bf16(o);
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) st[static_cast<int64_t>(16 * i + 4 * w + rg) * V] = S[i];
}

// The per-token inputs of the recurrence, prepared for all T tokens in parallel (kda_prep_kernel) into a
// workspace row per (token, head) of 3 K + 4 floats: q l2-normalised times the scale, k l2-normalised, the
// per-channel decay exp(gate(g)), then beta (the sigmoid applied when it comes as logits), q . k of the
// normalised vectors, and 2 zeros.
template <int K>
constexpr int kda_ws_row() { return 3 * K + 4; }

// The prepared inputs of token t, head h for the lane's channels lane + 64 j (one wave): q l2-normalised times the
// scale, k l2-normalised, the decay exp(gate(g)) (1 for a padding token), and, the same in every lane, beta (the
// sigmoid applied when it comes as logits; 0 for padding) and q . k of the normalised vectors.
template <int K>
__device__ __forceinline__ void kda_prep_token(const KdaArgs& a, int64_t t, int h, bool pad, float (&qn)[K / kWave],
                                               float (&kn)[K / kWave], float (&dv)[K / kWave], float& beta,
                                               float& qk) {
  constexpr int NJ = K / kWave;
  const int lane = lane_id();
  const int64_t hk = static_cast<int64_t>(h) * K;
  float qv[NJ], kv[NJ], gv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int64_t ch = hk + lane + kWave * j;
    qv[j] = bf16_to_f32(a.q[t * a.q_ts + ch]);
    kv[j] = bf16_to_f32(a.k[t * a.k_ts + ch]);
    gv[j] = ld_any(a.g, a.g_dtype, t * a.g_ts + ch);
  }
  float b = ld_any(a.beta, a.beta_dtype, t * a.b_ts + h);
  float qs = a.scale, ks = 1.f;
  if (a.use_l2norm) {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      sq = fmaf(qv[j], qv[j], sq);
      sk = fmaf(kv[j], kv[j], sk);
    }
    qs = a.scale / sqrtf(wave_sum(sq) + 1e-6f);
    ks = 1.f / sqrtf(wave_sum(sk) + 1e-6f);
  }
  const float nA = a.use_gate ? __expf(a.A_log[h]) : 0.f;
  float d = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    float gl = gv[j];
    if (a.use_gate) {
      const float x = gl + a.dt_bias[hk + lane + kWave * j];
      gl = isnan(a.lower_bound) ? -nA * softplus20(x) : a.lower_bound / (1.f + __expf(-nA * x));
    }
    qn[j] = qv[j] * qs;
    kn[j] = kv[j] * ks;
    dv[j] = pad ? 1.f : __expf(gl);
    d = fmaf(qn[j], kn[j], d);
  }
  qk = wave_sum(d);
  if (a.beta_logits) b = 1.f / (1.f + __expf(-b));
  beta = pad ? 0.f : b;
}

// Grid (T H / 4) x 4 waves: wave w prepares row (t, h) = divmod(4 blockIdx.x + w, H), lane i channels i + 64 j.
template <int K>
__global__ __launch_bounds__(256) void kda_prep_kernel(KdaArgs a, float* __restrict__ ws) {
  constexpr int NJ = K / kWave, ROW = kda_ws_row<K>();
  const int lane = lane_id();
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (idx >= static_cast<int64_t>(a.T) * a.H) return;  // whole waves
  const int64_t t = idx / a.H;
  const int h = static_cast<int>(idx % a.H);
  float qn[NJ], kn[NJ], dv[NJ], beta, qk;
  kda_prep_token<K>(a, t, h, t >= kda_valid(a), qn, kn, dv, beta, qk);
  float* row = ws + idx * ROW;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + kWave * j;
    row[c] = qn[j];
    row[K + c] = kn[j];
    row[2 * K + c] = dv[j];
  }
  if (lane < 4) row[3 * K + lane] = lane == 0 ? beta : lane == 1 ? qk : 0.f;
}

// NWB waves per (NWB CPW value columns, head): grid (V / (NWB CPW), H) x 64 NWB threads, CPW = 64 / RG with
// RG = K / RPL row groups. Each value column of the recurrence is independent (u and o of column v read only column
// v of S), so lane (c = lane / RG, rg = lane % RG) holds the RPL state rows rg RPL .. rg RPL + RPL - 1 of one
// column in registers for the whole prompt, and the sums over k are lane-internal, then over the RG lanes of a
// column (DPP steps, and one swizzle across rows of 16 lanes when RG = 32). The prepared rows of the head come into
// LDS 16 tokens at a time by global_load_lds, shared by the workgroup's waves and two chunk buffers deep (the
// next chunk loads while the recurrence runs on this one; one barrier per chunk), and each token's inputs of a lane
// are read from LDS within the chunk's unrolled token steps.
// Per token the two sums over k, k . S and q . S of the decayed state, are independent (pairwise within the
// lane, then their cross-lane steps interleaved), since o = S'^T q with S' = S + k u^T is q . S + u (q . k), q . k
// from the workspace: the token's latency is one chain of sums, not two.
template <int K, int RPL, int NWB>
__global__ __launch_bounds__(64 * NWB) void kda_recurrent_kernel(KdaArgs a, const float* __restrict__ ws) {
  constexpr int RG = K / RPL, CPW = kWave / RG, COLS = NWB * CPW, ROW = kda_ws_row<K>();
  constexpr int NT = NWB * kWave;
  constexpr int CHUNK_UNITS = kKdaChunk * ROW / 4;  // 16-byte pieces of a chunk
  constexpr int NU = (CHUNK_UNITS + NT - 1) / NT;
  constexpr int ROW_UNITS = ROW / 4;
  constexpr int VPT = (kKdaChunk * COLS + NT - 1) / NT;  // v values per thread per chunk
  static_assert(K == 64 || K == 128, "kda key dim");
  static_assert(RPL % 4 == 0 && RG <= kWave && (RG & (RG - 1)) == 0, "rows per lane");
  static_assert(ROW % 4 == 0, "16-byte workspace rows");
  // two chunk buffers (and v buffers: a wave writes the next chunk's values while the workgroup's other waves may
  // still read this chunk's), as separate arrays so that the compiler can tell a chunk's LDS reads from the next
  // chunk's loads in flight into the other buffer, and need not wait for those loads before the reads
  __shared__ __align__(16) float s_in0[kKdaChunk * ROW], s_in1[kKdaChunk * ROW];
  __shared__ float s_v0[kKdaChunk][COLS], s_v1[kKdaChunk][COLS];
  const int h = blockIdx.y, tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int c = lane / RG, rg = lane % RG;
  const int64_t V = a.V;
  const int64_t col0 = static_cast<int64_t>(blockIdx.x) * COLS;
  const int cw = wave * CPW + c;  // the lane's column within the workgroup
  float* st = a.state + static_cast<int64_t>(h) * K * V + col0 + cw;
  float S[RPL];
#pragma unroll
  for (int i = 0; i < RPL; ++i) S[i] = st[static_cast<int64_t>(RPL * rg + i) * V];
  const float* wsh = ws + static_cast<int64_t>(h) * ROW;
  const int64_t ts = static_cast<int64_t>(a.H) * ROW;  // workspace token stride
  uint16_t rv[VPT];  // raw bf16: converted once the chunk's loads are waited for, so the load needs no wait here
  auto issue = [&](int c0, float* dst) {
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const int u = tid + NT * j, tt = u / ROW_UNITS;
      if (u < CHUNK_UNITS && c0 + tt < a.T)
        load_lds16(wsh + (c0 + tt) * ts + (u % ROW_UNITS) * 4,
                   reinterpret_cast<char*>(dst) + (wave * kWave + NT * j) * 16);
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {  // no branch: rows past the prompt (never read) load its last token's row
      const int i = tid + NT * j, tt = min(c0 + i / COLS, a.T - 1);
      rv[j] = a.v[tt * a.v_ts + static_cast<int64_t>(h) * V + col0 + i % COLS];
    }
  };
  // one chunk from buffers (in, vb) while the next one loads into (in_next); called with the arrays themselves
  auto chunk = [&](int c0, const float* in, float (*vb)[COLS], float* in_next) {
    wait_vmcnt<0>();  // this wave's loads of the chunk (and the stores before them)
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int i = tid + NT * j;
      if (i < kKdaChunk * COLS) vb[i / COLS][i % COLS] = bf16_to_f32(rv[j]);
    }
    // every wave's loads of this chunk are in LDS, and every wave is done with the other buffer
    if constexpr (NWB == 1) wave_lds_fence(); else __syncthreads();
    if (c0 + kKdaChunk < a.T) issue(c0 + kKdaChunk, in_next);  // in flight during the recurrence below
    const int n = min(kKdaChunk, a.T - c0);
    const float* base = in + RPL * rg;
    // lane (c, rg) keeps the output of tokens rg, rg + RG, ... of the chunk (every lane of a column holds each
    // token's sum) and stores them after the chunk: the token steps have no branch
    constexpr int OPL = (kKdaChunk + RG - 1) / RG;
    float keep[OPL];
#pragma unroll
    for (int j = 0; j < OPL; ++j) keep[j] = 0.f;
    auto step = [&](int t) {
      const float* r = base + t * ROW;
      float qq[RPL], kk[RPL], dd[RPL];
#pragma unroll
      for (int i = 0; i < RPL; i += 4) {
        const float4 q4 = *reinterpret_cast<const float4*>(r + i);
        const float4 k4 = *reinterpret_cast<const float4*>(r + K + i);
        const float4 d4 = *reinterpret_cast<const float4*>(r + 2 * K + i);
        qq[i] = q4.x, qq[i + 1] = q4.y, qq[i + 2] = q4.z, qq[i + 3] = q4.w;
        kk[i] = k4.x, kk[i + 1] = k4.y, kk[i + 2] = k4.z, kk[i + 3] = k4.w;
        dd[i] = d4.x, dd[i + 1] = d4.y, dd[i + 2] = d4.z, dd[i + 3] = d4.w;
      }
      const float2 bq = *reinterpret_cast<const float2*>(in + t * ROW + 3 * K);  // beta, q . k
      const float vc = vb[t][cw];
      // decay; the part of v the state already predicts from k, and q . S of the decayed state
      float pk[RPL], pq[RPL];
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        S[i] *= dd[i];
        pk[i] = kk[i] * S[i];
        pq[i] = qq[i] * S[i];
      }
#pragma unroll
      for (int w = 1; w < RPL; w *= 2)  // pairwise: (0 + 1) + (2 + 3), ...
#pragma unroll
        for (int i = 0; i < RPL; i += 2 * w) {
          pk[i] += pk[i + w];
          pq[i] += pq[i + w];
        }
      const float pu = group_sum<RG>(pk[0]);
      const float qs = group_sum<RG>(pq[0]);
      const float u = (vc - pu) * bq.x;
      const float po = fmaf(u, bq.y, qs);
#pragma unroll
      for (int i = 0; i < RPL; ++i) S[i] = fmaf(kk[i], u, S[i]);
#pragma unroll
      for (int j = 0; j < OPL; ++j)
        if (t % RG == rg && t / RG == j) keep[j] = po;  // a select, no branch
    };
    if (n == kKdaChunk) {
#pragma unroll
      for (int t = 0; t < kKdaChunk; ++t) step(t);
    } else {
      for (int t = 0; t < n; ++t) step(t);
    }
#pragma unroll
    for (int j = 0; j < OPL; ++j) {
      const int t = rg + RG * j;
      if (t < n) a.o[(c0 + t) * a.o_ts + static_cast<int64_t>(h) * V + col0 + cw] = f32_to_bf16(keep[j]);
    }
    if constexpr (NWB == 1) wave_lds_fence();  // the chunk's reads before the loads two chunks on
  };
  issue(0, s_in0);
  for (int c0 = 0; c0 < a.T; c0 += 2 * kKdaChunk) {
    chunk(c0, s_in0, s_v0, s_in1);
    if (c0 + kKdaChunk < a.T) chunk(c0 + kKdaChunk, s_in1, s_v1, s_in0);
  }
#pragma unroll
  for (int i = 0; i < RPL; ++i) st[static_cast<int64_t>(RPL * rg + i) * V] = S[i];
}

// -------------------------------------------------------------------------------------- KDA, chunked form
//
// The same recurrence over a chunk of C = 16 tokens in closed form (the chunked form of fla's chunk_kda, which the
// engine selects past 192 tokens: engine.py:946-949, 964-967). With chunk-local tokens t = 0 .. C-1, S0 the state
// at the chunk start, d_t the per-channel decay of token t, P_t = d_0 ... d_t and D(j, t) = d_{j+1} ... d_t
// (per-channel products taken directly, never as ratios, so a strong decay underflows to zero instead of 0 / 0):
//   k_t . (the decayed state before token t's write) = a_t + sum_{j<t} A[t][j] u_j,
//       a_t = (k_t P_t) . S0,  A[t][j] = sum_c k_tc k_jc D(j, t)_c
//   u_t = beta_t (v_t - a_t - sum_{j<t} A[t][j] u_j)        (forward substitution, j in order)
//   o_t = q_t . S_t = b_t + sum_{j<=t} B[t][j] u_j,
//       b_t = (q_t P_t) . S0,  B[t][j] = sum_c q_tc k_jc D(j, t)_c (j < t),  B[t][t] = q_t . k_t
//   S_end = P_{C-1} S0 + sum_j (k_j D(j, C-1)) u_j^T
// Everything but S0 and v depends on the head alone, not on the value columns: kda_chunk_prep_kernel computes it
// for every (chunk, head) at once into a block of the workspace; kda_chunk_kernel then carries its value columns'
// state from chunk to chunk, and no token waits for a sum over k of the token before it. Padding tokens (past
// n_valid, or past T in the last chunk) have decay 1 and beta 0, so their u is 0 and the state passes them unchanged.

// A (chunk, head) block of the workspace, in floats: k P [C][K], q P [C][K], W = k D(., C-1) [C][K], P_{C-1} [K],
// A [C][C] with beta_t on its diagonal, B [C][C] (zero above the diagonal).
template <int K>
struct KdaBlk {
  static constexpr int C = kKdaChunk;
  static constexpr int KP = 0, QP = C * K, W = 2 * C * K, PC = 3 * C * K, A = PC + K, B = A + C * C;
  static constexpr int SIZE = B + C * C;
  static_assert(SIZE % 4 == 0, "blocks stay 16-byte aligned");
};

// 32 values over the 64 lanes of a wave: x[0] becomes the wave's total of value lane % 32 (the halves summed by
// v_permlane32_swap, then transposed over the rows and within them: 63 exchanges, against 192 for 32 separate sums).
__device__ __forceinline__ void wave_sums32(float (&x)[32]);

// Grid (chunks, H) x 16 waves. Wave w prepares token w of the chunk (kda_prep_token: q and k normalised, the decay,
// beta, q . k; a token past T gets q = k = 0, decay 1, beta 0) into LDS, then writes its rows: k P, q P and W of token
// w (the decay products over the other tokens' channels read back from LDS, taken as predicated products so that no
// register array is indexed at run time), P_{C-1} (wave C-1), and row w of A and B (entry j a wave sum over the
// channels, the 32 entries summed together by wave_sums32).
template <int K>
__global__ __launch_bounds__(64 * kKdaChunk) void kda_chunk_prep_kernel(KdaArgs a, float* __restrict__ blk) {
  using L = KdaBlk<K>;
  constexpr int C = L::C, NJ = K / kWave;
  __shared__ float s_k[C][K], s_d[C][K];
  const int ci = blockIdx.x, h = blockIdx.y;
  const int w = threadIdx.x / kWave, lane = lane_id();
  const int t0 = ci * C;
  const bool in = t0 + w < a.T;
  float qn[NJ], kn[NJ], dv[NJ], beta, qk;
  kda_prep_token<K>(a, in ? t0 + w : t0, h, t0 + w >= kda_valid(a), qn, kn, dv, beta, qk);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    qn[j] = in ? qn[j] : 0.f;
    kn[j] = in ? kn[j] : 0.f;
    dv[j] = in ? dv[j] : 1.f;
    s_k[w][lane + kWave * j] = kn[j];
    s_d[w][lane + kWave * j] = dv[j];
  }
  beta = in ? beta : 0.f;
  qk = in ? qk : 0.f;
  __syncthreads();
  // P_w = d_0 ... d_w and R_w = D(w, C-1) = d_{w+1} ... d_{C-1}; then, j running down, D(j, w) = d_{j+1} ... d_w
  float P[NJ], R[NJ], D[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) P[j] = R[j] = D[j] = 1.f;
  float x[32];  // the lane's parts of A[w][j] (x[j]) and B[w][j] (x[16 + j]), j < w
#pragma unroll
  for (int s2 = C - 1; s2 >= 0; --s2) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float ds = s_d[s2][lane + kWave * j];
      P[j] = s2 <= w ? P[j] * ds : P[j];
      R[j] = s2 > w ? R[j] * ds : R[j];
    }
  }
#pragma unroll
  for (int jj = C - 1; jj >= 0; --jj) {
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int ch = lane + kWave * j;
      if (jj + 1 < C) D[j] = jj + 1 <= w ? D[j] * s_d[jj + 1][ch] : D[j];
      const float kd = s_k[jj][ch] * D[j];
      sa = fmaf(kn[j], kd, sa);
      sb = fmaf(qn[j], kd, sb);
    }
    x[jj] = jj < w ? sa : 0.f;
    x[C + jj] = jj < w ? sb : 0.f;
  }
  float* out = blk + (static_cast<int64_t>(ci) * a.H + h) * L::SIZE;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int ch = lane + kWave * j;
    out[L::KP + w * K + ch] = kn[j] * P[j];
    out[L::QP + w * K + ch] = qn[j] * P[j];
    out[L::W + w * K + ch] = kn[j] * R[j];
    if (w == C - 1) out[L::PC + ch] = P[j];
  }
  wave_sums32(x);
  if (lane < 2 * C) {
    const int jj = lane % C;
    const float diag = lane < C ? beta : qk;
    out[(lane < C ? L::A : L::B) + w * C + jj] = jj < w ? x[0] : jj == w ? diag : 0.f;
  }
}

// Transposed sums over the lanes of a column. In a step the two lanes of a pair each keep the half of their values
// whose index has their lane bit, adding the partner's copy of it; the pairs are those of group_sum (v_permlane16_swap
// across rows of 16 for lane bit 4, then the DPP mirror, half mirror, xor 2 and xor 1 for bits 3 .. 0: a partner
// differs in the step's bit and agrees in every bit split before), so the lane's last value sums all the lanes.
// One step of 16-lane sums on x[0 .. 2H): pairs (v, v + H) split on lane bit `bit`.
template <int ctrl, int H>
__device__ __forceinline__ void col_step(float* x, int bit) {
  const bool hi = (lane_id() >> bit) & 1;
#pragma unroll
  for (int v = 0; v < H; ++v) {
    const float keep = hi ? x[v + H] : x[v], send = hi ? x[v] : x[v + H];
    x[v] = keep + dpp_f32<ctrl>(send);
  }
}

// 16 values over the 16 lanes of a row: x[0] becomes the row's total of value lane % 16 (15 exchanges, against 64
// for 16 separate sums).
__device__ __forceinline__ void row_sums16(float* x) {
  col_step<kDppMirror, 8>(x, 3);
  col_step<kDppHalfMirror, 4>(x, 2);
  col_step<kDppXor2, 2>(x, 1);
  col_step<kDppXor1, 1>(x, 0);
}

__device__ __forceinline__ void wave_sums32(float (&x)[32]) {
#pragma unroll
  for (int v = 0; v < 32; ++v) x[v] = half_pair_sum(x[v]);
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[v]), __float_as_uint(x[v + 16]), false, false);
    x[v] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  row_sums16(x);
}

// 32 values over the RG lanes of a column: RG = 32, x[0] = total of value rg; RG = 16, x[0] and x[16] = totals of
// values rg and 16 + rg.
template <int RG>
__device__ __forceinline__ void column_sums(float (&x)[32]) {
  if constexpr (RG == 32) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {  // row 0 keeps v, row 1 keeps v + 16, both at index v
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[v]), __float_as_uint(x[v + 16]), false, false);
      x[v] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    row_sums16(x);
  } else {
    row_sums16(x);
    row_sums16(x + 16);
  }
}

// Grid (V / COLS, H) x NWB waves, the layout of kda_recurrent_kernel: lane (c = lane / RG, rg = lane % RG) holds
// state rows 4 rg .. 4 rg + 3 of one value column. A chunk's block comes into LDS by global_load_lds (two buffers,
// the next chunk loading during this one). Per chunk a lane forms its parts of a_t and b_t for the 16 tokens and the
// column's lanes sum them transposed, so that one lane holds a_t ("A lane" of token t) and one b_t ("B lane"; for
// RG = 32 lanes 0-15 and 16-31, for RG = 16 every lane is both). The forward substitution then runs across the
// lanes: at step j the A lane of token j has all of its terms, forms u_j = beta_j r_j, and u_j goes to the column's
// lanes by readlane; every A lane of a later token subtracts A[t][j] u_j, every B lane adds B[t][j] u_j. Each lane
// keeps the 16 u for its rows of the state update; the B lanes store the outputs.
template <int K, int NWB>
__global__ __launch_bounds__(64 * NWB) void kda_chunk_kernel(KdaArgs a, const float* __restrict__ blk) {
  using L = KdaBlk<K>;
  constexpr int C = L::C, RPL = 4, RG = K / RPL, CPW = kWave / RG, COLS = NWB * CPW;
  constexpr int NT = NWB * kWave, UNITS = L::SIZE / 4, NU = (UNITS + NT - 1) / NT;
  constexpr int VPT = (C * COLS + NT - 1) / NT;
  constexpr bool DUAL = RG == C;  // every lane both an A and a B lane
  static_assert((RG == 32 || RG == 16) && C == 16, "column lanes");
  // separate arrays, so that a chunk's LDS reads need not wait for the next chunk's loads into the other one
  __shared__ __align__(16) float s_b0[L::SIZE], s_b1[L::SIZE];
  __shared__ float s_v0[C][COLS], s_v1[C][COLS];
  const int h = blockIdx.y, tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int c = lane / RG, rg = lane % RG, r0 = RPL * rg;
  const int64_t V = a.V;
  const int64_t col0 = static_cast<int64_t>(blockIdx.x) * COLS;
  const int cw = wave * CPW + c;
  const int tA = rg % C;                       // token of the lane's A role (RG = 32: lanes rg < 16)
  const bool isA = DUAL || rg < C, isB = DUAL || rg >= C;
  float* st = a.state + static_cast<int64_t>(h) * K * V + col0 + cw;
  float S[RPL];
#pragma unroll
  for (int i = 0; i < RPL; ++i) S[i] = st[static_cast<int64_t>(r0 + i) * V];
  const int nch = (a.T + C - 1) / C;
  const float* bh = blk + static_cast<int64_t>(h) * L::SIZE;
  const int64_t cs = static_cast<int64_t>(a.H) * L::SIZE;  // between the chunks of a head
  uint16_t rv[VPT];  // raw bf16 v, converted once the chunk's loads are waited for
  auto issue = [&](int ci, float* dst) {
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const int u = tid + NT * j;
      if (u < UNITS) load_lds16(bh + ci * cs + u * 4, reinterpret_cast<char*>(dst) + (wave * kWave + NT * j) * 16);
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {  // rows past the prompt (never used: beta 0) load its last token's row
      const int i = tid + NT * j, tt = min(ci * C + i / COLS, a.T - 1);
      rv[j] = a.v[tt * a.v_ts + static_cast<int64_t>(h) * V + col0 + i % COLS];
    }
  };
  // u_j of this lane's column: the value of its lane j (j wave-uniform)
  auto col_bcast = [&](float x, int j) {
    float r = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(x), j));
#pragma unroll
    for (int cc = 1; cc < CPW; ++cc) {
      const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(x), cc * RG + j));
      r = c == cc ? o : r;
    }
    return r;
  };
  auto chunk = [&](int ci, const float* in, float (*vb)[COLS], float* in_next) {
    wait_vmcnt<0>();
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int i = tid + NT * j;
      if (i < C * COLS) vb[i / COLS][i % COLS] = bf16_to_f32(rv[j]);
    }
    if constexpr (NWB == 1) wave_lds_fence(); else __syncthreads();
    if (ci + 1 < nch) issue(ci + 1, in_next);
    float x[32];  // the lane's parts of a_t (x[t]) and b_t (x[16 + t])
#pragma unroll
    for (int t = 0; t < C; ++t) {
      const float4 kp = *reinterpret_cast<const float4*>(in + L::KP + t * K + r0);
      const float4 qp = *reinterpret_cast<const float4*>(in + L::QP + t * K + r0);
      x[t] = fmaf(kp.x, S[0], kp.y * S[1]) + fmaf(kp.z, S[2], kp.w * S[3]);
      x[C + t] = fmaf(qp.x, S[0], qp.y * S[1]) + fmaf(qp.z, S[2], qp.w * S[3]);
    }
    column_sums<RG>(x);  // RG = 32: x[0] = a_rg or b_(rg-16); RG = 16: x[0] = a_rg, x[16] = b_rg
    // the lane's rows of A and B (A's diagonal holds beta)
    const float* arow = in + L::A + tA * C;
    const float* brow = in + L::B + (DUAL ? rg : (rg >= C ? rg - C : 0)) * C;
    float ca[C], cb[C];
#pragma unroll
    for (int j = 0; j < C; j += 4) {
      const float4 av = *reinterpret_cast<const float4*>(arow + j);
      const float4 bv = *reinterpret_cast<const float4*>(brow + j);
      ca[j] = av.x, ca[j + 1] = av.y, ca[j + 2] = av.z, ca[j + 3] = av.w;
      cb[j] = bv.x, cb[j + 1] = bv.y, cb[j + 2] = bv.z, cb[j + 3] = bv.w;
    }
    const float beta = arow[tA];
    float ra = isA ? vb[tA][cw] - x[0] : 0.f;  // v_t - a_t, less the earlier u's terms as they come
    float rb = DUAL ? x[16] : x[0];            // b_t, plus B[t][j] u_j
    float uall[C];
#pragma unroll
    for (int j = 0; j < C; ++j) {
      uall[j] = col_bcast(ra * beta, j);
      ra = tA > j ? fmaf(-ca[j], uall[j], ra) : ra;
      rb = fmaf(cb[j], uall[j], rb);
    }
    const float4 pc = *reinterpret_cast<const float4*>(in + L::PC + r0);
    S[0] *= pc.x;
    S[1] *= pc.y;
    S[2] *= pc.z;
    S[3] *= pc.w;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const float4 wv = *reinterpret_cast<const float4*>(in + L::W + j * K + r0);
      S[0] = fmaf(wv.x, uall[j], S[0]);
      S[1] = fmaf(wv.y, uall[j], S[1]);
      S[2] = fmaf(wv.z, uall[j], S[2]);
      S[3] = fmaf(wv.w, uall[j], S[3]);
    }
    const int t = ci * C + (DUAL ? rg : rg - C);
    if (isB && t < a.T) a.o[t * a.o_ts + static_cast<int64_t>(h) * V + col0 + cw] = f32_to_bf16(rb);
    if constexpr (NWB == 1) wave_lds_fence();  // the chunk's reads before the loads two chunks on
  };
  issue(0, s_b0);
  for (int ci = 0; ci < nch; ci += 2) {
    chunk(ci, s_b0, s_v0, s_b1);
    if (ci + 1 < nch) chunk(ci + 1, s_b1, s_v1, s_b0);
  }
#pragma unroll
  for (int i = 0; i < RPL; ++i) st[static_cast<int64_t>(r0 + i) * V] = S[i];
}

// ----------------------------------------------------------------------------------------- short conv

// y[t, ch] = silu(sum_j w[ch, j] * win_t[j] + b[ch]), win_t = the inputs t - W + 1 .. t of the channel (the cache
// holds the last W before the prompt, oldest first); the cache keeps the window after the last token. fp32 math,
// one rounding of y. Grid (C / 64, T / 16) x 64: a thread takes one channel for 16 tokens, all of whose inputs it
// loads at once; only the first token chunk reads the cache (16 >= W - 1), and its threads write the new window
// after their own reads of the old one.
constexpr int kConvTokens = 16;

template <int W>
__device__ __forceinline__ void short_conv_tile(const uint16_t* __restrict__ x, int64_t xs, int T, int64_t C,
                                                uint16_t* __restrict__ cache, const uint16_t* __restrict__ w,
                                                const uint16_t* __restrict__ b, int act, uint16_t* __restrict__ y,
                                                int64_t ys, const int64_t* __restrict__ n_valid, int bx, int by) {
  static_assert(kConvTokens >= W - 1, "only the first chunk may read the cache");
  const int64_t ch = static_cast<int64_t>(bx) * kWave + threadIdx.x;
  if (ch >= C) return;
  const int t0 = by * kConvTokens;
  float wt[W], in[kConvTokens + W - 1];  // inputs t0 - W + 1 .. t0 + 15
#pragma unroll
  for (int j = 0; j < W; ++j) wt[j] = bf16_to_f32(w[ch * W + j]);
  // every load unconditional (rows clamped into range, the value chosen after), so they all issue before the
  // first wait
#pragma unroll
  for (int i = 0; i < kConvTokens + W - 1; ++i) {
    const int t = t0 - (W - 1) + i;
    const float xv = bf16_to_f32(x[static_cast<int64_t>(t < 0 ? 0 : t < T ? t : T - 1) * xs + ch]);
    if (i < W - 1) {  // only these can precede the prompt (chunk 0)
      const float cv = bf16_to_f32(cache[ch * W + W + (t < 0 ? t : -1)]);
      in[i] = t < 0 ? cv : t < T ? xv : 0.f;
    } else {
      in[i] = t < T ? xv : 0.f;
    }
  }
  const float bias = b ? bf16_to_f32(b[ch]) : 0.f;
#pragma unroll
  for (int i = 0; i < kConvTokens; ++i) {
    if (t0 + i < T) {
      float acc = bias;
#pragma unroll
      for (int j = 0; j < W; ++j) acc = fmaf(wt[j], in[i + j], acc);
      if (act) acc = silu(acc);
      y[(t0 + i) * ys + ch] = f32_to_bf16(acc);
    }
  }
  if (by == 0) {
    // the window after the prompt's real tokens (the first n_valid, clamped to [0, T], when given: the padded
    // prefill's conv_idx, engine.py:261-262): inputs nv - W .. nv - 1, from the old cache where they precede it
    int nv = T;
    if (n_valid) nv = static_cast<int>(*n_valid < 0 ? 0 : *n_valid > T ? T : *n_valid);
    uint16_t nw[W];
#pragma unroll
    for (int j = 0; j < W; ++j) {
      const int t = nv - W + j;
      const uint16_t cv = cache[ch * W + (t < 0 ? W + t : j)];
      const uint16_t xv = x[static_cast<int64_t>(t < 0 ? 0 : t) * xs + ch];
      nw[j] = t < 0 ? cv : xv;
    }
#pragma unroll
    for (int j = 0; j < W; ++j) cache[ch * W + j] = nw[j];
  }
}


template <int W>
__global__ __launch_bounds__(64) void short_conv_kernel(const uint16_t* __restrict__ x, int64_t xs, int T, int64_t C,
                                                        uint16_t* __restrict__ cache, const uint16_t* __restrict__ w,
                                                        const uint16_t* __restrict__ b, int act,
                                                        uint16_t* __restrict__ y, int64_t ys,
                                                        const int64_t* __restrict__ n_valid) {
  short_conv_tile<W>(x, xs, T, C, cache, w, b, act, y, ys, n_valid, blockIdx.x, blockIdx.y);
}

// Up to kConvMany convolutions over the same tokens and width in one launch (a KDA layer's q, k and v):
// grid (channel blocks of the widest, token chunks, problems); a block past its problem's channels does nothing.
constexpr int kConvMany = 4;

struct ConvMany {
  const uint16_t* x[kConvMany];
  int64_t xs[kConvMany], C[kConvMany];
  uint16_t* cache[kConvMany];
  const uint16_t* w[kConvMany];
  uint16_t* y[kConvMany];
  int64_t ys[kConvMany];
  int T, act;
  const int64_t* n_valid;
};

template <int W>
__global__ __launch_bounds__(64) void short_conv_many_kernel(ConvMany m) {
  const int z = blockIdx.z;
  short_conv_tile<W>(m.x[z], m.xs[z], m.T, m.C[z], m.cache[z], m.w[z], nullptr, m.act, m.y[z], m.ys[z], m.n_valid,
                     blockIdx.x, blockIdx.y);
}

// --------------------------------------------------------------------------------------- gated RMSNorm

// One wave per row of n (<= 512) elements: y = bf16(x * rsqrt(mean(x^2) + eps) * w * sigmoid(g)), fp32 math.
__global__ __launch_bounds__(256) void rms_norm_gated_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                             const uint16_t* __restrict__ g, int64_t gs,
                                                             const uint16_t* __restrict__ w, int64_t rows, int n,
                                                             float eps, uint16_t* __restrict__ y, int64_t ys) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (row >= rows) return;
  const int lane = lane_id();
  // x, g and w of the row all requested first, through buffer resources over the row (an element past n reads
  // zero), so the wave waits for memory once (behind the range tests, each load was waited on in turn)
  const rsrc_t xr = make_rsrc(x + row * xs, static_cast<int64_t>(n) * 2), gr = make_rsrc(g + row * gs, static_cast<int64_t>(n) * 2),
               wr = make_rsrc(w, static_cast<int64_t>(n) * 2);
  float xv[8], gv[8], wv[8], ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = lane + kWave * j;
    const uint32_t off = i < n ? static_cast<uint32_t>(i) * 2u : kPast;
    xv[j] = bf16_to_f32(static_cast<uint16_t>(buf2(xr, off)));
    gv[j] = bf16_to_f32(static_cast<uint16_t>(buf2(gr, off)));
    wv[j] = bf16_to_f32(static_cast<uint16_t>(buf2(wr, off)));
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) ss = fmaf(xv[j], xv[j], ss);
  const float rstd = rsqrtf(wave_sum(ss) / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = lane + kWave * j;
    if (i < n) y[row * ys + i] = f32_to_bf16(xv[j] * rstd * wv[j] / (1.f + __expf(-gv[j])));
  }
}

// ------------------------------------------------------------------------------ one KDA decode token, one kernel
//
// The per-token core of a KDA layer (engine.py:242-263: the q/k/v short convolutions, the gate's LoRA up-projection
// f = f_b . fa, beta, fused_recurrent_kda, then g = g_b . ga and the gated output norm) in one launch instead of
// five, on the layer's projection row pr = [q | k (H K each) | v (H V) | fa | ga (R each) | beta logits (H)].
// kda_token_kernel: one workgroup of 16 waves per head, so every step that needs the whole head (the l2 norms over
// the key channels, the output norm over the value columns, the conv windows of the head's channels) stays inside
// the workgroup:
//   - the head's K key channels and V value channels are convolved over their cached windows (SiLU, rounded to
//     bf16 as short_conv_kernel stores them) and the windows shift in this token's inputs;
//   - f = bf16(sum_r f_b[ch, r] fa[r]) per key channel and g = bf16(sum_r g_b[ch, r] ga[r]) per value column
//     (two lanes per LoRA row, each over its half of R in order, one shuffle);
//   - one token of kda_short_kernel's recurrence, column block by column block (four waves per block of 16
//     value columns, the sums over key rows in kda_short_kernel's order);
//   - y = rms_norm_gated(bf16(o), g).
// Same arithmetic as the five kernels except the order of the f and g dots (small_linear reduces over more
// lanes), so f and g can differ in the last bf16 place.

struct KdaStepArgs {
  const uint16_t* pr;         // projection row
  const uint16_t* conv_w[3];  // q, k [H K, W] and v [H V, W] conv weights
  uint16_t* cache[3];         // the q, k and v conv caches of the same shapes, shifted in place
  const uint16_t* f_b;     // [H K, R]
  const uint16_t* g_b;     // [H V, R]
  const float* A_log;      // [H]
  const float* dt_bias;    // [H K]
  float lower_bound;       // NaN: the softplus gate
  float scale;
  float* state;            // [H, K, V] fp32, updated in place
  const uint16_t* o_norm;  // [V]
  float eps;
  uint16_t* y;             // [H, V]: the normed output
  int H, V, R;
};

// SiLU of a conv channel's window after the shift (cache cw[1..3], then the new input x), rounded to bf16 as
// short_conv_kernel stores it; ww the channel's 4 weights.
__device__ __forceinline__ float conv4(uint2 cw, uint2 ww, uint16_t x) {
  const float win[4] = {__uint_as_float(cw.x & 0xffff0000u), __uint_as_float(cw.y << 16),
                        __uint_as_float(cw.y & 0xffff0000u), bf16_to_f32(x)};
  const float wt[4] = {__uint_as_float(ww.x << 16), __uint_as_float(ww.x & 0xffff0000u), __uint_as_float(ww.y << 16),
                       __uint_as_float(ww.y & 0xffff0000u)};
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = fmaf(wt[j], win[j], acc);
  return round_bf16(silu(acc));
}

// The window after this token: the oldest input dropped, x appended.
__device__ __forceinline__ uint2 conv4_shift(uint2 cw, uint16_t x) {
  return make_uint2((cw.x >> 16) | (cw.y << 16), (cw.y >> 16) | (static_cast<uint32_t>(x) << 16));
}

constexpr int kKdaMaxR = 256;  // LoRA rank limit: one fa / ga element per thread of 256

// LoRA up-projection rows (row i at m + i * R, bf16, 16-byte aligned) times vec (fp32 in LDS, R entries):
// out[i] = bf16(sum_r m[i, r] vec[r]). R is taken in pieces of kLoraPiece; two neighbouring lanes share a row and
// a piece, each taking its half of it in r order (one wave load covers 32 rows x 256 bytes), and one shuffle adds
// the halves. lora_fetch issues a lane's loads for one piece, so that a kernel can issue its first piece with its
// other loads at the start; lora_piece does the arithmetic once vec is in LDS.
constexpr int kLoraPiece = 128;

struct LoraPart {
  uint4 v[kLoraPiece / 16];
};

__device__ __forceinline__ void lora_fetch(const uint16_t* m, int64_t i, bool ok, int R, int r0, LoraPart& lp) {
  const int rh = r0 + (threadIdx.x & 1) * (kLoraPiece / 2);
  const uint16_t* p = m + (ok ? i : 0) * R + rh;
#pragma unroll
  for (int j = 0; j < kLoraPiece / 16; ++j)
    lp.v[j] = ok && rh + 8 * j < R ? *reinterpret_cast<const uint4*>(p + 8 * j) : make_uint4(0u, 0u, 0u, 0u);
}

__device__ __forceinline__ float lora_piece(const LoraPart& lp, const float* vec, int R, int r0, float acc) {
  const int rh = r0 + (threadIdx.x & 1) * (kLoraPiece / 2);
#pragma unroll
  for (int j = 0; j < kLoraPiece / 16; ++j) {
    if (rh + 8 * j >= R) break;  // R is a multiple of 16: whole 8-element pieces
    const uint32_t u[4] = {lp.v[j].x, lp.v[j].y, lp.v[j].z, lp.v[j].w};
    const float* vv = vec + rh + 8 * j;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc = fmaf(__uint_as_float(u[q] << 16), vv[2 * q], acc);
      acc = fmaf(__uint_as_float(u[q] & 0xffff0000u), vv[2 * q + 1], acc);
    }
  }
  return acc;
}

// One row (i, shared by the lane pair threadIdx.x / 2) with its first piece already fetched into lp: the
// remaining pieces are fetched here. Both lanes of the pair hold the bf16-rounded result.
__device__ __forceinline__ float lora_row(const uint16_t* m, int64_t i, bool ok, int R, const float* vec,
                                          const LoraPart& first) {
  float acc = lora_piece(first, vec, R, 0, 0.f);
  for (int r0 = kLoraPiece; r0 < R; r0 += kLoraPiece) {
    LoraPart lp;
    lora_fetch(m, i, ok, R, r0, lp);
    acc = lora_piece(lp, vec, R, r0, acc);
  }
  return round_bf16(acc + __shfl_xor(acc, 1, kWave));
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// v + v of lane ^ m, element by element
__device__ __forceinline__ float4 xor_add4(float4 v, int m) {
  return make_float4(v.x + __shfl_xor(v.x, m, kWave), v.y + __shfl_xor(v.y, m, kWave), v.z + __shfl_xor(v.z, m, kWave),
                     v.w + __shfl_xor(v.w, m, kWave));
}

constexpr int kKdaThreads = 512;

// Grid H x 512 threads, K = 128, V <= 128 NP. Wave w, lane (rg = lane / 16, c4 = lane % 16): row group w4 = w % 4
// and column half hf = w / 4; in pass p the lane holds state rows r = 16 i + 4 w4 + rg (i < 8) of the four columns
// 128 p + 64 hf + 4 c4 .. + 3 (one 16-byte load per row). Each column's sums over rows keep kda_short_kernel's
// order: lane-internal over i, then over the 4 row groups of a wave (xor 16, then 32), then over the 4 waves of
// its half through LDS. Threads 0..255 take the f rows (K of them, a lane pair each), threads 256..511 the g rows,
// 128 per pass; threads < K the q and k channels, threads < V the v channels. Every global load is issued before
// the first barrier; column groups past V read zeros and write nothing (buffer bounds).
// prefetching workgroups per head: kda_token_kernel traced at 11.26 / 9.86 / 9.51 / 9.44 us per call with 0 / 3 / 7 /
// 15 of them (16 heads of 128 x 128, R = 128, inside the 28-layer hybrid step); with each helper thread's loads
// issued together (they had waited for one another) the 28-layer step took 1490 / 1484.5 / 1483 us per token with
// 3 / 7 / 15 helpers, against 1496 before
#ifndef MM_KDA_HELPERS
#define MM_KDA_HELPERS 7
#endif
constexpr int kKdaHelpers = MM_KDA_HELPERS;

// A helper workgroup of kda_token_kernel (blockIdx.x >= H): part `part` of kKdaHelpers of the head's state block
// and LoRA rows, read and dropped, so that the lines come into L2 through more CUs than the one running the head
// (whose own loads of them then find them there or in flight): one CU alone keeps too few misses outstanding to
// pull the head's 128 KB at HBM speed.
__device__ __forceinline__ void kda_token_prefetch(const KdaStepArgs& a, int h, int part) {
  constexpr int K = 128, B = 4;  // up to B pieces of each block per thread and batch, all blocks' batches at once
  const int64_t V = a.V;
  const void* blocks[3] = {a.state + static_cast<int64_t>(h) * K * V, a.f_b + static_cast<int64_t>(h) * K * a.R,
                           a.g_b + static_cast<int64_t>(h) * V * a.R};
  const int64_t bytes[3] = {K * V * 4, static_cast<int64_t>(K) * a.R * 2, V * a.R * 2};
  rsrc_t r[3];
  int64_t n[3];
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    r[b] = make_rsrc(blocks[b], bytes[b]);
    n[b] = bytes[b] / 16;  // whole 16-byte pieces (rows are 16-byte multiples)
  }
  const int64_t stride = static_cast<int64_t>(kKdaThreads) * kKdaHelpers;
  const int64_t most = n[0] > n[1] ? (n[0] > n[2] ? n[0] : n[2]) : (n[1] > n[2] ? n[1] : n[2]);
  uint32_t acc = 0;
  // every piece of a batch is requested before any is used (a load whose value the next one waits for keeps one
  // request per thread in flight); pieces past a block's end read nothing
  for (int64_t i0 = threadIdx.x + static_cast<int64_t>(part) * kKdaThreads; i0 < most; i0 += stride * B) {
    uint4 v[3][B];
#pragma unroll
    for (int b = 0; b < 3; ++b)
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const int64_t i = i0 + stride * j;
        v[b][j] = buf16(r[b], i < n[b] ? static_cast<uint32_t>(i) * 16u : kPast);
      }
#pragma unroll
    for (int b = 0; b < 3; ++b)
#pragma unroll
      for (int j = 0; j < B; ++j) acc ^= v[b][j].x;
  }
  asm volatile("" ::"v"(acc));  // keeps the loads; nothing is written
}

template <int NP>
__global__ __launch_bounds__(kKdaThreads) void kda_token_kernel(KdaStepArgs a) {
  constexpr int K = 128, RPT = K / 16, NV = 128 * NP;
  if (kKdaHelpers > 0 && static_cast<int>(blockIdx.x) >= a.H) {  // uniform: a helper workgroup
    const int hb = static_cast<int>(blockIdx.x) - a.H;
    kda_token_prefetch(a, hb % a.H, hb / a.H);
    return;
  }
  __shared__ float s_fga[2 * kKdaMaxR], s_f[K], s_q[K], s_k[K], s_dec[K], s_g[NV], s_vc[NV], s_nr[NV];
  __shared__ float s_red[K / kWave][2];
  __shared__ float4 part_u[NP][2][4][16], part_o[NP][2][4][16];
  __shared__ uint16_t s_o[NV];
  const int h = blockIdx.x;
  const int tid = threadIdx.x, w = tid / kWave, lane = lane_id();
  const int rg = lane / 16, c4 = lane % 16, w4 = w % 4, hf = w / 4;
  const int64_t V = a.V, HK = static_cast<int64_t>(a.H) * K, HV = static_cast<int64_t>(a.H) * V;
  const int64_t fa0 = 2 * HK + HV;  // fa, then ga, then the beta logits
  // fa (threads 0..255) and ga (256..511): R <= 256, one element per thread
  const int sec = tid >> 8, j8 = tid & 255;
  const uint16_t fga = a.pr[fa0 + sec * a.R + min(j8, a.R - 1)];
  // the first piece of this lane pair's f row (threads < 256) or g row
  const bool frow = tid < 256;
  const int gi0 = (tid - 256) >> 1;
  const uint16_t* lm = frow ? a.f_b + static_cast<int64_t>(h) * K * a.R : a.g_b + static_cast<int64_t>(h) * V * a.R;
  LoraPart lp;
  lora_fetch(lm, frow ? tid >> 1 : gi0, frow || gi0 < V, a.R, 0, lp);
  // the state rows of this lane's columns, through a resource over the head's [K, V] block (32-bit offsets)
  const rsrc_t srs = make_rsrc(a.state + static_cast<int64_t>(h) * K * V, static_cast<int64_t>(K) * V * 4);
  const uint32_t rstep = 16u * static_cast<uint32_t>(V) * 4u;
  uint32_t soff[NP];
  float4 S[NP][RPT];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int col = 128 * p + 64 * hf + 4 * c4;
    soff[p] = col < V ? (static_cast<uint32_t>(4 * w4 + rg) * static_cast<uint32_t>(V) + col) * 4u : kPast;
#pragma unroll
    for (int i = 0; i < RPT; ++i) S[p][i] = __builtin_bit_cast(float4, buf16(srs, soff[p] + i * rstep));
  }
  // conv channels: q and k channel tid (tid < K), v channel tid (tid < V); indices clamped, results unused past
  // the end
  const int64_t iq = static_cast<int64_t>(h) * K + min(tid, K - 1), iv = static_cast<int64_t>(h) * V + min<int64_t>(tid, V - 1);
  const uint2 cwq = *reinterpret_cast<const uint2*>(a.cache[0] + iq * 4), wq = *reinterpret_cast<const uint2*>(a.conv_w[0] + iq * 4);
  const uint2 cwk = *reinterpret_cast<const uint2*>(a.cache[1] + iq * 4), wk = *reinterpret_cast<const uint2*>(a.conv_w[1] + iq * 4);
  const uint2 cwv = *reinterpret_cast<const uint2*>(a.cache[2] + iv * 4), wv = *reinterpret_cast<const uint2*>(a.conv_w[2] + iv * 4);
  const uint16_t xq = a.pr[iq], xk = a.pr[HK + iq], xv = a.pr[2 * HK + iv];
  const float dtb = a.dt_bias[iq], nA = __expf(a.A_log[h]);
  const uint16_t nrm = a.o_norm[min<int64_t>(tid, V - 1)];  // the output norm's weight of column tid
  float beta = bf16_to_f32(a.pr[fa0 + 2 * a.R + h]);

  const bool chan = tid < K, vchan = tid < V;
  const float qv = conv4(cwq, wq, xq), kv = conv4(cwk, wk, xk);
  if (chan) {
    *reinterpret_cast<uint2*>(a.cache[0] + iq * 4) = conv4_shift(cwq, xq);
    *reinterpret_cast<uint2*>(a.cache[1] + iq * 4) = conv4_shift(cwk, xk);
  }
  if (vchan) {
    s_vc[tid] = conv4(cwv, wv, xv);
    s_nr[tid] = bf16_to_f32(nrm);
    *reinterpret_cast<uint2*>(a.cache[2] + iv * 4) = conv4_shift(cwv, xv);
  }
  if (j8 < a.R) s_fga[sec * kKdaMaxR + j8] = bf16_to_f32(fga);
  beta = 1.f / (1.f + __expf(-beta));
  __syncthreads();
  if (frow) {
    static_assert(K == 128, "one pass of 128 f rows over 256 threads");
    const float fv = lora_row(lm, tid >> 1, true, a.R, s_fga, lp);
    if ((tid & 1) == 0) s_f[tid >> 1] = fv;
  } else {
    for (int i0 = 0; i0 < V; i0 += 128) {  // wave-uniform trip count
      const int i = i0 + gi0;
      if (i0 > 0) lora_fetch(lm, i, i < V, a.R, 0, lp);
      const float gv = lora_row(lm, i, i < V, a.R, s_fga + kKdaMaxR, lp);
      if ((tid & 1) == 0 && i < V) s_g[i] = gv;
    }
  }
  __syncthreads();
  if (chan) {
    const float x = s_f[tid] + dtb;
    const float gl = isnan(a.lower_bound) ? -nA * softplus20(x) : a.lower_bound / (1.f + __expf(-nA * x));
    s_q[tid] = qv;
    s_k[tid] = kv;
    s_dec[tid] = __expf(gl);
    const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
    if (lane == 0) {
      s_red[w][0] = sq;
      s_red[w][1] = sk;
    }
  }
  __syncthreads();
  float sq = s_red[0][0], sk = s_red[0][1];
#pragma unroll
  for (int j = 1; j < K / kWave; ++j) {
    sq += s_red[j][0];
    sk += s_red[j][1];
  }
  const float qs = a.scale / sqrtf(sq + 1e-6f), ks = 1.f / sqrtf(sk + 1e-6f);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float4 pu = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = 16 * i + 4 * w4 + rg;
      const float d = s_dec[r], kk = s_k[r] * ks;
      S[p][i].x *= d;
      S[p][i].y *= d;
      S[p][i].z *= d;
      S[p][i].w *= d;
      pu.x = fmaf(kk, S[p][i].x, pu.x);
      pu.y = fmaf(kk, S[p][i].y, pu.y);
      pu.z = fmaf(kk, S[p][i].z, pu.z);
      pu.w = fmaf(kk, S[p][i].w, pu.w);
    }
    pu = xor_add4(pu, 16);
    pu = xor_add4(pu, 32);
    if (rg == 0) part_u[p][hf][w4][c4] = pu;
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int col = 128 * p + 64 * hf + 4 * c4;
    const float4 u0 = part_u[p][hf][0][c4], u1 = part_u[p][hf][1][c4], u2 = part_u[p][hf][2][c4], u3 = part_u[p][hf][3][c4];
    const float4 u = make_float4((s_vc[col] - (((u0.x + u1.x) + u2.x) + u3.x)) * beta,
                                 (s_vc[col + 1] - (((u0.y + u1.y) + u2.y) + u3.y)) * beta,
                                 (s_vc[col + 2] - (((u0.z + u1.z) + u2.z) + u3.z)) * beta,
                                 (s_vc[col + 3] - (((u0.w + u1.w) + u2.w) + u3.w)) * beta);
    float4 po = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int r = 16 * i + 4 * w4 + rg;
      const float kk = s_k[r] * ks, qq = s_q[r] * qs;
      S[p][i].x = fmaf(kk, u.x, S[p][i].x);
      S[p][i].y = fmaf(kk, u.y, S[p][i].y);
      S[p][i].z = fmaf(kk, u.z, S[p][i].z);
      S[p][i].w = fmaf(kk, u.w, S[p][i].w);
      po.x = fmaf(qq, S[p][i].x, po.x);
      po.y = fmaf(qq, S[p][i].y, po.y);
      po.z = fmaf(qq, S[p][i].z, po.z);
      po.w = fmaf(qq, S[p][i].w, po.w);
    }
    po = xor_add4(po, 16);
    po = xor_add4(po, 32);
    if (rg == 0) part_o[p][hf][w4][c4] = po;
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, S[p][i]), srs, static_cast<int>(soff[p] + i * rstep), 0, 0);
  }
  __syncthreads();
  if (w4 == 0 && rg == 0) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int col = 128 * p + 64 * hf + 4 * c4;
      const float4 o0 = part_o[p][hf][0][c4], o1 = part_o[p][hf][1][c4], o2 = part_o[p][hf][2][c4], o3 = part_o[p][hf][3][c4];
      s_o[col] = f32_to_bf16(((o0.x + o1.x) + o2.x) + o3.x);
      s_o[col + 1] = f32_to_bf16(((o0.y + o1.y) + o2.y) + o3.y);
      s_o[col + 2] = f32_to_bf16(((o0.z + o1.z) + o2.z) + o3.z);
      s_o[col + 3] = f32_to_bf16(((o0.w + o1.w) + o2.w) + o3.w);
    }
  }
  __syncthreads();
  // y = rms_norm_gated(bf16(o), g): wave 0, 8 elements per lane (V <= 512)
  if (w == 0) {
    float xo[8], ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = lane + kWave * j;
      xo[j] = i < V ? bf16_to_f32(s_o[min(i, NV - 1)]) : 0.f;
      ss = fmaf(xo[j], xo[j], ss);
    }
    const float rstd = rsqrtf(wave_sum(ss) / static_cast<float>(V) + a.eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = lane + kWave * j;
      if (i < V) a.y[static_cast<int64_t>(h) * V + i] = f32_to_bf16(xo[j] * rstd * s_nr[i] / (1.f + __expf(-s_g[i])));
    }
  }
}

// ------------------------------------------------------------------------------------ MLA decode attention

constexpr int kMlaChunk = 32;  // positions per workgroup: 4 waves of 8

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


// Grid (chunks, heads) x 4 waves; wave w owns positions t0 .. t0 + 7 (t0 = 32 chunk + 8 w), the new row standing
// in for row pos (and stored there by the wave that holds pos). First every lane issues its loads of the wave's
// value rows (LPR lanes x 8 dims per row, 64 / LPR rows per load), then the scores: 8 lanes per position, lane
// part taking the 16-byte pieces part, part + 8, ... of the q . k dot (KP of them at most), summed over the
// 8 lanes. Softmax over the chunk (a max over the 4 waves through LDS), p . V in the lanes' 8 dims, summed over
// a wave's row groups, then over the 4 waves in LDS; wave 0 writes the chunk's [dv] sums, max and sum of p.
template <int KP, int LPR>
__global__ __launch_bounds__(256) void mla_split_kernel(MlaArgs a) {
  constexpr int RPL = kWave / LPR;  // value rows per load
  constexpr int VI = 8 / RPL;       // loads covering a wave's 8 positions
  __shared__ float s_sc[kMlaChunk], s_max[4], s_l[4];
  __shared__ float s_acc[4][8 * LPR];
  const int tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int h = blockIdx.y, chunk = blockIdx.x;
  const int64_t pos = load_pos64(a.pos, a.pos_dtype);
  const int64_t c0 = static_cast<int64_t>(chunk) * kMlaChunk;
  if (pos < 0 || pos >= a.max_len || c0 > pos) return;  // uniform over the workgroup
  const int64_t t0 = c0 + wave * 8;
  const int64_t hk = static_cast<int64_t>(h) * a.max_len;
  // value rows t0 + vr + RPL i, dims 8 vd .. 8 vd + 7; rows past pos are not read (zeros: the cache there may
  // hold anything, and 0 * NaN would poison the sums)
  const int vr = lane / LPR, vd = lane % LPR;
  const bool vdim = vd * 8 < a.dv;
  uint4 vv[VI];
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int64_t tt = t0 + vr + RPL * i;
    const uint16_t* row = tt == pos ? a.v_new + static_cast<int64_t>(h) * a.dv : a.vc + (hk + tt) * a.dv;
    vv[i] = vdim && tt <= pos ? *reinterpret_cast<const uint4*>(row + vd * 8) : make_uint4(0, 0, 0, 0);
  }
  // scores: position t0 + sp, pieces part + 8 j (rows past pos are not read)
  const int sp = lane / 8, part = lane % 8;
  const int64_t t = t0 + sp;
  const int np = t <= pos ? a.dqk / 8 : 0;
  const uint16_t* krow = t == pos ? a.k_new + static_cast<int64_t>(h) * a.dqk : a.kc + (hk + t) * a.dqk;
  const uint16_t* qrow = a.q + static_cast<int64_t>(h) * a.dqk;
  uint4 kb[KP], qa[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int pc = part + 8 * j;
    if (pc < np) {
      kb[j] = *reinterpret_cast<const uint4*>(krow + pc * 8);
      qa[j] = *reinterpret_cast<const uint4*>(qrow + pc * 8);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < KP; ++j)
    if (part + 8 * j < np) s = dot8_bf16(kb[j], qa[j], s);
  s += dpp_f32<kDppXor1>(s);
  s += dpp_f32<kDppXor2>(s);
  s += dpp_f32<kDppHalfMirror>(s);
  const float sc = t <= pos ? s * a.scale : -INFINITY;
  const float wm = wave_max(sc);
  if (part == 0) s_sc[wave * 8 + sp] = sc;
  if (lane == 0) s_max[wave] = wm;
  // the wave holding pos stores the new rows into the cache
  if (pos >= t0 && pos < t0 + 8) {
    uint16_t* kd = a.kc + (hk + pos) * a.dqk;
    uint16_t* vd_ = a.vc + (hk + pos) * a.dv;
    for (int i = lane; i < a.dqk; i += kWave) kd[i] = a.k_new[static_cast<int64_t>(h) * a.dqk + i];
    for (int i = lane; i < a.dv; i += kWave) vd_[i] = a.v_new[static_cast<int64_t>(h) * a.dv + i];
  }
  __syncthreads();
  const float m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));  // finite: c0 <= pos is valid
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int r = vr + RPL * i;
    const float p = t0 + r <= pos ? __expf(s_sc[wave * 8 + r] - m) : 0.f;
    const uint32_t x[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] = fmaf(p, bf_lo(x[e]), acc[2 * e]);
      acc[2 * e + 1] = fmaf(p, bf_hi(x[e]), acc[2 * e + 1]);
    }
  }
#pragma unroll
  for (int off = LPR; off < kWave; off *= 2)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], off, kWave);
  if (lane < LPR && vdim) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_acc[wave][vd * 8 + e] = acc[e];
  }
  // the wave's sum of p: lane i < 8 for position t0 + i
  const float pl = lane < 8 && t0 + lane <= pos ? __expf(s_sc[wave * 8 + lane] - m) : 0.f;
  const float lsum = wave_sum(pl);
  if (lane == 0) s_l[wave] = lsum;
  __syncthreads();
  if (wave != 0) return;
  float* dst = a.ws + (static_cast<int64_t>(h) * a.nc + chunk) * (a.dv + 2);
  for (int d = lane; d < a.dv; d += kWave) dst[d] = ((s_acc[0][d] + s_acc[1][d]) + s_acc[2][d]) + s_acc[3][d];
  if (lane == 0) {
    dst[a.dv] = m;
    dst[a.dv + 1] = ((s_l[0] + s_l[1]) + s_l[2]) + s_l[3];
  }
}

// One workgroup of 4 waves per head merges the chunks 0 .. pos / 32: the max of the maxima (lanes over chunks),
// then wave w rescales and sums chunks w, w + 4, ... in that order (lane = value dimension), the 4 waves' sums
// added in LDS. The chunk states a wave needs for the first kMergeBatch of its chunks and the maxima of the first
// 256 chunks are loaded before pos arrives (chunks clamped into the workspace, the ones past pos dropped by
// selects), so the kernel waits for memory about once; longer prefixes load the rest afterwards.
// A position outside [0, max_len) writes NaN (and the split kernel wrote nothing).
constexpr int kMergeBatch = 8;  // chunks per wave loaded ahead: 4 waves x 8 x 32 positions = 1024 positions

template <int NDV>
__global__ __launch_bounds__(256) void mla_merge_kernel(MlaArgs a) {
  __shared__ float s_acc[4][kWave * NDV], s_l[4], s_m[4];
  const int h = blockIdx.x, tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int64_t cs = a.dv + 2;
  const float* base = a.ws + static_cast<int64_t>(h) * a.nc * cs;
  // loads that do not depend on pos
  const float m_first = base[static_cast<int64_t>(min(tid, a.nc - 1)) * cs + a.dv];
  float pm[kMergeBatch], pl[kMergeBatch], pv[kMergeBatch][NDV];
#pragma unroll
  for (int b = 0; b < kMergeBatch; ++b) {
    const float* p = base + static_cast<int64_t>(min(wave + 4 * b, a.nc - 1)) * cs;
    pm[b] = p[a.dv];
    pl[b] = p[a.dv + 1];
#pragma unroll
    for (int j = 0; j < NDV; ++j) pv[b][j] = p[min(lane + kWave * j, a.dv - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);  // pos (a scalar load) after the vector loads
  const int64_t pos = load_pos64(a.pos, a.pos_dtype);
  if (pos < 0 || pos >= a.max_len) {
    for (int d = tid; d < a.dv; d += 256) a.out[static_cast<int64_t>(h) * a.dv + d] = 0x7fc0;  // NaN
    return;
  }
  const int n = static_cast<int>(pos / kMlaChunk) + 1;
  float mx = tid < n ? m_first : -INFINITY;
  for (int c = tid + 256; c < n; c += 256) mx = fmaxf(mx, base[c * cs + a.dv]);
  mx = wave_max(mx);
  if (lane == 0) s_m[wave] = mx;
  __syncthreads();
  const float m = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
  float acc[NDV], l = 0.f;
#pragma unroll
  for (int j = 0; j < NDV; ++j) acc[j] = 0.f;
#pragma unroll
  for (int b = 0; b < kMergeBatch; ++b) {
    if (wave + 4 * b < n) {  // uniform
      const float wgt = __expf(pm[b] - m);
      l = fmaf(pl[b], wgt, l);
#pragma unroll
      for (int j = 0; j < NDV; ++j) {
        const int d = lane + kWave * j;
        if (d < a.dv) acc[j] = fmaf(pv[b][j], wgt, acc[j]);
      }
    }
  }
  for (int c = wave + 4 * kMergeBatch; c < n; c += 4) {
    const float* p = base + c * cs;
    const float wgt = __expf(p[a.dv] - m);
    l = fmaf(p[a.dv + 1], wgt, l);
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      const int d = lane + kWave * j;
      if (d < a.dv) acc[j] = fmaf(p[d], wgt, acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NDV; ++j) s_acc[wave][lane + kWave * j] = acc[j];
  if (lane == 0) s_l[wave] = l;
  __syncthreads();
  const float lt = ((s_l[0] + s_l[1]) + s_l[2]) + s_l[3];
  for (int d = tid; d < a.dv; d += 256) {
    const float o = ((s_acc[0][d] + s_acc[1][d]) + s_acc[2][d]) + s_acc[3][d];
    a.out[static_cast<int64_t>(h) * a.dv + d] = f32_to_bf16(o / lt);
  }
}

// ------------------------------------------------------------------------------- MLA prefill (T tokens)

struct MlaPrefillArgs {
  const uint16_t* q;      // token t's heads at q + t q_ts: [nh, dqk]
  const uint16_t* k_new;  // [nh, dqk] per token (token stride k_ts)
  const uint16_t* v_new;  // [nh, dv] per token (token stride v_ts)
  int64_t q_ts, k_ts, v_ts;
  uint16_t* kc;  // [nh, max_len, dqk]
  uint16_t* vc;  // [nh, max_len, dv]
  const void* pos;  // the first token's position
  int pos_dtype;
  int T, nh, dqk, dv;
  int64_t max_len;
  float scale;
  uint16_t* out;  // [nh, dv] per token (token stride out_ts)
  int64_t out_ts;
};

__device__ __forceinline__ bool mla_prefill_pos_ok(const MlaPrefillArgs& a, int64_t pos) {
  return pos >= 0 && pos + a.T <= a.max_len;
}

// Grid (T, nh) x 64: token t's key and value rows of head h go to cache row pos + t (engine.py:537-541,
// index_copy_ at the prompt's positions). A prompt that does not fit in [0, max_len) stores nothing.
__global__ __launch_bounds__(64) void mla_prefill_store_kernel(MlaPrefillArgs a) {
  const int t = blockIdx.x, h = blockIdx.y;
  const int64_t pos = load_pos64(a.pos, a.pos_dtype);
  if (!mla_prefill_pos_ok(a, pos)) return;
  const int64_t row = static_cast<int64_t>(h) * a.max_len + pos + t;
  const auto* ks = reinterpret_cast<const uint4*>(a.k_new + t * a.k_ts + static_cast<int64_t>(h) * a.dqk);
  const auto* vs = reinterpret_cast<const uint4*>(a.v_new + t * a.v_ts + static_cast<int64_t>(h) * a.dv);
  auto* kd = reinterpret_cast<uint4*>(a.kc + row * a.dqk);
  auto* vd = reinterpret_cast<uint4*>(a.vc + row * a.dv);
  for (int i = threadIdx.x; i < a.dqk / 8; i += kWave) kd[i] = ks[i];
  for (int i = threadIdx.x; i < a.dv / 8; i += kWave) vd[i] = vs[i];
}

constexpr int kMlaPKeys = 32;  // keys per tile
constexpr int kMlaPVtRow = 36;  // bf16 per transposed value row in LDS: 32 keys + 4 (72 bytes, see the stores)


// Causal attention of T prompt tokens over the static cache (the new rows already stored): token t at position
// pos + t takes softmax(scale q_t . K[0..pos+t]^T) . V[0..pos+t] (engine.py:679-682's mask). Grid (T / 16,
// nh) x NW waves (8 when the grid is small, else 4): a workgroup holds 16 queries of one head, and its waves take
// the 32-key tiles round robin (wave w: tiles w, w + NW, ...), each keeping its own running max, sum and output for
// the 16 queries; they are merged through LDS at the end. Per tile, on the 16x16x32 bf16 MFMA:
//   S^T [32 keys, 16 queries] = K Q^T, the key rows read straight from the cache into A fragments and the
//     queries held as B fragments (lane: query lane % 16, dims 32 kk + 8 (lane / 16) .. + 7);
//   the masked softmax update per query is lane-local (a lane of the S^T tiles holds 8 keys of its query
//     column: 4 (lane / 16) + v and 16 + 4 (lane / 16) + v), the tile max summed over the 4 lane quarters;
//   O^T [dv, 16 queries] += V^T P^T: the B fragment of P comes straight from the S^T registers, its 8 k slots
//     taking those 8 keys in that order, and the A fragment of V^T (dim lane % 16, the same 8 keys) from a
//     transposed copy of the value tile the wave stores in its own LDS ([dv][36], two keys per 4-byte store).
// O^T's lane layout (dims 4 (lane / 16) + v of each 16-dim tile, query lane % 16) keeps the rescaling by the
// query's exp(m_old - m_new) lane-local as well. Keys past the block's last query are not read (zeros, then
// masked); queries past T repeat the last token and are not stored. A prompt outside [0, max_len) writes NaN.
template <int NT, int NW>  // dv <= 16 NT; NW waves per workgroup
__global__ __launch_bounds__(NW * 64) void mla_prefill_attn_kernel(MlaPrefillArgs a) {
  constexpr int DVM = 16 * NT;
  constexpr int VT_BYTES = DVM * kMlaPVtRow * 2;
  constexpr int MERGE_BYTES = 16 * DVM * 4;  // the wave's O [16 queries][DVM] fp32
  constexpr int WAVE_BYTES = VT_BYTES > MERGE_BYTES ? VT_BYTES : MERGE_BYTES;
  __shared__ __align__(16) char s_buf[NW * WAVE_BYTES];
  __shared__ float s_m[NW][16], s_l[NW][16];
  const int tid = threadIdx.x, wave = tid / kWave, lane = lane_id();
  const int lr = lane & 15, lq = lane >> 4;
  const int h = blockIdx.y, tq0 = blockIdx.x * 16;
  const int64_t pos = load_pos64(a.pos, a.pos_dtype);
  const int n4 = a.dv / 4;
  if (!mla_prefill_pos_ok(a, pos)) {  // uniform over the workgroup
    for (int i = tid; i < 16 * a.dv; i += NW * kWave) {
      const int t = tq0 + i / a.dv;
      if (t < a.T) a.out[t * a.out_ts + static_cast<int64_t>(h) * a.dv + i % a.dv] = 0x7fc0;  // NaN
    }
    return;
  }
  const int tlast = min(tq0 + 15, a.T - 1);
  const int tq = min(tq0 + lr, a.T - 1);
  const int64_t qlim = pos + tq;          // the keys this lane's query attends: 0 .. qlim
  const int64_t kend = pos + tlast + 1;   // the keys any query of the workgroup attends: 0 .. kend - 1
  const int ntiles = static_cast<int>((kend + kMlaPKeys - 1) / kMlaPKeys);
  const int nkq = (a.dqk + 31) / 32;
  bf16x8_t qf[8];
  {
    const uint16_t* qrow = a.q + tq * a.q_ts + static_cast<int64_t>(h) * a.dqk;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int d = 32 * kk + 8 * lq;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (kk < nkq && d < a.dqk) x = *reinterpret_cast<const uint4*>(qrow + d);
      qf[kk] = __builtin_bit_cast(bf16x8_t, x);
    }
  }
  floatx4 o[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) o[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  uint16_t* vt = reinterpret_cast<uint16_t*>(s_buf + wave * WAVE_BYTES);
  const int64_t hk = static_cast<int64_t>(h) * a.max_len;
  constexpr int RV = (DVM + 31) / 32;  // value pieces (2 keys x 8 dims) per lane: 16 key pairs x dv / 8 groups
  const int ndg = a.dv / 8;
  for (int kt = wave; kt < ntiles; kt += NW) {
    const int64_t j0 = static_cast<int64_t>(kt) * kMlaPKeys;
    // every load of the tile first, unconditionally (rows and dims past the ends read the row's first piece and are
    // zeroed after), so the tile costs one trip to memory: where each load sat behind its own range test, the
    // compiler waited for each before the next (16 round trips per tile)
    // value tile: lane piece i = lane + 64 r -> key pair kp = i % 16, dim group dg = i / 16
    uint4 va[RV], vb[RV];
    bool oka[RV], okb[RV];
#pragma unroll
    for (int r = 0; r < RV; ++r) {
      const int i = lane + kWave * r, kp = i % 16, dg = i / 16;
      const int64_t ja = j0 + 2 * kp;
      const bool dok = dg < ndg;
      oka[r] = dok && ja < kend;
      okb[r] = dok && ja + 1 < kend;
      va[r] = *reinterpret_cast<const uint4*>(a.vc + (hk + (oka[r] ? ja : 0)) * a.dv + (oka[r] ? 8 * dg : 0));
      vb[r] = *reinterpret_cast<const uint4*>(a.vc + (hk + (okb[r] ? ja + 1 : 0)) * a.dv + (okb[r] ? 8 * dg : 0));
    }
    uint4 kx[2][8];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int64_t j = j0 + 16 * n + lr;
      const bool live = j < kend;
      const uint16_t* krow = a.kc + (hk + (live ? j : 0)) * a.dqk;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int d = 32 * kk + 8 * lq;
        const bool ok = live && d < a.dqk;
        kx[n][kk] = and_mask16(*reinterpret_cast<const uint4*>(krow + (ok ? d : 0)), ok);
      }
    }
#pragma unroll
    for (int r = 0; r < RV; ++r) {
      va[r] = and_mask16(va[r], oka[r]);
      vb[r] = and_mask16(vb[r], okb[r]);
    }
    floatx4 s[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      s[n] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        if (kk < nkq)
          s[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kx[n][kk]), qf[kk], s[n], 0, 0, 0);
    }
    // the transposed value tile: dword (dim 8 dg + e, keys 2 kp, 2 kp + 1); 16 consecutive key pairs per dim
    // row and 4 dim groups 8 x 18 dwords apart per store keep the 64 lanes on distinct banks
    wave_lds_fence();  // the previous tile's reads of vt are done
#pragma unroll
    for (int r = 0; r < RV; ++r) {
      const int i = lane + kWave * r, kp = i % 16, dg = i / 16;
      if (dg < ndg) {
        const uint32_t xa[4] = {va[r].x, va[r].y, va[r].z, va[r].w}, xb[4] = {vb[r].x, vb[r].y, vb[r].z, vb[r].w};
        auto* dst = reinterpret_cast<uint32_t*>(vt) + (8 * dg) * (kMlaPVtRow / 2) + kp;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dst[(2 * e) * (kMlaPVtRow / 2)] = __builtin_amdgcn_perm(xb[e], xa[e], 0x05040100u);      // low halves
          dst[(2 * e + 1) * (kMlaPVtRow / 2)] = __builtin_amdgcn_perm(xb[e], xa[e], 0x07060302u);  // high halves
        }
      }
    }
    // masked online softmax: slot e < 4 is key j0 + 4 lq + e, slot e >= 4 key j0 + 16 + 4 lq + e - 4
    float sv[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t key = j0 + (e < 4 ? 4 * lq + e : 16 + 4 * lq + e - 4);
      const float x = e < 4 ? s[0][e] : s[1][e - 4];
      sv[e] = key <= qlim ? x * a.scale : -INFINITY;
      tmax = fmaxf(tmax, sv[e]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float mn = fmaxf(m, tmax);
    const float mu = mn == -INFINITY ? 0.f : mn;  // a query with no key yet in this wave's tiles
    const float alpha = __expf(m - mu);
    m = mn;
    float ps = 0.f;
    uint32_t pw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p0 = __expf(sv[2 * e] - mu), p1 = __expf(sv[2 * e + 1] - mu);
      ps += p0 + p1;
      pw[e] = static_cast<uint32_t>(f32_to_bf16(p0)) | (static_cast<uint32_t>(f32_to_bf16(p1)) << 16);
    }
    l = fmaf(l, alpha, ps);
    const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, make_uint4(pw[0], pw[1], pw[2], pw[3]));
    wave_lds_fence();  // the stores of vt before the loads
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      o[nt] *= alpha;
      if (16 * nt < a.dv) {
        const uint16_t* row = vt + (16 * nt + lr) * kMlaPVtRow;
        const uint2 lo = *reinterpret_cast<const uint2*>(row + 4 * lq);
        const uint2 hi = *reinterpret_cast<const uint2*>(row + 16 + 4 * lq);
        o[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y)),
                                                        pf, o[nt], 0, 0, 0);
      }
    }
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  // the wave's state into its own LDS region (its value tile is no longer read), then the merge
  wave_lds_fence();
  float* so = reinterpret_cast<float*>(s_buf + wave * WAVE_BYTES);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    if (16 * nt < a.dv) *reinterpret_cast<floatx4*>(so + lr * DVM + 16 * nt + 4 * lq) = o[nt];
  if (lq == 0) {
    s_m[wave][lr] = m;
    s_l[wave][lr] = l;
  }
  __syncthreads();
  for (int i = tid; i < 16 * n4; i += NW * kWave) {
    const int qi = i / n4, d = 4 * (i % n4), t = tq0 + qi;
    if (t >= a.T) continue;
    float mx = s_m[0][qi];  // finite: wave 0 holds key 0
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, s_m[w][qi]);
    float lt = 0.f;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = __expf(s_m[w][qi] - mx);
      lt = fmaf(s_l[w][qi], wt, lt);
      acc += wt * *reinterpret_cast<const floatx4*>(reinterpret_cast<const float*>(s_buf + w * WAVE_BYTES) +
                                                    qi * DVM + d);
    }
    const float inv = 1.f / lt;
    uint16_t* dst = a.out + t * a.out_ts + static_cast<int64_t>(h) * a.dv + d;
    const uint32_t w0 = static_cast<uint32_t>(f32_to_bf16(acc[0] * inv)) | (static_cast<uint32_t>(f32_to_bf16(acc[1] * inv)) << 16);
    const uint32_t w1 = static_cast<uint32_t>(f32_to_bf16(acc[2] * inv)) | (static_cast<uint32_t>(f32_to_bf16(acc[3] * inv)) << 16);
    *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
  }
}

template <int K>
int launch_kda(const KdaArgs& a, float* ws, hipStream_t st) {
  if (a.T <= kKdaShortT) {
    hipLaunchKernelGGL((kda_short_kernel<K>), dim3(static_cast<unsigned>(a.V / kKdaCols), static_cast<unsigned>(a.H)),
                       dim3(256), 0, st, a);
    return mm::check_launch("kda_recurrent");
  }
  const int64_t rows = static_cast<int64_t>(a.T) * a.H;
  hipLaunchKernelGGL((kda_prep_kernel<K>), dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, st, a, ws);
  int rc = mm::check_launch("kda_recurrent prep");
  if (rc) return rc;
  constexpr int RPL = kKdaRpl, NWB = kKdaNwb, cols = NWB * kWave / (K / RPL);
  if (a.V % cols == 0) {
    hipLaunchKernelGGL((kda_recurrent_kernel<K, RPL, NWB>), dim3(static_cast<unsigned>(a.V / cols),
                       static_cast<unsigned>(a.H)), dim3(kWave * NWB), 0, st, a, static_cast<const float*>(ws));
  } else {  // V a multiple of 8 only: one wave of 8 rows per lane per workgroup
    hipLaunchKernelGGL((kda_recurrent_kernel<K, 8, 1>), dim3(static_cast<unsigned>(a.V / (kWave / (K / 8))),
                       static_cast<unsigned>(a.H)), dim3(kWave), 0, st, a, static_cast<const float*>(ws));
  }
  return mm::check_launch("kda_recurrent");
}

// The chunked form: token preparation, the (chunk, head) blocks after the token rows, then the chunk recurrence.
template <int K>
int launch_kda_chunk(const KdaArgs& a, float* ws, hipStream_t st) {
  if (a.T <= kKdaShortT) return launch_kda<K>(a, ws, st);  // a decode step: one launch, no workspace
  float* blk = ws;
  const unsigned nch = static_cast<unsigned>((a.T + kKdaChunk - 1) / kKdaChunk);
  hipLaunchKernelGGL((kda_chunk_prep_kernel<K>), dim3(nch, static_cast<unsigned>(a.H)), dim3(64 * kKdaChunk), 0, st, a,
                     blk);
  int rc = mm::check_launch("kda_chunk prep");
  if (rc) return rc;
  constexpr int NWB = kKdaNwb, cols = NWB * kWave / (K / 4);
  if (a.V % cols == 0) {
    hipLaunchKernelGGL((kda_chunk_kernel<K, NWB>), dim3(static_cast<unsigned>(a.V / cols), static_cast<unsigned>(a.H)),
                       dim3(kWave * NWB), 0, st, a, static_cast<const float*>(blk));
  } else {  // V a multiple of 8 only: one wave per workgroup
    hipLaunchKernelGGL((kda_chunk_kernel<K, 1>), dim3(static_cast<unsigned>(a.V / (cols / NWB)),
                       static_cast<unsigned>(a.H)), dim3(kWave), 0, st, a, static_cast<const float*>(blk));
  }
  return mm::check_launch("kda_chunk");
}

}  // namespace

extern "C" int64_t mm_kda_recurrent_workspace(int64_t T, int64_t H, int64_t K) {
  if (T < 0 || H < 1 || (K != 64 && K != 128)) return -1;
  if (T <= kKdaShortT) return 0;
  return T * H * (3 * K + 4) * static_cast<int64_t>(sizeof(float));
}

extern "C" int64_t mm_kda_chunk_workspace(int64_t T, int64_t H, int64_t K) {
  if (T < 0 || H < 1 || (K != 64 && K != 128)) return -1;
  if (T <= kKdaShortT) return 0;
  const int64_t blk = K == 64 ? KdaBlk<64>::SIZE : KdaBlk<128>::SIZE;
  return (T + kKdaChunk - 1) / kKdaChunk * H * blk * static_cast<int64_t>(sizeof(float));
}

// The argument checks and launches of mm_kda_recurrent and mm_kda_chunk (same arguments, same results up to the
// order of fp32 sums).
static int kda_entry(bool chunked, const void* q, int64_t q_ts, const void* k, int64_t k_ts, const void* v,
                     int64_t v_ts, const void* g, int g_dtype, int64_t g_ts, const void* beta, int beta_dtype,
                     int64_t beta_ts, const float* A_log, const float* dt_bias, float lower_bound, int use_qk_l2norm,
                     int use_gate, int beta_logits, float scale, int64_t T, int64_t H, int64_t K, int64_t V,
                     float* state, void* o, int64_t o_ts, const int64_t* n_valid, void* workspace,
                     int64_t workspace_bytes, void* stream) {
  const char* who = chunked ? "kda_chunk" : "kda_recurrent";
  MM_REQUIRE(T >= 0 && T <= (1 << 20) && H >= 1 && H <= 65535 && T * H <= (1LL << 31),
             "%s: bad T=%lld or H=%lld (T <= 2^20, H <= 65535, T H <= 2^31)", who, (long long)T, (long long)H);
  // a lane holds 8 state rows of one column; one wave per 64 / (K / 8) value columns
  MM_REQUIRE((K == 64 || K == 128) && V % (T <= kKdaShortT ? kKdaCols : 8) == 0 && V >= 8 && V <= 4096,
             "%s: head dims K=%lld (64 or 128), V=%lld (a multiple of 8 up to 4096; of 16 for T <= %d)", who,
             (long long)K, (long long)V, kKdaShortT);
  const int64_t need = chunked ? mm_kda_chunk_workspace(T, H, K) : mm_kda_recurrent_workspace(T, H, K);
  MM_REQUIRE(T <= kKdaShortT || (workspace && mm::aligned16(workspace) && workspace_bytes >= need),
             "%s: the workspace must be 16-byte aligned and hold mm_%s_workspace(T, H, K) bytes", who, who);
  MM_REQUIRE(g_dtype == MM_BF16 || g_dtype == MM_FP32, "%s: g must be bf16 or fp32", who);
  MM_REQUIRE(beta_dtype == MM_BF16 || beta_dtype == MM_FP32, "%s: beta must be bf16 or fp32", who);
  MM_REQUIRE(q && k && v && g && beta && state && o, "%s: null pointer", who);
  MM_REQUIRE(!use_gate || (A_log && dt_bias), "%s: the gate needs A_log and dt_bias", who);
  MM_REQUIRE(q_ts >= H * K && k_ts >= H * K && g_ts >= H * K && v_ts >= H * V && beta_ts >= H && o_ts >= H * V,
             "%s: token strides smaller than a token's heads", who);
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
  a.beta_logits = beta_logits;
  a.scale = scale;
  a.state = state;
  a.o = static_cast<uint16_t*>(o);
  a.o_ts = o_ts;
  a.T = static_cast<int>(T);
  a.H = static_cast<int>(H);
  a.V = static_cast<int>(V);
  a.n_valid = n_valid;
  hipStream_t st = MM_STREAM(stream);
  float* ws = static_cast<float*>(workspace);
  if (chunked) return K == 64 ? launch_kda_chunk<64>(a, ws, st) : launch_kda_chunk<128>(a, ws, st);
  return K == 64 ? launch_kda<64>(a, ws, st) : launch_kda<128>(a, ws, st);
}

extern "C" int mm_kda_recurrent(const void* q, int64_t q_ts, const void* k, int64_t k_ts, const void* v, int64_t v_ts,
                                const void* g, int g_dtype, int64_t g_ts, const void* beta, int beta_dtype,
                                int64_t beta_ts, const float* A_log, const float* dt_bias, float lower_bound,
                                int use_qk_l2norm, int use_gate, int beta_logits, float scale, int64_t T, int64_t H,
                                int64_t K, int64_t V, float* state, void* o, int64_t o_ts, const int64_t* n_valid,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  return kda_entry(false, q, q_ts, k, k_ts, v, v_ts, g, g_dtype, g_ts, beta, beta_dtype, beta_ts, A_log, dt_bias,
                   lower_bound, use_qk_l2norm, use_gate, beta_logits, scale, T, H, K, V, state, o, o_ts, n_valid,
                   workspace, workspace_bytes, stream);
}

extern "C" int mm_kda_chunk(const void* q, int64_t q_ts, const void* k, int64_t k_ts, const void* v, int64_t v_ts,
                            const void* g, int g_dtype, int64_t g_ts, const void* beta, int beta_dtype, int64_t beta_ts,
                            const float* A_log, const float* dt_bias, float lower_bound, int use_qk_l2norm,
                            int use_gate, int beta_logits, float scale, int64_t T, int64_t H, int64_t K, int64_t V,
                            float* state, void* o, int64_t o_ts, const int64_t* n_valid, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  return kda_entry(true, q, q_ts, k, k_ts, v, v_ts, g, g_dtype, g_ts, beta, beta_dtype, beta_ts, A_log, dt_bias,
                   lower_bound, use_qk_l2norm, use_gate, beta_logits, scale, T, H, K, V, state, o, o_ts, n_valid,
                   workspace, workspace_bytes, stream);
}

extern "C" int mm_short_conv(const void* x, int64_t x_ts, int64_t T, int64_t C, void* cache, int64_t W, const void* w,
                             const void* b, int act, void* y, int64_t y_ts, const int64_t* n_valid, void* stream) {
  MM_REQUIRE(T >= 0 && T <= 65535LL * kConvTokens && C >= 1 && C <= (1LL << 31) / 8, "short_conv: bad T=%lld or C=%lld",
             (long long)T, (long long)C);
  MM_REQUIRE(W >= 2 && W <= 8, "short_conv: kernel width %lld must be in [2, 8]", (long long)W);
  MM_REQUIRE(x && cache && w && y, "short_conv: null pointer");
  MM_REQUIRE(x_ts >= C && y_ts >= C, "short_conv: token strides smaller than the channels");
  if (T == 0) return MM_OK;
  const auto* xp = static_cast<const uint16_t*>(x);
  auto* cp = static_cast<uint16_t*>(cache);
  const auto* wp = static_cast<const uint16_t*>(w);
  const auto* bp = static_cast<const uint16_t*>(b);
  auto* yp = static_cast<uint16_t*>(y);
  const int64_t* nv = n_valid;
  dim3 grid(static_cast<unsigned>((C + kWave - 1) / kWave), static_cast<unsigned>((T + kConvTokens - 1) / kConvTokens));
  hipStream_t st = MM_STREAM(stream);
  switch (W) {
    case 2: hipLaunchKernelGGL(short_conv_kernel<2>, grid, dim3(kWave), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts, nv); break;
    case 3: hipLaunchKernelGGL(short_conv_kernel<3>, grid, dim3(kWave), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts, nv); break;
    case 4: hipLaunchKernelGGL(short_conv_kernel<4>, grid, dim3(kWave), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts, nv); break;
    case 5: hipLaunchKernelGGL(short_conv_kernel<5>, grid, dim3(kWave), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts, nv); break;
    case 6: hipLaunchKernelGGL(short_conv_kernel<6>, grid, dim3(kWave), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts, nv); break;
    case 7: hipLaunchKernelGGL(short_conv_kernel<7>, grid, dim3(kWave), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts, nv); break;
    default: hipLaunchKernelGGL(short_conv_kernel<8>, grid, dim3(kWave), 0, st, xp, x_ts, (int)T, C, cp, wp, bp, act, yp, y_ts, nv); break;
  }
  return mm::check_launch("short_conv");
}

extern "C" int mm_short_conv_many(int64_t n, const void* const* x, const int64_t* x_ts, const int64_t* C,
                                  void* const* cache, const void* const* w, void* const* y, const int64_t* y_ts,
                                  int64_t T, int64_t W, int act, const int64_t* n_valid, void* stream) {
  MM_REQUIRE(n >= 1 && n <= kConvMany, "short_conv_many: %lld convolutions (1 to %d)", (long long)n, kConvMany);
  MM_REQUIRE(x && x_ts && C && cache && w && y && y_ts, "short_conv_many: null array");
  MM_REQUIRE(T >= 0 && T <= 65535LL * kConvTokens, "short_conv_many: bad T=%lld", (long long)T);
  MM_REQUIRE(W >= 2 && W <= 8, "short_conv_many: kernel width %lld must be in [2, 8]", (long long)W);
  ConvMany m{};
  int64_t cmax = 0;
  for (int64_t i = 0; i < n; ++i) {
    MM_REQUIRE(C[i] >= 1 && C[i] <= (1LL << 31) / 8, "short_conv_many: bad C=%lld (convolution %lld)", (long long)C[i],
               (long long)i);
    MM_REQUIRE(x[i] && cache[i] && w[i] && y[i], "short_conv_many: null pointer (convolution %lld)", (long long)i);
    MM_REQUIRE(x_ts[i] >= C[i] && y_ts[i] >= C[i], "short_conv_many: token strides smaller than the channels "
               "(convolution %lld)", (long long)i);
    m.x[i] = static_cast<const uint16_t*>(x[i]);
    m.xs[i] = x_ts[i];
    m.C[i] = C[i];
    m.cache[i] = static_cast<uint16_t*>(cache[i]);
    m.w[i] = static_cast<const uint16_t*>(w[i]);
    m.y[i] = static_cast<uint16_t*>(y[i]);
    m.ys[i] = y_ts[i];
    cmax = C[i] > cmax ? C[i] : cmax;
  }
  if (T == 0) return MM_OK;
  m.T = static_cast<int>(T);
  m.act = act;
  m.n_valid = n_valid;
  dim3 grid(static_cast<unsigned>((cmax + kWave - 1) / kWave), static_cast<unsigned>((T + kConvTokens - 1) / kConvTokens),
            static_cast<unsigned>(n));
  hipStream_t st = MM_STREAM(stream);
  switch (W) {
    case 2: hipLaunchKernelGGL(short_conv_many_kernel<2>, grid, dim3(kWave), 0, st, m); break;
    case 3: hipLaunchKernelGGL(short_conv_many_kernel<3>, grid, dim3(kWave), 0, st, m); break;
    case 4: hipLaunchKernelGGL(short_conv_many_kernel<4>, grid, dim3(kWave), 0, st, m); break;
    case 5: hipLaunchKernelGGL(short_conv_many_kernel<5>, grid, dim3(kWave), 0, st, m); break;
    case 6: hipLaunchKernelGGL(short_conv_many_kernel<6>, grid, dim3(kWave), 0, st, m); break;
    case 7: hipLaunchKernelGGL(short_conv_many_kernel<7>, grid, dim3(kWave), 0, st, m); break;
    default: hipLaunchKernelGGL(short_conv_many_kernel<8>, grid, dim3(kWave), 0, st, m); break;
  }
  return mm::check_launch("short_conv_many");
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

extern "C" int mm_kda_decode_step(const void* pr, int64_t pr_len, const void* const* conv_w, void* const* conv_cache,
                                  int64_t W, const void* f_b, const void* g_b, int64_t R, const float* A_log,
                                  const float* dt_bias, float lower_bound, float scale, float* state, int64_t H,
                                  int64_t K, int64_t V, const void* o_norm, float eps, void* y, void* stream) {
  MM_REQUIRE(H >= 1 && H <= 65535, "kda_decode_step: bad H=%lld", (long long)H);
  MM_REQUIRE(K == 128 && V % kKdaCols == 0 && V >= kKdaCols && V <= 512,
             "kda_decode_step: head dims K=%lld (128), V=%lld (a multiple of 16 up to 512)", (long long)K, (long long)V);
  MM_REQUIRE(W == 4, "kda_decode_step: conv window %lld (4)", (long long)W);
  MM_REQUIRE(R >= 16 && R <= kKdaMaxR && R % 16 == 0, "kda_decode_step: LoRA rank %lld (a multiple of 16 up to %d)",
             (long long)R, kKdaMaxR);
  MM_REQUIRE(pr_len == 2 * H * K + H * V + 2 * R + H,
             "kda_decode_step: projection row of %lld elements, expected 2 H K + H V + 2 R + H = %lld", (long long)pr_len,
             (long long)(2 * H * K + H * V + 2 * R + H));
  MM_REQUIRE(pr && conv_w && conv_cache && f_b && g_b && A_log && dt_bias && state && o_norm && y,
             "kda_decode_step: null pointer");
  MM_REQUIRE(mm::aligned16(f_b) && mm::aligned16(g_b) && mm::aligned16(state),
             "kda_decode_step: f_b, g_b and state must be 16-byte aligned");
  KdaStepArgs a;
  for (int i = 0; i < 3; ++i) {
    MM_REQUIRE(conv_w[i] && conv_cache[i] && (reinterpret_cast<uintptr_t>(conv_w[i]) & 7) == 0 &&
                   (reinterpret_cast<uintptr_t>(conv_cache[i]) & 7) == 0,
               "kda_decode_step: conv weight / cache %d null or not 8-byte aligned", i);
    a.conv_w[i] = static_cast<const uint16_t*>(conv_w[i]);
    a.cache[i] = static_cast<uint16_t*>(conv_cache[i]);
  }
  a.pr = static_cast<const uint16_t*>(pr);
  a.f_b = static_cast<const uint16_t*>(f_b);
  a.g_b = static_cast<const uint16_t*>(g_b);
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.lower_bound = lower_bound;
  a.scale = scale;
  a.state = state;
  a.o_norm = static_cast<const uint16_t*>(o_norm);
  a.eps = eps;
  a.y = static_cast<uint16_t*>(y);
  a.H = static_cast<int>(H);
  a.V = static_cast<int>(V);
  a.R = static_cast<int>(R);
  hipStream_t st = MM_STREAM(stream);
  const dim3 grid(static_cast<unsigned>(H * (1 + kKdaHelpers))), block(kKdaThreads);
  if (V <= 128) hipLaunchKernelGGL(kda_token_kernel<1>, grid, block, 0, st, a);
  else if (V <= 256) hipLaunchKernelGGL(kda_token_kernel<2>, grid, block, 0, st, a);
  else hipLaunchKernelGGL(kda_token_kernel<4>, grid, block, 0, st, a);
  return mm::check_launch("kda_decode_step");
}

extern "C" int64_t mm_mla_attn_workspace(int nh, int dv, int64_t max_len) {
  if (nh < 1 || dv < 1 || max_len < 1) return 0;
  return static_cast<int64_t>(nh) * ((max_len + kMlaChunk - 1) / kMlaChunk) * (dv + 2) * 4;
}

extern "C" int mm_mla_decode_attn(const void* q, const void* k_new, const void* v_new, int nh, int dqk, int dv,
                                  void* k_cache, void* v_cache, int64_t max_len, const void* pos, int pos_dtype,
                                  float scale, void* out, void* workspace, int64_t workspace_bytes, void* stream) {
  MM_REQUIRE(nh >= 1 && nh <= 65535 && max_len >= 1 && max_len <= (1LL << 24), "mla_decode_attn: bad nh or max_len");
  MM_REQUIRE(dqk % 8 == 0 && dqk >= 8 && dqk <= 512, "mla_decode_attn: dqk=%d must be a multiple of 8 in [8, 512]",
             dqk);
  MM_REQUIRE(dv % 8 == 0 && dv >= 8 && dv <= 256, "mla_decode_attn: dv=%d must be a multiple of 8 in [8, 256]", dv);
  MM_REQUIRE(pos_dtype == MM_INT64 || pos_dtype == MM_INT32, "mla_decode_attn: pos must be int64 or int32");
  MM_REQUIRE(q && k_new && v_new && k_cache && v_cache && pos && out && workspace, "mla_decode_attn: null pointer");
  MM_REQUIRE(mm::aligned16(q) && mm::aligned16(k_new) && mm::aligned16(v_new) && mm::aligned16(k_cache) &&
                 mm::aligned16(v_cache) && mm::aligned16(workspace),
             "mla_decode_attn: q, k_new, v_new, the caches and the workspace must be 16-byte aligned");
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
  const int kp = (dqk / 8 + 7) / 8;  // 16-byte pieces of a k row per lane, 8 lanes per position
  if (dv <= 128) {
    if (kp <= 1) hipLaunchKernelGGL((mla_split_kernel<1, 16>), grid, dim3(256), 0, st, a);
    else if (kp <= 2) hipLaunchKernelGGL((mla_split_kernel<2, 16>), grid, dim3(256), 0, st, a);
    else if (kp <= 4) hipLaunchKernelGGL((mla_split_kernel<4, 16>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((mla_split_kernel<8, 16>), grid, dim3(256), 0, st, a);
  } else {
    if (kp <= 2) hipLaunchKernelGGL((mla_split_kernel<2, 32>), grid, dim3(256), 0, st, a);
    else if (kp <= 4) hipLaunchKernelGGL((mla_split_kernel<4, 32>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((mla_split_kernel<8, 32>), grid, dim3(256), 0, st, a);
  }
  int rc = mm::check_launch("mla_decode_attn split");
  if (rc) return rc;
  if (dv <= 64) hipLaunchKernelGGL(mla_merge_kernel<1>, dim3(static_cast<unsigned>(nh)), dim3(256), 0, st, a);
  else if (dv <= 128) hipLaunchKernelGGL(mla_merge_kernel<2>, dim3(static_cast<unsigned>(nh)), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(mla_merge_kernel<4>, dim3(static_cast<unsigned>(nh)), dim3(256), 0, st, a);
  return mm::check_launch("mla_decode_attn merge");
}

extern "C" int mm_mla_prefill_attn(const void* q, int64_t q_ts, const void* k_new, int64_t k_ts, const void* v_new,
                                   int64_t v_ts, int64_t T, int nh, int dqk, int dv, void* k_cache, void* v_cache,
                                   int64_t max_len, const void* pos, int pos_dtype, float scale, void* out,
                                   int64_t out_ts, void* stream) {
  MM_REQUIRE(T >= 0 && T <= (1 << 20), "mla_prefill_attn: bad T=%lld", (long long)T);
  MM_REQUIRE(nh >= 1 && nh <= 65535 && max_len >= 1 && max_len <= (1LL << 24), "mla_prefill_attn: bad nh or max_len");
  MM_REQUIRE(dqk % 8 == 0 && dqk >= 8 && dqk <= 256, "mla_prefill_attn: dqk=%d must be a multiple of 8 in [8, 256]",
             dqk);
  MM_REQUIRE(dv % 8 == 0 && dv >= 8 && dv <= 128, "mla_prefill_attn: dv=%d must be a multiple of 8 in [8, 128]", dv);
  MM_REQUIRE(pos_dtype == MM_INT64 || pos_dtype == MM_INT32, "mla_prefill_attn: pos must be int64 or int32");
  MM_REQUIRE(q && k_new && v_new && k_cache && v_cache && pos && out, "mla_prefill_attn: null pointer");
  MM_REQUIRE(q_ts >= static_cast<int64_t>(nh) * dqk && k_ts >= static_cast<int64_t>(nh) * dqk &&
                 v_ts >= static_cast<int64_t>(nh) * dv && out_ts >= static_cast<int64_t>(nh) * dv,
             "mla_prefill_attn: token strides smaller than a token's heads");
  MM_REQUIRE(q_ts % 8 == 0 && k_ts % 8 == 0 && v_ts % 8 == 0 && out_ts % 4 == 0,
             "mla_prefill_attn: token strides must keep rows 16-byte aligned (8-byte for out)");
  MM_REQUIRE(mm::aligned16(q) && mm::aligned16(k_new) && mm::aligned16(v_new) && mm::aligned16(k_cache) &&
                 mm::aligned16(v_cache) && (reinterpret_cast<uintptr_t>(out) & 7) == 0,
             "mla_prefill_attn: q, k_new, v_new and the caches must be 16-byte aligned, out 8-byte aligned");
  if (T == 0) return MM_OK;
  MlaPrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.q_ts = q_ts;
  a.k_ts = k_ts;
  a.v_ts = v_ts;
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.pos = pos;
  a.pos_dtype = pos_dtype;
  a.T = static_cast<int>(T);
  a.nh = nh;
  a.dqk = dqk;
  a.dv = dv;
  a.max_len = max_len;
  a.scale = scale;
  a.out = static_cast<uint16_t*>(out);
  a.out_ts = out_ts;
  hipStream_t st = MM_STREAM(stream);
  hipLaunchKernelGGL(mla_prefill_store_kernel, dim3(static_cast<unsigned>(T), static_cast<unsigned>(nh)), dim3(kWave),
                     0, st, a);
  int rc = mm::check_launch("mla_prefill_attn store");
  if (rc) return rc;
  const dim3 grid(static_cast<unsigned>((T + 15) / 16), static_cast<unsigned>(nh));
  // fewer workgroups than two per CU: 8 waves each, so that each wave walks half as many key tiles
  const bool wide = static_cast<int64_t>(grid.x) * grid.y < 2 * mm::cu_count();
  if (dv <= 64) {
    if (wide) hipLaunchKernelGGL((mla_prefill_attn_kernel<4, 8>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((mla_prefill_attn_kernel<4, 4>), grid, dim3(256), 0, st, a);
  } else {
    if (wide) hipLaunchKernelGGL((mla_prefill_attn_kernel<8, 8>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((mla_prefill_attn_kernel<8, 4>), grid, dim3(256), 0, st, a);
  }
  return mm::check_launch("mla_prefill_attn");
}
