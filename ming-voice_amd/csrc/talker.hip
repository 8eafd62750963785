// The Talker's three small kernels (fast_talker.py): interleaved-rotary attention over 2-3 tokens per
// (batch, head) for the DiT and aggregator blocks, single-token GQA decode attention over the Qwen2 KV
// cache, and the SiLU-gated product of the Qwen2 MLP. All three are latency-bound: a few KB to a few
// hundred KB per call. The decode attention spreads the cached positions over many workgroups (64
// positions each, QK^T on bf16 MFMA) and merges their partial softmax states in a second small kernel,
// so a long prefix is read by many CUs at once instead of one program per head walking it serially; both
// kernels issue their loads before the position arrives, so each costs about one memory round trip.
#include "mm_common.h"

namespace {

using namespace mmd;

// ----------------------------------------------------------------------------------------- rope_attn

constexpr int kRopeMaxS = 8;
constexpr int kRopeMaxHd = 256;

// One wave per (batch, head); lane d (+64 t) owns element d of every row. The pair partner of element d
// is d ^ 1, which is lane ^ 1 of the same t because 64 is even.
// fast_talker.py:34-69: x' = (xe cos - xo sin, xo cos + xe sin) rounded to bf16 for q and k; softmax of
// scale * q'.k' over the S keys; p rounded to bf16; out = p . v rounded to bf16.
template <int SP, int NT>
__global__ __launch_bounds__(64) void rope_attn_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ cs,
                                                       const float* __restrict__ sn, uint16_t* __restrict__ out,
                                                       int S, int H, int D, int HD, float scale) {
  const int lane = lane_id();
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int P = HD / 2;
  float q2[SP][NT], k2[SP][NT], v[SP][NT];
#pragma unroll
  for (int s = 0; s < SP; ++s) {
    const uint16_t* row = qkv + (static_cast<int64_t>(b) * S + s) * 3 * D + static_cast<int64_t>(h) * HD;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d = lane + 64 * t;
      const bool ok = s < S && d < HD;
      const float q = ok ? bf16_to_f32(row[d]) : 0.f;
      const float k = ok ? bf16_to_f32(row[D + d]) : 0.f;
      v[s][t] = ok ? bf16_to_f32(row[2 * D + d]) : 0.f;
      const float c = ok ? cs[s * P + (d >> 1)] : 1.f;
      const float si = ok ? sn[s * P + (d >> 1)] : 0.f;
      const float qp = __shfl_xor(q, 1, kWave), kp = __shfl_xor(k, 1, kWave);
      const float sg = (d & 1) ? si : -si;  // even: x cos - partner sin; odd: x cos + partner sin
      q2[s][t] = round_bf16(fmaf(qp, sg, q * c));
      k2[s][t] = round_bf16(fmaf(kp, sg, k * c));
    }
  }
  float o[SP][NT];
#pragma unroll
  for (int i = 0; i < SP; ++i) {
    float sc[SP];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < SP; ++j) {
      float part = 0.f;
#pragma unroll
      for (int t = 0; t < NT; ++t) part = fmaf(q2[i][t], k2[j][t], part);
      sc[j] = j < S ? wave_sum(part) * scale : -INFINITY;
      mx = fmaxf(mx, sc[j]);
    }
    float den = 0.f;
#pragma unroll
    for (int j = 0; j < SP; ++j) {
      sc[j] = __expf(sc[j] - mx);
      den += sc[j];
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) o[i][t] = 0.f;
#pragma unroll
    for (int j = 0; j < SP; ++j) {
      const float p = round_bf16(sc[j] / den);
#pragma unroll
      for (int t = 0; t < NT; ++t) o[i][t] = fmaf(p, v[j][t], o[i][t]);
    }
  }
#pragma unroll
  for (int s = 0; s < SP; ++s) {
    uint16_t* orow = out + (static_cast<int64_t>(b) * S + s) * D + static_cast<int64_t>(h) * HD;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d = lane + 64 * t;
      if (s < S && d < HD) orow[d] = f32_to_bf16(o[s][t]);
    }
  }
}

template <int SP>
int launch_rope(int nt, dim3 grid, hipStream_t st, const uint16_t* qkv, const float* cs, const float* sn,
                uint16_t* out, int S, int H, int D, int HD, float scale) {
  if (nt == 1)
    hipLaunchKernelGGL((rope_attn_kernel<SP, 1>), grid, dim3(64), 0, st, qkv, cs, sn, out, S, H, D, HD, scale);
  else if (nt == 2)
    hipLaunchKernelGGL((rope_attn_kernel<SP, 2>), grid, dim3(64), 0, st, qkv, cs, sn, out, S, H, D, HD, scale);
  else
    hipLaunchKernelGGL((rope_attn_kernel<SP, 4>), grid, dim3(64), 0, st, qkv, cs, sn, out, S, H, D, HD, scale);
  return mm::check_launch("rope_attn");
}

// ------------------------------------------------------------------------------------- decode attention

constexpr int kTile = 16;                 // cached positions per MFMA tile
constexpr int kTilesPerChunk = 4;
constexpr int kChunk = kTile * kTilesPerChunk;  // positions per split workgroup
constexpr int kAttnMaxHd = 256;
constexpr int kMaxGroup = 16;             // query heads per KV head (rows of one MFMA tile)
constexpr int kMaxChunks = 1024;          // max_len <= 65536

struct AttnArgs {
  const uint16_t* qkv;
  uint16_t* kc;
  uint16_t* vc;
  const void* pos;
  int pos_dtype;
  const float* inv_freq;
  int64_t max_len;
  int nh, nkv, hd, nc;
  float scale;
  float* ws_m;    // [nh, nc] running max of each chunk
  float* ws_l;    // [nh, nc] softmax denominator relative to that max
  float* ws_acc;  // [nh, nc, hd] unnormalised p . V relative to that max
  uint16_t* out;
};

__device__ __forceinline__ int64_t load_pos(const AttnArgs& a) {
  return a.pos_dtype == MM_INT64 ? *static_cast<const int64_t*>(a.pos) : *static_cast<const int32_t*>(a.pos);
}

__device__ __forceinline__ float group16_max(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  return fmaxf(v, dpp_f32<kDppMirror>(v));
}

// Rotary of 8 consecutive elements d0..d0+7 of one head (rotate-half form, fast_talker.py:176-187):
// x'[d] = bf16(x[d] c[d] + sign(d) x[(d + hd/2) % hd] s[d]), sign -1 below hd/2; xv holds x[d0..d0+7], pv the
// partners x[(d0 + hd/2) % hd ..]; c, s are the bf16-rounded cos / sin of pos * inv_freq[d % (hd/2)] in LDS.
__device__ __forceinline__ bf16x8_t rotate8(uint4 xv, uint4 pv, int d0, int half, const float* lc, const float* ls) {
  const int fi = d0 % half;
  const float sgn = d0 < half ? -1.f : 1.f;
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, pw[4] = {pv.x, pv.y, pv.z, pv.w};
  uint32_t r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x0 = __uint_as_float(xw[i] << 16), x1 = __uint_as_float(xw[i] & 0xffff0000u);
    const float p0 = __uint_as_float(pw[i] << 16), p1 = __uint_as_float(pw[i] & 0xffff0000u);
    const float y0 = fmaf(sgn * p0, ls[fi + 2 * i], x0 * lc[fi + 2 * i]);
    const float y1 = fmaf(sgn * p1, ls[fi + 2 * i + 1], x1 * lc[fi + 2 * i + 1]);
    r[i] = static_cast<uint32_t>(f32_to_bf16(y0)) | (static_cast<uint32_t>(f32_to_bf16(y1)) << 16);
  }
  return __builtin_bit_cast(bf16x8_t, make_uint4(r[0], r[1], r[2], r[3]));
}

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Split phase: workgroup (chunk c, KV head kvh) covers positions [64c, 64c + 64) with 4 waves, one 16-position
// tile each. The kernel is latency-bound, so every global load that does not need pos (the K / V rows of the
// tile, clamped to the cache, and this token's q / k / v) is issued before pos arrives, unconditionally; rows
// that turn out to lie beyond pos are discarded by selects. The current position's k / v come from qkv
// (rotated here); the wave whose tile holds pos also writes them into the cache at pos
// (fast_talker.py:191-193). No workgroup reads cache row pos, so the write does not race with the reads.
// Scores: one 16x16x32 bf16 MFMA per 32 head dims, rows = the G query heads of the group, columns = the tile's
// positions. p . V runs on the VALU with lane = head dim, in fp32 like the reference (fast_talker.py:199-211).
// The 4 waves' softmax states are merged in LDS into the chunk's (m, l, acc), written to the workspace.
// Chunks wholly beyond pos write nothing; the merge kernel never uses them.
template <int NDV, int G4>
__global__ __launch_bounds__(256) void decode_attn_split_kernel(AttnArgs a) {
  constexpr int KSM = 2 * NDV;  // max 32-wide k steps (hd <= 64 * NDV)
  constexpr int kWaves = kTilesPerChunk;
  constexpr int GP = 4 * G4;    // query heads of the group, padded to a multiple of 4
  __shared__ __align__(16) float lc[kAttnMaxHd / 2];
  __shared__ __align__(16) float ls[kAttnMaxHd / 2];
  __shared__ __align__(16) float lp[kWaves][kTile * kMaxGroup];  // p[position][head] per wave
  __shared__ float lm[kWaves][kMaxGroup], ll[kWaves][kMaxGroup];
  __shared__ __align__(16) float lacc[kWaves - 1][GP * 64 * NDV];  // waves 1..3: acc[head][d]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = blockIdx.x, kvh = blockIdx.y;
  const int hd = a.hd, half = hd / 2, ks_n = hd / 32, G = a.nh / a.nkv;
  const int r = lane & 15, q4 = lane >> 4;
  const int64_t c0 = static_cast<int64_t>(c) * kChunk, t0 = c0 + wave * kTile, last = a.max_len - 1;
  const uint16_t* kcache = a.kc + static_cast<int64_t>(kvh) * a.max_len * hd;
  const uint16_t* vcache = a.vc + static_cast<int64_t>(kvh) * a.max_len * hd;
  const uint16_t* qrow = a.qkv + static_cast<int64_t>(kvh * G + min(r, G - 1)) * hd;
  const uint16_t* krow_new = a.qkv + static_cast<int64_t>(a.nh + kvh) * hd;
  const uint16_t* vrow_new = a.qkv + static_cast<int64_t>(a.nh + a.nkv + kvh) * hd;

  // ---- loads that do not depend on pos (all unconditional, addresses clamped into the buffers)
  const float invf = a.inv_freq[min(tid, half - 1)];
  const int64_t krow = min(t0 + r, last);
  uint4 kb[KSM], qx[KSM], qp[KSM], kx[KSM], kp[KSM], vx[KSM];
#pragma unroll
  for (int ks = 0; ks < KSM; ++ks) {
    const int d0 = min(32 * ks, hd - 32) + 8 * q4, pd0 = (d0 + half) % hd;
    kb[ks] = ld16(kcache + krow * hd + d0);
    qx[ks] = ld16(qrow + d0);
    qp[ks] = ld16(qrow + pd0);
    kx[ks] = ld16(krow_new + d0);
    kp[ks] = ld16(krow_new + pd0);
    vx[ks] = ld16(vrow_new + d0);
  }
  uint16_t vraw[kTile][NDV];
#pragma unroll
  for (int tt = 0; tt < kTile; ++tt) {
    const int64_t row = min(t0 + tt, last);
#pragma unroll
    for (int j = 0; j < NDV; ++j) vraw[tt][j] = vcache[row * hd + min(lane + 64 * j, hd - 1)];
  }
  float vcur[NDV];
#pragma unroll
  for (int j = 0; j < NDV; ++j) vcur[j] = bf16_to_f32(vrow_new[min(lane + 64 * j, hd - 1)]);
  // pos is a scalar load: issued after the vector loads, or its wait would hold them back
  __builtin_amdgcn_sched_barrier(0);
  const int64_t pos = load_pos(a);

  // ---- pos-dependent part. The exit test comes after the barrier: a branch before it would let the compiler
  // sink the loads above into the live path, behind the wait for pos.
  const bool live = pos >= 0 && pos < a.max_len && c0 <= pos;
  if (tid < half) {
    float s, co;
    sincosf(static_cast<float>(live ? pos : 0) * invf, &s, &co);
    lc[tid] = round_bf16(co);
    ls[tid] = round_bf16(s);
  }
  __syncthreads();
  if (!live) return;  // uniform across the workgroup
  bf16x8_t qa[KSM], kcur[KSM];
#pragma unroll
  for (int ks = 0; ks < KSM; ++ks) {
    const int d0 = min(32 * ks, hd - 32) + 8 * q4;
    const bf16x8_t qr = rotate8(qx[ks], qp[ks], d0, half, lc, ls);
    qa[ks] = r < G ? qr : bf16x8_t{};
    kcur[ks] = rotate8(kx[ks], kp[ks], d0, half, lc, ls);
  }
  if (pos >= t0 && pos < t0 + kTile && r == 0) {  // this wave's tile holds pos: write the new cache row
    uint16_t* kdst = a.kc + (static_cast<int64_t>(kvh) * a.max_len + pos) * hd;
    uint16_t* vdst = a.vc + (static_cast<int64_t>(kvh) * a.max_len + pos) * hd;
#pragma unroll
    for (int ks = 0; ks < KSM; ++ks) {
      if (ks < ks_n) {
        const int d0 = 32 * ks + 8 * q4;
        *reinterpret_cast<uint4*>(kdst + d0) = __builtin_bit_cast(uint4, kcur[ks]);
        *reinterpret_cast<uint4*>(vdst + d0) = vx[ks];
      }
    }
  }
  floatx4 s4 = {0.f, 0.f, 0.f, 0.f};
  const bool cached = t0 + r < pos;
#pragma unroll
  for (int ks = 0; ks < KSM; ++ks)
    if (ks < ks_n) s4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], cached ? __builtin_bit_cast(bf16x8_t, kb[ks]) : kcur[ks], s4, 0, 0, 0);
  // s4[v]: head 4 * q4 + v, position t0 + r
  const bool valid = t0 + r <= pos;
  float p[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float sc = valid ? s4[v] * a.scale : -INFINITY;
    const float m = group16_max(sc);  // -inf only when the whole tile lies beyond pos
    p[v] = valid ? __expf(sc - m) : 0.f;
    const float l = group_sum<16>(p[v]);
    if (r == 0) {
      lm[wave][4 * q4 + v] = m;
      ll[wave][4 * q4 + v] = l;
    }
  }
  *reinterpret_cast<float4*>(&lp[wave][r * kMaxGroup + 4 * q4]) = make_float4(p[0], p[1], p[2], p[3]);
  __syncthreads();
  // p . V with lane = head dim; the padded heads (G..GP-1) compute harmless values that are never stored
  float acc[GP][NDV];
#pragma unroll
  for (int g = 0; g < GP; ++g)
#pragma unroll
    for (int j = 0; j < NDV; ++j) acc[g][j] = 0.f;
#pragma unroll
  for (int tt = 0; tt < kTile; ++tt) {
    float vt[NDV];
#pragma unroll
    for (int j = 0; j < NDV; ++j) vt[j] = t0 + tt < pos ? bf16_to_f32(vraw[tt][j]) : t0 + tt == pos ? vcur[j] : 0.f;
#pragma unroll
    for (int g4 = 0; g4 < G4; ++g4) {
      const float4 pp = *reinterpret_cast<const float4*>(&lp[wave][tt * kMaxGroup + 4 * g4]);
      const float pg[4] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < NDV; ++j) acc[4 * g4 + u][j] = fmaf(pg[u], vt[j], acc[4 * g4 + u][j]);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int g = 0; g < GP; ++g)
#pragma unroll
      for (int j = 0; j < NDV; ++j) lacc[wave - 1][g * 64 * NDV + lane + 64 * j] = acc[g][j];
  }
  __syncthreads();
  if (wave != 0) return;
  // wave 0 holds position c0 <= pos, so its max is finite and so is the chunk's
  const int64_t hbase = static_cast<int64_t>(kvh) * G;
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    const float m = fmaxf(fmaxf(lm[0][g], lm[1][g]), fmaxf(lm[2][g], lm[3][g]));
    float w[kWaves];
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) w[wv] = lm[wv][g] == -INFINITY ? 0.f : __expf(lm[wv][g] - m);
    float s[NDV];
#pragma unroll
    for (int j = 0; j < NDV; ++j) {
      s[j] = acc[g][j] * w[0];
#pragma unroll
      for (int wv = 1; wv < kWaves; ++wv) s[j] = fmaf(lacc[wv - 1][g * 64 * NDV + lane + 64 * j], w[wv], s[j]);
    }
    if (g < G) {
      float* dst = a.ws_acc + ((hbase + g) * a.nc + c) * hd;
#pragma unroll
      for (int j = 0; j < NDV; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) dst[d] = s[j];
      }
      if (lane == 0) {
        a.ws_m[(hbase + g) * a.nc + c] = m;
        a.ws_l[(hbase + g) * a.nc + c] = ((ll[0][g] * w[0] + ll[1][g] * w[1]) + ll[2][g] * w[2]) + ll[3][g] * w[3];
      }
    }
  }
}

// Merge phase: one wave per query head merges the states of chunks 0 .. pos/64:
// M = max m_c, w_c = exp(m_c - M), out = bf16(sum_c w_c acc_c / sum_c w_c l_c). The workspace is read for
// every chunk before pos arrives; chunks beyond pos (not written by this call) are dropped by selects.
// An out-of-range pos (outside [0, max_len)) leaves the cache untouched and makes the output NaN.
template <int NDV>
__global__ __launch_bounds__(64) void decode_attn_merge_kernel(AttnArgs a) {
  constexpr int kBatch = 16;
  __shared__ float lw[kMaxChunks];
  const int lane = lane_id(), h = blockIdx.x, hd = a.hd, nc = a.nc;
  const float* wm = a.ws_m + static_cast<int64_t>(h) * nc;
  const float* wl = a.ws_l + static_cast<int64_t>(h) * nc;
  const float* wa = a.ws_acc + static_cast<int64_t>(h) * nc * hd;
  // first batch of partial sums, loaded before pos is known
  float first[kBatch][NDV];
#pragma unroll
  for (int c = 0; c < kBatch; ++c)
#pragma unroll
    for (int j = 0; j < NDV; ++j) first[c][j] = wa[static_cast<int64_t>(min(c, nc - 1)) * hd + min(lane + 64 * j, hd - 1)];
  float m0 = wm[min(lane, nc - 1)], l0 = wl[min(lane, nc - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const int64_t pos = load_pos(a);
  uint16_t* o = a.out + static_cast<int64_t>(h) * hd;
  // no branch on pos before the arithmetic (it would let the loads above sink behind the wait for pos)
  const bool bad = pos < 0 || pos >= a.max_len;
  const int nv = static_cast<int>((bad ? 0 : pos) / kChunk) + 1;
  float mx = lane < nv ? m0 : -INFINITY;
  for (int c = lane + kWave; c < nv; c += kWave) mx = fmaxf(mx, wm[c]);
  mx = wave_max(mx);
  float den = 0.f;
  if (lane < nv) {
    const float w = __expf(m0 - mx);
    lw[lane] = w;
    den = l0 * w;
  }
  for (int c = lane + kWave; c < nv; c += kWave) {
    const float w = __expf(wm[c] - mx);
    lw[c] = w;
    den = fmaf(wl[c], w, den);
  }
  den = wave_sum(den);
  __syncthreads();
  float s[NDV];
#pragma unroll
  for (int j = 0; j < NDV; ++j) s[j] = 0.f;
#pragma unroll
  for (int c = 0; c < kBatch; ++c)
#pragma unroll
    for (int j = 0; j < NDV; ++j) s[j] = c < nv ? fmaf(first[c][j], lw[c], s[j]) : s[j];
  for (int c = kBatch; c < nv; ++c)
#pragma unroll
    for (int j = 0; j < NDV; ++j) s[j] = fmaf(wa[static_cast<int64_t>(c) * hd + min(lane + 64 * j, hd - 1)], lw[c], s[j]);
#pragma unroll
  for (int j = 0; j < NDV; ++j) {
    const int d = lane + 64 * j;
    if (d < hd) o[d] = bad ? static_cast<uint16_t>(0x7fc0) : f32_to_bf16(s[j] / den);  // 0x7fc0: bf16 quiet NaN
  }
}

int64_t attn_chunks(int64_t max_len) { return (max_len + kChunk - 1) / kChunk; }

template <int NDV, int G4>
void launch_split(const AttnArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((decode_attn_split_kernel<NDV, G4>), dim3(static_cast<unsigned>(a.nc), static_cast<unsigned>(a.nkv)),
                     dim3(64 * kTilesPerChunk), 0, st, a);
}

template <int NDV>
int launch_decode(const AttnArgs& a, hipStream_t st) {
  const int g4 = (a.nh / a.nkv + 3) / 4;
  if (g4 == 1) launch_split<NDV, 1>(a, st);
  else if (g4 == 2) launch_split<NDV, 2>(a, st);
  else if (g4 == 3) launch_split<NDV, 3>(a, st);
  else launch_split<NDV, 4>(a, st);
  int rc = mm::check_launch("qwen_decode_attn split");
  if (rc) return rc;
  hipLaunchKernelGGL(decode_attn_merge_kernel<NDV>, dim3(static_cast<unsigned>(a.nh)), dim3(64), 0, st, a);
  return mm::check_launch("qwen_decode_attn merge");
}

// ------------------------------------------------------------------------------------------ silu_mul

// out = bf16(bf16(silu(g)) * u) for gu = [g | u] rows (fast_talker.py:215-222); 8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(const uint16_t* __restrict__ gu, int64_t gs, int64_t I,
                                                           uint16_t* __restrict__ out, int64_t os) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c * 8 >= I) return;
  const uint16_t* row = gu + blockIdx.y * gs;
  const uint4 gv = *reinterpret_cast<const uint4*>(row + c * 8);
  const uint4 uv = *reinterpret_cast<const uint4*>(row + I + c * 8);
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float g0 = round_bf16(silu(__uint_as_float(gw[i] << 16)));
    const float g1 = round_bf16(silu(__uint_as_float(gw[i] & 0xffff0000u)));
    const float y0 = g0 * __uint_as_float(uw[i] << 16), y1 = g1 * __uint_as_float(uw[i] & 0xffff0000u);
    r[i] = static_cast<uint32_t>(f32_to_bf16(y0)) | (static_cast<uint32_t>(f32_to_bf16(y1)) << 16);
  }
  *reinterpret_cast<uint4*>(out + blockIdx.y * os + c * 8) = make_uint4(r[0], r[1], r[2], r[3]);
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t gs, int64_t I,
                                                       uint16_t* __restrict__ out, int64_t os) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= I) return;
  const uint16_t* row = gu + blockIdx.y * gs;
  const float g = round_bf16(silu(bf16_to_f32(row[i])));
  out[blockIdx.y * os + i] = f32_to_bf16(g * bf16_to_f32(row[I + i]));
}

// ------------------------------------------------------------------------------------------ CFG update

// y_out = bf16(y + bf16(bf16(pred + bf16(bf16(pred - null) * cfg)) * dt)): the bf16 torch expression
// y + (pred + (pred - null) * cfg) * dt (fast_talker.py:151-152), one rounding per operation.
__global__ __launch_bounds__(256) void cfg_update_kernel(const uint16_t* __restrict__ y, const uint16_t* __restrict__ pn,
                                                         int64_t ps, int64_t n, float cfg, const void* __restrict__ dt,
                                                         int dt_dtype, uint16_t* y_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float d = dt_dtype == MM_FP32 ? *static_cast<const float*>(dt) : bf16_to_f32(*static_cast<const uint16_t*>(dt));
  const float pred = bf16_to_f32(pn[i]), null = bf16_to_f32(pn[ps + i]);
  const float t = round_bf16(round_bf16(pred + round_bf16(round_bf16(pred - null) * cfg)) * d);
  y_out[i] = f32_to_bf16(bf16_to_f32(y[i]) + t);
}

}  // namespace

extern "C" int mm_cfg_update(const void* y, const void* pred_null, int64_t pn_row_stride, int64_t n, float cfg,
                             const void* dt, int dt_dtype, void* y_out, void* stream) {
  MM_REQUIRE(y && pred_null && dt && y_out, "cfg_update: null pointer");
  MM_REQUIRE(n >= 1 && n <= (1LL << 31) && pn_row_stride >= n, "cfg_update: n=%lld, pred/null row stride %lld",
             (long long)n, (long long)pn_row_stride);
  MM_REQUIRE(dt_dtype == MM_BF16 || dt_dtype == MM_FP32, "cfg_update: dt must be bf16 or fp32");
  hipLaunchKernelGGL(cfg_update_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, MM_STREAM(stream),
                     static_cast<const uint16_t*>(y), static_cast<const uint16_t*>(pred_null), pn_row_stride, n, cfg, dt,
                     dt_dtype, static_cast<uint16_t*>(y_out));
  return mm::check_launch("cfg_update");
}

extern "C" int mm_rope_attn(const void* qkv, int64_t batch, int64_t seq, int64_t dim, int heads, const float* cos_t,
                            const float* sin_t, void* out, void* stream) {
  MM_REQUIRE(qkv && cos_t && sin_t && out, "rope_attn: null pointer");
  MM_REQUIRE(batch >= 1 && seq >= 1 && seq <= kRopeMaxS, "rope_attn: batch=%lld, seq=%lld (1..%d) bad shape",
             (long long)batch, (long long)seq, kRopeMaxS);
  MM_REQUIRE(heads >= 1 && dim >= 2 && dim % heads == 0, "rope_attn: dim=%lld not divisible by heads=%d",
             (long long)dim, heads);
  const int64_t hd = dim / heads;
  MM_REQUIRE(hd % 2 == 0 && hd <= kRopeMaxHd, "rope_attn: head dim %lld must be even and <= %d", (long long)hd,
             kRopeMaxHd);
  MM_REQUIRE(batch * heads <= 0x7fffffffLL && batch * seq * 3 * dim < (1LL << 40), "rope_attn: too large");
  const int nt = hd <= 64 ? 1 : hd <= 128 ? 2 : 4;
  const dim3 grid(static_cast<unsigned>(batch * heads));
  hipStream_t st = MM_STREAM(stream);
  auto q = static_cast<const uint16_t*>(qkv);
  auto o = static_cast<uint16_t*>(out);
  const int S = static_cast<int>(seq), D = static_cast<int>(dim), HD = static_cast<int>(hd);
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  if (S <= 2) return launch_rope<2>(nt, grid, st, q, cos_t, sin_t, o, S, heads, D, HD, scale);
  if (S <= 4) return launch_rope<4>(nt, grid, st, q, cos_t, sin_t, o, S, heads, D, HD, scale);
  return launch_rope<8>(nt, grid, st, q, cos_t, sin_t, o, S, heads, D, HD, scale);
}

extern "C" int64_t mm_decode_attn_workspace(int nh, int hd, int64_t max_len) {
  if (nh <= 0 || hd <= 0 || max_len <= 0) return 0;
  return static_cast<int64_t>(nh) * attn_chunks(max_len) * (hd + 2) * static_cast<int64_t>(sizeof(float));
}

extern "C" int mm_qwen_decode_attn(const void* qkv, int nh, int nkv, int hd, void* k_cache, void* v_cache,
                                   int64_t max_len, const void* pos, int pos_dtype, const float* inv_freq,
                                   float scale, void* out, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  MM_REQUIRE(qkv && k_cache && v_cache && pos && inv_freq && out && workspace, "qwen_decode_attn: null pointer");
  MM_REQUIRE(nh >= 1 && nkv >= 1 && nh % nkv == 0 && nh / nkv <= kMaxGroup,
             "qwen_decode_attn: nh=%d, nkv=%d: nh must be a multiple of nkv with at most %d query heads per KV head",
             nh, nkv, kMaxGroup);
  MM_REQUIRE(hd >= 32 && hd <= kAttnMaxHd && hd % 32 == 0, "qwen_decode_attn: head dim %d must be a multiple of 32 "
             "in [32, %d]", hd, kAttnMaxHd);
  MM_REQUIRE(max_len >= 1 && max_len <= static_cast<int64_t>(kMaxChunks) * kChunk,
             "qwen_decode_attn: max_len=%lld must be in [1, %d]", (long long)max_len, kMaxChunks * kChunk);
  MM_REQUIRE(pos_dtype == MM_INT64 || pos_dtype == MM_INT32, "qwen_decode_attn: pos must be int32 or int64");
  MM_REQUIRE(mm::aligned16(qkv) && mm::aligned16(k_cache) && mm::aligned16(v_cache),
             "qwen_decode_attn: qkv and the caches must be 16-byte aligned");
  const int64_t need = mm_decode_attn_workspace(nh, hd, max_len);
  MM_REQUIRE(workspace_bytes >= need && mm::aligned16(workspace),
             "qwen_decode_attn: workspace needs %lld bytes, 16-byte aligned (got %lld)", (long long)need,
             (long long)workspace_bytes);
  const int64_t nc = attn_chunks(max_len);
  float* ws = static_cast<float*>(workspace);
  AttnArgs a{static_cast<const uint16_t*>(qkv), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
             pos, pos_dtype, inv_freq, max_len, nh, nkv, hd, static_cast<int>(nc), scale,
             ws, ws + nh * nc, ws + 2 * nh * nc, static_cast<uint16_t*>(out)};
  hipStream_t st = MM_STREAM(stream);
  const int ndv = (hd + 63) / 64;
  if (ndv == 1) return launch_decode<1>(a, st);
  if (ndv == 2) return launch_decode<2>(a, st);
  if (ndv == 3) return launch_decode<3>(a, st);
  return launch_decode<4>(a, st);
}

extern "C" int mm_silu_mul(const void* gu, int64_t rows, int64_t inter, int64_t gu_row_stride, void* out,
                           int64_t out_row_stride, void* stream) {
  MM_REQUIRE(gu && out, "silu_mul: null pointer");
  MM_REQUIRE(rows >= 1 && rows <= 65535 && inter >= 1, "silu_mul: bad shape rows=%lld inter=%lld", (long long)rows,
             (long long)inter);
  MM_REQUIRE(gu_row_stride >= 2 * inter && out_row_stride >= inter, "silu_mul: row stride too small");
  hipStream_t st = MM_STREAM(stream);
  auto g = static_cast<const uint16_t*>(gu);
  auto o = static_cast<uint16_t*>(out);
  const bool vec = inter % 8 == 0 && gu_row_stride % 8 == 0 && out_row_stride % 8 == 0 && mm::aligned16(gu) &&
                   mm::aligned16(out);
  if (vec) {
    const dim3 grid(static_cast<unsigned>((inter / 8 + 255) / 256), static_cast<unsigned>(rows));
    hipLaunchKernelGGL(silu_mul_vec_kernel, grid, dim3(256), 0, st, g, gu_row_stride, inter, o, out_row_stride);
  } else {
    const dim3 grid(static_cast<unsigned>((inter + 255) / 256), static_cast<unsigned>(rows));
    hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(256), 0, st, g, gu_row_stride, inter, o, out_row_stride);
  }
  return mm::check_launch("silu_mul");
}
