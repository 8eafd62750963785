// Router selection for one token on one wave (fused_ops.py:53-93 and the softmax router of the configs).
// Shared by the router kernels (logits + selection for small batches, selection alone), so every path
// picks identical experts.
#pragma once

#include "mm_common.h"

namespace mmd {

struct SelectParams {
  const float* bias;  // [E] or null
  int E, scoring, n_group, topk_group, top_k;
  float scale;
  int append_shared;
};

// Arg-max over the lane-held slots then across the wave; lowest expert index wins ties. The maximum comes from
// DPP row reductions (wave_max), the index from one ballot per slot: expert e = lane + 64 j, so the lowest index
// holding the maximum lies in the lowest slot j whose ballot is non-empty, at that ballot's lowest set lane. A
// maximum that no lane matches (NaN keys) falls back to the lowest valid slot. Slots past the valid range hold
// -inf and larger indices, so an all -inf input yields the lowest index.
template <int NS>
__device__ __forceinline__ void slots_argmax(const float (&v)[NS], int nslots, float& best, int& bidx) {
  float m = v[0];
#pragma unroll
  for (int j = 1; j < NS; ++j)
    if (j < nslots) m = fmaxf(m, v[j]);
  best = wave_max(m);
  bidx = -1;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (bidx < 0 && j < nslots) {
      const unsigned long long hit = __ballot(v[j] == best);
      if (hit) bidx = __ffsll(static_cast<long long>(hit)) - 1 + kWave * j;
    }
  }
  if (bidx < 0) bidx = 0;
}

// Fast path of select_token for at most 64 experts without group limits: one expert per lane. Each of the top_k
// rounds takes the maximum key of the lanes not yet picked (DPP reductions), then the lowest such lane with a
// ballot, so the picks come in the order of a stable descending sort (value descending, index ascending). Same
// picks, order and arithmetic as the general path.
__device__ __forceinline__ void select_token64(const SelectParams& a, const float* lg, int& id, float& w, bool& has) {
  const int lane = lane_id();
  const int E = a.E;
  const bool valid = lane < E;
  float score = 0.f, key = -INFINITY;
  // the logit and bias of this lane through buffer resources (a null bias has size zero and reads zero), with no
  // branch before the loads: behind the lane and null tests each load was waited on by itself
  const rsrc_t lr = make_rsrc(lg, static_cast<int64_t>(E) * 4), br = make_rsrc(a.bias, a.bias ? E * 4 : 0);
  const uint32_t off = valid ? static_cast<uint32_t>(lane) * 4u : kPast;
  const float l = __uint_as_float(buf4(lr, off)), b = __uint_as_float(buf4(br, off));
  if (valid) {
    if (a.scoring == MM_SCORE_SIGMOID_GROUP) {
      score = 1.0f / (1.0f + __expf(-l));
      key = score + b;
    } else {
      key = l + b;
    }
  }
  if (a.scoring == MM_SCORE_SOFTMAX) {
    const float m = wave_max(key);
    if (valid) score = __expf(key - m);
    const float den = wave_sum(valid ? score : 0.f);
    score = score / den;
  }
  // lane k gathers the k-th pick; the weights' sum runs over the picks in order
  bool taken = !valid;
  float total = 0.f, sel_w = 0.f;
  int sel_e = 0;
  const int sb = __float_as_int(score);
  for (int k = 0; k < a.top_k; ++k) {
    const float m = wave_max(taken ? -INFINITY : key);
    unsigned long long hit = __ballot(!taken && key == m);
    if (!hit) hit = __ballot(!taken);  // NaN keys: the lowest lane not yet picked
    const int src = __ffsll(static_cast<long long>(hit)) - 1;
    const float s = __int_as_float(__builtin_amdgcn_readlane(sb, src));
    total += s;
    if (lane == k) { sel_w = s; sel_e = src; }
    if (lane == src) taken = true;
  }
  has = false;
  w = 0.f;
  id = 0;
  if (lane < a.top_k) {
    w = sel_w / (total + 1e-20f) * a.scale;
    id = sel_e;
    has = true;
  } else if (lane == a.top_k && a.append_shared) {
    w = 1.0f;
    id = E;
    has = true;
  }
}

// Selects the experts of one token from its logits `lg` (whole wave). On return lane k < top_k holds the
// k-th pick (id, weight), lane top_k the shared expert when append_shared; `has` tells which lanes hold
// an entry. rbuf: NS*64 floats of LDS private to this wave.
//   sigmoid: s = sigmoid(l); key = s + bias; group-limited (n_group > 1: groups ranked by the sum of
//            their two largest keys, topk_group kept); top_k by key; w = s / (sum s + 1e-20) * scale
//   softmax: key = l + bias; top_k by key; p = softmax(key); w = p / (sum p_sel + 1e-20) * scale
template <int NS>
__device__ __forceinline__ void select_token(const SelectParams& a, const float* lg, float* rbuf, int& id, float& w,
                                             bool& has) {
  const int lane = lane_id();
  const int E = a.E;
  const int nslots = (E + kWave - 1) / kWave;
  float score[NS], key[NS];  // score: weight source; key: selection value
  // every slot's logit and bias loaded first, with no branch before them (as in select_token64)
  const rsrc_t lr = make_rsrc(lg, static_cast<int64_t>(E) * 4), br = make_rsrc(a.bias, a.bias ? E * 4 : 0);
  float lv[NS], bv[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int e = lane + kWave * j;
    const uint32_t off = j < nslots && e < E ? static_cast<uint32_t>(e) * 4u : kPast;
    lv[j] = __uint_as_float(buf4(lr, off));
    bv[j] = __uint_as_float(buf4(br, off));
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int e = lane + kWave * j;
    score[j] = 0.f;
    key[j] = -INFINITY;
    if (j < nslots && e < E) {
      const float l = lv[j];
      const float b = bv[j];
      if (a.scoring == MM_SCORE_SIGMOID_GROUP) {
        score[j] = 1.0f / (1.0f + __expf(-l));
        key[j] = score[j] + b;
      } else {
        key[j] = l + b;
      }
    }
  }
  if (a.scoring == MM_SCORE_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NS; ++j) m = fmaxf(m, key[j]);
    m = wave_max(m);
    float den = 0.f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int e = lane + kWave * j;
      if (j < nslots && e < E) {
        score[j] = __expf(key[j] - m);
        den += score[j];
      }
    }
    den = wave_sum(den);
#pragma unroll
    for (int j = 0; j < NS; ++j) score[j] = score[j] / den;
  } else if (a.n_group > 1) {
    // group score = sum of the two largest keys of the group (first max excluded once)
    const int G = a.n_group, GS = E / G;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int e = lane + kWave * j;
      if (j < nslots && e < E) rbuf[e] = key[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float gscore[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int g = lane + kWave * j;
      gscore[j] = -INFINITY;
      if (g < G) {
        float m1 = -INFINITY;
        int a1 = 0;
        for (int i = 0; i < GS; ++i) {
          const float v = rbuf[g * GS + i];
          if (v > m1 || i == 0) { m1 = v; a1 = i; }
        }
        float m2 = -INFINITY;
        for (int i = 0; i < GS; ++i)
          if (i != a1) m2 = fmaxf(m2, rbuf[g * GS + i]);
        gscore[j] = m1 + m2;
      }
    }
    // keep the topk_group best groups (iterative arg-max, lowest group index on ties)
    bool keep[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) keep[j] = false;
    for (int it = 0; it < a.topk_group; ++it) {
      float bv;
      int bi;
      slots_argmax(gscore, NS, bv, bi);
#pragma unroll
      for (int j = 0; j < NS; ++j)
        if (lane + kWave * j == bi) { keep[j] = true; gscore[j] = -INFINITY; }
    }
    // broadcast the kept-group flags through LDS and mask the keys of dropped groups
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int g = lane + kWave * j;
      if (g < G) rbuf[g] = keep[j] ? 1.f : 0.f;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int e = lane + kWave * j;
      if (j < nslots && e < E && rbuf[e / GS] == 0.f) key[j] = -INFINITY;
    }
    __builtin_amdgcn_wave_barrier();  // rbuf may be reused by the caller
  }
  // top_k by iterative arg-max on the keys; weights come from the scores
  float sel_w = 0.f;  // lane k holds the score of the k-th pick
  int sel_e = 0;
  float total = 0.f;
  for (int k = 0; k < a.top_k; ++k) {
    float bv;
    int bi;
    slots_argmax(key, nslots, bv, bi);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NS; ++j)
      if (lane + kWave * j == bi) { s = score[j]; key[j] = -INFINITY; }
    s = wave_sum(s);  // exactly one lane contributes
    total += s;
    if (lane == k) { sel_w = s; sel_e = bi; }
  }
  has = false;
  w = 0.f;
  id = 0;
  if (lane < a.top_k) {
    w = sel_w / (total + 1e-20f) * a.scale;
    id = sel_e;
    has = true;
  } else if (lane == a.top_k && a.append_shared) {
    w = 1.0f;
    id = E;
    has = true;
  }
}

// Selection entry used by every kernel: the one-expert-per-lane path when it applies, else the general one.
template <int NS>
__device__ __forceinline__ void select_any(const SelectParams& a, const float* lg, float* rbuf, int& id, float& w,
                                           bool& has) {
  if (a.E <= kWave && a.n_group <= 1) select_token64(a, lg, id, w, has);
  else select_token<NS>(a, lg, rbuf, id, w, has);
}

// Slots per lane (NS) needed for E experts and G groups.
inline int select_slots(int64_t E, int64_t G) {
  const int64_t need = E > G ? E : G;
  return need <= 64 ? 1 : need <= 128 ? 2 : need <= 256 ? 4 : 16;
}

// Sum of squares of elements 8c .. 8c+7 (those below n) of a row, added to ss in element order.
template <class TX>
__device__ __forceinline__ float chunk_ss(const typename TX::T* xr, int64_t c, int64_t n, float ss) {
  const int64_t i0 = c * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i0 + i < n) {
      const float v = TX::ld(xr, i0 + i);
      ss = fmaf(v, v, ss);
    }
  }
  return ss;
}

// The same for a whole, 16-byte aligned chunk of bf16 (one load, same order).
__device__ __forceinline__ float chunk_ss_bf16x8(const uint4& v, float ss) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = __uint_as_float(w[i] << 16), hi = __uint_as_float(w[i] & 0xffff0000u);
    ss = fmaf(lo, lo, ss);
    ss = fmaf(hi, hi, ss);
  }
  return ss;
}

// Whether rows of TX at xr with n elements (row stride xs) can be read in whole aligned bf16 chunks.
template <class TX>
__device__ __forceinline__ bool rows_bf16x8(const typename TX::T* xr, int64_t n, int64_t xs) {
  return TX::kBf16 && (n & 7) == 0 && (xs & 7) == 0 && (reinterpret_cast<uintptr_t>(xr) & 15) == 0;
}

// 1 / sqrt(mean(x^2) + eps) of one row, computed the same way by every kernel that normalises a row (so
// fused and standalone RMSNorm produce identical bits): thread i < 256 sums the 8-element chunks i,
// i + 256, ... (elements in order), each of the 4 waves reduces by butterflies, and waves 0..3 are summed
// in order. Every thread of the workgroup (256 or more) must call it; every thread gets the result.
// red: 4 floats of LDS.
template <class TX>
__device__ __forceinline__ float row_rstd256(const typename TX::T* xr, int64_t n, float eps, float* red) {
  if (threadIdx.x < 256) {
    float ss = 0.f;
    if (rows_bf16x8<TX>(xr, n, 8)) {
      for (int64_t c = threadIdx.x; c * 8 < n; c += 256)
        ss = chunk_ss_bf16x8(reinterpret_cast<const uint4*>(xr)[c], ss);
    } else {
      for (int64_t c = threadIdx.x; c * 8 < n; c += 256) ss = chunk_ss<TX>(xr, c, n, ss);
    }
    ss = wave_sum(ss);
    if (lane_id() == 0) red[threadIdx.x / kWave] = ss;
  }
  __syncthreads();
  const float t = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return rsqrtf(t / static_cast<float>(n) + eps);
}

// The same normalisation by one wave holding a whole bf16 row: lane l holds chunks l + 64 j (j < NC; zero
// past the row). Chunk l + 64 j is chunk (l + 64 j) % 256 of row_rstd256's thread of that index, in its
// wave j % 4, and a thread adds its chunks in j order, so summing per j % 4, reducing each by wave_sum and
// adding the four in order gives row_rstd256's bits. The chunks become bf16(w * bf16(x * rstd)) in place,
// as mm_rms_norm writes them (nv: the norm weight's chunks, bf16).
template <int NC>
__device__ __forceinline__ void norm_row_chunks64(uint4 (&xv)[NC], const uint4 (&nv)[NC], int64_t n, float eps) {
  float ssw[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NC; ++j) ssw[j % 4] = chunk_ss_bf16x8(xv[j], ssw[j % 4]);
  const float tot = ((wave_sum(ssw[0]) + wave_sum(ssw[1])) + wave_sum(ssw[2])) + wave_sum(ssw[3]);
  const float rstd = rsqrtf(tot / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const uint32_t xq[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
    const uint32_t nq[4] = {nv[j].x, nv[j].y, nv[j].z, nv[j].w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = round_bf16(__uint_as_float(nq[i] << 16) * round_bf16(__uint_as_float(xq[i] << 16) * rstd));
      const float hi =
          round_bf16(__uint_as_float(nq[i] & 0xffff0000u) * round_bf16(__uint_as_float(xq[i] & 0xffff0000u) * rstd));
      o[i] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
    }
    xv[j] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

}  // namespace mmd
