// Shared host and device helpers of libmingmoe (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <mutex>

#include "mingmoe.h"

// ------------------------------------------------------------------------------------------ host side

namespace mm {

// Records a printf-style message as this thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch; returns MM_OK or MM_ERR_HIP with "HIP error: ..." recorded.
int check_launch(const char* what);

// Size in bytes of a dtype code, 0 when unknown.
size_t dtype_size(int dtype);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Largest byte span a buffer resource (mmd::make_rsrc) may describe: the kernels address it with 32-bit
// offsets and use 2^31 (mmd::kPast) as the offset that reads zero, so every valid offset must stay below it.
constexpr int64_t kMaxRsrcBytes = 0x7fffffffLL;
inline bool rsrc_fits(int64_t bytes) { return bytes >= 0 && bytes <= kMaxRsrcBytes; }

// Number of compute units of the current device (queried once per device, thread-safe).
int cu_count();

// Dynamic LDS above the default limit needs an opt-in per kernel and device: the attribute is set the first
// time a kernel is launched on a device with a given size, and again whenever a launch needs more than the
// size set so far (state keyed by the kernel's address and the device, thread-safe).
int allow_lds_ptr(const void* kernel, size_t bytes, const char* what);

template <class K>
int allow_lds(K kernel, size_t bytes, const char* what) {
  return allow_lds_ptr(reinterpret_cast<const void*>(kernel), bytes, what);
}

}  // namespace mm

#define MM_REQUIRE(cond, ...)                                 \
  do {                                                        \
    if (!(cond)) return ::mm::set_error(MM_ERR_ARG, __VA_ARGS__); \
  } while (0)

#define MM_STREAM(s) (reinterpret_cast<hipStream_t>(s))

// ---------------------------------------------------------------------------------------- device side

namespace mmd {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even float -> bf16 (a single v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Round a float through bf16 and back, the `.to(bfloat16).to(float32)` of the reference kernels.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// Typed scalar load / store through dtype tags.
struct BF16 { typedef uint16_t T; static constexpr bool kBf16 = true; static __device__ __forceinline__ float ld(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
              static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = f32_to_bf16(v); } };
struct FP16 { typedef uint16_t T; static constexpr bool kBf16 = false; static __device__ __forceinline__ float ld(const T* p, int64_t i) { return f16_to_f32(p[i]); }
              static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = f32_to_f16(v); } };
struct FP32 { typedef float T; static constexpr bool kBf16 = false; static __device__ __forceinline__ float ld(const T* p, int64_t i) { return p[i]; }
              static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = v; } };

// Scale loads for int8 weights (fp32 or bf16 scale tensors).
__device__ __forceinline__ float load_scale(const void* s, int s_dtype, int64_t i) {
  return s_dtype == MM_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(s)[i]) : static_cast<const float*>(s)[i];
}

__device__ __forceinline__ int64_t load_id(const void* ids, int ids_dtype, int64_t i) {
  return ids_dtype == MM_INT64 ? static_cast<const int64_t*>(ids)[i] : static_cast<int64_t>(static_cast<const int32_t*>(ids)[i]);
}

// 2 x bf16 (packed in a dword) dot 2 x bf16, accumulated in fp32 (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// Dot of 8 bf16 weights (uint4) with 8 bf16 activations (uint4).
__device__ __forceinline__ float dot8_bf16(const uint4& w, const uint4& x, float acc) {
  acc = dot2_bf16(w.x, x.x, acc);
  acc = dot2_bf16(w.y, x.y, acc);
  acc = dot2_bf16(w.z, x.z, acc);
  acc = dot2_bf16(w.w, x.w, acc);
  return acc;
}

// Signed byte b (0..3) of a dword as float (a single SDWA v_cvt_f32_i32 on gfx950).
__device__ __forceinline__ float sbyte(uint32_t v, int b) { return static_cast<float>(static_cast<int8_t>(v >> (8 * b))); }

// Dot of 4 int8 weights (one dword) with 4 activations given as two packed bf16 pairs.
__device__ __forceinline__ float dot4_i8_bf16(uint32_t w, uint32_t x01, uint32_t x23, float acc) {
  acc = fmaf(sbyte(w, 0), __uint_as_float(x01 << 16), acc);
  acc = fmaf(sbyte(w, 1), __uint_as_float(x01 & 0xffff0000u), acc);
  acc = fmaf(sbyte(w, 2), __uint_as_float(x23 << 16), acc);
  acc = fmaf(sbyte(w, 3), __uint_as_float(x23 & 0xffff0000u), acc);
  return acc;
}

// Two fp32 values whose low 16 bits are zero -> packed bf16 pair (lo in bits 0-15): the high halves, one v_perm_b32.
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 16 int8 -> 16 bf16 (exact), as two uint4 of packed bf16 pairs. |q| <= 127 has at most 7 significant bits, so
// fp32(q) has a zero low half and its high half is bf16(q): a byte convert per element and one permute per pair
// (1.5 VALU ops per element, against 3 for a rounding convert of each value and a shift-or to pack).
__device__ __forceinline__ void widen_i8(const uint4& q, uint4& lo, uint4& hi) {
  const uint32_t in[4] = {q.x, q.y, q.z, q.w};
  uint32_t out[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = in[i];
    out[2 * i] = pack_hi16(sbyte(v, 0), sbyte(v, 1));
    out[2 * i + 1] = pack_hi16(sbyte(v, 2), sbyte(v, 3));
  }
  lo = make_uint4(out[0], out[1], out[2], out[3]);
  hi = make_uint4(out[4], out[5], out[6], out[7]);
}

// Dot of 16 int8 weights (uint4) with 16 bf16 activations (two uint4).
__device__ __forceinline__ float dot16_i8_bf16(const uint4& w, const uint4& xa, const uint4& xb, float acc) {
  acc = dot4_i8_bf16(w.x, xa.x, xa.y, acc);
  acc = dot4_i8_bf16(w.y, xa.z, xa.w, acc);
  acc = dot4_i8_bf16(w.z, xb.x, xb.y, acc);
  acc = dot4_i8_bf16(w.w, xb.z, xb.w, acc);
  return acc;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Cross-lane moves inside rows of 16 lanes by DPP (no LDS round trip).
template <int ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]: lane i <-> i ^ 1
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]: lane i <-> i ^ 2
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16 lanes

// Sum over aligned groups of `width` lanes (a power of two <= 64); every lane of a group gets the group's
// total, with one fixed association: pairs, then quads, then halves and rows of 16 (each step adds a lane
// of the partner group, whose lanes hold equal values by then), then the row totals as (r0 + r1) + (r2 + r3).
// The steps across rows use gfx950's v_permlane16_swap / v_permlane32_swap of a register with itself: the first
// result holds rows (0, 0, 2, 2) of it, the second rows (1, 1, 3, 3) (16-swap), or the low and high 32 lanes
// in both halves (32-swap), so their sum is the pair's total in every lane (lane layouts checked on the device),
// all in the VALU with no trip through the LDS crossbar or the scalar unit.
__device__ __forceinline__ float row_pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), true, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float half_pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), true, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int width>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(width >= 1 && width <= 64 && (width & (width - 1)) == 0, "group width");
  if constexpr (width >= 2) v += dpp_f32<kDppXor1>(v);
  if constexpr (width >= 4) v += dpp_f32<kDppXor2>(v);
  if constexpr (width >= 8) v += dpp_f32<kDppHalfMirror>(v);
  if constexpr (width >= 16) v += dpp_f32<kDppMirror>(v);
  if constexpr (width >= 32) v = row_pair_sum(v);   // r0 + r1 | r2 + r3
  if constexpr (width == 64) v = half_pair_sum(v);  // (r0 + r1) + (r2 + r3)
  return v;
}

// Sum over the lanes of a wave (all lanes get the total).
__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// Transposed sums (group_sums below) keep, in their step on lane bit B of groups of W lanes, the half of a lane's
// values that this bit selects (1: the upper half). It is the lane bit itself, xor a higher bit that the later
// mirror steps flip along with it: 0, 1 take bit 2 (flipped by the half mirror and the mirror), 2 takes bit 3
// (the mirror), so that the half mirror (lane i <-> 7 - i) and mirror (i <-> 15 - i) partners of group_sum hold the
// same values' partials as the lane.
template <int B, int W>
__device__ __forceinline__ int sums_hi(int lane) {
  const int b = (lane >> B) & 1;
  if constexpr (B <= 1) return b ^ (W > 4 ? (lane >> 2) & 1 : 0);
  else if constexpr (B == 2) return b ^ (W > 8 ? (lane >> 3) & 1 : 0);
  else return b;
}

// group_sum's pair step on lane bit B: partner xor 1, xor 2, half mirror, mirror, across rows, across halves.
template <int B>
__device__ __forceinline__ float pair_sum_bit(float v) {
  if constexpr (B == 0) return v + dpp_f32<kDppXor1>(v);
  else if constexpr (B == 1) return v + dpp_f32<kDppXor2>(v);
  else if constexpr (B == 2) return v + dpp_f32<kDppHalfMirror>(v);
  else if constexpr (B == 3) return v + dpp_f32<kDppMirror>(v);
  else if constexpr (B == 4) return row_pair_sum(v);
  else return half_pair_sum(v);
}

// One transposed step on lane bit B: 2H values -> H, each lane of a pair keeping the half its select bit names and
// adding the partner's copy of it.
template <int B, int W, int H>
__device__ __forceinline__ void group_sums_step(float* x) {
  if constexpr (B < 4) {
    const bool hi = sums_hi<B, W>(lane_id());
#pragma unroll
    for (int v = 0; v < H; ++v) {
      const float keep = hi ? x[v + H] : x[v], send = hi ? x[v] : x[v + H];
      constexpr int ctrl = B == 0 ? kDppXor1 : B == 1 ? kDppXor2 : B == 2 ? kDppHalfMirror : kDppMirror;
      x[v] = keep + dpp_f32<ctrl>(send);
    }
  } else {
#pragma unroll
    for (int v = 0; v < H; ++v) {  // rows 0 / 2 (bit 4) or lanes 0-31 (bit 5) keep v, the others v + H
      const auto r = B == 4 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x[v]), __float_as_uint(x[v + H]), false, false)
                            : __builtin_amdgcn_permlane32_swap(__float_as_uint(x[v]), __float_as_uint(x[v + H]), false, false);
      x[v] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  }
}

template <int B, int W, int N>
__device__ __forceinline__ void group_sums_from(float* x) {
  if constexpr ((1 << B) < W) {
    if constexpr (N > 1) group_sums_step<B, W, N / 2>(x);
    else x[0] = pair_sum_bit<B>(x[0]);
    group_sums_from<B + 1, W, (N > 1 ? N / 2 : 1)>(x);
  }
}

// Sums of N values over aligned groups of W lanes (powers of two, N <= W <= 64), transposed: on lane bits 0, 1, ...
// in turn, the lanes of each pair split their values in half while more than one is left (group_sums_step), then
// sum the last one (pair_sum_bit). Every step pairs the lanes as group_sum's does and adds the partials of one value
// over the same two lane sets, so each total is group_sum's of that value, bit for bit; a lane makes N - 1 +
// log2 W - log2 N exchanges, where N group_sum calls take N log2 W. Lane l's x[0] ends as the total of value
// sums_index<W, N>(l).
template <int W, int N>
__device__ __forceinline__ void group_sums(float (&x)[N]) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0 && N >= 1 && N <= W && (N & (N - 1)) == 0, "group sums");
  group_sums_from<0, W, N>(x);
}

template <int B, int W, int N>
__device__ __forceinline__ int sums_index_from(int lane) {
  if constexpr ((1 << B) < N) return sums_hi<B, W>(lane) * (N >> (B + 1)) + sums_index_from<B + 1, W, N>(lane);
  else return 0;
}

// The value whose total lane `lane` holds after group_sums<W, N>: sum over b < log2 N of its select bit b times
// N / 2^(b+1). Lane ^ 1 holds value index +- N / 2 (only select bit 0 differs).
template <int W, int N>
__device__ __forceinline__ int sums_index(int lane) {
  return sums_index_from<0, W, N>(lane);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppMirror>(v));
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), true, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), true, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}


// Global operands of the latency-bound kernels are read through buffer resources (a wave-uniform base and
// byte size): a load at an offset past the end returns zero, so a lane past a row's end is given kPast as
// its offset instead of a branch or a mask, and all of a lane's loads issue back to back.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kPast = 0x80000000u;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ uint4 buf16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}

__device__ __forceinline__ uint32_t buf4(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0));
}

__device__ __forceinline__ uint32_t buf2(rsrc_t r, uint32_t off) {
  return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, 0));
}

// Loads of a tensor whose dtype is one of two, chosen at run time, without a branch on it: one buffer resource per
// dtype over the same memory, the other dtype's of size zero (its loads read zero and touch no memory), and the
// two results combined. A load behind a branch makes the wave wait for it, and for every load issued before it,
// right away; these wait only where their value is used.
// A row of n fp32 or bf16 scales starting at element `first` of s.
struct ScaleRow {
  rsrc_t r16, r32;
};

__device__ __forceinline__ ScaleRow scale_row(const void* s, int s_dtype, int64_t first, int64_t n) {
  const bool b16 = s_dtype == MM_BF16;
  const char* row = static_cast<const char*>(s) + first * (b16 ? 2 : 4);
  return {make_rsrc(row, b16 ? n * 2 : 0), make_rsrc(row, b16 ? 0 : n * 4)};
}

__device__ __forceinline__ float scale_at(const ScaleRow& r, uint32_t i) {
  return __uint_as_float((buf2(r.r16, i * 2u) << 16) | buf4(r.r32, i * 4u));
}


typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

// global_load_lds_dwordx4: lane i copies 16 bytes from src into LDS at lds_wave_base + 16 i (the base is
// wave-uniform); the data is there once the wave's vector-memory count says the load is done (wait_vmcnt).
__device__ __forceinline__ void load_lds16(const void* src, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)lds_wave_base, 16, 0, 0);
}

// Wait until at most n vector-memory operations of this wave are outstanding (n a compile-time constant).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

}  // namespace mmd
