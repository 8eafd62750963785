// The two ends of a greedy decode step (engine.py:685-689): the embedding lookup of the previous token
// (word_embeddings(tok_buf)) and the greedy pick logits.argmax(-1) written back for the next step.
//
//   embed_rows_kernel   out[i] = table[ids[i]] (a row copy in 16-byte pieces; an id outside [0, V) gives a row
//                       of zeros, where torch's embedding would stop on a device-side assert).
//   argmax_rows_kernel  one workgroup of 1024 threads per row: every 16-byte load of the row is issued before
//                       the first comparison (one trip to memory), then the (value, index) pairs are reduced
//                       lane -> wave -> workgroup. torch.argmax's order: the largest value, NaN above every
//                       number, the lowest index among equals; so the result does not depend on the
//                       reduction's shape.
//   argmax_part_kernel  (with a workspace) the row split over many workgroups, each writing its best (value,
//   argmax_final_kernel index) to the workspace, then one wave per row merges them: one CU draws a long row at
//                       the rate its few outstanding lines allow (126464 bf16 logits: 17 us traced), many CUs
//                       draw it in one round trip each.
#include <algorithm>

#include "mm_common.h"

namespace {

using namespace mmd;

// (v, i) beats (bv, bi) in torch.argmax's order: the larger value, NaN above every number, the lower index
// among equals (and among NaNs). Branch-free.
__device__ __forceinline__ bool beats(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  const bool num = !vn && !bn && (v > bv || (v == bv && i < bi));
  return num || (vn && (!bn || i < bi));
}

// A thread's scan visits indices in increasing order, so a later element wins only when strictly larger or the
// first NaN; bi < 0 marks "nothing yet".
__device__ __forceinline__ void scan(float& bv, int& bi, float v, int i) {
  const bool vn = v != v, bn = bv != bv;
  const bool b = bi < 0 || (vn ? !bn : (!bn && v > bv));
  bv = b ? v : bv;
  bi = b ? i : bi;
}

__device__ __forceinline__ void merge(float& bv, int& bi, float v, int i) {
  const bool b = i >= 0 && (bi < 0 || beats(v, i, bv, bi));
  bv = b ? v : bv;
  bi = b ? i : bi;
}

constexpr int kArgThreads = 1024;
constexpr int kArgLoads = 16;  // 16-byte loads in flight per thread

// VEC: rows 16-byte aligned and n a multiple of the elements per 16 bytes; otherwise one element per load.
template <bool F32, bool VEC>
__global__ __launch_bounds__(kArgThreads) void argmax_rows_kernel(const void* __restrict__ x, int n, int64_t rs,
                                                                  int64_t* __restrict__ out) {
  __shared__ float s_v[kArgThreads / kWave];
  __shared__ int s_i[kArgThreads / kWave];
  constexpr int EPC = F32 ? 4 : 8;  // elements per 16-byte chunk
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  float bv = 0.f;
  int bi = -1;
  if constexpr (VEC) {
    const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * rs * (F32 ? 4 : 2));
    const int nch = n / EPC;
    for (int c0 = 0; c0 < nch; c0 += kArgThreads * kArgLoads) {
      uint4 v[kArgLoads];
#pragma unroll
      for (int j = 0; j < kArgLoads; ++j) {
        const int c = c0 + tid + kArgThreads * j;
        v[j] = xr[c < nch ? c : nch - 1];  // clamped: the value is not used past the end
      }
#pragma unroll
      for (int j = 0; j < kArgLoads; ++j) {
        const int c = c0 + tid + kArgThreads * j;
        if (c < nch) {  // uniform for all but the last chunks
          const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if constexpr (F32) {
              scan(bv, bi, __uint_as_float(w[q]), c * EPC + q);
            } else {
              scan(bv, bi, __uint_as_float(w[q] << 16), c * EPC + 2 * q);
              scan(bv, bi, __uint_as_float(w[q] & 0xffff0000u), c * EPC + 2 * q + 1);
            }
          }
        }
      }
    }
  } else {
    const char* xr = static_cast<const char*>(x) + row * rs * (F32 ? 4 : 2);
    for (int i = tid; i < n; i += kArgThreads)
      scan(bv, bi, F32 ? reinterpret_cast<const float*>(xr)[i] : bf16_to_f32(reinterpret_cast<const uint16_t*>(xr)[i]),
           i);
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const int oi = __shfl_xor(bi, m, kWave);
    merge(bv, bi, ov, oi);
  }
  if (lane == 0) {
    s_v[wave] = bv;
    s_i[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgThreads / kWave; ++w) merge(bv, bi, s_v[w], s_i[w]);
    out[row] = bi;
  }
}

struct ArgPart {
  float v;
  int i;
};
constexpr int kArgPartThreads = 256;
constexpr int kArgPartLoads = 2;  // 16-byte chunks per thread and pass
constexpr int kArgPartChunks = kArgPartThreads * kArgPartLoads;
constexpr int kArgMaxParts = 1024;

int arg_parts(int64_t n, bool f32) {
  const int64_t nch = n / (f32 ? 4 : 8);
  return static_cast<int>(std::min<int64_t>((nch + kArgPartChunks - 1) / kArgPartChunks, kArgMaxParts));
}

// Grid (parts, rows), rows 16-byte aligned and n a multiple of the elements per chunk: workgroup g scans the chunks
// g * kArgPartChunks + [0, kArgPartChunks) of its row (and every parts * kArgPartChunks after), each pass's loads
// issued before its comparisons, and writes its best (value, index) to part[row * parts + g].
template <bool F32>
__global__ __launch_bounds__(kArgPartThreads) void argmax_part_kernel(const void* __restrict__ x, int n, int64_t rs,
                                                                      ArgPart* __restrict__ part) {
  __shared__ float s_v[kArgPartThreads / kWave];
  __shared__ int s_i[kArgPartThreads / kWave];
  constexpr int EPC = F32 ? 4 : 8;
  const int64_t row = blockIdx.y;
  const int g = blockIdx.x, parts = gridDim.x;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * rs * (F32 ? 4 : 2));
  const int nch = n / EPC;
  float bv = 0.f;
  int bi = -1;
  for (int c0 = g * kArgPartChunks; c0 < nch; c0 += parts * kArgPartChunks) {
    uint4 v[kArgPartLoads];
#pragma unroll
    for (int j = 0; j < kArgPartLoads; ++j) {
      const int c = c0 + tid + kArgPartThreads * j;
      v[j] = xr[c < nch ? c : nch - 1];  // clamped: the value is not used past the end
    }
#pragma unroll
    for (int j = 0; j < kArgPartLoads; ++j) {
      const int c = c0 + tid + kArgPartThreads * j;
      if (c < nch) {
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (F32) {
            scan(bv, bi, __uint_as_float(w[q]), c * EPC + q);
          } else {
            scan(bv, bi, __uint_as_float(w[q] << 16), c * EPC + 2 * q);
            scan(bv, bi, __uint_as_float(w[q] & 0xffff0000u), c * EPC + 2 * q + 1);
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const int oi = __shfl_xor(bi, m, kWave);
    merge(bv, bi, ov, oi);
  }
  if (lane == 0) {
    s_v[wave] = bv;
    s_i[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgPartThreads / kWave; ++w) merge(bv, bi, s_v[w], s_i[w]);
    part[row * parts + g] = ArgPart{bv, bi};
  }
}

// Grid rows, one wave: lane l merges parts l, l + 64, ... of its row, then the wave merges the lanes.
__global__ __launch_bounds__(kWave) void argmax_final_kernel(const ArgPart* __restrict__ part, int parts,
                                                             int64_t* __restrict__ out) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  float bv = 0.f;
  int bi = -1;
  for (int p = lane; p < parts; p += kWave) {
    const ArgPart q = part[row * parts + p];
    merge(bv, bi, q.v, q.i);
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const int oi = __shfl_xor(bi, m, kWave);
    merge(bv, bi, ov, oi);
  }
  if (lane == 0) out[row] = bi;
}

// Grid (pieces of a row / 256, rows): thread = one 16-byte piece of the output row.
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint4* __restrict__ table, int64_t V, int64_t pieces,
                                                         int64_t trs, const void* ids, int ids_dtype,
                                                         uint4* __restrict__ out, int64_t ors) {
  const int64_t i = blockIdx.y;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= pieces) return;
  const int64_t id = load_id(ids, ids_dtype, i);
  const bool ok = id >= 0 && id < V;
  out[i * ors + c] = ok ? table[id * trs + c] : make_uint4(0u, 0u, 0u, 0u);
}

int dtype_bytes(int dt) { return dt == MM_FP32 ? 4 : (dt == MM_BF16 || dt == MM_FP16 ? 2 : 0); }

}  // namespace

extern "C" int64_t mm_argmax_rows_workspace_bytes(int64_t rows, int64_t n, int x_dtype) {
  if (rows < 0 || n < 1 || (x_dtype != MM_BF16 && x_dtype != MM_FP32)) return -1;
  return rows * arg_parts(n, x_dtype == MM_FP32) * static_cast<int64_t>(sizeof(ArgPart));
}

extern "C" int mm_argmax_rows_ws(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t x_row_stride,
                                 int64_t* out, void* workspace, int64_t workspace_bytes, void* stream) {
  MM_REQUIRE(x_dtype == MM_BF16 || x_dtype == MM_FP32, "argmax_rows: x must be bf16 or fp32");
  MM_REQUIRE(rows >= 0 && rows <= 65535 && n >= 1 && n <= 0x7fffffffLL,
             "argmax_rows: rows=%lld, n=%lld (rows <= 65535, 1 <= n < 2^31)", (long long)rows, (long long)n);
  MM_REQUIRE(x_row_stride >= n || rows <= 1, "argmax_rows: row stride %lld smaller than n=%lld", (long long)x_row_stride,
             (long long)n);
  MM_REQUIRE(x && out && workspace, "argmax_rows: null pointer");
  const bool f32 = x_dtype == MM_FP32;
  const int es = f32 ? 4 : 2, epc = 16 / es;
  const bool vec = mm::aligned16(x) && (x_row_stride * es) % 16 == 0 && n % epc == 0;
  const int parts = arg_parts(n, f32);
  // short or unaligned rows: the one-workgroup kernel (the same result)
  if (!vec || parts < 2) return mm_argmax_rows(x, x_dtype, rows, n, x_row_stride, out, stream);
  const int64_t need = rows * parts * static_cast<int64_t>(sizeof(ArgPart));
  MM_REQUIRE(workspace_bytes >= need && mm::aligned16(workspace),
             "argmax_rows: workspace of %lld bytes, %lld needed (16-byte aligned)", (long long)workspace_bytes,
             (long long)need);
  if (rows == 0) return MM_OK;
  hipStream_t st = MM_STREAM(stream);
  ArgPart* part = static_cast<ArgPart*>(workspace);
  const dim3 grid(static_cast<unsigned>(parts), static_cast<unsigned>(rows));
  if (f32) hipLaunchKernelGGL((argmax_part_kernel<true>), grid, dim3(kArgPartThreads), 0, st, x, static_cast<int>(n), x_row_stride, part);
  else hipLaunchKernelGGL((argmax_part_kernel<false>), grid, dim3(kArgPartThreads), 0, st, x, static_cast<int>(n), x_row_stride, part);
  if (const int rc = mm::check_launch("argmax_rows")) return rc;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(static_cast<unsigned>(rows)), dim3(kWave), 0, st, part, parts, out);
  return mm::check_launch("argmax_rows");
}

extern "C" int mm_argmax_rows(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t x_row_stride, int64_t* out,
                              void* stream) {
  MM_REQUIRE(x_dtype == MM_BF16 || x_dtype == MM_FP32, "argmax_rows: x must be bf16 or fp32");
  MM_REQUIRE(rows >= 0 && rows <= 0x7fffffffLL && n >= 1 && n <= 0x7fffffffLL,
             "argmax_rows: rows=%lld, n=%lld (1 <= n < 2^31)", (long long)rows, (long long)n);
  MM_REQUIRE(x_row_stride >= n || rows <= 1, "argmax_rows: row stride %lld smaller than n=%lld", (long long)x_row_stride,
             (long long)n);
  MM_REQUIRE(x && out, "argmax_rows: null pointer");
  if (rows == 0) return MM_OK;
  hipStream_t st = MM_STREAM(stream);
  const bool f32 = x_dtype == MM_FP32;
  const int es = f32 ? 4 : 2, epc = 16 / es;
  const bool vec = mm::aligned16(x) && (x_row_stride * es) % 16 == 0 && n % epc == 0;
  const dim3 grid(static_cast<unsigned>(rows)), block(kArgThreads);
  if (f32) {
    if (vec) hipLaunchKernelGGL((argmax_rows_kernel<true, true>), grid, block, 0, st, x, static_cast<int>(n), x_row_stride, out);
    else hipLaunchKernelGGL((argmax_rows_kernel<true, false>), grid, block, 0, st, x, static_cast<int>(n), x_row_stride, out);
  } else {
    if (vec) hipLaunchKernelGGL((argmax_rows_kernel<false, true>), grid, block, 0, st, x, static_cast<int>(n), x_row_stride, out);
    else hipLaunchKernelGGL((argmax_rows_kernel<false, false>), grid, block, 0, st, x, static_cast<int>(n), x_row_stride, out);
  }
  return mm::check_launch("argmax_rows");
}

extern "C" int mm_embed_rows(const void* table, int dtype, int64_t V, int64_t H, int64_t table_row_stride,
                             const void* ids, int ids_dtype, int64_t n, void* out, int64_t out_row_stride,
                             void* stream) {
  const int es = dtype_bytes(dtype);
  MM_REQUIRE(es > 0, "embed_rows: table must be bf16, fp16 or fp32");
  MM_REQUIRE(ids_dtype == MM_INT32 || ids_dtype == MM_INT64, "embed_rows: ids must be int32 or int64");
  MM_REQUIRE(V >= 1 && H >= 1 && n >= 0 && n <= 65535, "embed_rows: V=%lld, H=%lld, n=%lld (n <= 65535)",
             (long long)V, (long long)H, (long long)n);
  MM_REQUIRE(table_row_stride >= H && out_row_stride >= H, "embed_rows: row stride smaller than H");
  MM_REQUIRE(table && ids && out, "embed_rows: null pointer");
  MM_REQUIRE(mm::aligned16(table) && mm::aligned16(out) && (H * es) % 16 == 0 && (table_row_stride * es) % 16 == 0 &&
                 (out_row_stride * es) % 16 == 0,
             "embed_rows: table and out rows must be 16-byte aligned and H * element size a multiple of 16");
  if (n == 0) return MM_OK;
  const int64_t pieces = H * es / 16;
  hipStream_t st = MM_STREAM(stream);
  hipLaunchKernelGGL(embed_rows_kernel, dim3(static_cast<unsigned>((pieces + 255) / 256), static_cast<unsigned>(n)),
                     dim3(256), 0, st, static_cast<const uint4*>(table), V, pieces, table_row_stride * es / 16, ids,
                     ids_dtype, static_cast<uint4*>(out), out_row_stride * es / 16);
  return mm::check_launch("embed_rows");
}
