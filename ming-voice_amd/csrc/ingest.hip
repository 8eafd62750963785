// Expert ingestion from safetensors shards into the stacked layout (engine.py:126-188, direct_load.py:81-131):
// every expert matrix (gate, up, down of each routed expert, and the shared expert in the last slot) is read
// from its file range and written into w_gu[slot, 0:I] / w_gu[slot, I:2I] / w_d[slot] of an mm_experts
// descriptor, as bf16 or as int8 with per-row scales (quantised on the GPU as it arrives).
//
// Host side: n_threads workers take items in file order. Each worker owns two pinned host staging slots
// and one device staging slot; it reads an item with pread into a host slot, copies it to the GPU on its
// own stream, and either lands it in place (bf16 file data into a bf16 stack needs no conversion) or converts
// it there: a bf16 rounding cast (fp16 / fp32 file data) or the int8 quantiser. Reading item k+1 overlaps
// the copy and the kernel of item k; a host slot is refilled only after its copy has completed.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "mm_common.h"

namespace {

using namespace mmd;

// out[r, c] = bf16(in[r, c]) (round to nearest even), out rows with stride os.
template <class TX>
__global__ __launch_bounds__(256) void cast_rows_kernel(const typename TX::T* __restrict__ in, int64_t cols,
                                                        uint16_t* __restrict__ out, int64_t os) {
  const int64_t r = blockIdx.y;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; c < cols; c += static_cast<int64_t>(gridDim.x) * 256)
    out[r * os + c] = f32_to_bf16(TX::ld(in, r * cols + c));
}

struct Dest {
  char* base;        // first row of the matrix in the stack
  int64_t row_stride;  // elements
  void* scale;       // int8: first scale of the matrix
};

Dest dest_of(const mm_experts& ex, const mm_ingest_item& it) {
  const bool q = ex.w_dtype == MM_INT8;
  const size_t es = q ? 1 : 2;
  const size_t ss = ex.s_dtype == MM_BF16 ? 2 : 4;
  Dest d{};
  if (it.part == MM_PART_DOWN) {
    d.base = static_cast<char*>(const_cast<void*>(ex.w_d)) + (it.slot * ex.d_stride_e) * es;
    d.row_stride = ex.d_stride_n;
    if (q) d.scale = static_cast<char*>(const_cast<void*>(ex.s_d)) + (it.slot * ex.sd_stride_e) * ss;
  } else {
    const int64_t row0 = it.part == MM_PART_UP ? ex.inter : 0;
    d.base = static_cast<char*>(const_cast<void*>(ex.w_gu)) + (it.slot * ex.gu_stride_e + row0 * ex.gu_stride_n) * es;
    d.row_stride = ex.gu_stride_n;
    if (q) d.scale = static_cast<char*>(const_cast<void*>(ex.s_gu)) + (it.slot * ex.sgu_stride_e + row0) * ss;
  }
  return d;
}

struct Shared {
  std::atomic<int64_t> next{0};
  std::atomic<bool> failed{false};
  std::mutex mu;
  std::string error;
  int code = MM_OK;
  void fail(int c, const std::string& msg) {
    std::lock_guard<std::mutex> lock(mu);
    if (!failed.exchange(true)) {
      code = c;
      error = msg;
    }
  }
};

bool read_range(int fd, char* dst, int64_t n, int64_t off, std::string& err) {
  int64_t got = 0;
  while (got < n) {
    const ssize_t r = pread(fd, dst + got, static_cast<size_t>(n - got), static_cast<off_t>(off + got));
    if (r < 0) {
      if (errno == EINTR) continue;
      err = std::string("read failed: ") + strerror(errno);
      return false;
    }
    if (r == 0) {
      err = "file ends before the tensor's data range";
      return false;
    }
    got += r;
  }
  return true;
}

#define HIP_OR_FAIL(call, what)                                                                              \
  do {                                                                                                       \
    hipError_t e_ = (call);                                                                                  \
    if (e_ != hipSuccess) {                                                                                  \
      sh.fail(MM_ERR_HIP, std::string("HIP error in ingest_experts (") + (what) + "): " + hipGetErrorString(e_)); \
      return;                                                                                                \
    }                                                                                                        \
  } while (0)

void worker(int dev, int t, const mm_ingest_item* items, const int64_t* order, int64_t n, const mm_experts& ex,
            char* host, char* devbuf, int64_t slot_bytes, Shared& sh) {
  HIP_OR_FAIL(hipSetDevice(dev), "set device");
  hipStream_t st = nullptr;
  HIP_OR_FAIL(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "stream");
  hipEvent_t copied[2] = {nullptr, nullptr};
  bool pending[2] = {false, false};
  for (auto& e : copied) {
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      sh.fail(MM_ERR_HIP, "HIP error in ingest_experts (event)");
      (void)hipStreamDestroy(st);
      return;
    }
  }
  char* hslot[2] = {host + (2 * t) * slot_bytes, host + (2 * t + 1) * slot_bytes};
  char* dslot = devbuf + t * slot_bytes;
  const char* open_path = nullptr;
  int fd = -1;
  int k = 0;
  auto cleanup = [&]() {
    if (fd >= 0) close(fd);
    (void)hipStreamSynchronize(st);
    for (auto& e : copied) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(st);
  };
  for (;;) {
    if (sh.failed.load()) break;
    const int64_t i = sh.next.fetch_add(1);
    if (i >= n) break;
    const mm_ingest_item& it = items[order[i]];
    if (open_path == nullptr || strcmp(open_path, it.path) != 0) {
      if (fd >= 0) close(fd);
      fd = open(it.path, O_RDONLY);
      if (fd < 0) {
        sh.fail(MM_ERR_ARG, std::string("ingest_experts: cannot open ") + it.path + ": " + strerror(errno));
        break;
      }
      open_path = it.path;
    }
    const int b = k++ & 1;
    if (pending[b]) {  // this host slot's previous copy must have left it
      if (hipEventSynchronize(copied[b]) != hipSuccess) {
        sh.fail(MM_ERR_HIP, "HIP error in ingest_experts (event wait)");
        break;
      }
      pending[b] = false;
    }
    std::string err;
    if (!read_range(fd, hslot[b], it.nbytes, it.offset, err)) {
      sh.fail(MM_ERR_ARG, std::string("ingest_experts: ") + it.path + ": " + err);
      break;
    }
    const Dest d = dest_of(ex, it);
    const bool direct = ex.w_dtype == MM_BF16 && it.src_dtype == MM_BF16;
    hipError_t e = hipSuccess;
    if (direct && d.row_stride == it.cols) {  // the matrix is one contiguous block of the stack
      e = hipMemcpyAsync(d.base, hslot[b], it.nbytes, hipMemcpyHostToDevice, st);
    } else if (direct) {
      e = hipMemcpy2DAsync(d.base, d.row_stride * 2, hslot[b], it.cols * 2, it.cols * 2, it.rows,
                           hipMemcpyHostToDevice, st);
    } else {
      e = hipMemcpyAsync(dslot, hslot[b], it.nbytes, hipMemcpyHostToDevice, st);
    }
    if (e == hipSuccess) e = hipEventRecord(copied[b], st);
    if (e != hipSuccess) {
      sh.fail(MM_ERR_HIP, std::string("HIP error in ingest_experts (copy): ") + hipGetErrorString(e));
      break;
    }
    pending[b] = true;
    if (direct) continue;
    if (ex.w_dtype == MM_INT8) {
      const int rc = mm_quantize_rows_int8(dslot, it.src_dtype, it.rows, it.cols, it.cols, reinterpret_cast<int8_t*>(d.base),
                                           d.row_stride, d.scale, ex.s_dtype, st);
      if (rc != MM_OK) {
        char msg[1024];
        mm_last_error(msg, sizeof msg);
        sh.fail(rc, msg);
        break;
      }
    } else {
      const dim3 grid(static_cast<unsigned>((it.cols + 255) / 256 < 8 ? (it.cols + 255) / 256 : 8),
                      static_cast<unsigned>(it.rows));
      if (it.src_dtype == MM_FP32)
        hipLaunchKernelGGL(cast_rows_kernel<FP32>, grid, dim3(256), 0, st, reinterpret_cast<const float*>(dslot), it.cols,
                           reinterpret_cast<uint16_t*>(d.base), d.row_stride);
      else
        hipLaunchKernelGGL(cast_rows_kernel<FP16>, grid, dim3(256), 0, st, reinterpret_cast<const uint16_t*>(dslot),
                           it.cols, reinterpret_cast<uint16_t*>(d.base), d.row_stride);
      e = hipGetLastError();
      if (e != hipSuccess) {
        sh.fail(MM_ERR_HIP, std::string("HIP error in ingest_experts (cast): ") + hipGetErrorString(e));
        break;
      }
    }
  }
  if (hipStreamSynchronize(st) != hipSuccess) sh.fail(MM_ERR_HIP, "HIP error in ingest_experts (stream sync)");
  cleanup();
}

}  // namespace

extern "C" int mm_ingest_experts(const mm_ingest_item* items, int64_t n_items, const mm_experts* ex, void* host_staging,
                                 void* dev_staging, int64_t slot_bytes, int n_threads) {
  MM_REQUIRE(ex && (n_items == 0 || items), "ingest_experts: null pointer");
  MM_REQUIRE(n_items >= 0 && n_threads >= 1 && n_threads <= 64, "ingest_experts: n_items=%lld, n_threads=%d",
             (long long)n_items, n_threads);
  MM_REQUIRE(ex->w_dtype == MM_BF16 || ex->w_dtype == MM_INT8, "ingest_experts: the stack must be bf16 or int8");
  MM_REQUIRE(ex->w_dtype != MM_INT8 || (ex->s_gu && ex->s_d && (ex->s_dtype == MM_FP32 || ex->s_dtype == MM_BF16)),
             "ingest_experts: an int8 stack needs fp32 or bf16 scales");
  MM_REQUIRE(ex->w_gu && ex->w_d && ex->inter > 0 && ex->hidden > 0 && ex->n_slots > 0, "ingest_experts: bad stack");
  MM_REQUIRE(host_staging && dev_staging && slot_bytes > 0, "ingest_experts: staging buffers missing");
  for (int64_t i = 0; i < n_items; ++i) {
    const mm_ingest_item& it = items[i];
    const size_t es = mm::dtype_size(it.src_dtype);
    MM_REQUIRE(it.path && (it.src_dtype == MM_BF16 || it.src_dtype == MM_FP16 || it.src_dtype == MM_FP32),
               "ingest_experts: item %lld: file dtype must be BF16, F16 or F32", (long long)i);
    MM_REQUIRE(it.part == MM_PART_GATE || it.part == MM_PART_UP || it.part == MM_PART_DOWN,
               "ingest_experts: item %lld: part %d", (long long)i, it.part);
    MM_REQUIRE(it.slot >= 0 && it.slot < ex->n_slots, "ingest_experts: item %lld: slot %lld outside [0, %lld)",
               (long long)i, (long long)it.slot, (long long)ex->n_slots);
    const int64_t want_r = it.part == MM_PART_DOWN ? ex->hidden : ex->inter;
    const int64_t want_c = it.part == MM_PART_DOWN ? ex->inter : ex->hidden;
    MM_REQUIRE(it.rows == want_r && it.cols == want_c,
               "ingest_experts: item %lld: shape [%lld, %lld] does not fit the stack (want [%lld, %lld])", (long long)i,
               (long long)it.rows, (long long)it.cols, (long long)want_r, (long long)want_c);
    MM_REQUIRE(it.offset >= 0 && it.nbytes == it.rows * it.cols * static_cast<int64_t>(es),
               "ingest_experts: item %lld: %lld bytes for a [%lld, %lld] tensor", (long long)i, (long long)it.nbytes,
               (long long)it.rows, (long long)it.cols);
    MM_REQUIRE(it.nbytes <= slot_bytes, "ingest_experts: item %lld: %lld bytes exceed the staging slot (%lld)",
               (long long)i, (long long)it.nbytes, (long long)slot_bytes);
  }
  if (n_items == 0) return MM_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mm::set_error(MM_ERR_HIP, "HIP error in ingest_experts: %s", hipGetErrorString(e));
  // file order: items of one file by offset, so each worker reads forward
  std::vector<int64_t> order(static_cast<size_t>(n_items));
  for (int64_t i = 0; i < n_items; ++i) order[static_cast<size_t>(i)] = i;
  std::stable_sort(order.begin(), order.end(), [&](int64_t x, int64_t y) {
    const int c = strcmp(items[x].path, items[y].path);
    return c != 0 ? c < 0 : items[x].offset < items[y].offset;
  });
  Shared sh;
  const int nt = static_cast<int>(n_threads < n_items ? n_threads : n_items);
  std::vector<std::thread> pool;
  pool.reserve(static_cast<size_t>(nt));
  for (int t = 0; t < nt; ++t)
    pool.emplace_back(worker, dev, t, items, order.data(), n_items, std::cref(*ex), static_cast<char*>(host_staging),
                      static_cast<char*>(dev_staging), slot_bytes, std::ref(sh));
  for (auto& th : pool) th.join();
  if (sh.failed.load()) return mm::set_error(sh.code, "%s", sh.error.c_str());
  return MM_OK;
}
