// Grouped prefill MoE on bf16 MFMA (fused_moe.py:92-196).
//
// mm_align_blocks groups the (token, slot) pairs by expert into blocks of BM rows (64, or 128 for bf16
// experts averaging at least 128 pairs) and reports each expert's padded row range. A tile is (expert block
// of BM pairs) x (BN = 128 or 256 output columns):
//   GATE_UP: columns are BN/2 gate + the matching BN/2 up rows of W_gu[e]; the epilogue writes
//            a[pair] = bf16(bf16(silu(bf16(g))) * bf16(u)) (int8: row scale on the fp32 accumulator first).
//   DOWN:    columns are BN rows of W_d[e]; the epilogue writes part[pair] = bf16(a . Wd^T [* s]).
//   COMBINE: y[t] = bf16(sum_k w[t,k] * part[t*nk+k]) (fp32, slots in order) (+ residual, rounded again),
//            the reference's f32(bf16(acc)) * w summed over slots (fused_moe.py:147-148, 196).
// Tiles are ordered expert-major, then column tile, then block, and dealt out to the 8 XCDs in contiguous
// runs, so the blocks that share a weight tile run together on one XCD and hit its L2. The k loop copies
// 64-wide slabs of the activation rows and of the weight rows straight into LDS (global_load_lds, several
// slabs in flight) and feeds v_mfma_f32_16x16x32_bf16 from there. int8 weights stay int8 in LDS and are
// widened to bf16 (exact for |q| <= 127) as fragments are read.
#include "mm_common.h"
#include "mm_select.h"

namespace {

using namespace mmd;

// Rows (pairs) per expert block, = align block_m: 64, or 128 for bf16 weights when experts average at least
// 128 pairs (then every weight slab feeds twice the MFMA rows: the 2048-token Zipf block runs 18% faster,
// while a 512-token block, about 55 pairs per expert, runs 8% slower). kBM is the largest.
constexpr int kBM = 128;
constexpr int kBMSmall = 64;
constexpr int kXcds = 8;
// Tile shape per weight type and GEMM: output columns per tile (BN) and waves per workgroup. The k-slab is
// 64 elements, with 2 slabs in flight (LDS = slabs x (BM x 128 B + BN x 64 x weight bytes): three 64-pair
// bf16 workgroups share a CU, two of 128-pair tiles), except the gate/up GEMM on the row layout, whose
// 64-pair bf16 tiles keep 3 in flight (two workgroups per CU; slabs_in_flight). Waves
// split the BM x BN tile as 1 x 4 (4 waves, each BM rows x BN/4) or 2 x NW/2 (8 waves, or 64-column
// tiles). Measured on the 512-token block: 8-wave 128-column bf16 tiles are the fastest of 64/128/256
// columns x 4/8 waves x 2/3 slabs; on the 2048-token Zipf block the same shape with 128-pair blocks beats
// 16 waves, 4 waves of 64 x 64, 3-4 slabs, 32-k slabs and 256-column tiles.
#ifndef MM_PREFILL_GU_BN_BF16
#define MM_PREFILL_GU_BN_BF16 128
#endif
#ifndef MM_PREFILL_DOWN_BN_BF16
#define MM_PREFILL_DOWN_BN_BF16 128
#endif
#ifndef MM_PREFILL_GU_BN_INT8
#define MM_PREFILL_GU_BN_INT8 256
#endif
#ifndef MM_PREFILL_DOWN_BN_INT8
#define MM_PREFILL_DOWN_BN_INT8 256
#endif
#ifndef MM_PREFILL_GU_WAVES_BF16
#define MM_PREFILL_GU_WAVES_BF16 8
#endif
#ifndef MM_PREFILL_DOWN_WAVES_BF16
#define MM_PREFILL_DOWN_WAVES_BF16 8
#endif
#ifndef MM_PREFILL_GU_WAVES_INT8
#define MM_PREFILL_GU_WAVES_INT8 4
#endif
#ifndef MM_PREFILL_DOWN_WAVES_INT8
#define MM_PREFILL_DOWN_WAVES_INT8 4
#endif

// Rows per piece of the prefill copy of w_gu: [E1][2I/R][H/64][R][64], so a 64-k slab of R consecutive rows is
// one piece of R * 64 weights. bf16: R = 8 makes a piece the 1 KB that one direct-load instruction of a wave fills
// (8 rows x 128 bytes): measured on the 512-token block, gate/up 163.5 us with the row layout, 156-157 / 146-149 /
// 140-143 / 142-145 us with R = 2 / 4 / 8 / 16. int8: R = 16, the same 1 KB (16 rows x 64 bytes).
#ifndef MM_SLAB_ROWS
#define MM_SLAB_ROWS 8
#endif
constexpr int kSlabRows = MM_SLAB_ROWS;
constexpr int kSlabRowsI8 = 2 * kSlabRows;
constexpr int slab_rows(bool q) { return q ? kSlabRowsI8 : kSlabRows; }

// The gated activations a (gate/up output, down input) in 64-column slabs per expert block: [nb][ceil(I/64)][BM][64],
// so that each A slab of a down tile is one contiguous BM x 128-byte piece (read by 1 KB direct loads, as the weight
// copies are) instead of BM row pieces scattered by pair index. 0: rows by pair index, [P][I].
#ifndef MM_PREFILL_A_SLABS
#define MM_PREFILL_A_SLABS 1
#endif

struct PrefillArgs {
  const uint16_t* x;
  int64_t xs;
  int n_tokens, nk, P, E1;
  const void* ids;
  int ids_dtype;
  const float* wts;
  const int32_t* sorted_ids;
  const int32_t* bexp;
  const int32_t* offsets;  // [E1+1] padded start row of each expert, used rows last
  const void* w_gu;
  const void* w_d;
  const void* s_gu;
  const void* s_d;
  int s_dtype;
  int64_t H, I;
  int64_t gu_se, gu_sn, d_se, d_sn, sgu_se, sd_se;
  int gu_slabs;  // w_gu is the prefill copy: [E1][2I/R][H/64][R][64], R = slab_rows(int8)
  int d_slabs;   // w_d is the prefill copy: [E1][H/R][I/64][R][64]
  const uint16_t* res;
  int64_t res_rs;
  uint16_t* a_buf;
  uint16_t* part;
  uint16_t* y;
  int64_t ys;
};

// Tile of this workgroup: expert e, block blk (rows blk*BM ..), column tile nt. False: no tile.
template <int BM>
__device__ __forceinline__ bool map_tile(const PrefillArgs& a, int NT, int& e, int& blk, int& nt) {
  const int used_blocks = a.offsets[a.E1] / BM;
  const int G = used_blocks * NT;
  const int per = (G + kXcds - 1) / kXcds;
  const int w = blockIdx.x;
  const int idx = w / kXcds, xcd = w % kXcds;  // workgroups are dealt to XCDs round robin
  if (idx >= per) return false;
  const int L = xcd * per + idx;
  if (L >= G) return false;
  e = a.bexp[L / NT];
  const int b0 = a.offsets[e] / BM, nblk = a.offsets[e + 1] / BM - b0;
  const int local = L - b0 * NT;
  nt = local / nblk;
  blk = b0 + local % nblk;
  return true;
}

// ---------------------------------------------------------------------------------- k-slab pipeline
//
// Each k-slab (BK k) of the tile is copied global -> LDS by global_load_lds_dwordx4: one wave instruction
// fills 1 KB of LDS in lane order, and each lane picks the 16-byte global chunk that belongs at its LDS
// position. Rows and k past the operand (padding pairs, columns past the weight, the k tail) read a
// zero chunk. NS slabs are in flight; the wave waits on vmcnt for the oldest and a barrier makes it
// visible to every wave. Rows of R bytes (bf16: 2*BK, int8 weights: BK) hold R/16 chunks; chunk c of row
// r sits at r*R + (c ^ s(r))*16 with s(r) = (r / rows-per-256-bytes) mod min(R/16, 16), so the 16 rows
// that one MFMA fragment reads (same logical chunk) fall on distinct bank groups.
// A lane's MFMA k-chunk for step ks of lane quarter lq is ks*4 + lq (bf16 weights) or, for int8 weights
// (one 16-byte int8 chunk widens into two steps), 8g + 2lq + ks in 64-k group g; A follows the same choice.

__device__ __attribute__((aligned(16))) uint4 g_zero_chunk[1];  // 16 zero bytes for masked lanes

// Slabs in flight. Measured on the 512-token block (µs): the gate/up GEMM on the row layout 163.3-166.0 with 3
// (two workgroups per CU) against 168.3-169.2 with 2 (three per CU); on the prefill copy 141.6-144.8 with 3
// against 137.7-139.1 with 2; the down GEMM 80.6-81.3 with 3 against 77.1-78.1 with 2.
constexpr int slabs_in_flight(bool q, int bn, int bm, bool row_gate_up) {
  return row_gate_up && !q && bn < 256 && bm <= kBMSmall ? 3 : 2;
}

template <bool Quant, int TileN, int Waves = 4, int BlockM = kBMSmall, bool RowGateUp = false>
struct Geo {
  static constexpr bool Q = Quant;
  static constexpr int BM = BlockM;                   // rows (pairs) per tile
  static constexpr int BN = TileN;                    // output columns per tile
  static constexpr int NW = Waves;                    // waves per workgroup
  static constexpr int BK = 64;                       // k elements per slab
  static constexpr int NS = slabs_in_flight(Q, BN, BM, RowGateUp);
  static constexpr int WM = (BN <= 64 || NW == 8) ? 2 : 1;  // wave rows
  static constexpr int WN = NW / WM;                  // wave columns
  static constexpr int FM = BM / WM / 16;             // 16-row fragments per wave
  static constexpr int FN = BN / WN / 16;             // 16-column fragments per wave
  static constexpr int AROW = BK * 2;                 // activation (bf16) bytes per row per slab
  static constexpr int ROWB = Q ? BK : BK * 2;        // weight bytes per row per slab
  static constexpr int A_BYTES = BM * AROW;
  static constexpr int B_BYTES = BN * ROWB;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr size_t LDS = static_cast<size_t>(NS) * STAGE;
  static constexpr int A_INSTR = A_BYTES / 1024 / NW;  // direct-load instructions per wave per slab
  static constexpr int B_INSTR = B_BYTES / 1024 / NW;
  static constexpr int LOADS = A_INSTR + B_INSTR;
  static constexpr int KSTEPS = BK / 32;              // MFMA k-steps per slab
  static_assert((BN == 64 || BN == 128 || BN == 256) && (NW == 4 || NW == 8) && FN % 2 == 0, "tile shape");
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "slab must split over the waves in 1 KB pieces");
};

// LDS byte position of 16-byte chunk c of row r in a slab with rows of `rowb` bytes. The XOR swizzle puts
// the 16 rows read by one MFMA fragment (same logical chunk) on distinct 16-byte bank groups.
template <int rowb>
__device__ __forceinline__ int pos_row(int r, int c) {
  constexpr int ch = rowb / 16;                     // chunks per row
  constexpr int rp = rowb >= 256 ? 1 : 256 / rowb;  // rows per 256 bytes (one pass over the banks)
  constexpr int mask = ch < 16 ? ch - 1 : 15;
  return r * rowb + ((c ^ ((r / rp) & mask)) << 4);
}


// Per-thread source rows of the direct loads: for A instruction j the lane fills tile row ra[j], logical
// chunk ca[j]; for B instruction j tile row rb[j], logical chunk cb[j].
template <class G>
struct LoadMap {
  int ra[G::A_INSTR], ca[G::A_INSTR];
  int rb[G::B_INSTR], cb[G::B_INSTR];
  __device__ __forceinline__ LoadMap() {
    constexpr int ACH = G::AROW / 16, BCH = G::ROWB / 16;  // chunks per row
    const int w = threadIdx.x / kWave, l = lane_id();
#pragma unroll
    for (int j = 0; j < G::A_INSTR; ++j) {
      ra[j] = (w * G::A_INSTR + j) * (64 / ACH) + l / ACH;
      // the lane's LDS position holds physical chunk l % ACH; the swizzle is an involution, so the
      // logical chunk is the position the swizzle gives that physical chunk
      ca[j] = (pos_row<G::AROW>(ra[j], l % ACH) - ra[j] * G::AROW) >> 4;
    }
#pragma unroll
    for (int j = 0; j < G::B_INSTR; ++j) {
      rb[j] = (w * G::B_INSTR + j) * (64 / BCH) + l / BCH;
      cb[j] = (pos_row<G::ROWB>(rb[j], l % BCH) - rb[j] * G::ROWB) >> 4;
    }
  }
};

// Issues the direct loads of slab kt into LDS stage `st` (arow/brow: this thread's source row starts,
// null for masked rows; k counted in elements; slab kt of an activation row starts kt * aslab elements in, of a
// weight row kt * bslab).
template <class G>
__device__ __forceinline__ void issue_slab(char* lds, int st, int kt, int64_t K, const LoadMap<G>& m,
                                           const uint16_t* const* arow, const char* const* brow, int64_t aslab,
                                           int64_t bslab) {
  constexpr int ES = G::Q ? 1 : 2;
  char* sa = lds + st * G::STAGE;
  char* sb = sa + G::A_BYTES;
  const int w = threadIdx.x / kWave;
  const int64_t k0 = static_cast<int64_t>(kt) * G::BK;
#pragma unroll
  for (int j = 0; j < G::A_INSTR; ++j) {
    const int64_t k = k0 + m.ca[j] * 8, ka = kt * aslab + m.ca[j] * 8;
    const void* src = (arow[j] && k < K) ? static_cast<const void*>(arow[j] + ka) : static_cast<const void*>(g_zero_chunk);
    load_lds16(src, sa + (w * G::A_INSTR + j) * 1024);
  }
#pragma unroll
  for (int j = 0; j < G::B_INSTR; ++j) {
    const int64_t k = k0 + m.cb[j] * (16 / ES), kb = kt * bslab + m.cb[j] * (16 / ES);
    const void* src = (brow[j] && k < K) ? static_cast<const void*>(brow[j] + kb * ES) : static_cast<const void*>(g_zero_chunk);
    load_lds16(src, sb + (w * G::B_INSTR + j) * 1024);
  }
}

__device__ __forceinline__ bf16x8_t lds_frag16(const char* base, int pos) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(base + pos));
}

// Rows of the expert block in spair that hold pairs (< P). align pads each expert's rows at the end of
// its run, so they are a prefix of the block. Wave-uniform.
template <int BM>
__device__ __forceinline__ int valid_rows(const int* spair, int P) {
  int n = 0;
#pragma unroll
  for (int r = 0; r < BM; r += kWave) n += __popcll(__ballot(spair[r + lane_id()] < P));
  return __builtin_amdgcn_readfirstlane(n);
}

// The shared GEMM body: acc[i][j] (i: 16-row fragment of the wave's rows starting at tile row r0, j: its
// 16-column fragments) over K; bcol(j) is the tile row (B row) of column fragment j; xrow(r) / wrow(r) is
// where activation / weight row r's first slab starts and aslab / bslab the elements between its slabs. Row fragments at or
// past fm_live (wave-uniform) hold only padding rows: their LDS reads and MFMAs are skipped and their
// accumulators stay zero (the epilogues store no padding row).
template <class G, class XRowFn, class WRowFn, class BColFn>
__device__ __forceinline__ void tile_gemm(floatx4 (&acc)[G::FM][G::FN], int64_t K, XRowFn xrow, int64_t aslab,
                                          WRowFn wrow, int64_t bslab, char* lds, int r0, BColFn bcol, int fm_live) {
  constexpr int NS = G::NS, LOADS = G::LOADS, FM = G::FM, FN = G::FN;
  const int lane = lane_id();
  const int lr = lane & 15, lq = lane >> 4;
  const LoadMap<G> m;
  const uint16_t* arow[G::A_INSTR];
  const char* brow[G::B_INSTR];
#pragma unroll
  for (int j = 0; j < G::A_INSTR; ++j) arow[j] = xrow(m.ra[j]);
#pragma unroll
  for (int j = 0; j < G::B_INSTR; ++j) brow[j] = wrow(m.rb[j]);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int nk = static_cast<int>((K + G::BK - 1) / G::BK);
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue_slab<G>(lds, s, s, K, m, arow, brow, aslab, bslab);
  for (int kt = 0; kt < nk; ++kt) {
    // slabs issued after kt so far: min(nk - 1 - kt, NS - 2); wait for kt's own loads
    const int pending = min(nk - 1 - kt, NS - 2);
    static_assert(NS >= 2 && NS <= 6 && (NS - 2) * LOADS < 64, "slab count");
    switch (pending) {
      case 4: wait_vmcnt<(NS >= 6 ? 4 : 0) * LOADS>(); break;
      case 3: wait_vmcnt<(NS >= 5 ? 3 : 0) * LOADS>(); break;
      case 2: wait_vmcnt<(NS >= 4 ? 2 : 0) * LOADS>(); break;
      case 1: wait_vmcnt<LOADS>(); break;
      default: wait_vmcnt<0>(); break;
    }
    // slab kt visible to all waves; every wave is done with slab kt-1. A plain barrier: the loads of
    // slab kt were waited for above, and a memory fence would also wait for the later slabs' loads.
    __builtin_amdgcn_s_barrier();
    if (kt + NS - 1 < nk) issue_slab<G>(lds, (kt + NS - 1) % NS, kt + NS - 1, K, m, arow, brow, aslab, bslab);
    const char* sa = lds + (kt % NS) * G::STAGE;
    const char* sb = sa + G::A_BYTES;
    if constexpr (G::Q) {
      // one 16-byte int8 chunk (16 k) per lane and fragment feeds two 32-wide steps: in 64-k group g the
      // lane quarter lq takes int8 chunk 4g + lq, i.e. bf16 activation chunks 8g + 2lq (+1)
#pragma unroll
      for (int g = 0; g < G::BK / 64; ++g) {
        bf16x8_t fb[2][FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          uint4 lo, hi;
          widen_i8(*reinterpret_cast<const uint4*>(sb + pos_row<G::ROWB>(bcol(j) + lr, 4 * g + lq)), lo, hi);
          fb[0][j] = __builtin_bit_cast(bf16x8_t, lo);
          fb[1][j] = __builtin_bit_cast(bf16x8_t, hi);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          bf16x8_t fa[FM];
#pragma unroll
          for (int i = 0; i < FM; ++i)
            if (i < fm_live) fa[i] = lds_frag16(sa, pos_row<G::AROW>(r0 + 16 * i + lr, 8 * g + 2 * lq + ks));
#pragma unroll
          for (int i = 0; i < FM; ++i)
            if (i < fm_live)
#pragma unroll
              for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[ks][j], acc[i][j], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < G::KSTEPS; ++ks) {
        const int ch = ks * 4 + lq;
        bf16x8_t fa[FM], fb[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          if (i < fm_live) fa[i] = lds_frag16(sa, pos_row<G::AROW>(r0 + 16 * i + lr, ch));
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j] = lds_frag16(sb, pos_row<G::ROWB>(bcol(j) + lr, ch));
#pragma unroll
        for (int i = 0; i < FM; ++i)
          if (i < fm_live)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
    }
  }
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Epilogue store: the tile's bf16 outputs sit in LDS as [BM][NC] rows (row stride os elements); each thread
// writes 16-byte chunks of them to dst[pair][col0 + ...] (row stride ld), consecutive threads along a row, so a
// row goes out as one NC * 2-byte run. Padding rows (pair >= P) and chunks past ncols (a multiple of 8) are
// skipped. NTS: nontemporal stores, for outputs that the next kernel reads back from memory anyway (2 us of the
// 512-token down GEMM; against one 2-byte store per element and lane, which wrote 4 rows x 32 bytes per
// instruction, the rows cost 2 us less at 512 tokens and 8 us less on the 2048-token Zipf block).
template <int BM, int NC, int NT, bool NTS = false>
__device__ __forceinline__ void store_rows(const uint16_t* ot, int os, const int* spair, int P, uint16_t* dst,
                                           int64_t ld, int64_t col0, int64_t ncols) {
  constexpr int CPR = NC / 8;  // 16-byte chunks per row
  static_assert(NC % 8 == 0, "whole chunks");
#pragma unroll
  for (int q = threadIdx.x; q < BM * CPR; q += NT) {
    const int r = q / CPR, cc = q % CPR;
    const int p = spair[r];
    const int64_t col = col0 + cc * 8;
    if (p < P && col < ncols) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ot + r * os + cc * 8);
      u32x4_t* d = reinterpret_cast<u32x4_t*>(dst + static_cast<int64_t>(p) * ld + col);
      if constexpr (NTS) __builtin_nontemporal_store(v, d);
      else *d = v;
    }
  }
}

// The gated activations of a gate/up tile into the block's slabs (dst: the block's first slab; column col of row r at
// ((col / 64) * BM + r) * 64 + col % 64): consecutive threads write consecutive 16-byte chunks, so 8 rows of a
// 64-column slab go out as 1 KB. Padding rows (pair >= P) and chunks past ncols are skipped.
template <int BM, int NC, int NT>
__device__ __forceinline__ void store_slab_rows(const uint16_t* ot, int os, const int* spair, int P, uint16_t* dst,
                                                int64_t col0, int64_t ncols) {
  constexpr int CPR = NC / 8;
  static_assert(NC % 8 == 0, "whole chunks");
#pragma unroll
  for (int q = threadIdx.x; q < BM * CPR; q += NT) {
    const int r = q / CPR, cc = q % CPR;
    const int64_t col = col0 + cc * 8;
    if (spair[r] < P && col < ncols) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ot + r * os + cc * 8);
      *reinterpret_cast<u32x4_t*>(dst + ((col >> 6) * BM + r) * 64 + (col & 63)) = v;
    }
  }
}

// ------------------------------------------------------------------------------------------- gate / up

// SL: the weights are the prefill copy of w_gu (kSlabRows-row pieces), else the row layout.
template <bool Q, int BN, int NW, int BM, bool SL = false>
__global__ __launch_bounds__(NW * 64) void prefill_gate_up_kernel(PrefillArgs a) {
  using G = Geo<Q, BN, NW, BM, !SL>;
  constexpr int HALF = G::BN / 2;  // gate columns per tile (and as many up columns)
  extern __shared__ uint4 lds_raw[];
  __shared__ int spair[BM];
  const int NT = static_cast<int>((a.I + HALF - 1) / HALF);
  int e, blk, nt;
  if (!map_tile<BM>(a, NT, e, blk, nt)) return;
  constexpr int ES = Q ? 1 : 2;
  const int64_t I = a.I, n0 = static_cast<int64_t>(nt) * HALF;
  if (threadIdx.x < BM) spair[threadIdx.x] = a.sorted_ids[static_cast<int64_t>(blk) * BM + threadIdx.x];
  __syncthreads();
  // activation row of tile row r (token of pair spair[r]); weight row of tile column r (gate columns
  // first, then the matching up rows); null = masked
  auto xrow = [&](int r) -> const uint16_t* {
    const int p = spair[r];
    return p < a.P ? a.x + static_cast<int64_t>(p / a.nk) * a.xs : nullptr;
  };
  constexpr int R = slab_rows(Q);
  const char* wbase = static_cast<const char*>(a.w_gu) + static_cast<int64_t>(e) * a.gu_se * ES;
  auto wrow = [&](int r) -> const char* {
    const int64_t col = n0 + (r % HALF), rr = r < HALF ? col : I + col;
    // the prefill copy: row rr is row rr % R of piece group rr / R, whose 64-k slabs are R * 64 elements apart
    const int64_t off = SL ? (rr / R) * R * a.H + (rr % R) * 64 : rr * a.gu_sn;
    return col < I ? wbase + off * ES : nullptr;
  };
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int wm = wave / G::WN, wn = wave % G::WN;
  const int r0 = wm * (BM / G::WM);
  constexpr int FG = G::FN / 2;      // gate fragments of the wave; the next FG are the matching up ones
  const int g0 = wn * FG * 16;       // first gate column of the wave, relative to n0
  floatx4 acc[G::FM][G::FN];
  const int fm_live = min(max((valid_rows<BM>(spair, a.P) - r0 + 15) / 16, 0), G::FM);
  tile_gemm<G>(acc, a.H, xrow, G::BK, wrow, SL ? R * G::BK : G::BK, reinterpret_cast<char*>(lds_raw), r0,
               [&](int j) { return (j < FG ? 0 : HALF) + g0 + 16 * (j % FG); }, fm_live);
  // the output tile [BM][HALF] goes through LDS (free once every wave is past the last slab), then out in rows
  constexpr int OS = HALF + 8;  // row stride (elements): rows 4 apart start 64 bytes apart on the banks
  static_assert(static_cast<size_t>(BM) * OS * 2 <= G::LDS, "gate/up output tile must fit in the k-slab LDS");
  uint16_t* ot = reinterpret_cast<uint16_t*>(lds_raw);
  // int8: the row scales of the wave's columns, all requested before the first is used and without a branch on the
  // scale type (one trip to memory; loaded per fragment behind that branch, each waited on in turn)
  float sgv[FG], suv[FG];
#pragma unroll
  for (int j = 0; j < FG; ++j) sgv[j] = suv[j] = 1.f;
  if constexpr (Q) {
    const ScaleRow sr = scale_row(a.s_gu, a.s_dtype, static_cast<int64_t>(e) * a.sgu_se, 2 * I);
#pragma unroll
    for (int j = 0; j < FG; ++j) {
      const uint32_t col = static_cast<uint32_t>(min(n0 + g0 + 16 * j + (lane & 15), I - 1));
      sgv[j] = scale_at(sr, col);
      suv[j] = scale_at(sr, col + static_cast<uint32_t>(I));
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < FG; ++j) {
    const int c = g0 + 16 * j + (lane & 15);  // tile column; columns past I are never stored
    const float sg = sgv[j], su = suv[j];
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = r0 + 16 * i + 4 * (lane >> 4) + v;  // D[row = 4*(lane/16) + v][col = lane%16]
        float g = acc[i][j][v], u = acc[i][j + FG][v];
        if (Q) { g *= sg; u *= su; }
        const float gg = round_bf16(g), uu = round_bf16(u);
        ot[r * OS + c] = f32_to_bf16(round_bf16(silu(gg)) * uu);
      }
  }
  __syncthreads();
  if constexpr (MM_PREFILL_A_SLABS)
    store_slab_rows<BM, HALF, NW * 64>(ot, OS, spair, a.P, a.a_buf + static_cast<int64_t>(blk) * ((I + 63) / 64) * BM * 64,
                                       n0, I);
  else
    store_rows<BM, HALF, NW * 64>(ot, OS, spair, a.P, a.a_buf, I, n0, I);
}

// ----------------------------------------------------------------------------------------------- down

// SL: the weights are the prefill copy of w_d (kSlabRows-row pieces), else the row layout.
template <bool Q, int BN, int NW, int BM, bool SL = false>
__global__ __launch_bounds__(NW * 64) void prefill_down_kernel(PrefillArgs a) {
  using G = Geo<Q, BN, NW, BM>;
  extern __shared__ uint4 lds_raw[];
  __shared__ int spair[BM];
  const int NT = static_cast<int>((a.H + G::BN - 1) / G::BN);
  int e, blk, nt;
  if (!map_tile<BM>(a, NT, e, blk, nt)) return;
  constexpr int ES = Q ? 1 : 2;
  const int64_t H = a.H, I = a.I, h0 = static_cast<int64_t>(nt) * G::BN;
  if (threadIdx.x < BM) spair[threadIdx.x] = a.sorted_ids[static_cast<int64_t>(blk) * BM + threadIdx.x];
  __syncthreads();
  // the block's slabs of a (row r of slab kt at (kt * BM + r) * 64), or rows by pair index
  const uint16_t* ablk = a.a_buf + static_cast<int64_t>(blk) * ((I + 63) / 64) * BM * 64;
  auto xrow = [&](int r) -> const uint16_t* {
    const int p = spair[r];
    if constexpr (MM_PREFILL_A_SLABS) return p < a.P ? ablk + r * 64 : nullptr;
    else return p < a.P ? a.a_buf + static_cast<int64_t>(p) * I : nullptr;
  };
  constexpr int R = slab_rows(Q);
  const char* wbase = static_cast<const char*>(a.w_d) + static_cast<int64_t>(e) * a.d_se * ES;
  auto wrow = [&](int r) -> const char* {
    const int64_t h = h0 + r;
    const int64_t off = SL ? (h / R) * R * I + (h % R) * 64 : h * a.d_sn;
    return h < H ? wbase + off * ES : nullptr;
  };
  const int wave = threadIdx.x / kWave, lane = lane_id();
  const int wm = wave / G::WN, wn = wave % G::WN;
  const int r0 = wm * (BM / G::WM);
  const int c0 = wn * G::FN * 16;
  floatx4 acc[G::FM][G::FN];
  const int fm_live = min(max((valid_rows<BM>(spair, a.P) - r0 + 15) / 16, 0), G::FM);
  tile_gemm<G>(acc, I, xrow, MM_PREFILL_A_SLABS ? BM * 64 : G::BK, wrow, SL ? R * G::BK : G::BK,
               reinterpret_cast<char*>(lds_raw), r0, [&](int j) { return c0 + 16 * j; }, fm_live);
  // the output tile [BM][BN] goes through LDS, then out in rows (as in gate/up)
  constexpr int OS = G::BN + 8;
  static_assert(static_cast<size_t>(BM) * OS * 2 <= G::LDS, "down output tile must fit in the k-slab LDS");
  uint16_t* ot = reinterpret_cast<uint16_t*>(lds_raw);
  float scv[G::FN];  // int8: the wave's row scales, requested together (as in gate/up)
#pragma unroll
  for (int j = 0; j < G::FN; ++j) scv[j] = 1.f;
  if constexpr (Q) {
    const ScaleRow sr = scale_row(a.s_d, a.s_dtype, static_cast<int64_t>(e) * a.sd_se, H);
#pragma unroll
    for (int j = 0; j < G::FN; ++j) scv[j] = scale_at(sr, static_cast<uint32_t>(min(h0 + c0 + 16 * j + (lane & 15), H - 1)));
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < G::FN; ++j) {
    const int c = c0 + 16 * j + (lane & 15);
    const float sc = scv[j];
#pragma unroll
    for (int i = 0; i < G::FM; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = r0 + 16 * i + 4 * (lane >> 4) + v;
        ot[r * OS + c] = f32_to_bf16(Q ? acc[i][j][v] * sc : acc[i][j][v]);
      }
  }
  __syncthreads();
  store_rows<BM, G::BN, NW * 64, true>(ot, OS, spair, a.P, a.part, H, h0, H);  // read back by the combine
}

// -------------------------------------------------------------------------------------------- combine

// One thread per 8 consecutive outputs of a token: y = bf16(sum_k w_k * part_k) (+ residual, rounded again), slots
// in order. MAXK > 0: up to MAXK slots, every slot's id, weight and part chunk loaded before the first sum (a dropped
// pair's part row is never written: its term is skipped by a select, not multiplied by zero), so the thread waits
// for memory once; MAXK = 0: any number of slots, one at a time.
template <int MAXK, bool I64>
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillArgs a) {
  const int64_t H8 = a.H / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(a.n_tokens) * H8) return;
  const int64_t t = idx / H8, h = (idx % H8) * 8;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  auto add = [&](bool ok, float w, const uint4& v) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = ok ? fmaf(w, __uint_as_float(u[i] << 16), acc[2 * i]) : acc[2 * i];
      acc[2 * i + 1] = ok ? fmaf(w, __uint_as_float(u[i] & 0xffff0000u), acc[2 * i + 1]) : acc[2 * i + 1];
    }
  };
  uint16_t rraw[8];  // the residual, fetched with the slots' loads
  if (a.res) {
    const uint16_t* rr = a.res + t * a.res_rs + h;
    if ((reinterpret_cast<uintptr_t>(a.res) & 15) == 0 && (a.res_rs & 7) == 0) {  // uniform
      const uint4 r = *reinterpret_cast<const uint4*>(rr);
      const uint32_t ru[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rraw[2 * i] = static_cast<uint16_t>(ru[i] & 0xffff);
        rraw[2 * i + 1] = static_cast<uint16_t>(ru[i] >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) rraw[i] = rr[i];
    }
  }
  if constexpr (MAXK > 0) {
    int64_t id[MAXK];
    float w[MAXK];
    uint4 v[MAXK];
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {  // slots past nk load the last slot again (not used)
      const int64_t p = t * a.nk + min(k, a.nk - 1);
      id[k] = I64 ? static_cast<const int64_t*>(a.ids)[p] : static_cast<const int32_t*>(a.ids)[p];
      w[k] = a.wts[p];
      v[k] = *reinterpret_cast<const uint4*>(a.part + p * a.H + h);
    }
#pragma unroll
    for (int k = 0; k < MAXK; ++k) add(k < a.nk && id[k] >= 0 && id[k] < a.E1, w[k], v[k]);
  } else {
    for (int k = 0; k < a.nk; ++k) {
      const int64_t p = t * a.nk + k;
      const int64_t id = load_id(a.ids, a.ids_dtype, p);
      if (id < 0 || id >= a.E1) continue;  // dropped pairs have no row
      add(true, a.wts[p], *reinterpret_cast<const uint4*>(a.part + p * a.H + h));
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float lo = round_bf16(acc[2 * i]), hi = round_bf16(acc[2 * i + 1]);
    if (a.res) {
      lo += bf16_to_f32(rraw[2 * i]);
      hi += bf16_to_f32(rraw[2 * i + 1]);
    }
    o[i] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
  }
  uint16_t* yr = a.y + t * a.ys + h;
  if ((reinterpret_cast<uintptr_t>(yr) & 15) == 0) {
    *reinterpret_cast<uint4*>(yr) = make_uint4(o[0], o[1], o[2], o[3]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      yr[2 * i] = static_cast<uint16_t>(o[i] & 0xffff);
      yr[2 * i + 1] = static_cast<uint16_t>(o[i] >> 16);
    }
  }
}

constexpr int kCombineMaxK = 16;

template <bool Q, int BN, int NW, int BM, bool SL>
int launch_gate_up(const PrefillArgs& a, int64_t nb, hipStream_t st) {
  using G = Geo<Q, BN, NW, BM, !SL>;
  const int64_t nt = (a.I + G::BN / 2 - 1) / (G::BN / 2);
  const int64_t g = (nb * nt + kXcds - 1) / kXcds * kXcds;
  int rc = mm::allow_lds(prefill_gate_up_kernel<Q, BN, NW, BM, SL>, G::LDS, "prefill_gate_up");
  if (rc) return rc;
  hipLaunchKernelGGL((prefill_gate_up_kernel<Q, BN, NW, BM, SL>), dim3(static_cast<unsigned>(g)), dim3(NW * 64), G::LDS,
                     st, a);
  return mm::check_launch("moe_prefill gate_up");
}

template <bool Q, int BN, int NW, int BM, bool SL>
int launch_down(const PrefillArgs& a, int64_t nb, hipStream_t st) {
  using G = Geo<Q, BN, NW, BM>;
  const int64_t nt = (a.H + G::BN - 1) / G::BN;
  const int64_t g = (nb * nt + kXcds - 1) / kXcds * kXcds;
  int rc = mm::allow_lds(prefill_down_kernel<Q, BN, NW, BM, SL>, G::LDS, "prefill_down");
  if (rc) return rc;
  hipLaunchKernelGGL((prefill_down_kernel<Q, BN, NW, BM, SL>), dim3(static_cast<unsigned>(g)), dim3(NW * 64), G::LDS, st,
                     a);
  return mm::check_launch("moe_prefill down");
}

template <bool Q, int BM>
int launch_gemms(const PrefillArgs& a, int64_t nb, int phases, hipStream_t st) {
  constexpr int GU_BN = Q ? MM_PREFILL_GU_BN_INT8 : MM_PREFILL_GU_BN_BF16;
  constexpr int DOWN_BN = Q ? MM_PREFILL_DOWN_BN_INT8 : MM_PREFILL_DOWN_BN_BF16;
  constexpr int GU_NW = Q ? MM_PREFILL_GU_WAVES_INT8 : MM_PREFILL_GU_WAVES_BF16;
  constexpr int DOWN_NW = Q ? MM_PREFILL_DOWN_WAVES_INT8 : MM_PREFILL_DOWN_WAVES_BF16;
  int rc;
  if (phases & MM_PHASE_GATE_UP) {
    rc = a.gu_slabs ? launch_gate_up<Q, GU_BN, GU_NW, BM, true>(a, nb, st) : launch_gate_up<Q, GU_BN, GU_NW, BM, false>(a, nb, st);
    if (rc) return rc;
  }
  if (phases & MM_PHASE_DOWN) {
    rc = a.d_slabs ? launch_down<Q, DOWN_BN, DOWN_NW, BM, true>(a, nb, st) : launch_down<Q, DOWN_BN, DOWN_NW, BM, false>(a, nb, st);
    if (rc) return rc;
  }
  return MM_OK;
}

// The prefill copy of a weight stack w [E1, rows, K] of ES-byte weights (w_gu: rows 2I, K = H; w_d: rows H, K = I),
// one 16-byte chunk per thread in output order (grid-stride). A piece (64 chunks, 1 KB) holds the 64-k slab of R
// rows, C = 64 * ES / 16 chunks per row: chunk c of expert e is chunk c % C of row j = (c / C) % R of k-slab
// t = (c / 64) % KT of row group q = c / (64 KT), KT = K / 64, R = 64 / C.
template <int ES>
__global__ __launch_bounds__(256) void slab_copy_kernel(const char* __restrict__ w, int64_t se, int64_t sn,
                                                       int64_t rows, int64_t K, int64_t total, uint4* __restrict__ out) {
  constexpr int C = 64 * ES / 16, R = 64 / C;
  static_assert(R == slab_rows(ES == 1), "piece rows");
  const int64_t per = rows * K * ES / 16, KT = K / 64;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; c < total;
       c += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t e = c / per, ce = c - e * per;
    const int64_t ch = ce % C, j = (ce / C) % R, t = (ce / 64) % KT, q = ce / (64 * KT);
    out[c] = *reinterpret_cast<const uint4*>(w + (e * se + (R * q + j) * sn + 64 * t) * ES + ch * 16);
  }
}

// Launches the copy of one stack (ES from the descriptor's weight type).
int launch_slab_copy(const void* w, int w_dtype, int64_t se, int64_t sn, int64_t rows, int64_t K, int64_t bytes,
                     void* out, void* stream, const char* what) {
  const int64_t total = bytes / 16;
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
  if (w_dtype == MM_INT8)
    hipLaunchKernelGGL(slab_copy_kernel<1>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, MM_STREAM(stream),
                       static_cast<const char*>(w), se, sn, rows, K, total, static_cast<uint4*>(out));
  else
    hipLaunchKernelGGL(slab_copy_kernel<2>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, MM_STREAM(stream),
                       static_cast<const char*>(w), se, sn, rows, K, total, static_cast<uint4*>(out));
  return mm::check_launch(what);
}

}  // namespace

namespace mm {
int check_experts(const char* who, const mm_experts* ex);
}

static int64_t weight_bytes(const mm_experts* ex) {
  return ex->w_dtype == MM_INT8 ? 1 : ex->w_dtype == MM_BF16 ? 2 : 0;
}

extern "C" int64_t mm_gate_up_slabs_bytes(const mm_experts* ex) {
  if (!ex || weight_bytes(ex) == 0 || ex->hidden <= 0 || ex->hidden % 64 != 0 || ex->inter <= 0 ||
      (2 * ex->inter) % slab_rows(ex->w_dtype == MM_INT8) != 0 || ex->n_slots <= 0)
    return 0;
  return ex->n_slots * 2 * ex->inter * ex->hidden * weight_bytes(ex);
}

extern "C" int mm_gate_up_slabs(const mm_experts* ex, void* out, void* stream) {
  // only w_gu is read: w_d, the scales and w_gu_slabs may be unset
  MM_REQUIRE(ex && ex->w_gu, "gate_up_slabs: null expert descriptor or w_gu");
  const int64_t bytes = mm_gate_up_slabs_bytes(ex);
  MM_REQUIRE(bytes > 0,
             "gate_up_slabs: needs bf16 or int8 experts, hidden a multiple of 64 and 2 * inter a multiple of %d (bf16) "
             "or %d (int8)", kSlabRows, kSlabRowsI8);
  const int64_t es = weight_bytes(ex);
  MM_REQUIRE(ex->gu_stride_n >= ex->hidden && ex->gu_stride_e >= 2 * ex->inter * ex->gu_stride_n,
             "gate_up_slabs: w_gu strides do not describe [E, 2I, H] with a contiguous last dim");
  MM_REQUIRE(mm::aligned16(ex->w_gu) && (ex->gu_stride_n * es) % 16 == 0 && (ex->gu_stride_e * es) % 16 == 0,
             "gate_up_slabs: w_gu rows must be 16-byte aligned");
  MM_REQUIRE(out && mm::aligned16(out), "gate_up_slabs: out must be a 16-byte aligned buffer");
  return launch_slab_copy(ex->w_gu, ex->w_dtype, ex->gu_stride_e, ex->gu_stride_n, 2 * ex->inter, ex->hidden, bytes, out,
                          stream, "gate_up_slabs");
}

extern "C" int64_t mm_down_slabs_bytes(const mm_experts* ex) {
  if (!ex || weight_bytes(ex) == 0 || ex->inter <= 0 || ex->inter % 64 != 0 || ex->hidden <= 0 ||
      ex->hidden % slab_rows(ex->w_dtype == MM_INT8) != 0 || ex->n_slots <= 0)
    return 0;
  return ex->n_slots * ex->hidden * ex->inter * weight_bytes(ex);
}

extern "C" int mm_down_slabs(const mm_experts* ex, void* out, void* stream) {
  // only w_d is read: w_gu, the scales and the copies may be unset
  MM_REQUIRE(ex && ex->w_d, "down_slabs: null expert descriptor or w_d");
  const int64_t bytes = mm_down_slabs_bytes(ex);
  MM_REQUIRE(bytes > 0,
             "down_slabs: needs bf16 or int8 experts, inter a multiple of 64 and hidden a multiple of %d (bf16) or %d "
             "(int8)", kSlabRows, kSlabRowsI8);
  const int64_t es = weight_bytes(ex);
  MM_REQUIRE(ex->d_stride_n >= ex->inter && ex->d_stride_e >= ex->hidden * ex->d_stride_n,
             "down_slabs: w_d strides do not describe [E, H, I] with a contiguous last dim");
  MM_REQUIRE(mm::aligned16(ex->w_d) && (ex->d_stride_n * es) % 16 == 0 && (ex->d_stride_e * es) % 16 == 0,
             "down_slabs: w_d rows must be 16-byte aligned");
  MM_REQUIRE(out && mm::aligned16(out), "down_slabs: out must be a 16-byte aligned buffer");
  return launch_slab_copy(ex->w_d, ex->w_dtype, ex->d_stride_e, ex->d_stride_n, ex->hidden, ex->inter, bytes, out, stream,
                          "down_slabs");
}

extern "C" int32_t mm_prefill_block_m(int64_t n_tokens, int64_t nk, int64_t n_slots, int w_dtype) {
  // bf16 experts averaging at least 128 pairs take 128-row blocks; everything else 64
  return w_dtype == MM_BF16 && n_slots > 0 && n_tokens * nk >= static_cast<int64_t>(kBM) * n_slots ? kBM : kBMSmall;
}

extern "C" int mm_moe_prefill(const void* x, int64_t n_tokens, int64_t x_row_stride, const mm_experts* ex, int64_t nk,
                              const void* ids, int ids_dtype, const float* wts, const int32_t* sorted_ids,
                              const int32_t* bexp, const int32_t* expert_offsets, int64_t nb, int32_t block_m,
                              const void* residual, int64_t res_row_stride, void* a_buf, void* part_buf, void* y,
                              int64_t y_row_stride, int phases, void* stream) {
  int rc = mm::check_experts("moe_prefill", ex);
  if (rc) return rc;
  MM_REQUIRE(block_m == kBMSmall || (block_m == kBM && ex->w_dtype == MM_BF16),
             "moe_prefill: block_m must be %d (or %d for bf16 experts; got %d)", kBMSmall, kBM, block_m);
  MM_REQUIRE(n_tokens >= 0 && nk >= 1 && n_tokens * nk <= (1LL << 30), "moe_prefill: bad token/slot counts");
  MM_REQUIRE(nb >= 0 && nb * 16 <= 0x7fffffffLL, "moe_prefill: bad block count");
  MM_REQUIRE(ex->n_slots <= 0x7fffffff && ex->hidden % 8 == 0, "moe_prefill: hidden must be a multiple of 8");
  if (n_tokens == 0) return MM_OK;
  MM_REQUIRE(ids_dtype == MM_INT32 || ids_dtype == MM_INT64, "moe_prefill: ids must be int32 or int64");
  MM_REQUIRE(x && ids && wts && sorted_ids && bexp && expert_offsets && a_buf && part_buf && y,
             "moe_prefill: null pointer");
  MM_REQUIRE(x_row_stride >= ex->hidden && y_row_stride >= ex->hidden, "moe_prefill: row stride smaller than hidden");
  MM_REQUIRE(mm::aligned16(x) && (x_row_stride * 2) % 16 == 0, "moe_prefill: x rows must be 16-byte aligned");
  MM_REQUIRE(mm::aligned16(a_buf) && mm::aligned16(part_buf), "moe_prefill: a_buf and part_buf must be 16-byte aligned");
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
  a.offsets = expert_offsets;
  // experts with a prefill copy of w_gu: the gate/up GEMM reads that copy (64-k slabs 64 R elements apart)
  a.gu_slabs = ex->w_gu_slabs ? 1 : 0;
  a.w_gu = a.gu_slabs ? ex->w_gu_slabs : ex->w_gu;
  // the same for w_d and the down GEMM
  a.d_slabs = ex->w_d_slabs ? 1 : 0;
  a.w_d = a.d_slabs ? ex->w_d_slabs : ex->w_d;
  a.s_gu = ex->s_gu;
  a.s_d = ex->s_d;
  a.s_dtype = ex->s_dtype;
  a.H = ex->hidden;
  a.I = ex->inter;
  a.gu_se = a.gu_slabs ? 2 * ex->inter * ex->hidden : ex->gu_stride_e;
  a.gu_sn = a.gu_slabs ? 0 : ex->gu_stride_n;
  a.d_se = a.d_slabs ? ex->hidden * ex->inter : ex->d_stride_e;
  a.d_sn = a.d_slabs ? 0 : ex->d_stride_n;
  a.sgu_se = ex->sgu_stride_e;
  a.sd_se = ex->sd_stride_e;
  a.res = static_cast<const uint16_t*>(residual);
  a.res_rs = res_row_stride;
  a.a_buf = static_cast<uint16_t*>(a_buf);
  a.part = static_cast<uint16_t*>(part_buf);
  a.y = static_cast<uint16_t*>(y);
  a.ys = y_row_stride;
  hipStream_t st = MM_STREAM(stream);
  if (phases == MM_PHASE_ALL) phases = MM_PHASE_GATE_UP | MM_PHASE_DOWN | MM_PHASE_COMBINE;
  if (nb > 0) {
    if (ex->w_dtype == MM_INT8) rc = launch_gemms<true, kBMSmall>(a, nb, phases, st);
    else if (block_m == kBM) rc = launch_gemms<false, kBM>(a, nb, phases, st);
    else rc = launch_gemms<false, kBMSmall>(a, nb, phases, st);
    if (rc) return rc;
  }
  if (!(phases & MM_PHASE_COMBINE)) return MM_OK;
  const int64_t total = n_tokens * (a.H / 8);
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  const bool i64 = ids_dtype == MM_INT64;
  if (nk <= 8 && i64) hipLaunchKernelGGL((prefill_combine_kernel<8, true>), grid, dim3(256), 0, st, a);
  else if (nk <= 8) hipLaunchKernelGGL((prefill_combine_kernel<8, false>), grid, dim3(256), 0, st, a);
  else if (nk <= kCombineMaxK && i64) hipLaunchKernelGGL((prefill_combine_kernel<kCombineMaxK, true>), grid, dim3(256), 0, st, a);
  else if (nk <= kCombineMaxK) hipLaunchKernelGGL((prefill_combine_kernel<kCombineMaxK, false>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((prefill_combine_kernel<0, false>), grid, dim3(256), 0, st, a);
  return mm::check_launch("moe_prefill combine");
}

namespace mm {
int check_router_args(int64_t n_tokens, int64_t E, int scoring, int n_group, int topk_group, int top_k,
                      int append_shared, const void* ids, int ids_dtype, const float* wts, int64_t out_row_stride);
int router_front(const void* x, int64_t n_tokens, int64_t H, int64_t xs, const void* norm_w, float eps,
                 const float* w32, const mmd::SelectParams& sp, float* logits, void* ids, int ids_dtype, float* wts,
                 int64_t out_row_stride, void* xn_out, hipStream_t s, bool with_select = true);
}  // namespace mm

// Whole MoE block for a prefill batch: RMSNorm into xn, router logits, selection, align, gate/up and down
// over the expert blocks, combine with the raw rows as residual.
extern "C" int mm_moe_block_prefill(const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w, float eps,
                                    const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                                    int topk_group, int top_k, float scale, const mm_experts* ex, float* logits,
                                    void* ids, int ids_dtype, float* wts, void* xn, int32_t* sorted_ids, int32_t* bexp,
                                    int32_t* expert_offsets, int64_t nb, void* a_buf, void* part_buf, int add_residual,
                                    void* y, int64_t y_row_stride, void* stream) {
  int rc = mm::check_experts("moe_block_prefill", ex);
  if (rc) return rc;
  const int64_t nk = static_cast<int64_t>(top_k) + 1;
  rc = mm::check_router_args(n_tokens, n_experts, scoring, n_group, topk_group, top_k, 1, ids, ids_dtype, wts, nk);
  if (rc) return rc;
  MM_REQUIRE(ex->n_slots == n_experts + 1, "moe_block_prefill: expert slots (%lld) must be n_experts + 1 (shared last)",
             (long long)ex->n_slots);
  MM_REQUIRE(x && norm_w && w32 && logits && xn, "moe_block_prefill: null pointer");
  MM_REQUIRE(mm::aligned16(xn), "moe_block_prefill: xn must be 16-byte aligned");
  if (n_tokens == 0) return MM_OK;
  hipStream_t st = MM_STREAM(stream);
  const mmd::SelectParams sp{bias, static_cast<int>(n_experts), scoring, n_group, topk_group, top_k, scale, 1};
  rc = mm::router_front(x, n_tokens, ex->hidden, x_row_stride, norm_w, eps, w32, sp, logits, ids, ids_dtype, wts, nk, xn,
                        st);
  if (rc) return rc;
  const int32_t bm = mm_prefill_block_m(n_tokens, nk, ex->n_slots, ex->w_dtype);
  rc = mm_align_blocks(ids, ids_dtype, n_tokens * nk, static_cast<int32_t>(ex->n_slots), bm, sorted_ids, bexp, nb,
                       expert_offsets, stream);
  if (rc) return rc;
  return mm_moe_prefill(xn, n_tokens, ex->hidden, ex, nk, ids, ids_dtype, wts, sorted_ids, bexp, expert_offsets, nb, bm,
                        add_residual ? x : nullptr, x_row_stride, a_buf, part_buf, y, y_row_stride, MM_PHASE_ALL,
                        stream);
}
