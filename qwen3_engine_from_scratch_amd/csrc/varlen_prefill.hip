// Varlen causal flash-attention prefill for gfx950 (packed sequences, GQA).
//
// Semantics follow flash_attention_varlen_kernel
// (qwen3/kernels/flash_attention_varlen.py:25-123): query row i of sequence s
// attends keys j <= i of the same sequence; query head h reads KV head
// h / G; online softmax in fp32, P rounded to bf16 for the PV product,
// bf16 output.
//
// Design (MI355X-first):
//  * One 256-thread workgroup (4 wave64s) per (query tile, head group,
//    sequence).  The head group holds HG query heads that share one KV head
//    (HG = the largest of 4, 2, 1 dividing G), so a K/V tile staged in LDS
//    serves every head of the group; each wave owns 32 query rows of one
//    head.  Two workgroups share a CU (two waves per SIMD), so one wave's
//    softmax overlaps the other's matrix-core work.
//  * K/V tiles of 64 keys go from HBM straight into LDS with buffer loads
//    that write LDS (no staging registers), double-buffered: the next tile's
//    loads are issued before the current tile's math, with one barrier per
//    tile.  The buffer descriptor covers only the sequence's rows, so rows
//    past its end read as zero without a branch.
//  * LDS tile layout: 64 key rows of 256 B, the 16-byte chunk c of row r at
//    slot c ^ swz(r).  K uses swz = r % 16 (the QK operand reads one chunk
//    of 16 consecutive rows per LDS cycle); V uses swz = 4 (r % 4) (the PV
//    operand reads 64 B of 4 consecutive rows).  Both are conflict-free.
//  * Scores are computed transposed, S^T(32 keys x 32 queries) = K Q^T with
//    mfma_f32_32x32x16_bf16: each lane owns one query column and 16 of its
//    keys, so the row max needs one cross-lane step, and the S^T register
//    layout is directly the B operand (P^T) of O^T = V^T P^T.  The V^T A
//    operand comes from the row-major V tile with ds_read_b64_tr_b16, two
//    transposing 8-byte reads per MFMA.
//  * Softmax in the exp2 domain with the scale folded into one FMA; the
//    running max is only raised (and the accumulator rescaled) when a new
//    score exceeds it by more than 2^8, which keeps every P <= 256 and makes
//    rescales rare; masking runs only on diagonal and tail tiles.
#include "common.hpp"

namespace {

constexpr int kD = 128;
constexpr int kBN = 64;                   // keys per staged K/V tile
constexpr int kRowBytes = kD * 2;         // one staged key row (256 B)
constexpr int kTileElems = kBN * kD;      // one staged K or V tile (16 KiB)
// Workgroups of W = 4 or 8 waves (one or two per CU): eight waves share each
// staged K/V tile among twice the query rows, halving the tile traffic per
// flop, but hold items twice as large (fewer, coarser work items).
template <int W>
constexpr int dma_per_wave() { return kBN * kRowBytes / (W * 64 * 16); }  // 16-byte lanes
constexpr int kMaxDma = 4;
constexpr float kRescaleSlack = 8.f;      // log2 headroom before the max is raised
constexpr int kMaxSeqs = 256;             // persistent path: sequences ranked in LDS
constexpr int kScanMax = 1024;            // persistent path: query-tile ranks in LDS
constexpr int kPools = 8;                 // dynamic schedule: one item pool per XCD
constexpr int kPoolStride = 32;           // counters 128 bytes apart
constexpr int kMaxSplits = 256;           // work items cut in two per call, at most
constexpr int kSplitSlotFloats = 8 * 64 * 66;  // eight waves x 64 lanes x (64 sums, max, sum)
static_assert(dma_per_wave<4>() == kMaxDma && dma_per_wave<8>() == 2, "tile / workgroup shape");

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short i16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4_t;

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* k;
  int64_t k_st, k_sh;
  const uint16_t* v;
  int64_t v_st, v_sh;
  uint16_t* o;
  int64_t o_st, o_sh;
  const int32_t* cu;
  int num_seqs;
  int64_t total;
  int Hq, G, HG;
  int groups;    // query-head groups (Hq / HG)
  int rows;      // query rows per head per workgroup (32 * W / HG)
  int n_mtiles;  // query tiles of the longest sequence
  float scale_log2;
  int causal;
  uint32_t* ctr;  // nullable: [32 p] next item of pool p, [32 kPools] workgroups done (zero between calls)
  // Split work items (split kernel only): per slot a ticket and a ready
  // flag (zero between calls) and the first finisher's partial state.
  uint32_t* split_ctr;  // [kMaxSplits][2]
  float* split_buf;     // [kMaxSplits][kSplitSlotFloats]
};

// The staged tiles of one workgroup: two K and two V buffers.
struct TileBufs {
  uint16_t* k0;
  uint16_t* v0;
  uint16_t* k1;
  uint16_t* v1;
};

// Per-lane byte offsets that do not change from tile to tile.
struct LaneOffsets {
  uint32_t kdma[kMaxDma];  // source offset of this lane's K chunk, load j
  uint32_t vdma[kMaxDma];  // same for V
  uint32_t kread[8];           // LDS offset of the QK operand, d step t (key block 0)
  uint32_t vread[4];           // LDS offset of the PV operand, d block db (key chunk 0)
};

template <int W>
__device__ __forceinline__ LaneOffsets lane_offsets(int lane, int wave, int64_t k_row_bytes,
                                                    int64_t v_row_bytes) {
  LaneOffsets o;
  // Load j of wave w fills LDS block n = D w + j (rows 4n .. 4n+3, D loads
  // per wave); lane i writes slot i % 16 of row 4n + i / 16, i.e. source
  // chunk slot ^ swz(row).
  constexpr int D = dma_per_wave<W>();
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int row = 4 * (D * wave + j) + (lane >> 4);
    const int slot = lane & 15;
    o.kdma[j] = static_cast<uint32_t>(row * k_row_bytes) + ((slot ^ (row & 15)) << 4);
    o.vdma[j] = static_cast<uint32_t>(row * v_row_bytes) + ((slot ^ (4 * (row & 3))) << 4);
  }
  // QK A operand (mfma 32x32x16): lane reads key row lane % 32, chunk 2t + lane / 32.
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int t = 0; t < 8; ++t) o.kread[t] = r * kRowBytes + ((((2 * t) | h) ^ (r & 15)) << 4);
  // PV A operand (V^T) through ds_read_b64_tr_b16: in 16-lane group g, lane
  // m supplies row 4 (g / 2) + m / 4 (+ 8 for the second read, + 16 per key
  // chunk) and dims 32 db + 16 (g % 2) + 4 (m % 4) .. +3.
  const int g = lane >> 4, m = lane & 15;
  const int vrow = 4 * (g >> 1) + (m >> 2);
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const int slot = 4 * (db ^ (m >> 2)) + 2 * (g & 1) + ((m & 3) >> 1);
    o.vread[db] = vrow * kRowBytes + slot * 16 + 8 * (m & 1);
  }
  return o;
}

// Issues this wave's share of the loads of key tile n0 into (sk, sv).
template <int W>
__device__ __forceinline__ void tile_dma(const PrefillArgs& a, const LaneOffsets& off,
                                         int64_t start, int len, int kvh, int n0, uint16_t* sk,
                                         uint16_t* sv, int wave) {
  const int rows = min(kBN, len - n0);
  const uint16_t* kb = a.k + (start + n0) * a.k_st + static_cast<int64_t>(kvh) * a.k_sh;
  const uint16_t* vb = a.v + (start + n0) * a.v_st + static_cast<int64_t>(kvh) * a.v_sh;
  // Rows past `rows` are outside the descriptor and read as zero.
  const int k_bytes = static_cast<int>((rows - 1) * a.k_st * 2) + kRowBytes;
  const int v_bytes = static_cast<int>((rows - 1) * a.v_st * 2) + kRowBytes;
  const __amdgpu_buffer_rsrc_t kr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kb), 0, k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vb), 0, v_bytes, 0x00020000);
  constexpr int D = dma_per_wave<W>();
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int blk = (D * wave + j) * 512;  // elements: 1 KiB per load
    __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void_t*)(sk + blk), 16, off.kdma[j], 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_void_t*)(sv + blk), 16, off.vdma[j], 0, 0, 0);
  }
}

__device__ __forceinline__ q3::bf16x8 lds_ld16(const uint16_t* base, uint32_t byte_off) {
  return q3::as_bf16x8(
      *reinterpret_cast<const q3::u32x4*>(reinterpret_cast<const char*>(base) + byte_off));
}

// V^T operand: two transposing 8-byte reads (keys +0..3 and +8..11 of the
// lane half's key set).
__device__ __forceinline__ q3::bf16x8 lds_vt(const uint16_t* base, uint32_t byte_off) {
  const char* p = reinterpret_cast<const char*>(base) + byte_off;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + 8 * kRowBytes));
  typedef short i16x8 __attribute__((__vector_size__(8 * sizeof(short))));
  const i16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(q3::bf16x8, both);
}

// LDS operand distance of the MFMA loops (steps read ahead).
constexpr int kAhead = 4;

// Byte offset of the K operand of QK step u (key block u % 2, d step u / 2).
__device__ __forceinline__ uint32_t qk_operand(const LaneOffsets& off, int u) {
  return off.kread[u >> 1] + (u & 1) * 32 * kRowBytes;
}

// Byte offset of the V^T operand of PV step u (key chunk u / 4, d block u % 4).
__device__ __forceinline__ uint32_t pv_operand(const LaneOffsets& off, int u) {
  return off.vread[u & 3] + (u >> 2) * 16 * kRowBytes;
}

// Maximum of the 32 scores s[0..1][0..15] of one lane: four interleaved
// v_max3 chains of eight scores and a final combine (depth 6).  Written as
// one asm block because fmaxf would first canonicalize every MFMA result;
// a NaN score makes P, and so the output, NaN either way.
__device__ __forceinline__ float max3_scores(const q3::f32x16 (&s)[2]) {
  const q3::f32x16& a = s[0];
  const q3::f32x16& b = s[1];
  float m, t1, t2, t3;
  asm volatile(
      "v_max3_f32 %0, %4, %5, %6\n\t"
      "v_max3_f32 %1, %12, %13, %14\n\t"
      "v_max3_f32 %2, %20, %21, %22\n\t"
      "v_max3_f32 %3, %28, %29, %30\n\t"
      "v_max3_f32 %0, %0, %7, %8\n\t"
      "v_max3_f32 %1, %1, %15, %16\n\t"
      "v_max3_f32 %2, %2, %23, %24\n\t"
      "v_max3_f32 %3, %3, %31, %32\n\t"
      "v_max3_f32 %0, %0, %9, %10\n\t"
      "v_max3_f32 %1, %1, %17, %18\n\t"
      "v_max3_f32 %2, %2, %25, %26\n\t"
      "v_max3_f32 %3, %3, %33, %34\n\t"
      "v_max3_f32 %0, %0, %11, %19\n\t"
      "v_max3_f32 %2, %2, %27, %35\n\t"
      "v_max3_f32 %0, %0, %1, %2\n\t"
      "v_max_f32 %0, %0, %3"
      : "=&v"(m), "=&v"(t1), "=&v"(t2), "=&v"(t3)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
        "v"(a[8]), "v"(a[9]), "v"(a[10]), "v"(a[11]), "v"(a[12]), "v"(a[13]), "v"(a[14]),
        "v"(a[15]), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(b[4]), "v"(b[5]), "v"(b[6]),
        "v"(b[7]), "v"(b[8]), "v"(b[9]), "v"(b[10]), "v"(b[11]), "v"(b[12]), "v"(b[13]),
        "v"(b[14]), "v"(b[15]));
  return m;
}

// x combined with the value lane l ^ 32 holds: v_permlane32_swap of x with
// itself leaves the lower-half value in r[0] and the upper-half value in
// r[1] on every lane.
__device__ __forceinline__ float cross_half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float cross_half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ void wait_loads() {
  // vmcnt(0) with expcnt / lgkmcnt left at their maxima.
  __builtin_amdgcn_s_waitcnt(0x0f70);
}

// Partial state of one wave of a split item, in its slot: accumulators as
// 16 float4 rows of 64 lanes, then (max, sum share) per lane.  Written and
// read with device-scope accesses (sc1: written through to, and read from,
// the point where all XCDs' L2s agree), so the hand-off needs no L2
// write-back or invalidation, which would stall the whole XCD.
constexpr int kCpolDevice = 16;  // sc1
constexpr int kSlotMlOffset = 8 * 64 * 64 * 4;  // bytes before the (max, sum) pairs

__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(float* slot) {
  return __builtin_amdgcn_make_buffer_rsrc(slot, 0, kSplitSlotFloats * 4, 0x00020000);
}

__device__ __forceinline__ void save_partial(__amdgpu_buffer_rsrc_t slot, int wave, int lane,
                                             float m_run, float l_run, const q3::f32x16 (&acc)[4]) {
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const q3::f32x4 v = {acc[db][4 * r4], acc[db][4 * r4 + 1], acc[db][4 * r4 + 2],
                           acc[db][4 * r4 + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(q3::u32x4, v), slot,
          static_cast<uint32_t>(((wave * 16 + db * 4 + r4) * 64 + lane) * 16), 0, kCpolDevice);
    }
  const uint32_t ml = kSlotMlOffset + (wave * 64 + lane) * 8;
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_run), slot, ml, 0, kCpolDevice);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l_run), slot, ml + 4, 0, kCpolDevice);
}

// Folds the other part's saved state into (m_run, l_run, acc) (both
// relative to their own running max; the result is relative to the larger
// one).  The sums are
// formed as part 0 * its weight + part 1 * its weight whichever part merges,
// so the output does not depend on which part finished first.
__device__ __forceinline__ void merge_partial(__amdgpu_buffer_rsrc_t slot, int wave, int lane,
                                              bool own_first, float& m_run, float& l_run,
                                              q3::f32x16 (&acc)[4]) {
  // Every load in flight at once: one memory round trip.
  const uint32_t ml = kSlotMlOffset + (wave * 64 + lane) * 8;
  const float om = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(slot, ml, 0, kCpolDevice));
  const float ol =
      __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(slot, ml + 4, 0, kCpolDevice));
  q3::f32x4 v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    v[i] = __builtin_bit_cast(
        q3::f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       slot, static_cast<uint32_t>(((wave * 16 + i) * 64 + lane) * 16), 0,
                       kCpolDevice));
  __builtin_amdgcn_sched_barrier(0);
  const float m = fmaxf(m_run, om);
  if (m == q3::kNegInf) return;  // no key reached this row in either part
  const float a_own = q3::fast_exp2(m_run - m);  // exp2(-inf) = 0
  const float a_oth = q3::fast_exp2(om - m);
  const float w0 = own_first ? a_own : a_oth, w1 = own_first ? a_oth : a_own;
  m_run = m;
  {
    const float x0 = own_first ? l_run : ol, x1 = own_first ? ol : l_run;
    l_run = __builtin_fmaf(x1, w1, x0 * w0);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float own = acc[i >> 2][4 * (i & 3) + e];
      const float x0 = own_first ? own : v[i][e], x1 = own_first ? v[i][e] : own;
      acc[i >> 2][4 * (i & 3) + e] = __builtin_fmaf(x1, w1, x0 * w0);
    }
}

// One work item: query tile mt of sequence seq for head group hg, over all
// of its key tiles (part < 0) or, in the split kernel, over the first
// (part 0) or second (part 1) half of them.  The two parts of a split item
// meet through split slot `slot`: the first to finish saves its partial
// state and raises the slot's ready flag; the second waits for that flag
// (the first is past all its work by then, so the wait is short), merges
// and writes the output, then leaves the slot's ticket and flag at zero.
// Every thread of the workgroup calls it.
template <int W, bool Split = false>
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, const LaneOffsets& off,
                                             int64_t start, int len, int hg, int mt,
                                             const TileBufs& tb, int part = -1, int slot = 0,
                                             uint32_t* s_role = nullptr) {
  const int m0 = mt * a.rows;
  if (m0 >= len) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const int l32 = lane & 31;
  const int hl = lane >> 5;
  const int wph = W / a.HG;  // waves per head
  const int head = hg * a.HG + wave / wph;
  const int kvh = (hg * a.HG) / a.G;
  const int q0 = m0 + (wave % wph) * 32;  // first query row of this wave
  const int qrow = q0 + l32;               // the query column this lane owns

  const int kend = a.causal ? min(len, m0 + a.rows) : len;
  const int n_tiles = (kend + kBN - 1) / kBN;
  const int t0 = Split && part == 1 ? n_tiles / 2 : 0;
  const int t1 = Split && part == 0 ? n_tiles / 2 : n_tiles;

  tile_dma<W>(a, off, start, len, kvh, t0 * kBN, tb.k0, tb.v0, wave);

  // Q^T as the B operand: lane (query l32, k-group hl), chunk c: dims
  // c*16 + 8*hl .. +7.
  q3::bf16x8 qv[8];
  {
    const q3::u32x4 z = {0u, 0u, 0u, 0u};
    const bool ok = qrow < len;
    const uint16_t* qp =
        a.q + (start + (ok ? qrow : 0)) * a.q_st + static_cast<int64_t>(head) * a.q_sh + 8 * hl;
#pragma unroll
    for (int c = 0; c < 8; ++c) qv[c] = q3::as_bf16x8(ok ? q3::ld16(qp + c * 16) : z);
  }

  float m_run = q3::kNegInf;  // running max (log2 domain) of this query
  float l_run = 0.f;          // this lane's share of the denominator
  q3::f32x16 acc[4];          // acc[db][r] = O[qrow][32*db + 8*(r/4) + 4*hl + r%4]
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

  const bool wave_active = q0 < len;
  const int wave_last_q = min(q0 + 31, len - 1);
  const float c = a.scale_log2;

  wait_loads();
  __syncthreads();

  auto tile = [&](int it, const uint16_t* kt, const uint16_t* vt, uint16_t* nk, uint16_t* nv) {
    const int n0 = it * kBN;
    if (it + 1 < t1) tile_dma<W>(a, off, start, len, kvh, n0 + kBN, nk, nv, wave);

    // Causal: the tile is entirely above this wave's last query row.
    const bool wave_skip = !wave_active || (a.causal && n0 > wave_last_q);
    if (!wave_skip) {
      // ---- S^T = K Q^T for two 32-key blocks ----
      // Step u covers key block u % 2, dims 16 (u / 2) .. +15; the two
      // blocks' chains alternate and K operands are read 4 steps ahead (the
      // scheduling fences keep that distance).
      q3::f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
      {
        q3::bf16x8 kf[kAhead];
#pragma unroll
        for (int u = 0; u < kAhead; ++u) kf[u] = lds_ld16(kt, qk_operand(off, u));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          s[u & 1] = q3::mfma32x32x16(kf[u % kAhead], qv[u >> 1], s[u & 1]);
          if (u + kAhead < 16) kf[u % kAhead] = lds_ld16(kt, qk_operand(off, u + kAhead));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // ---- mask (diagonal / tail tiles only) and block max ----
      const bool need_mask = (n0 + kBN > len) || (a.causal && n0 + kBN - 1 > q0);
      if (need_mask) {
        // score (kb, r) is key n0 + 4 hl + kr with kr = 32 kb + 8 (r / 4) +
        // r % 4 (an inline constant): compare kr with per-lane limits
        const int lim_len = len - n0 - 4 * hl;                   // kr < lim_len
        const int lim_q = a.causal ? qrow - n0 - 4 * hl : kBN;  // kr <= lim_q
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kr = kb * 32 + 8 * (r / 4) + (r % 4);
            const bool valid = kr < lim_len && kr <= lim_q;
            s[kb][r] = valid ? s[kb][r] : q3::kNegInf;
          }
      }
      // Row max as a v_max3 chain over the lane's 32 scores.  Written as asm
      // because fmaxf would first canonicalize every MFMA result (one more
      // VALU op per score); a NaN score makes P, and so the output, NaN
      // either way.  The scores were written by the QK MFMAs just above:
      // 24 wait states cover the MFMA-to-VALU dependency.
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
      float bm = max3_scores(s);
      bm = cross_half_max(bm);
      const float m_cand = bm * c;
      const bool raise = m_cand > m_run + kRescaleSlack;
      if (__any(raise)) {
        const float m_new = raise ? m_cand : m_run;
        const float alpha = raise ? q3::fast_exp2(m_run - m_new) : 1.f;
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] *= alpha;
      }
      // V^T operands of the first PV steps are read before the exponentials,
      // which hide their latency.
      q3::bf16x8 vf[kAhead];
#pragma unroll
      for (int u = 0; u < kAhead; ++u) vf[u] = lds_vt(vt, pv_operand(off, u));
      __builtin_amdgcn_sched_barrier(0);
      const float m_use = m_run == q3::kNegInf ? 0.f : m_run;
      // ---- P = exp2(s * c - m) as P^T B operands (chunk g = 2 kb + kc:
      // scores s[kb][8 kc .. 8 kc + 7]) and O^T += V^T P^T, step u covering
      // key chunk u / 4, dims 32 (u % 4) .. +31.  Chunk 0 is computed
      // first; the exponentials of chunk g + 1 are issued between the four
      // MFMAs of chunk g, two per step, so the VALU works while the matrix
      // core runs.
      q3::u32x4 pk[4];
      float psum[4];  // four independent sum chains, started by chunk 0
      auto exp_pair = [&](int g, int h) {  // scores 2h, 2h + 1 of chunk g
        const int kb = g >> 1, kc = g & 1;
        const float e0 = q3::fast_exp2(__builtin_fmaf(s[kb][8 * kc + 2 * h], c, -m_use));
        const float e1 = q3::fast_exp2(__builtin_fmaf(s[kb][8 * kc + 2 * h + 1], c, -m_use));
        if (g == 0 && h < 2) {
          psum[2 * h] = e0;
          psum[2 * h + 1] = e1;
        } else {
          psum[(2 * h) & 3] += e0;
          psum[(2 * h + 1) & 3] += e1;
        }
        pk[g][h] = q3::pack_bf16x2(e0, e1);
      };
#pragma unroll
      for (int h = 0; h < 4; ++h) exp_pair(0, h);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        acc[u & 3] = q3::mfma32x32x16(vf[u % kAhead], q3::as_bf16x8(pk[u >> 2]), acc[u & 3]);
        if (u + kAhead < 16) vf[u % kAhead] = lds_vt(vt, pv_operand(off, u + kAhead));
        if (u < 12) exp_pair((u >> 2) + 1, u & 3);
        __builtin_amdgcn_sched_barrier(0);
      }
      l_run += (psum[0] + psum[1]) + (psum[2] + psum[3]);
    }
    wait_loads();
    __syncthreads();
  };

  for (int it = t0; it < t1; it += 2) {
    tile(it, tb.k0, tb.v0, tb.k1, tb.v1);
    if (it + 1 < t1) tile(it + 1, tb.k1, tb.v1, tb.k0, tb.v0);
  }

  if constexpr (Split) {
    if (part >= 0) {
      uint32_t* ticket = a.split_ctr + 2 * slot;
      uint32_t* ready = ticket + 1;
      const __amdgpu_buffer_rsrc_t saved =
          slot_rsrc(a.split_buf + static_cast<int64_t>(slot) * kSplitSlotFloats);
      if (tid == 0)
        *s_role = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      if (*s_role == 0) {
        save_partial(saved, wave, lane, m_run, l_run, acc);
        wait_loads();  // this wave's device-scope saves are complete
        __syncthreads();
        if (tid == 0) __hip_atomic_store(ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      if (tid == 0) {
        // Bounded: with the ticket taken, the other part only has its
        // saves left.  (A workspace not zeroed before its first call could
        // leave the flag down; the cap ends the wait all the same.)
        for (int spin = 0; spin < (1 << 22); ++spin) {
          if (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
      __syncthreads();  // the saves are read (device scope) only after the flag
      merge_partial(saved, wave, lane, part == 0, m_run, l_run, acc);
      if (tid == 0) {
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ready, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  l_run = cross_half_sum(l_run);
  if (!wave_active) return;
  // The output goes through LDS so that each global store writes whole
  // 256-byte rows (four per instruction) instead of 16 bytes of 32 rows:
  // every tile buffer is free after the loop's last barrier, and the
  // caller's barrier follows before the next item's loads refill them.
  // Wave w stages its 32 x 128 tile in 8 KiB of buffer w / 2, chunk c of
  // row r at chunk c ^ (r % 16) (conflict-free for both directions).
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;  // 0 for rows past the end
  const int sb = wave >> 1;
  char* stage = reinterpret_cast<char*>(sb == 0 ? tb.k0 : sb == 1 ? tb.v0 : sb == 2 ? tb.k1 : tb.v1) +
                (wave & 1) * 8192;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int ch = 4 * db + g4;
      q3::u32x2 w = {q3::pack_bf16x2(acc[db][4 * g4] * inv, acc[db][4 * g4 + 1] * inv),
                     q3::pack_bf16x2(acc[db][4 * g4 + 2] * inv, acc[db][4 * g4 + 3] * inv)};
      *reinterpret_cast<q3::u32x2*>(stage + l32 * 256 + ((ch ^ (l32 & 15)) << 4) + hl * 8) = w;
    }
  const int oc = lane & 15;  // this lane's 16-byte chunk of a row
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rr = 4 * j + (lane >> 4);
    const q3::u32x4 v =
        *reinterpret_cast<const q3::u32x4*>(stage + rr * 256 + ((oc ^ (rr & 15)) << 4));
    const int row = q0 + rr;
    if (row < len)
      q3::st16(a.o + (start + row) * a.o_st + static_cast<int64_t>(head) * a.o_sh + oc * 8, v);
  }
}

// The four staged tile buffers, as separate LDS arrays so loads into one
// buffer are known not to alias reads of the other.
#define Q3_PREFILL_TILE_BUFFERS                                        \
  __shared__ __attribute__((aligned(1024))) uint16_t s_k0[kTileElems]; \
  __shared__ __attribute__((aligned(1024))) uint16_t s_v0[kTileElems]; \
  __shared__ __attribute__((aligned(1024))) uint16_t s_k1[kTileElems]; \
  __shared__ __attribute__((aligned(1024))) uint16_t s_v1[kTileElems]; \
  const TileBufs tb{s_k0, s_v0, s_k1, s_v1};                           \
  const LaneOffsets off = lane_offsets<W>(threadIdx.x & 63, threadIdx.x >> 6, a.k_st * 2, a.v_st * 2)

// Flat grid (fallback for many sequences / very long ones): one workgroup
// per virtual item, head group fastest so consecutive workgroups go to
// different XCDs and all items of one KV head share an XCD's L2; query tiles
// heaviest first.  Items past a sequence's end exit at once.
template <int W>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void varlen_prefill_flat_kernel(PrefillArgs a) {
  Q3_PREFILL_TILE_BUFFERS;
  const int64_t id = blockIdx.x;
  const int hg = static_cast<int>(id % a.groups);
  const int seq = static_cast<int>((id / a.groups) % a.num_seqs);
  const int mt =
      a.n_mtiles - 1 - static_cast<int>(id / (static_cast<int64_t>(a.groups) * a.num_seqs));
  const int64_t start = a.cu[seq];
  const int64_t end = a.cu[seq + 1];
  if (start < 0 || end > a.total || end <= start) return;
  prefill_item<W>(a, off, start, static_cast<int>(end - start), hg, mt, tb);
}

// Exclusive prefix sum over n <= kScanMax ints held in LDS (in place); returns
// the total.  Called by all threads of the workgroup.
template <int W>
__device__ __forceinline__ int block_exclusive_scan(int* v, int n, int* s_wsum) {
  constexpr int kPer = kScanMax / (W * 64);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int local[kPer];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = tid * kPer + i;
    local[i] = j < n ? v[j] : 0;
    sum += local[i];
  }
  int incl = sum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  int run = incl - sum, total = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    if (w < wave) run += s_wsum[w];
    total += s_wsum[w];
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = tid * kPer + i;
    if (j < n) v[j] = run;
    run += local[i];
  }
  __syncthreads();
  return total;
}

// Builds, in every workgroup's LDS, the compact list of the non-empty items
// (query tile, sequence, head group) ordered heaviest first: query tiles of
// the highest index first; within one, longest sequences first (ties by
// index), head group fastest.  s_first[r] = items before query-tile rank r
// (r = n_mtiles - 1 - mt); s_len[t] = sequence t's length (0 for a range
// outside the batch) and s_start[t] its first row.  Returns the number of items.  Called by all threads
// of the workgroup.
template <int W>
__device__ __forceinline__ int build_items(const PrefillArgs& a, int* s_len, int* s_start,
                                           int* s_sorted, int* s_first, int* s_wsum) {
  const int tid = threadIdx.x;
  const int S = a.num_seqs;
  const int nm = a.n_mtiles;
  for (int t = tid; t < S; t += W * 64) {
    const int64_t s0 = a.cu[t], s1 = a.cu[t + 1];
    const bool ok = s0 >= 0 && s1 <= a.total && s1 > s0;
    s_len[t] = ok ? static_cast<int>(s1 - s0) : 0;
    s_start[t] = ok ? static_cast<int>(s0) : 0;
  }
  __syncthreads();
  // Rank by length, longest first (ties by index).
  for (int t = tid; t < S; t += W * 64) {
    const int lt = s_len[t];
    int rank = 0;
    for (int u = 0; u < S; ++u) {
      const int lu = s_len[u];
      rank += (lu > lt || (lu == lt && u < t)) ? 1 : 0;
    }
    s_sorted[rank] = t;
  }
  __syncthreads();
  // Items of m-tile rank r: groups x (number of sequences longer than mt*rows).
  for (int r = tid; r < nm; r += W * 64) {
    const int mt = nm - 1 - r;
    const int64_t thr = static_cast<int64_t>(mt) * a.rows;
    int lo = 0, hi = S;  // first sorted index with len <= thr
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_len[s_sorted[mid]] > thr) lo = mid + 1; else hi = mid;
    }
    s_first[r] = lo * a.groups;
  }
  __syncthreads();
  return block_exclusive_scan<W>(s_first, nm, s_wsum);
}

// Coordinates of item i of that list (uniform, read from LDS): made scalar
// with readfirstlane so the item's indices and bounds live in SGPRs.
__device__ __forceinline__ void item_at(const PrefillArgs& a, int64_t i64, const int* s_first,
                                        const int* s_sorted, int& seq, int& hg, int& mt) {
  const int nm = a.n_mtiles;
  const int i = __builtin_amdgcn_readfirstlane(static_cast<int>(i64));
  int lo = 0, hi = nm - 1;  // largest rank r with s_first[r] <= i
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (__builtin_amdgcn_readfirstlane(s_first[mid]) <= i) lo = mid; else hi = mid - 1;
  }
  const int j = i - __builtin_amdgcn_readfirstlane(s_first[lo]);
  seq = __builtin_amdgcn_readfirstlane(s_sorted[j / a.groups]);
  hg = j % a.groups;
  mt = nm - 1 - lo;
}

// Persistent grid (CUs x resident workgroups).  Every workgroup builds the
// same compact list of non-empty items ordered heaviest first (query tiles
// of the highest index first; within one, longest sequences first, head
// group fastest), and item i goes to XCD i % 8, so one head group's K/V
// tiles stay in one XCD's L2.  Workgroup w takes item w first (the
// heaviest items, one per workgroup).  With counters in the workspace (and
// a multiple of 8 head groups) each XCD's workgroups then take that XCD's
// remaining items from its pool as they finish -- longest-processing-time-
// first list scheduling: a workgroup busy with a heavy item takes no more
// until the others have theirs -- asking for the next one while the current
// one runs, and take what other pools have left once theirs is empty.
// Without them they take their share in a snake order over rounds
// (mirroring whole groups of 8 positions so item i stays on XCD i % 8).
#ifndef Q3_PREFILL_PERSISTENT_WAVES_PER_EU
#define Q3_PREFILL_PERSISTENT_WAVES_PER_EU 2
#endif
template <int W>
__global__ __launch_bounds__(W * 64)
__attribute__((amdgpu_waves_per_eu(Q3_PREFILL_PERSISTENT_WAVES_PER_EU, Q3_PREFILL_PERSISTENT_WAVES_PER_EU)))
void varlen_prefill_persistent_kernel(PrefillArgs a) {
  Q3_PREFILL_TILE_BUFFERS;
  __shared__ int s_len[kMaxSeqs];
  __shared__ int s_start[kMaxSeqs];
  __shared__ int s_sorted[kMaxSeqs];
  __shared__ int s_first[kScanMax];  // items before m-tile rank r (r = n_mtiles-1-mt)
  __shared__ int s_wsum[W];
  const int tid = threadIdx.x;
  // Workgroup 0 clears the counters before its first barrier (a workspace
  // never used, or left mid-call, still gives every item to some workgroup:
  // workgroup 0 takes items, from every pool, until all are done, and an
  // item taken twice is computed twice with the same result).
  if (a.ctr && blockIdx.x == 0 && tid <= kPools) {
    const uint32_t prev = atomicExch(a.ctr + tid * kPoolStride, 0u);
    asm volatile("" ::"v"(prev));  // performed before this thread reaches the barriers below
  }

  const int T = build_items<W>(a, s_len, s_start, s_sorted, s_first, s_wsum);

  auto run = [&](int64_t i64) {
    int seq, hg, mt;
    item_at(a, i64, s_first, s_sorted, seq, hg, mt);
    // the sequence's rows from LDS, as scalars (no global load per item)
    prefill_item<W>(a, off, __builtin_amdgcn_readfirstlane(s_start[seq]),
                    __builtin_amdgcn_readfirstlane(s_len[seq]), hg, mt, tb);
  };
  // One loop and one inlined item body for both orders (each extra call
  // site of `run` costs registers in the tile loop).
  //  - static: round r takes item r * nwg + w, mirrored on odd rounds
  //    (w' = the same XCD, the opposite end of the CU order), which pairs
  //    heavy items with light ones, and on a last round that does not
  //    fill the grid (its items go to the workgroups whose first items
  //    were the lightest, not to those holding the heaviest);
  //  - counters (eight-wave path, given a workspace): the first round is
  //    the static one; pool p holds the later items with i % 8 == p
  //    (ticket j is item nwg + j * 8 + p), a workgroup draws from the pool
  //    of its XCD and, once that is empty, from the fullest pool.
  const int64_t nwg = gridDim.x;
  const int w = blockIdx.x;
  const int w_mirror = (gridDim.x / 8 - 1 - w / 8) * 8 + w % 8;
  const bool counters = a.ctr && a.groups % kPools == 0 && gridDim.x % kPools == 0;
  auto pool_items = [&](int q) -> int64_t {
    return T > nwg + q ? (T - nwg - q + kPools - 1) / kPools : 0;
  };
  __shared__ int64_t s_item;
  int pool = static_cast<int>(blockIdx.x % kPools);  // the XCD the dispatcher placed it on
  uint32_t mine = 0;                                  // thread 0: the next ticket, drawn ahead
  // Counter order: the next item for the workgroup (every thread calls it).
  auto draw = [&]() -> int64_t {
    if (tid == 0) {
      int64_t item = -1;
      int64_t j = mine;
      // an empty pool: read every pool's count (coherent loads) and ask the
      // one with the most items left; a failed ask leaves that pool visibly
      // empty, so this ends
      while (j >= pool_items(pool)) {
        int best_q = -1;
        int64_t best = 0;
        for (int q = 0; q < kPools; ++q) {
          const int64_t left = pool_items(q) - static_cast<int64_t>(__hip_atomic_load(
              a.ctr + q * kPoolStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          if (left > best) {
            best = left;
            best_q = q;
          }
        }
        if (best_q < 0) break;
        pool = best_q;
        j = atomicAdd(a.ctr + pool * kPoolStride, 1u);
      }
      if (j < pool_items(pool)) {
        item = nwg + j * kPools + pool;
        mine = atomicAdd(a.ctr + pool * kPoolStride, 1u);  // the next, one item ahead
      }
      s_item = item;
    }
    __syncthreads();  // every thread has finished the previous item
    const int64_t i = s_item;
    __syncthreads();  // every thread has read s_item
    return i;
  };
  if (counters && tid == 0) mine = atomicAdd(a.ctr + pool * kPoolStride, 1u);
  int64_t i = w < T ? w : (counters ? draw() : -1);
  for (int round = 1; i >= 0; ++round) {
    run(i);
    if (counters) {
      i = draw();
    } else {
      const bool mirror = (round & 1) || static_cast<int64_t>(round + 1) * nwg > T;
      i = static_cast<int64_t>(round) * nwg + (mirror ? w_mirror : w);
      if (i >= T) i = -1;
      __syncthreads();  // the item's LDS tiles are no longer read
    }
  }
  if (counters && tid == 0 &&
      atomicAdd(a.ctr + kPools * kPoolStride, 1u) == gridDim.x - 1) {
    // the last workgroup to finish leaves every counter at zero
    for (int q = 0; q <= kPools; ++q) atomicExch(a.ctr + q * kPoolStride, 0u);
  }
}

// Sizes the items for W waves and launches the persistent grid (CUs x
// resident workgroups, from the occupancy API) or, past its LDS tables, the
// flat grid.
// Split plan of a causal batch (with split slots in the workspace).  An
// item's work is its key tiles, about (mt + 1) rows / 64 for query tile mt,
// so the heaviest items are those of the highest query tiles -- the first
// ranks of the list.  The items of query tiles mt >= ms are cut in two at
// their middle key tile, ms being the lowest query tile whose items are
// heavier than the batch's mean work per workgroup (and have at least four
// key tiles, and fit the slots); a split item's slot is its list index.
// Entries are then ordered by work in half-tile classes: class k holds the
// whole items of query tile k / 2 - 1 (k even, below ms) followed by the
// two parts of each item of query tile k - 1 (at or above ms), classes
// heaviest first.  s_cls[j] = entries before class 2 n_mtiles - j.
struct SplitPlan {
  int ms;  // first split query tile (n_mtiles: none)
  int E;   // work entries
  int T;   // items
};

template <int W>
__device__ __forceinline__ SplitPlan plan_splits(const PrefillArgs& a, const int* s_len,
                                                 const int* s_first, int T, int nwg, int* s_cls,
                                                 int* s_wsum, unsigned long long* s_work) {
  const int nm = a.n_mtiles;
  const int tid = threadIdx.x;
  SplitPlan p{nm, T, T};
  if (!a.split_buf || !a.causal || 2 * nm > kScanMax) return p;
  // Key tiles of all items, per head group.
  if (tid == 0) *s_work = 0ull;
  __syncthreads();
  unsigned long long mine = 0;
  for (int t = tid; t < a.num_seqs; t += W * 64) {
    const int len = s_len[t];
    for (int m0 = 0; m0 < len; m0 += a.rows) mine += (min(len, m0 + a.rows) + kBN - 1) / kBN;
  }
  if (mine) atomicAdd(s_work, mine);
  __syncthreads();
  const unsigned long long work = *s_work * a.groups;
  const unsigned long long mean = (work + nwg - 1) / nwg;  // key tiles per workgroup
  // Lowest mt with (mt + 1) rows > mean * 64 and at least four key tiles.
  int ms = static_cast<int>(min<unsigned long long>(mean * kBN / a.rows, nm));
  ms = max(ms, 4 * kBN / a.rows - 1);
  auto before = [&](int r) { return r < nm ? s_first[r] : T; };  // items before rank r
  while (ms < nm && before(nm - ms) > kMaxSplits) ++ms;
  if (ms >= nm) return p;
  p.ms = ms;
  const int K = 2 * nm;
  for (int j = tid; j < K; j += W * 64) {
    const int k = K - j;
    int cnt = 0;
    const int mu = k / 2 - 1;  // whole items of query tile mu
    if ((k & 1) == 0 && mu < ms) cnt += before(nm - mu) - before(nm - 1 - mu);
    const int mp = k - 1;      // parts of the items of query tile mp
    if (mp >= ms && mp < nm) cnt += 2 * (before(nm - mp) - before(nm - 1 - mp));
    s_cls[j] = cnt;
  }
  __syncthreads();
  p.E = block_exclusive_scan<W>(s_cls, K, s_wsum);
  return p;
}

// Coordinates of work entry e (uniform): the item (seq, hg, mt), its part
// (-1: whole) and split slot.
__device__ __forceinline__ void entry_at(const PrefillArgs& a, const SplitPlan& p, int64_t e64,
                                         const int* s_first, const int* s_sorted, const int* s_cls,
                                         int& seq, int& hg, int& mt, int& part, int& slot) {
  const int nm = a.n_mtiles;
  part = -1;
  slot = 0;
  if (p.ms >= nm) {
    item_at(a, e64, s_first, s_sorted, seq, hg, mt);
    return;
  }
  const int e = __builtin_amdgcn_readfirstlane(static_cast<int>(e64));
  const int K = 2 * nm;
  int lo = 0, hi = K - 1;  // largest class index j with s_cls[j] <= e
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (__builtin_amdgcn_readfirstlane(s_cls[mid]) <= e) lo = mid; else hi = mid - 1;
  }
  const int k = K - lo;
  int o = e - __builtin_amdgcn_readfirstlane(s_cls[lo]);
  auto before = [&](int r) {  // items before rank r
    return r < nm ? __builtin_amdgcn_readfirstlane(s_first[r]) : p.T;
  };
  int r;
  const int mu = k / 2 - 1;
  bool whole = false;
  if ((k & 1) == 0 && mu < p.ms) {
    r = nm - 1 - mu;
    const int n_whole = before(r + 1) - before(r);
    whole = o < n_whole;
    if (!whole) o -= n_whole;
  }
  int j;
  if (whole) {
    mt = mu;
    j = o;
  } else {
    mt = k - 1;
    r = nm - 1 - mt;
    j = o >> 1;
    part = o & 1;
    slot = before(r) + j;
  }
  seq = __builtin_amdgcn_readfirstlane(s_sorted[j / a.groups]);
  hg = j % a.groups;
}

// Small causal batches (fewer items than resident workgroups, so most CUs
// would otherwise idle while the longest items finish): the same item list,
// with the heaviest items cut in two (split plan above) and handed out in
// the snake order of the persistent grid.  A part waits only for a part
// that has finished its key tiles, so every wait ends.
template <int W>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void varlen_prefill_split_kernel(PrefillArgs a) {
  Q3_PREFILL_TILE_BUFFERS;
  __shared__ int s_len[kMaxSeqs];
  __shared__ int s_start[kMaxSeqs];
  __shared__ int s_sorted[kMaxSeqs];
  __shared__ int s_first[kScanMax];  // items before m-tile rank r (r = n_mtiles-1-mt)
  __shared__ int s_cls[kScanMax];    // entries before work class 2 n_mtiles - j
  __shared__ int s_wsum[W];
  __shared__ unsigned long long s_work;
  __shared__ uint32_t s_role;
  const int T_items = build_items<W>(a, s_len, s_start, s_sorted, s_first, s_wsum);
  const SplitPlan plan =
      plan_splits<W>(a, s_len, s_first, T_items, gridDim.x, s_cls, s_wsum, &s_work);
  const int64_t nwg = gridDim.x;
  const int w = blockIdx.x;
  const int w_mirror = (gridDim.x / 8 - 1 - w / 8) * 8 + w % 8;
  int64_t i = w;
  for (int round = 1; i < plan.E; ++round) {
    int seq, hg, mt, part, slot;
    entry_at(a, plan, i, s_first, s_sorted, s_cls, seq, hg, mt, part, slot);
    const int64_t start = a.cu[seq];  // a valid range: the entry exists
    prefill_item<W, true>(a, off, start, static_cast<int>(a.cu[seq + 1] - start), hg, mt, tb,
                          part, slot, &s_role);
    i = static_cast<int64_t>(round) * nwg + ((round & 1) ? w_mirror : w);
    __syncthreads();  // the entry's LDS tiles are no longer read
  }
}

template <int W>
int launch_prefill(PrefillArgs a, int num_seqs, int max_seqlen, int dev, int cus,
                   hipStream_t s, const char* who) {
  a.rows = 32 * W / a.HG;
  a.n_mtiles = static_cast<int>(q3::cdiv(max_seqlen, a.rows));
  const int64_t blocks = static_cast<int64_t>(a.groups) * num_seqs * a.n_mtiles;
  if (blocks > 0x7fffffff)
    return q3::fail(QWEN3_EINVAL, "%s: grid too large (heads %d, seqs %d, max_seqlen %d)", who,
                    a.Hq, num_seqs, max_seqlen);
  // Resident workgroups per CU, queried once per device (a host-side cost
  // of every call otherwise).
  static int occupancy[64] = {0};
  int per_cu = dev >= 0 && dev < 64 ? occupancy[dev] : 0;
  if (per_cu == 0 &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void*>(varlen_prefill_persistent_kernel<W>), W * 64,
          0) == hipSuccess &&
      per_cu > 0 && dev >= 0 && dev < 64)
    occupancy[dev] = per_cu;
  const bool persistent =
      num_seqs <= kMaxSeqs && a.n_mtiles <= kScanMax && cus > 0 && per_cu > 0;
  // At most this many items: groups x (query tiles of all rows + one
  // ragged tile per sequence).
  const int64_t items_max = static_cast<int64_t>(a.groups) *
                            (q3::cdiv(a.total, a.rows) + static_cast<int64_t>(num_seqs));
  if (persistent && a.split_buf && a.causal && 2 * a.n_mtiles <= kScanMax &&
      items_max < static_cast<int64_t>(cus) * per_cu) {
    const int wgs = ((cus * per_cu + 7) / 8) * 8;
    hipLaunchKernelGGL(varlen_prefill_split_kernel<W>, dim3(wgs), dim3(W * 64), 0, s, a);
  } else if (persistent) {
    const int wgs = ((cus * per_cu + 7) / 8) * 8;  // multiple of 8 for the XCD-preserving snake
    hipLaunchKernelGGL(varlen_prefill_persistent_kernel<W>, dim3(wgs), dim3(W * 64), 0, s, a);
  } else {
    hipLaunchKernelGGL(varlen_prefill_flat_kernel<W>, dim3(static_cast<unsigned>(blocks)),
                       dim3(W * 64), 0, s, a);
  }
  return q3::launch_status(who);
}

// Workspace: schedule counters, split tickets / flags, then split partials.
constexpr size_t kCtrBytes = (kPools + 1) * kPoolStride * sizeof(uint32_t);
constexpr size_t kSplitCtrBytes = kMaxSplits * 2 * sizeof(uint32_t);
constexpr size_t kSplitBufOffset = (kCtrBytes + kSplitCtrBytes + 255) / 256 * 256;
constexpr size_t kWorkspaceBytes =
    kSplitBufOffset + static_cast<size_t>(kMaxSplits) * kSplitSlotFloats * sizeof(float);

}  // namespace

extern "C" size_t qwen3_varlen_prefill_workspace_bytes(void) { return kWorkspaceBytes; }

extern "C" int qwen3_varlen_prefill_bf16(const void* q, const int64_t q_strides[2],
                                         const void* k, const int64_t k_strides[2],
                                         const void* v, const int64_t v_strides[2], void* o,
                                         const int64_t o_strides[2], const int32_t* cu_seqlens,
                                         int num_seqs, int max_seqlen, int64_t total_tokens,
                                         int num_heads, int num_kv_heads, int head_dim,
                                         float scale, int causal, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  const char* who = "qwen3_varlen_prefill_bf16";
  if (!q || !k || !v || !o || !cu_seqlens || !q_strides || !k_strides || !v_strides ||
      !o_strides)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (head_dim != kD)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: head_dim %d not supported (built for %d)", who,
                    head_dim, kD);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > 16)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: num_heads %d / num_kv_heads %d unsupported", who,
                    num_heads, num_kv_heads);
  if (num_seqs < 0 || max_seqlen < 0 || total_tokens < 0)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (num_seqs == 0 || max_seqlen == 0 || total_tokens == 0) return QWEN3_OK;
  const int64_t vec_strides[] = {q_strides[0], q_strides[1], k_strides[0], k_strides[1],
                                 v_strides[0], v_strides[1], o_strides[0], o_strides[1]};
  bool ok = q3::aligned16(q) && q3::aligned16(k) && q3::aligned16(v) && q3::aligned16(o);
  for (int64_t s : vec_strides) ok = ok && s % 8 == 0;
  if (!ok)
    return q3::fail(QWEN3_EALIGN, "%s: q/k/v/o need 16-byte aligned rows (strides multiple "
                    "of 8 elements)", who);

  PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_strides[0];
  a.q_sh = q_strides[1];
  a.k = static_cast<const uint16_t*>(k);
  a.k_st = k_strides[0];
  a.k_sh = k_strides[1];
  a.v = static_cast<const uint16_t*>(v);
  a.v_st = v_strides[0];
  a.v_sh = v_strides[1];
  a.o = static_cast<uint16_t*>(o);
  a.o_st = o_strides[0];
  a.o_sh = o_strides[1];
  a.cu = cu_seqlens;
  a.num_seqs = num_seqs;
  a.total = total_tokens;
  a.Hq = num_heads;
  a.G = num_heads / num_kv_heads;
  a.HG = a.G % 4 == 0 ? 4 : (a.G % 2 == 0 ? 2 : 1);
  a.scale_log2 = scale * q3::kLog2e;
  a.causal = causal ? 1 : 0;
  a.groups = num_heads / a.HG;
  if (workspace) {
    if (workspace_bytes < qwen3_varlen_prefill_workspace_bytes())
      return q3::fail(QWEN3_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who,
                      qwen3_varlen_prefill_workspace_bytes(), workspace_bytes);
    if (!q3::aligned16(workspace))
      return q3::fail(QWEN3_EALIGN, "%s: workspace must be 16-byte aligned", who);
  }

  q3::clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = -1, cus = 0;
  static int cu_cache[64] = {0};
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    cus = cu_cache[dev];
    if (cus == 0 &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      cu_cache[dev] = cus;
  }
  // Eight-wave workgroups once the batch holds enough of their (twice as
  // large) work items to give every CU four: they halve the K/V tile
  // traffic per flop, but a batch of a few short sequences needs the finer
  // four-wave items to spread its causal work.
  const int64_t rows8 = 32 * 8 / a.HG;
  const int64_t items8 = static_cast<int64_t>(a.groups) * q3::cdiv(total_tokens, rows8);
  const bool wide = cus > 0 && items8 >= 4 * static_cast<int64_t>(cus);
  // Items handed out from the counters only on the eight-wave path: over
  // many rounds of mixed-length items they finish 1-2% sooner (64 prompts
  // of 128..1024 tokens: 229 -> 224 us), while the few rounds of a small
  // batch are paired better by the static snake.
  if (workspace && wide) a.ctr = static_cast<uint32_t*>(workspace);
  if (workspace) {
    char* ws = static_cast<char*>(workspace);
    a.split_ctr = reinterpret_cast<uint32_t*>(ws + kCtrBytes);
    a.split_buf = reinterpret_cast<float*>(ws + kSplitBufOffset);
  }
  return wide ? launch_prefill<8>(a, num_seqs, max_seqlen, dev, cus, s, who)
              : launch_prefill<4>(a, num_seqs, max_seqlen, dev, cus, s, who);
}
