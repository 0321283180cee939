// Varlen causal flash-attention prefill for gfx950 (packed sequences, GQA).
//
// Semantics follow flash_attention_varlen_kernel
// (qwen3/kernels/flash_attention_varlen.py:25-123): query row i of sequence s
// attends keys j <= i of the same sequence; query head h reads KV head
// h / G; online softmax in fp32, P rounded to bf16 for the PV product,
// bf16 output.
//
// Design (MI355X-first):
//  * A work item is (query tile, head group, sequence).  The head group
//    holds HG query heads that share one KV head (HG = the largest of 4, 2,
//    1 dividing G), so a K/V tile staged in LDS serves every head of the
//    group; each wave of a workgroup owns 32 query rows of one head.  Two
//    256-thread workgroups share a CU (two waves per SIMD), so one wave's
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
//  * Range schedule (varlen_prefill_range_kernel): the items' key tiles,
//    each weighted by its cost plus a fixed cost per item, are laid end to
//    end and cut into equal ranges, one per resident workgroup.  A
//    workgroup streams its range as a chain of segments (runs of one
//    item's key tiles), each starting with the loads of its first K/V tile
//    and its Q rows.  An item whose tiles fall in several ranges leaves one
//    partial softmax state per range in the workspace; the last part to
//    arrive folds them in key order.
//  * Wave-specialised tile (varlen_prefill_ws_kernel, QWEN3_PREFILL_TILE=ws):
//    matrix waves issue only MFMAs, softmax waves turn scores into P^T
//    operands, both through LDS; it moves 1.75 times the LDS bytes per MFMA
//    of the tile above and runs slower (LDS-bound), so it is not the
//    default.
#include <cstdlib>
#include <cstring>

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
constexpr int kMaxSeqs = 256;             // persistent / range paths: sequences ranked in LDS
constexpr int kScanMax = 1024;            // persistent path: query-tile ranks in LDS
constexpr int kPools = 8;                 // dynamic schedule: one item pool per XCD
constexpr int kPoolStride = 32;           // counters 128 bytes apart
static_assert(dma_per_wave<4>() == kMaxDma && dma_per_wave<8>() == 2, "tile / workgroup shape");

// Range schedule weights: a key tile is kUnits, an item adds kItemUnits,
// its start and output (measured per-workgroup timelines: about 2.5 tiles'
// time from one item's last tile to the next item's first).  Items of at
// most kAtomicTiles key tiles are never cut (so a prompt of at most 256
// tokens is computed the same way in any batch); a range holds at least
// kMinRangeTiles tiles' weight.
constexpr int kUnits = 16;
constexpr int kItemUnits = 40;
constexpr int kAtomicTiles = 4;
constexpr int kMinRangeTiles = 4;
// Partial softmax state of one workgroup in the workspace: per wave and
// lane 64 accumulators (16 float4 rows), then (running max, sum share).
template <int W>
constexpr int slot_floats() { return W * 64 * 66; }
template <int W>
constexpr int slot_ml_offset() { return W * 64 * 64 * 4; }  // bytes before the (max, sum) pairs

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
  // Range path: per range that holds the first tile of a cut item, the
  // number of its parts that have arrived (zero between calls), and two
  // partial-state slots per range (its first and its last segment).
  uint32_t* tickets;  // [max_ranges]
  float* slots;       // [2 * max_ranges][slot_floats<W>()]
  int max_ranges;
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
  uint32_t kread;              // LDS offset of the QK operand, d step 0 (key block 0)
  uint32_t vread;              // LDS offset of the PV operand, d block 0 (key chunk 0)
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
  // QK A operand (mfma 32x32x16): lane reads key row lane % 32, chunk 2t + lane / 32
  // at chunk (2t + h) ^ (r % 16) = (h ^ (r % 16)) ^ 2t: d step t is kread ^ (t << 5)
  // (the XOR stays inside the row's 256 bytes).
  const int r = lane & 31, h = lane >> 5;
  o.kread = r * kRowBytes + ((h ^ (r & 15)) << 4);
  // PV A operand (V^T) through ds_read_b64_tr_b16: in 16-lane group g, lane
  // m supplies row 4 (g / 2) + m / 4 (+ 8 for the second read, + 16 per key
  // chunk) and dims 32 db + 16 (g % 2) + 4 (m % 4) .. +3.
  // Slot 4 (db ^ (m / 4)) + ..: d block db is vread ^ (db << 6).
  const int g = lane >> 4, m = lane & 15;
  const int vrow = 4 * (g >> 1) + (m >> 2);
  const int slot = 4 * (m >> 2) + 2 * (g & 1) + ((m & 3) >> 1);
  o.vread = vrow * kRowBytes + slot * 16 + 8 * (m & 1);
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
constexpr int kAhead = 2;

// Byte offset of the K operand of QK step u (key block u % 2, d step u / 2).
__device__ __forceinline__ uint32_t qk_operand(const LaneOffsets& off, int u) {
  return (off.kread ^ static_cast<uint32_t>((u >> 1) << 5)) + (u & 1) * 32 * kRowBytes;
}

// Byte offset of the V^T operand of PV step u (key chunk u / 4, d block u % 4).
__device__ __forceinline__ uint32_t pv_operand(const LaneOffsets& off, int u) {
  return (off.vread ^ static_cast<uint32_t>((u & 3) << 6)) + (u >> 2) * 16 * kRowBytes;
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

// One wave's share of a work item: the sequence's rows, this wave's 32
// query rows of one head (wave-uniform).
struct WaveItem {
  int64_t start;  // first row of the sequence
  int len;        // its length
  int head;       // query head of this wave
  int kvh;        // its KV head
  int q0;         // first query row of this wave (lane l owns row q0 + l % 32)
  __device__ __forceinline__ bool active() const { return q0 < len; }
  __device__ __forceinline__ int last_q() const { return min(q0 + 31, len - 1); }
};

template <int W>
__device__ __forceinline__ WaveItem wave_item(const PrefillArgs& a, int64_t start, int len, int hg,
                                              int mt, int wave, int lane) {
  WaveItem wi;
  const int wph = W / a.HG;  // waves per head
  wi.start = start;
  wi.len = len;
  wi.head = hg * a.HG + wave / wph;
  wi.kvh = (hg * a.HG) / a.G;
  wi.q0 = mt * a.rows + (wave % wph) * 32;
  return wi;
}

// Q^T as the B operand: lane (query l32, k-group hl), chunk c: dims
// c*16 + 8*hl .. +7.  The wave's 32 rows are read through a buffer
// descriptor that ends at the sequence's last row, so rows past it read as
// zero; q_lane is the lane's byte offset l32 * row stride + 16 hl, the
// same for every item.  The chunk offset c * 32 goes in the scalar offset,
// which the range check does not cover: the lane's row start (in the
// vector offset) decides, and a row in range is in range up to its end.
__device__ __forceinline__ uint32_t q_lane_offset(const PrefillArgs& a, int lane) {
  return static_cast<uint32_t>((lane & 31) * a.q_st * 2 + 16 * (lane >> 5));
}
__device__ __forceinline__ void load_q(const PrefillArgs& a, const WaveItem& wi, uint32_t q_lane,
                                       q3::bf16x8 (&qv)[8]) {
  const int rows = min(32, wi.len - wi.q0);
  const uint16_t* base =
      a.q + (wi.start + wi.q0) * a.q_st + static_cast<int64_t>(wi.head) * a.q_sh;
  const int bytes = rows > 0 ? static_cast<int>((rows - 1) * a.q_st * 2) + kRowBytes : 0;
  const __amdgpu_buffer_rsrc_t qr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, bytes, 0x00020000);
#pragma unroll
  for (int c = 0; c < 8; ++c)
    qv[c] = q3::as_bf16x8(__builtin_bit_cast(
        q3::u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, q_lane, c * 32, 0)));
}

// One 64-key tile (first key n0, staged in kt / vt) folded into this wave's
// online softmax state.  Prio: the wave runs its two MFMA chains at raised
// issue priority, so of the two waves on a SIMD the one feeding the matrix
// core issues first (measured: 1 µs faster on one 2,048-token prompt in the
// range schedule, 3-4 µs slower on the Qwen3-0.6B batch in the persistent
// one, so only the range schedule sets it).
template <bool Prio>
__device__ __forceinline__ void tile_math(const PrefillArgs& a, const LaneOffsets& off,
                                          const WaveItem& wi, int lane, int n0,
                                          const uint16_t* kt, const uint16_t* vt,
                                          const q3::bf16x8 (&qv)[8], float& m_run, float& l_run,
                                          q3::f32x16 (&acc)[4]) {
  const int hl = lane >> 5;
  const float c = a.scale_log2;
  // Causal: the tile is entirely above this wave's last query row.
  const bool wave_skip = !wi.active() || (a.causal && n0 > wi.last_q());
  if (wave_skip) return;
  // ---- S^T = K Q^T for two 32-key blocks ----
  // Step u covers key block u % 2, dims 16 (u / 2) .. +15; the two blocks'
  // chains alternate and K operands are read 4 steps ahead (the scheduling
  // fences keep that distance).
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
    if constexpr (Prio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      s[u & 1] = q3::mfma32x32x16(kf[u % kAhead], qv[u >> 1], s[u & 1]);
      if (u + kAhead < 16) kf[u % kAhead] = lds_ld16(kt, qk_operand(off, u + kAhead));
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (Prio) __builtin_amdgcn_s_setprio(0);
  }
  // ---- mask (diagonal / tail tiles only) and block max ----
  const bool need_mask = (n0 + kBN > wi.len) || (a.causal && n0 + kBN - 1 > wi.q0);
  if (need_mask) {
    // score (kb, r) is key n0 + 4 hl + kr with kr = 32 kb + 8 (r / 4) + r %
    // 4 (an inline constant): valid iff kr <= lim, one per-lane limit for
    // the sequence end and the causal diagonal.
    int lim = wi.len - 1 - n0 - 4 * hl;
    if (a.causal) lim = min(lim, wi.q0 + (lane & 31) - n0 - 4 * hl);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = kb * 32 + 8 * (r / 4) + (r % 4);
        s[kb][r] = kr <= lim ? s[kb][r] : q3::kNegInf;
      }
  }
  // Row max as a v_max3 chain over the lane's 32 scores.  The scores were
  // written by the QK MFMAs just above: 24 wait states cover the
  // MFMA-to-VALU dependency.
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
  // key chunk u / 4, dims 32 (u % 4) .. +31.  Chunk 0 is computed first;
  // the exponentials of chunk g + 1 are issued between the four MFMAs of
  // chunk g, two per step, so the VALU works while the matrix core runs.
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
  if constexpr (Prio) __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    acc[u & 3] = q3::mfma32x32x16(vf[u % kAhead], q3::as_bf16x8(pk[u >> 2]), acc[u & 3]);
    if (u + kAhead < 16) vf[u % kAhead] = lds_vt(vt, pv_operand(off, u + kAhead));
    if (u < 12) exp_pair((u >> 2) + 1, u & 3);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (Prio) __builtin_amdgcn_s_setprio(0);
  l_run += (psum[0] + psum[1]) + (psum[2] + psum[3]);
}

// Byte offset of this lane's 16-byte output chunk in the first of the four
// rows one store instruction writes (lane / 16 selects the row, lane % 16
// the chunk), the same for every item.
__device__ __forceinline__ uint32_t o_lane_offset(const PrefillArgs& a, int lane) {
  return static_cast<uint32_t>((lane >> 4) * a.o_st * 2 + 16 * (lane & 15));
}

// Normalises this wave's 32 x 128 output tile (l: the row's full sum) and
// writes its valid rows.  The tile goes through 8 KiB of LDS at `stage`
// (chunk c of row r at chunk c ^ (r % 16), conflict-free both ways) so
// that each store writes four whole 256-byte rows; the stores go through a
// buffer descriptor that ends at the sequence's last row, so rows past it
// are dropped without a branch.  The caller's barrier must follow before
// `stage` is written again.
__device__ __forceinline__ void store_output(const PrefillArgs& a, const WaveItem& wi, int lane,
                                             uint32_t o_lane, float l,
                                             const q3::f32x16 (&acc)[4], char* stage) {
  const int l32 = lane & 31, hl = lane >> 5;
  const float inv = l > 0.f ? 1.f / l : 0.f;  // 0 for rows past the end
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int ch = 4 * db + g4;
      q3::u32x2 w = {q3::pack_bf16x2(acc[db][4 * g4] * inv, acc[db][4 * g4 + 1] * inv),
                     q3::pack_bf16x2(acc[db][4 * g4 + 2] * inv, acc[db][4 * g4 + 3] * inv)};
      *reinterpret_cast<q3::u32x2*>(stage + l32 * 256 + ((ch ^ (l32 & 15)) << 4) + hl * 8) = w;
    }
  const int rows = min(32, wi.len - wi.q0);
  uint16_t* base = a.o + (wi.start + wi.q0) * a.o_st + static_cast<int64_t>(wi.head) * a.o_sh;
  const int bytes = rows > 0 ? static_cast<int>((rows - 1) * a.o_st * 2) + kRowBytes : 0;
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
  const int oc = lane & 15;  // this lane's 16-byte chunk of a row
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rr = 4 * j + (lane >> 4);
    const q3::u32x4 v =
        *reinterpret_cast<const q3::u32x4*>(stage + rr * 256 + ((oc ^ (rr & 15)) << 4));
    // the row offset in the vector offset: the range check covers it (it
    // does not cover the scalar offset)
    __builtin_amdgcn_raw_buffer_store_b128(
        v, orr, o_lane + static_cast<uint32_t>(4 * j * a.o_st * 2), 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Whole items (flat and persistent grids).

// Key tiles [t0, t1) of one work item folded into a fresh online softmax
// state (m_run, l_run, acc): the first tile and the Q rows load, then each
// tile's loads are issued before the previous tile's math (two buffer
// pairs, one barrier per tile).  Every thread of the workgroup calls it;
// all four tile buffers are free when it returns.
template <int W, bool Prio = false>
__device__ __forceinline__ void run_tiles(const PrefillArgs& a, const LaneOffsets& off,
                                          const WaveItem& wi, int t0, int t1, const TileBufs& tb,
                                          int lane, int wave, float& m_run, float& l_run,
                                          q3::f32x16 (&acc)[4]) {
  tile_dma<W>(a, off, wi.start, wi.len, wi.kvh, t0 * kBN, tb.k0, tb.v0, wave);
  q3::bf16x8 qv[8];
  load_q(a, wi, q_lane_offset(a, lane), qv);
  m_run = q3::kNegInf;  // running max (log2 domain) of this query
  l_run = 0.f;          // this lane's share of the denominator
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
  wait_loads();
  __syncthreads();
  auto tile = [&](int it, const uint16_t* kt, const uint16_t* vt, uint16_t* nk, uint16_t* nv) {
    if (it + 1 < t1) tile_dma<W>(a, off, wi.start, wi.len, wi.kvh, (it + 1) * kBN, nk, nv, wave);
    tile_math<Prio>(a, off, wi, lane, it * kBN, kt, vt, qv, m_run, l_run, acc);
    wait_loads();
    __syncthreads();
  };
  for (int it = t0; it < t1; it += 2) {
    tile(it, tb.k0, tb.v0, tb.k1, tb.v1);
    if (it + 1 < t1) tile(it + 1, tb.k1, tb.v1, tb.k0, tb.v0);
  }
}

// This wave's 8 KiB output staging area: wave w in half w % 2 of buffer
// w / 2 (the tile buffers are free after run_tiles).
__device__ __forceinline__ char* stage_of(const TileBufs& tb, int wave) {
  const int sb = wave >> 1;
  return reinterpret_cast<char*>(sb == 0 ? tb.k0 : sb == 1 ? tb.v0 : sb == 2 ? tb.k1 : tb.v1) +
         (wave & 1) * 8192;
}

// One work item: query tile mt of sequence seq for head group hg, over all
// of its key tiles.  Every thread of the workgroup calls it; the caller's
// barrier must follow before the tile buffers are loaded again.
template <int W>
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, const LaneOffsets& off,
                                             int64_t start, int len, int hg, int mt,
                                             const TileBufs& tb) {
  if (mt * a.rows >= len) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  const WaveItem wi = wave_item<W>(a, start, len, hg, mt, wave, lane);
  const int kend = a.causal ? min(len, mt * a.rows + a.rows) : len;
  float m_run, l_run;
  q3::f32x16 acc[4];  // acc[db][r] = O[q0 + l32][32*db + 8*(r/4) + 4*hl + r%4]
  run_tiles<W>(a, off, wi, 0, (kend + kBN - 1) / kBN, tb, lane, wave, m_run, l_run, acc);
  l_run = cross_half_sum(l_run);
  if (!wi.active()) return;
  store_output(a, wi, lane, o_lane_offset(a, lane), l_run, acc, stage_of(tb, wave));
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

// ---------------------------------------------------------------------------
// Wave-specialised tile (varlen_prefill_ws_kernel): one 768-thread workgroup
// per CU, four matrix waves and eight softmax waves, so each SIMD holds one
// matrix wave and the two softmax waves that serve it.  A matrix wave owns
// 32 query rows (Q and the O^T accumulator in registers) and issues only the
// MFMA products; each of its two softmax waves owns 16 of those query
// columns (their running max and sum) and turns the fp32 scores into bf16
// P^T operands.  Scores and P go through LDS, in a three-stage pipeline
// with one barrier per phase: in phase k the matrix waves run QK of tile k
// and PV of tile k - 2, the softmax waves the softmax of tile k - 1 and the
// loads of K(k + 1) and V(k - 1).
//
// LDS (160 KiB, all of it): K and V double buffers (4 x 16 KiB), scores
// (2 x 4 x 8 KiB: [32 queries][64 keys] fp32 per matrix wave, 16-byte chunk
// c of row q at c ^ (q % 16)), P^T operands (2 x 4 x 4 KiB: [4 key chunks]
// [64 lanes] x 16 B per matrix wave).  A softmax wave's rescale factor of
// query q goes into float 2 q of row q of the score buffer it has just read
// (the matrix wave reads it before it writes that buffer again; 32 rows on
// 32 distinct banks), its final sum into float 2 q + 1 after the last phase.
constexpr int kWsMatrix = 4;
constexpr int kWsSoft = 8;
constexpr int kWsWaves = kWsMatrix + kWsSoft;

// Loads one K or V tile of this softmax wave's share (eight waves, two
// 16-byte loads each per lane) into dst.
__device__ __forceinline__ void ws_dma(const uint16_t* base, int64_t row_st, int rows,
                                       const uint32_t (&offs)[kMaxDma], uint16_t* dst, int si) {
  const int bytes = static_cast<int>((rows - 1) * row_st * 2) + kRowBytes;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, bytes, 0x00020000);
  constexpr int D = dma_per_wave<8>();
#pragma unroll
  for (int j = 0; j < D; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(dst + (D * si + j) * 512), 16,
                                             offs[j], 0, 0, 0);
}

// Maximum of 16 scores (v_max3 chains; fmaxf would canonicalize each input).
__device__ __forceinline__ float max3_16(const q3::f32x4 (&x)[4]) {
  float m, t;
  asm volatile(
      "v_max3_f32 %0, %2, %3, %4\n\t"
      "v_max3_f32 %1, %10, %11, %12\n\t"
      "v_max3_f32 %0, %0, %5, %6\n\t"
      "v_max3_f32 %1, %1, %13, %14\n\t"
      "v_max3_f32 %0, %0, %7, %8\n\t"
      "v_max3_f32 %1, %1, %15, %16\n\t"
      "v_max3_f32 %0, %0, %9, %17\n\t"
      "v_max_f32 %0, %0, %1"
      : "=&v"(m), "=&v"(t)
      : "v"(x[0][0]), "v"(x[0][1]), "v"(x[0][2]), "v"(x[0][3]), "v"(x[1][0]), "v"(x[1][1]),
        "v"(x[1][2]), "v"(x[1][3]), "v"(x[2][0]), "v"(x[2][1]), "v"(x[2][2]), "v"(x[2][3]),
        "v"(x[3][0]), "v"(x[3][1]), "v"(x[3][2]), "v"(x[3][3]));
  return m;
}

__global__ __launch_bounds__(kWsWaves * 64) __attribute__((amdgpu_waves_per_eu(3, 3)))
void varlen_prefill_ws_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t s_k0[kTileElems];
  __shared__ __attribute__((aligned(1024))) uint16_t s_k1[kTileElems];
  __shared__ __attribute__((aligned(1024))) uint16_t s_v0[kTileElems];
  __shared__ __attribute__((aligned(1024))) uint16_t s_v1[kTileElems];
  __shared__ __attribute__((aligned(1024))) float s_sc[2][kWsMatrix][32 * kBN];
  __shared__ __attribute__((aligned(1024))) q3::u32x4 s_pt[2][kWsMatrix][4 * 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the item: as the flat grid of four-wave workgroups
  const int64_t id = blockIdx.x;
  const int hg = static_cast<int>(id % a.groups);
  const int seq = static_cast<int>((id / a.groups) % a.num_seqs);
  const int mt =
      a.n_mtiles - 1 - static_cast<int>(id / (static_cast<int64_t>(a.groups) * a.num_seqs));
  const int64_t start = a.cu[seq];
  const int64_t end = a.cu[seq + 1];
  if (start < 0 || end > a.total || end <= start) return;
  const int len = static_cast<int>(end - start);
  if (mt * a.rows >= len) return;
  const int kend = a.causal ? min(len, mt * a.rows + a.rows) : len;
  const int n = (kend + kBN - 1) / kBN;
  const float c = a.scale_log2;
  const bool matrix = wave < kWsMatrix;
  const int si = wave - kWsMatrix;                 // softmax wave index
  const int mi = matrix ? wave : si >> 1;          // the matrix wave served
  const WaveItem wi = wave_item<4>(a, start, len, hg, mt, mi, lane);
  const uint16_t* kb = a.k + start * a.k_st + static_cast<int64_t>(wi.kvh) * a.k_sh;
  const uint16_t* vb = a.v + start * a.v_st + static_cast<int64_t>(wi.kvh) * a.v_sh;
  auto kbuf = [&](int i) { return i ? s_k1 : s_k0; };
  auto vbuf = [&](int i) { return i ? s_v1 : s_v0; };

  if (matrix) {
    // ---------------- matrix wave ----------------
    const LaneOffsets off = lane_offsets<4>(lane, 0, a.k_st * 2, a.v_st * 2);
    const int q = lane & 31;
    q3::bf16x8 qv[8];
    load_q(a, wi, q_lane_offset(a, lane), qv);
    q3::f32x16 acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    wait_loads();
    __syncthreads();  // K(0) staged
    for (int k = 0; k < n + 2; ++k) {
      const bool qk = k < n, pv = k >= 2;
      const int b = k & 1;  // buffers of tile k (K, scores) and of tile k - 2 (V, scores, P)
      float* sc = s_sc[b][mi];
      if (pv) {  // the softmax waves' rescale of tile k - 2, read before S(k) overwrites it
        const float alpha = sc[q * kBN + 2 * q];
        if (__any(alpha != 1.f)) {
#pragma unroll
          for (int db = 0; db < 4; ++db) acc[db] *= alpha;
        }
      }
      if (qk) {
        const uint16_t* kt = kbuf(b);
        q3::f32x16 s[2];
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[kb2][r] = 0.f;
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
        // S^T -> the score buffer: lane (q, hl) holds keys 32 kb2 + 8 j + 4 hl
        // + 0..3 in s[kb2][4 j .. 4 j + 3], chunk 8 kb2 + 2 j + hl of row q.
        const int hl = lane >> 5;
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int ch = 8 * kb2 + 2 * j + hl;
            *reinterpret_cast<q3::f32x4*>(sc + q * kBN + 4 * (ch ^ (q & 15))) =
                q3::f32x4{s[kb2][4 * j], s[kb2][4 * j + 1], s[kb2][4 * j + 2], s[kb2][4 * j + 3]};
          }
      }
      if (pv) {
        const uint16_t* vt = vbuf(b);
        const q3::u32x4* pt = s_pt[b][mi];
        q3::bf16x8 vf[kAhead];
        q3::bf16x8 pf[2];  // P^T operand of key chunk u / 4, one chunk ahead
        pf[0] = q3::as_bf16x8(pt[lane]);
#pragma unroll
        for (int u = 0; u < kAhead; ++u) vf[u] = lds_vt(vt, pv_operand(off, u));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          if ((u & 3) == 0 && u + 4 < 16) pf[((u >> 2) + 1) & 1] = q3::as_bf16x8(pt[(u >> 2) * 64 + 64 + lane]);
          acc[u & 3] = q3::mfma32x32x16(vf[u % kAhead], pf[(u >> 2) & 1], acc[u & 3]);
          if (u + kAhead < 16) vf[u % kAhead] = lds_vt(vt, pv_operand(off, u + kAhead));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      wait_loads();
      __syncthreads();
    }
    __syncthreads();  // the softmax waves' final sums are in
    const float l = s_sc[0][mi][q * kBN + 2 * q + 1];
    if (!wi.active()) return;
    // staging: this wave's half of a K buffer (no reads or loads of it remain)
    char* stage = reinterpret_cast<char*>(mi < 2 ? s_k0 : s_k1) + (mi & 1) * 8192;
    store_output(a, wi, lane, o_lane_offset(a, lane), l, acc, stage);
    return;
  }
  // ---------------- softmax wave ----------------
  const LaneOffsets off8 = lane_offsets<8>(lane, si, a.k_st * 2, a.v_st * 2);
  const int ql = lane & 15, g = lane >> 4;
  const int qm = 16 * (si & 1) + ql;  // query column within the matrix wave
  float m_run = q3::kNegInf, l_run = 0.f;
  ws_dma(kb, a.k_st, min(kBN, len), off8.kdma, s_k0, si);
  wait_loads();
  __syncthreads();  // K(0) staged
  for (int k = 0; k < n + 2; ++k) {
    if (k + 1 < n) {
      const int n0 = (k + 1) * kBN;
      ws_dma(kb + n0 * a.k_st, a.k_st, min(kBN, len - n0), off8.kdma, kbuf((k + 1) & 1), si);
    }
    if (k >= 1 && k - 1 < n) {
      const int n0 = (k - 1) * kBN;
      ws_dma(vb + n0 * a.v_st, a.v_st, min(kBN, len - n0), off8.vdma, vbuf((k - 1) & 1), si);
    }
    if (k >= 1 && k <= n) {
      const int t = k - 1, b = t & 1, n0 = t * kBN;
      float* sc = s_sc[b][mi];
      q3::f32x4 x[4];  // keys n0 + 16 g + 4 i + e
#pragma unroll
      for (int i = 0; i < 4; ++i)
        x[i] = *reinterpret_cast<const q3::f32x4*>(sc + qm * kBN + 4 * ((4 * g + i) ^ (qm & 15)));
      const bool need_mask = (n0 + kBN > len) || (a.causal && n0 + kBN - 1 > wi.q0);
      if (need_mask) {
        int lim = len - 1 - n0 - 16 * g;
        if (a.causal) lim = min(lim, wi.q0 + qm - n0 - 16 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) x[i][e] = 4 * i + e <= lim ? x[i][e] : q3::kNegInf;
      }
      float bm = max3_16(x);
      bm = q3::max_xor32(q3::max_xor16(bm));
      const float m_cand = bm * c;
      const bool raise = m_cand > m_run + kRescaleSlack;
      const float m_new = raise ? m_cand : m_run;
      const float alpha = raise ? q3::fast_exp2(m_run - m_new) : 1.f;
      m_run = m_new;
      const float m_use = m_run == q3::kNegInf ? 0.f : m_run;
      float e[4][4];
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          e[i][j] = q3::fast_exp2(__builtin_fmaf(x[i][j], c, -m_use));
          ps += e[i][j];
        }
      ps = q3::sum_xor32(q3::sum_xor16(ps));
      l_run = __builtin_fmaf(l_run, alpha, ps);
      // P^T operands of key chunk g: lane slot qm + 32 hl holds keys
      // 16 g + 4 hl + {0..3, 8..11}.
      q3::u32x4* pt = s_pt[b][mi] + g * 64 + qm;
      pt[0] = q3::u32x4{q3::pack_bf16x2(e[0][0], e[0][1]), q3::pack_bf16x2(e[0][2], e[0][3]),
                        q3::pack_bf16x2(e[2][0], e[2][1]), q3::pack_bf16x2(e[2][2], e[2][3])};
      pt[32] = q3::u32x4{q3::pack_bf16x2(e[1][0], e[1][1]), q3::pack_bf16x2(e[1][2], e[1][3]),
                         q3::pack_bf16x2(e[3][0], e[3][1]), q3::pack_bf16x2(e[3][2], e[3][3])};
      if (g == 0) sc[qm * kBN + 2 * qm] = alpha;  // read by the matrix wave before PV of this tile
    }
    wait_loads();
    __syncthreads();
  }
  if (g == 0) s_sc[0][mi][qm * kBN + 2 * qm + 1] = l_run;
  __syncthreads();
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
template <int W>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
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

// ---------------------------------------------------------------------------
// Range schedule.
//
// Items are ordered head group first (so with a multiple of 8 groups each
// XCD's contiguous share of the ranges reads one KV head's tiles from its
// L2), then sequences longest first, then query tiles in order.  Item
// (hg, rank r, mt) sits at weight position hg H + pos[r] + f_r(mt), where
// f(mt) = kUnits (key tiles of query tiles < mt) + kItemUnits mt, and its
// tile j's midpoint at that + kItemUnits + kUnits j + kUnits / 2.  Range v
// of N owns the positions p with floor(p N / U) = v (U: the total weight).
// A tile belongs to the range holding its midpoint; an item of at most
// kAtomicTiles tiles goes whole to the range holding its own midpoint.

// Key tiles of query tile mt.
__device__ __forceinline__ int item_tiles(int len, int mt, int rows, int causal) {
  const int kend = causal ? min(len, (mt + 1) * rows) : len;
  return (kend + kBN - 1) / kBN;
}
// Key tiles of query tiles 0 .. mt - 1, for mt below the sequence's query
// tile count (whole query tiles only; rows is 32 or a multiple of 64).
__device__ __forceinline__ int64_t tiles_before(int len, int mt, int rows, int causal) {
  if (!causal) return static_cast<int64_t>(mt) * ((len + kBN - 1) / kBN);
  if (rows >= kBN) return static_cast<int64_t>(rows / kBN) * mt * (mt + 1) / 2;
  return (static_cast<int64_t>(mt) + 1) * (mt + 1) / 4;  // rows 32: sum of ceil(m / 2), m = 1..mt
}
__device__ __forceinline__ int64_t item_pos_in_seq(int len, int mt, int rows, int causal) {
  return kUnits * tiles_before(len, mt, rows, causal) + static_cast<int64_t>(kItemUnits) * mt;
}
__device__ __forceinline__ int64_t seq_weight(int len, int rows, int causal) {
  if (len <= 0) return 0;
  const int n = (len + rows - 1) / rows;
  return item_pos_in_seq(len, n - 1, rows, causal) +
         kUnits * static_cast<int64_t>(item_tiles(len, n - 1, rows, causal)) + kItemUnits;
}

// One segment of a range: key tiles [j0, j1) of item (hg, rank r, mt),
// wave-uniform.
struct RangeSeg {
  int valid;
  int hg, r, mt;
  int64_t P;       // the item's weight position
  int64_t start;   // first row of its sequence
  int len;         // the sequence's length
  int n;           // its query tiles
  int kt;          // key tiles of the item
  int j0, j1;      // the tiles this range owns
  int cut;         // its tiles span several ranges
};

struct RangeCtx {
  int64_t H;       // weight of one head group
  int64_t U;       // total weight
  int N;           // ranges
  int v;           // this workgroup's range
  int64_t p_lo, p_hi;  // its positions
  int n_ranked;    // sequences of non-zero length (ranks 0 .. n_ranked - 1)
  const int* rlen;
  const int* rstart;
  const int64_t* rpos;
  // floor(p N / U), the range owning position p.  In double precision the
  // quotient is exact here: p N < 2^53, and U < 2^43 keeps a non-integer
  // quotient at least 2^-43 from the next integer, more than the rounding
  // error (N 2^-53 <= 2^-43 for N <= 1024).
  __device__ __forceinline__ int owner(int64_t p) const {
    return static_cast<int>(__builtin_floor(static_cast<double>(p * N) / static_cast<double>(U)));
  }
};

__device__ __forceinline__ int uread(const int* p) {
  return __builtin_amdgcn_readfirstlane(*p);
}
__device__ __forceinline__ int64_t uread64(const int64_t* p) {
  const uint64_t x = static_cast<uint64_t>(*p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Fills kt and the tiles the range owns (item coordinates, P and the
// sequence already set).
__device__ __forceinline__ void own_tiles(const PrefillArgs& a, const RangeCtx& rc, RangeSeg& sg) {
  sg.kt = item_tiles(sg.len, sg.mt, a.rows, a.causal);
  sg.cut = 0;
  if (sg.kt <= kAtomicTiles) {
    const int64_t mid = sg.P + (kUnits * sg.kt + kItemUnits) / 2;
    const bool own = mid >= rc.p_lo && mid < rc.p_hi;
    sg.j0 = 0;
    sg.j1 = own ? sg.kt : 0;
    return;
  }
  const int64_t base = sg.P + kItemUnits + kUnits / 2;  // tile 0's midpoint
  auto first_at = [&](int64_t p) -> int {  // first tile with midpoint >= p
    if (p <= base) return 0;
    const int64_t j = (p - base + kUnits - 1) / kUnits;
    return static_cast<int>(j < sg.kt ? j : sg.kt);
  };
  sg.j0 = first_at(rc.p_lo);
  sg.j1 = first_at(rc.p_hi);
  sg.cut = sg.j0 < sg.j1 && (sg.j0 > 0 || sg.j1 < sg.kt);
}

// A cut item's first range (the one holding tile 0) and its number of
// ranges.
__device__ __forceinline__ void cut_ranges(const RangeCtx& rc, const RangeSeg& sg, int& vfirst,
                                           int& nseg) {
  const int64_t base = sg.P + kItemUnits + kUnits / 2;
  vfirst = sg.j0 == 0 ? rc.v : rc.owner(base);
  const int vlast =
      sg.j1 == sg.kt ? rc.v : rc.owner(base + static_cast<int64_t>(kUnits) * (sg.kt - 1));
  nseg = vlast - vfirst + 1;
}

__device__ __forceinline__ void seq_of_rank(const PrefillArgs& a, const RangeCtx& rc, RangeSeg& sg) {
  sg.len = uread(rc.rlen + sg.r);
  sg.start = uread(rc.rstart + sg.r);
  sg.n = (sg.len + a.rows - 1) / a.rows;
}

// The item holding weight position p (0 <= p < U).
__device__ __forceinline__ RangeSeg locate(const PrefillArgs& a, const RangeCtx& rc, int64_t p) {
  RangeSeg sg;
  sg.valid = 1;
  sg.hg = static_cast<int>(p / rc.H);
  const int64_t p1 = p - sg.hg * rc.H;
  int lo = 0, hi = rc.n_ranked - 1;  // largest rank with pos <= p1
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (uread64(rc.rpos + mid) <= p1) lo = mid; else hi = mid - 1;
  }
  sg.r = lo;
  seq_of_rank(a, rc, sg);
  const int64_t p2 = p1 - uread64(rc.rpos + lo);
  int mlo = 0, mhi = sg.n - 1;  // largest query tile with f(mt) <= p2
  while (mlo < mhi) {
    const int mid = (mlo + mhi + 1) >> 1;
    if (item_pos_in_seq(sg.len, mid, a.rows, a.causal) <= p2) mlo = mid; else mhi = mid - 1;
  }
  sg.mt = mlo;
  sg.P = p - p2 + item_pos_in_seq(sg.len, mlo, a.rows, a.causal);
  own_tiles(a, rc, sg);
  return sg;
}

// The item after sg's (LDS is read only when it starts another sequence).
__device__ __forceinline__ RangeSeg next_item(const PrefillArgs& a, const RangeCtx& rc,
                                              const RangeSeg& sg) {
  RangeSeg nx = sg;
  nx.P = sg.P + static_cast<int64_t>(kUnits) * sg.kt + kItemUnits;
  nx.valid = nx.P < rc.p_hi;
  if (!nx.valid) return nx;
  if (++nx.mt == sg.n) {
    nx.mt = 0;
    if (++nx.r == rc.n_ranked) {
      nx.r = 0;
      if (++nx.hg == a.groups) {
        nx.valid = 0;
        return nx;
      }
    }
    seq_of_rank(a, rc, nx);
  }
  own_tiles(a, rc, nx);
  return nx;
}

// sg itself if the range owns some of its tiles, else the next such item
// (items the range does not own lie only at its two ends).
__device__ __forceinline__ RangeSeg next_owned(const PrefillArgs& a, const RangeCtx& rc,
                                               RangeSeg sg) {
  while (sg.valid && sg.j0 >= sg.j1) sg = next_item(a, rc, sg);
  return sg;
}

// Partial state hand-off of cut items.  Written and read with device-scope
// accesses (sc1: through to, and from, the point where all XCDs' L2s
// agree), so no L2 write-back or invalidation is needed (those stall the
// whole XCD).  A part's saves complete (vmcnt(0)) before its ticket is
// taken, and the part that takes the last ticket reads the others' saves
// only after that, so it sees them whole.
constexpr int kCpolDevice = 16;  // sc1

template <int W>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(const PrefillArgs& a, int slot) {
  return __builtin_amdgcn_make_buffer_rsrc(a.slots + static_cast<int64_t>(slot) * slot_floats<W>(),
                                           0, slot_floats<W>() * 4, 0x00020000);
}

template <int W>
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
  const uint32_t ml = slot_ml_offset<W>() + (wave * 64 + lane) * 8;
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_run), slot, ml, 0, kCpolDevice);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l_run), slot, ml + 4, 0, kCpolDevice);
}

// One saved part of a cut item, as this lane holds it: the running max,
// the sum and 16 x 4 accumulator floats.
struct PartState {
  float m, l;
  q3::f32x4 x[16];
};

// Issues every load of a saved part at once (one memory round trip).
template <int W>
__device__ __forceinline__ PartState load_part(__amdgpu_buffer_rsrc_t slot, int wave, int lane) {
  PartState st;
  const uint32_t ml = slot_ml_offset<W>() + (wave * 64 + lane) * 8;
  st.m = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(slot, ml, 0, kCpolDevice));
  st.l = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(slot, ml + 4, 0, kCpolDevice));
#pragma unroll
  for (int i = 0; i < 16; ++i)
    st.x[i] = __builtin_bit_cast(
        q3::f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       slot, static_cast<uint32_t>(((wave * 16 + i) * 64 + lane) * 16), 0,
                       kCpolDevice));
  return st;
}

// Folds a part into (m_run, l_run, acc): the state becomes relative to the
// larger running max, state * 2^(m_state - m) + part * 2^(m_part - m).
// From the empty state (m_run = -inf, l_run = 0, acc = 0) the result is the
// part itself (factors 0 and exp2(0) = 1).
__device__ __forceinline__ void fold_state(const PartState& st, float& m_run, float& l_run,
                                           q3::f32x16 (&acc)[4]) {
  const float m = fmaxf(m_run, st.m);
  const float m_use = m == q3::kNegInf ? 0.f : m;
  const float a_s = q3::fast_exp2(m_run - m_use);  // exp2(-inf) = 0: an empty side adds nothing
  const float a_p = q3::fast_exp2(st.m - m_use);
  m_run = m;
  l_run = __builtin_fmaf(st.l, a_p, l_run * a_s);
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y = acc[i >> 2][4 * (i & 3) + e];
      acc[i >> 2][4 * (i & 3) + e] = __builtin_fmaf(st.x[i][e], a_p, y * a_s);
    }
}

// Folds parts p0 .. nseg - 1 of the cut item whose first range is vfirst
// (part 0: slot 2 vfirst + 1, part p > 0: slot 2 (vfirst + p)), in key
// order, so the bits depend only on the parts: one memory round trip per
// part (two parts in flight would not fit the tile loop's registers).
template <int W>
__device__ __forceinline__ void fold_parts(const PrefillArgs& a, int vfirst, int p0, int nseg,
                                           int wave, int lane, float& m_run, float& l_run,
                                           q3::f32x16 (&acc)[4]) {
  for (int p = p0; p < nseg; ++p)
    fold_state(load_part<W>(slot_rsrc<W>(a, p == 0 ? 2 * vfirst + 1 : 2 * (vfirst + p)), wave,
                            lane),
               m_run, l_run, acc);
}

// Range grid (CUs x resident workgroups, a multiple of 8): range v of N
// (ranges of workgroups on one XCD adjacent when every workgroup has one)
// is streamed as a chain of segments, each starting with the loads of its
// first K/V tile and its Q rows.  A segment of a cut item
// saves its partial state in slot 2 v (the range's first segment) or
// 2 v + 1 (its last, the part holding the item's tile 0), then takes the
// item's ticket; the part taking the last ticket folds every part in key
// order and writes the output.  The part holding tile 0 (normally the
// last to finish: it ends its range) first checks the ticket and, when the
// others are all in, folds without saving.  No part waits for another.
template <int W>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void varlen_prefill_range_kernel(PrefillArgs a) {
  Q3_PREFILL_TILE_BUFFERS;
  __shared__ int s_rlen[kMaxSeqs];
  __shared__ int s_rstart[kMaxSeqs];
  __shared__ int64_t s_rpos[kMaxSeqs + 1];
  __shared__ uint32_t s_ticket;
  static_assert(kMaxSeqs == 4 * 64, "one wave scans the ranked weights, four per lane");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = a.num_seqs;
  // ---- sequence tables: lengths ranked longest first, weight prefix ----
  int* s_len0 = reinterpret_cast<int*>(s_k0);  // tile buffers are free until the first load
  int* s_start0 = reinterpret_cast<int*>(s_v0);
  for (int t = tid; t < S; t += W * 64) {
    const int64_t s0 = a.cu[t], s1 = a.cu[t + 1];
    const bool ok = s0 >= 0 && s1 <= a.total && s1 > s0;
    s_len0[t] = ok ? static_cast<int>(s1 - s0) : 0;
    s_start0[t] = ok ? static_cast<int>(s0) : 0;
  }
  __syncthreads();
  for (int t = tid; t < S; t += W * 64) {
    const int lt = s_len0[t];
    int rank = 0;
    for (int u = 0; u < S; ++u) {
      const int lu = s_len0[u];
      rank += (lu > lt || (lu == lt && u < t)) ? 1 : 0;
    }
    s_rlen[rank] = lt;
    s_rstart[rank] = s_start0[t];
  }
  __syncthreads();
  if (wave == 0) {
    int64_t w4[4], sum = 0;
    int nz = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = lane * 4 + i;
      const int len = r < S ? s_rlen[r] : 0;
      w4[i] = seq_weight(len, a.rows, a.causal);
      sum += w4[i];
      nz += len > 0 ? 1 : 0;
    }
    int64_t incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    int64_t run = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = lane * 4 + i;
      if (r < kMaxSeqs) s_rpos[r] = run;
      run += w4[i];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) nz += __shfl_xor(nz, o, 64);
    if (lane == 63) s_rpos[kMaxSeqs] = incl;
    if (lane == 0) s_ticket = static_cast<uint32_t>(nz);
  }
  __syncthreads();
  RangeCtx rc;
  rc.rlen = s_rlen;
  rc.rstart = s_rstart;
  rc.rpos = s_rpos;
  rc.H = uread64(s_rpos + kMaxSeqs);
  rc.n_ranked = static_cast<int>(__builtin_amdgcn_readfirstlane(s_ticket));
  rc.U = rc.H * a.groups;
  if (rc.U == 0) return;
  const int nwg = gridDim.x;
  int64_t N = rc.U / (kMinRangeTiles * kUnits);
  N = N < 1 ? 1 : N;
  N = N < nwg ? N : nwg;
  N = N < a.max_ranges ? N : a.max_ranges;
  rc.N = static_cast<int>(N);
  const int w = blockIdx.x;
  // every workgroup busy: XCD x (workgroups w % 8 == x) holds ranges
  // x * nwg / 8 .. , adjacent items sharing its L2; fewer ranges: spread.
  const int v = rc.N == nwg && nwg % 8 == 0 ? (w % 8) * (nwg / 8) + w / 8 : w;
  if (v >= rc.N) return;
  rc.v = v;
  rc.p_lo = (static_cast<int64_t>(v) * rc.U + rc.N - 1) / rc.N;
  rc.p_hi = (static_cast<int64_t>(v + 1) * rc.U + rc.N - 1) / rc.N;
  __syncthreads();  // s_ticket is reused below
  if (rc.p_lo >= rc.p_hi) return;

  const uint32_t o_lane = o_lane_offset(a, lane);
  for (RangeSeg cur = next_owned(a, rc, locate(a, rc, rc.p_lo)); cur.valid;
       cur = next_owned(a, rc, next_item(a, rc, cur))) {
    const WaveItem wi = wave_item<W>(a, cur.start, cur.len, cur.hg, cur.mt, wave, lane);
    float m_run, l_run;
    q3::f32x16 acc[4];  // acc[db][r] = O[q0 + l32][32*db + 8*(r/4) + 4*hl + r%4]
    run_tiles<W, true>(a, off, wi, cur.j0, cur.j1, tb, lane, wave, m_run, l_run, acc);
    bool write = !cur.cut;
    if (cur.cut) {
      int vfirst, nseg;
      cut_ranges(rc, cur, vfirst, nseg);
      uint32_t* ticket = a.tickets + vfirst;
      const bool first_part = v == vfirst;  // holds tile 0, ends this range
      const uint32_t last = static_cast<uint32_t>(nseg - 1);
      bool merged = false;
      if (first_part) {
        if (tid == 0) s_ticket = __hip_atomic_load(ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s_ticket == last) {  // every other part has saved: fold them in without saving
          fold_parts<W>(a, vfirst, 1, nseg, wave, lane, m_run, l_run, acc);
          merged = true;
        }
        __syncthreads();  // s_ticket is reused below
      }
      if (!merged) {
        save_partial<W>(slot_rsrc<W>(a, first_part ? 2 * v + 1 : 2 * v), wave, lane, m_run, l_run,
                        acc);
        wait_loads();  // this wave's saves are complete
        __syncthreads();
        if (tid == 0)
          s_ticket = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s_ticket == last) {  // the last part in: fold all saved parts, in key order
          m_run = q3::kNegInf;
          l_run = 0.f;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
          fold_parts<W>(a, vfirst, 0, nseg, wave, lane, m_run, l_run, acc);
          merged = true;
        }
      }
      if (merged && tid == 0)
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      write = merged;
    }
    if (write) {
      l_run = cross_half_sum(l_run);
      if (wi.active()) store_output(a, wi, lane, o_lane, l_run, acc, stage_of(tb, wave));
    }
    __syncthreads();  // the staging buffers are read before the next segment's loads refill them
  }
}

// QWEN3_PREFILL_TILE=ws selects the wave-specialised tile (flat grid of
// four-wave items) for batches that would take the four-wave path; read at
// every call.
bool ws_tile_selected() {
  const char* e = std::getenv("QWEN3_PREFILL_TILE");
  return e && std::strcmp(e, "ws") == 0;
}

// Resident workgroups per CU of a kernel, queried once per device (a
// host-side cost of every call otherwise).
template <int W>
int resident_per_cu(const void* kernel, int dev, int* cache) {
  int per_cu = dev >= 0 && dev < 64 ? cache[dev] : 0;
  if (per_cu == 0 &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, W * 64, 0) == hipSuccess &&
      per_cu > 0 && dev >= 0 && dev < 64)
    cache[dev] = per_cu;
  return per_cu;
}

// Sizes the items for W waves and launches the range grid (four waves,
// given a workspace, fewer items than resident workgroups), the persistent
// grid (CUs x resident workgroups, from the occupancy API) or, past their
// LDS tables, the flat grid.
template <int W>
int launch_prefill(PrefillArgs a, int num_seqs, int max_seqlen, int dev, int cus,
                   hipStream_t s, const char* who) {
  a.rows = 32 * W / a.HG;
  a.n_mtiles = static_cast<int>(q3::cdiv(max_seqlen, a.rows));
  const int64_t blocks = static_cast<int64_t>(a.groups) * num_seqs * a.n_mtiles;
  if (blocks > 0x7fffffff)
    return q3::fail(QWEN3_EINVAL, "%s: grid too large (heads %d, seqs %d, max_seqlen %d)", who,
                    a.Hq, num_seqs, max_seqlen);
  static int occ_persistent[64] = {0};
  static int occ_range[64] = {0};
  // At most this many items: groups x (query tiles of all rows + one
  // ragged tile per sequence).
  const int64_t items_max = static_cast<int64_t>(a.groups) *
                            (q3::cdiv(a.total, a.rows) + static_cast<int64_t>(num_seqs));
  if constexpr (W == 4) {
    // Fewer items than resident workgroups (a few long prompts): the range
    // schedule, which cuts the heaviest items across workgroups.  With
    // more, whole items in the persistent grid finish sooner: an item
    // switch costs about 2.5 tiles' time and a cut item more, which the
    // better balance of equal ranges does not win back (measured on the
    // Qwen3-0.6B batch: 59 us persistent against 70 us in ranges).
    if (a.tickets && num_seqs <= kMaxSeqs && cus > 0) {
      const int per_cu = resident_per_cu<W>(
          reinterpret_cast<const void*>(varlen_prefill_range_kernel<W>), dev, occ_range);
      const int wgs = (cus * per_cu) / 8 * 8;
      a.max_ranges = a.max_ranges < wgs ? a.max_ranges : wgs;
      if (per_cu > 0 && a.max_ranges > 0 && items_max < static_cast<int64_t>(cus) * per_cu) {
        hipLaunchKernelGGL(varlen_prefill_range_kernel<W>, dim3(wgs), dim3(W * 64), 0, s, a);
        return q3::launch_status(who);
      }
    }
  }
  const int per_cu = resident_per_cu<W>(
      reinterpret_cast<const void*>(varlen_prefill_persistent_kernel<W>), dev, occ_persistent);
  const bool persistent =
      num_seqs <= kMaxSeqs && a.n_mtiles <= kScanMax && cus > 0 && per_cu > 0;
  if (persistent) {
    const int wgs = ((cus * per_cu + 7) / 8) * 8;  // multiple of 8 for the XCD-preserving snake
    hipLaunchKernelGGL(varlen_prefill_persistent_kernel<W>, dim3(wgs), dim3(W * 64), 0, s, a);
  } else {
    hipLaunchKernelGGL(varlen_prefill_flat_kernel<W>, dim3(static_cast<unsigned>(blocks)),
                       dim3(W * 64), 0, s, a);
  }
  return q3::launch_status(who);
}

// Workspace: schedule counters, then range tickets, then range slots; the
// range part is sized for two four-wave workgroups per CU.
constexpr size_t kCtrBytes = (kPools + 1) * kPoolStride * sizeof(uint32_t);
constexpr int kMaxCus = 1024;
size_t ranges_for(int cus) { return static_cast<size_t>(2) * static_cast<size_t>(cus); }
size_t ticket_bytes(size_t ranges) { return (ranges * sizeof(uint32_t) + 255) / 256 * 256; }
size_t workspace_bytes_for(int cus) {
  const size_t n = ranges_for(cus);
  return kCtrBytes + ticket_bytes(n) + 2 * n * slot_floats<4>() * sizeof(float);
}

int device_cus() {
  static int cu_cache[64] = {0};
  int dev = -1, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cu_cache[dev]) return cu_cache[dev];
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  if (dev < 64) cu_cache[dev] = cus;
  return cus;
}

}  // namespace

extern "C" size_t qwen3_varlen_prefill_workspace_bytes(void) {
  const int cus = device_cus();
  return workspace_bytes_for(cus > 0 && cus <= kMaxCus ? cus : 256);
}

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
  const int cus = device_cus();
  if (workspace) {
    const size_t need = workspace_bytes_for(cus > 0 && cus <= kMaxCus ? cus : 256);
    if (workspace_bytes < need)
      return q3::fail(QWEN3_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who,
                      need, workspace_bytes);
    if (!q3::aligned16(workspace))
      return q3::fail(QWEN3_EALIGN, "%s: workspace must be 16-byte aligned", who);
  }

  q3::clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  // Eight-wave workgroups once the batch holds enough of their (twice as
  // large) work items to give every CU four: they halve the K/V tile
  // traffic per flop; smaller batches take the range schedule of four-wave
  // workgroups, which cuts the heaviest items across workgroups.
  const int64_t rows8 = 32 * 8 / a.HG;
  const int64_t items8 = static_cast<int64_t>(a.groups) * q3::cdiv(total_tokens, rows8);
  const bool wide = cus > 0 && items8 >= 4 * static_cast<int64_t>(cus);
  if (workspace) {
    char* ws = static_cast<char*>(workspace);
    // Items handed out from the counters only on the eight-wave path: over
    // many rounds of mixed-length items they finish 1-2% sooner.
    if (wide) a.ctr = reinterpret_cast<uint32_t*>(ws);
    const size_t n = ranges_for(cus > 0 && cus <= kMaxCus ? cus : 256);
    a.tickets = reinterpret_cast<uint32_t*>(ws + kCtrBytes);
    a.slots = reinterpret_cast<float*>(ws + kCtrBytes + ticket_bytes(n));
    a.max_ranges = static_cast<int>(n);
  }
  if (ws_tile_selected()) {  // flat grid of four-wave items on the wave-specialised tile
    a.rows = 32 * 4 / a.HG;
    a.n_mtiles = static_cast<int>(q3::cdiv(max_seqlen, a.rows));
    const int64_t blocks = static_cast<int64_t>(a.groups) * num_seqs * a.n_mtiles;
    if (blocks > 0x7fffffff)
      return q3::fail(QWEN3_EINVAL, "%s: grid too large (heads %d, seqs %d, max_seqlen %d)", who,
                      a.Hq, num_seqs, max_seqlen);
    hipLaunchKernelGGL(varlen_prefill_ws_kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(kWsWaves * 64), 0, s, a);
    return q3::launch_status(who);
  }
  return wide ? launch_prefill<8>(a, num_seqs, max_seqlen, dev, cus, s, who)
              : launch_prefill<4>(a, num_seqs, max_seqlen, dev, cus, s, who);
}
