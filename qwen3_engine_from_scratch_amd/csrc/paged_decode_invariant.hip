// Batch-invariant paged decode attention for gfx950: the same attention as
// paged_decode.hip (qwen3/kernels/paged_attention.py:27-129), computed so
// that a sequence's output bits depend only on its own query, K/V and
// length, never on the batch around it.
//
//  * Every sequence-head is cut into canonical partitions from its first
//    tile: 16 tiles (256 tokens), or 32 tiles (512 tokens) for
//    sequence-heads of 4,096 tokens or more (fewer hand-offs where they are
//    long; the size depends on the sequence's own length only).  A
//    partition's softmax state starts fresh and folds its tiles in load
//    batches of kChunk from its first tile; the output is the left fold of
//    the partition states in ascending order, with one fold formula
//    everywhere.
//  * The batch only decides which wave owns which partitions (persistent
//    waves over the flat tile list, as in the default path, with ranges
//    rounded to partition starts), so work stays balanced to within one
//    partition per wave.
//  * A sequence-head split across waves is handed on through workspace
//    slots with tickets (no wave ever waits for another): waves visit their
//    segments from the last to the first, so the first part's fold is
//    written early and the last part usually folds everything straight into
//    the output.
//  * Batches above kStreamMaxB use one wave per partition and a merge kernel
//    with the same fold.
#include "paged_decode_tile.hpp"

namespace {

// Tiles of one canonical partition of a sequence-head of n tiles: the unit
// of work a wave owns, and of the merge.
constexpr int kPartTiles = 16;       // the smallest (slots are sized for it)
constexpr int kLongPartTiles = 32;
constexpr int kLongTiles = 256;      // from 4,096 tokens on
__host__ __device__ constexpr int part_tiles(int n) {
  return n >= kLongTiles ? kLongPartTiles : kPartTiles;
}

// ---------------------------------------------------------------------------
// Canonical partitions.  Every sequence-head is cut into partitions of
// part_tiles(n) tiles from its first tile; a partition's softmax state starts
// fresh and folds its tiles in load batches of kChunk tiles from its first
// tile, and the output is the left fold of the partition states in
// ascending partition order.  Both launch paths and the merge compute
// exactly this, whatever batch a sequence is in and wherever the waves'
// ranges fall, so a sequence's output bits depend on its own data only.

// Weights of the union of two softmax states with running maxima mF and mp
// (log2 domain).  The fold below is the one formula every kernel uses.
struct FoldW {
  float m, a, b;
};

__device__ __forceinline__ FoldW fold_weights(float mF, float mp) {
  FoldW w;
  w.m = fmaxf(mF, mp);
  const float mu = w.m == q3::kNegInf ? 0.f : w.m;
  w.a = q3::fast_exp2(mF - mu);
  w.b = q3::fast_exp2(mp - mu);
  return w;
}

__device__ __forceinline__ float fold_val(float f, float a, float p, float b) {
  return __builtin_fmaf(f, a, p * b);
}

__device__ __forceinline__ int64_t slot_of(const DecodeArgs& a, int b, int hkv, int j) {
  return (static_cast<int64_t>(b) * a.Hkv + hkv) * a.max_parts + j;
}

// Writes the state of column lo (lane (lo, hi) holds dims 32*hi .. +31 of the
// unnormalised output; m, l complete) to workspace slot `slot`.
__device__ __forceinline__ void store_state(const DecodeArgs& a, int64_t slot, int lo, int hi,
                                            const q3::f32x4 (&acc)[8], float m, float l) {
  if (lo >= a.G) return;
  float* po = a.s_acc + (slot * a.G + lo) * kD + 32 * hi;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    q3::f32x4 v0 = {acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
    q3::f32x4 v1 = {acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
    *reinterpret_cast<q3::f32x4*>(po + 8 * r) = v0;
    *reinterpret_cast<q3::f32x4*>(po + 8 * r + 4) = v1;
  }
  if (hi == 0) a.s_ml[slot * a.G + lo] = float2{m, l};
}

// ---------------------------------------------------------------------------
// Stream path: persistent waves over the flat tile list.
//
// Every wave owns the partitions whose first tile falls in its range of pw
// tiles and visits the sequence-head segments of its range from the last to
// the first.  A sequence-head split across waves is handed on through the
// workspace: the wave holding its first partitions (the segment that ends
// its range, so visited first) writes the fold of its partitions early;
// a wave holding a middle part writes each partition's state; the wave
// holding the last partitions (the segment that starts its range, visited
// last) usually finds every other part already written and folds them and
// its own partitions straight into the output.  Otherwise each part takes
// a ticket after writing its states, and the part taking the last ticket
// merges.  Nothing ever waits for another wave.

// Load-side cursor of a wave: the segment being fetched (tiles [t_lo, t_hi)
// of sequence-head (b, hkv), whose first tile is flat tile S) and its next tile.
struct Cursor {
  int64_t S;
  int b, hkv, t, t_lo, t_hi;
  int n;  // tiles of sequence b
  int L;  // context length of sequence b
  bool done;
};

// Hand-off through the workspace: slots are written and read with
// device-scope accesses (sc1: through to, and from, the point where all
// XCDs' L2s agree), so no L2 write-back or invalidation is needed.  A part's
// stores complete (vmcnt(0)) before it takes its ticket, and a wave reads
// other parts' slots only after their tickets are in.
constexpr int kCpolDevice = 16;  // sc1
constexpr uint32_t kMergeLater = 0x80000000u;  // ticket mark: left for the merge kernel
// Longest hand-off folded inside the stream kernel (slots read by one wave);
// longer ones go to the merge kernel, which runs only when a table row can
// hold more partitions than this.
constexpr int kInlineSlots = 32;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t acc_rsrc(const DecodeArgs& a, int64_t slot) {
  return __builtin_amdgcn_make_buffer_rsrc(a.s_acc + slot * a.G * kD, 0, a.G * kD * 4, 0x00020000);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ml_rsrc(const DecodeArgs& a, int64_t slot) {
  return __builtin_amdgcn_make_buffer_rsrc(a.s_ml + slot * a.G, 0, a.G * 8, 0x00020000);
}

// How a sequence-head of n tiles whose first tile is flat tile S is shared
// when wave w owns the partitions starting in [w * pw, (w + 1) * pw): N waves
// take part and the first owns partitions [0, j1) of k.
struct Split {
  int k, N, j1;
};

__device__ __forceinline__ Split split_of(int64_t S, int n, int64_t pw) {
  Split s;
  const int P = part_tiles(n);
  s.k = (n + P - 1) / P;
  const int64_t w0 = S / pw;
  if (P > pw) {  // every partition starts in another wave's range
    s.N = s.k;
    s.j1 = 1;
    return s;
  }
  s.N = static_cast<int>((S + static_cast<int64_t>(s.k - 1) * P) / pw - w0 + 1);
  const int64_t x = (w0 + 1) * pw - S;
  s.j1 = x >= n ? s.k : static_cast<int>((x + P - 1) / P);
  return s;
}

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void paged_decode_inv_stream_kernel(DecodeArgs a) {
  __shared__ int32_t s_pref[kStreamMaxB + 1];
  __shared__ int32_t s_row[kStreamMaxB];
  __shared__ int32_t s_len[kStreamMaxB];
  __shared__ int32_t s_wsum[kWaves];
  // Each wave's running fold in slot order (query head g, dim d at g * kD + d)
  // and its (m, l) per query head.
  __shared__ q3::f32x4 s_f[kWaves][kMaxG * kD / 4];
  __shared__ float2 s_fml[kWaves][kMaxG];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lo = lane & 15;
  const int hi = lane >> 4;
  const int B = a.B;
  const int G = a.G;
  // Wave-uniform reads of the LDS tables (scalar registers and branches).
  auto pref = [&](int b) { return __builtin_amdgcn_readfirstlane(s_pref[b]); };

  // ---- prologue: rows, lengths and the exclusive tile prefix of every sequence ----
  constexpr int kPer = kStreamMaxB / (kWaves * 64);
  int cnt[kPer];
  int local = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = tid * kPer + i;
    int n = 0;
    if (b < B) {
      const int64_t row = row_of(a, b);
      const int64_t L = row >= 0 ? clamp_len(a, a.seq_lens[row]) : 0;
      s_row[b] = static_cast<int32_t>(row);
      s_len[b] = static_cast<int32_t>(L);
      n = static_cast<int>(q3::cdiv(L, kTile));
    }
    cnt[i] = n;
    local += n;
  }
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  int run = incl - local;
  int total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) run += s_wsum[w];
    total += s_wsum[w];
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = tid * kPer + i;
    if (b < B) s_pref[b] = run;
    run += cnt[i];
  }
  if (tid == 0) s_pref[B] = total;
  __syncthreads();

  // empty contexts: zero rows, spread over the workgroups
  for (int b = blockIdx.x; b < B; b += gridDim.x) {
    if (s_len[b] != 0) continue;
    for (int e = tid; e < a.Hq * (kD / 8); e += kWaves * 64)
      q3::st16(a.out + b * a.o_sb + static_cast<int64_t>(e / (kD / 8)) * a.o_sh + 8 * (e % (kD / 8)),
               q3::u32x4{0u, 0u, 0u, 0u});
  }

  const int64_t T = static_cast<int64_t>(a.Hkv) * total;
  const int64_t W = static_cast<int64_t>(gridDim.x) * kWaves;
  int64_t pw = q3::cdiv(T, W);
  pw = pw < kMinTilesPerWave ? kMinTilesPerWave : pw;
  if (blockIdx.x == 0) {
    for (int b = tid; b <= B; b += kWaves * 64) a.s_pref[b] = s_pref[b];
    if (tid == 0) a.s_pw[0] = pw;
  }
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (w * pw >= T) return;

  // Sequence holding flat tile g < T: the largest b with Hkv * pref[b] <= g
  // (never an empty one: an empty b shares its prefix with b + 1).
  auto seq_at = [&](int64_t g) -> int {
    int lo_b = 0, hi_b = B - 1;
    while (lo_b < hi_b) {
      const int mid = (lo_b + hi_b + 1) >> 1;
      if (static_cast<int64_t>(a.Hkv) * pref(mid) <= g) lo_b = mid; else hi_b = mid - 1;
    }
    return lo_b;
  };
  // First partition start at or after flat tile g (T if none).
  auto part_align = [&](int64_t g) -> int64_t {
    if (g >= T) return T;
    const int b = seq_at(g);
    const int n = pref(b + 1) - pref(b);
    const int64_t off = g - static_cast<int64_t>(a.Hkv) * pref(b);
    const int64_t start = g - off % n;  // first tile of the sequence-head
    const int P = part_tiles(n);
    const int64_t j = q3::cdiv(off % n, P);
    return j * P >= n ? start + n : start + j * P;
  };
  // The wave owns the partitions whose first tile lies in [w*pw, (w+1)*pw).
  const int64_t g0 = part_align(w * pw);
  const int64_t g1 = part_align((w + 1) * pw < T ? (w + 1) * pw : T);
  if (g0 >= g1) return;

  // The segment of the range that holds flat tile g (g0 <= g < g1).
  Cursor cur;
  auto seg_at = [&](int64_t g) __attribute__((always_inline)) {
    const int b = seq_at(g);
    cur.b = b;
    cur.n = pref(b + 1) - pref(b);
    cur.L = __builtin_amdgcn_readfirstlane(s_len[b]);
    const int64_t base = static_cast<int64_t>(a.Hkv) * pref(b);
    cur.hkv = static_cast<int>((g - base) / cur.n);
    cur.S = base + static_cast<int64_t>(cur.hkv) * cur.n;
    cur.t_lo = static_cast<int>((g0 > cur.S ? g0 : cur.S) - cur.S);
    cur.t_hi = static_cast<int>((g1 < cur.S + cur.n ? g1 : cur.S + cur.n) - cur.S);
    cur.t = cur.t_lo;
  };
  seg_at(g1 - 1);
  cur.done = false;
  TableWindow tw;
  window_load(tw, a, __builtin_amdgcn_readfirstlane(s_row[cur.b]), (cur.t * kTile) / a.bs, lane);

  // Issues the next batch of at most kChunk tiles: the rest of the current
  // segment, then the segment before it.
  auto issue = [&](Chunk& c) {
    c.n = 0;
    if (cur.done) return;
    if (cur.t >= cur.t_hi) {
      if (cur.S <= g0) {
        cur.done = true;
        return;
      }
      seg_at(cur.S - 1);
      tw.row = __builtin_amdgcn_readfirstlane(s_row[cur.b]);
      window_load(tw, a, tw.row, (cur.t * kTile) / a.bs, lane);
    }
    int n = cur.t_hi - cur.t;
    n = n < kChunk ? n : kChunk;
    c.n = n;
    c.t0 = cur.t;
    c.seg = cur.b * a.Hkv + cur.hkv;
    c.ntiles = cur.n;
    c.L = cur.L;
    const uint16_t* kbase = a.k + static_cast<int64_t>(cur.hkv) * a.k_sh;
    const uint16_t* vbase = a.v + static_cast<int64_t>(cur.hkv) * a.v_sh;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      int64_t phys = -1;
      int sub = 0;
      if (i < n) {
        const int tok0 = (cur.t + i) * kTile;
        phys = window_phys(tw, a, tok0 / a.bs, lane);
        sub = tok0 % a.bs;
      }
      load_tile(c, i, a, kbase, vbase, phys, sub, lo, hi);
    }
    cur.t += n;
  };

  // ---- compute side ----
  int cseg = -1, cb = 0, chkv = 0, cn = 0, pstart = 0, ct_hi = 0, seg_hi = 0;
  int cP = kPartTiles;  // partition tiles of the sequence-head
  bool own = false;       // the segment starts at the sequence-head's first tile
  bool complete = false;  // the segment ends at its last tile
  bool emit = false;      // each partition state goes to its slot
  bool have_f = false;    // s_f holds the fold of the partitions so far
  Split sp{1, 1, 1};
  int nmerge = 0, mseg0 = 0, mseg1 = 0;  // sequence-heads this wave merges last
  q3::bf16x8 qv[4];
  SoftmaxState st;
  reset(st);

  // The partition state in registers becomes the fold in s_f.
  auto state_to_lds = [&]() __attribute__((always_inline)) {
    if (lo < G) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = lo * kD + 32 * hi + 8 * r;
        s_f[wave][f / 4] = q3::f32x4{st.acc[0][r], st.acc[1][r], st.acc[2][r], st.acc[3][r]};
        s_f[wave][f / 4 + 1] = q3::f32x4{st.acc[4][r], st.acc[5][r], st.acc[6][r], st.acc[7][r]};
      }
      if (hi == 0) s_fml[wave][lo] = float2{st.m, st.l};
    }
  };
  // The partition state in registers is folded into s_f.
  auto fold_state = [&]() __attribute__((always_inline)) {
    if (lo < G) {
      const float2 ml = s_fml[wave][lo];
      const FoldW fw = fold_weights(ml.x, st.m);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = lo * kD + 32 * hi + 8 * r;
        q3::f32x4 x = s_f[wave][f / 4];
        x[0] = fold_val(x[0], fw.a, st.acc[0][r], fw.b);
        x[1] = fold_val(x[1], fw.a, st.acc[1][r], fw.b);
        x[2] = fold_val(x[2], fw.a, st.acc[2][r], fw.b);
        x[3] = fold_val(x[3], fw.a, st.acc[3][r], fw.b);
        s_f[wave][f / 4] = x;
        q3::f32x4 y = s_f[wave][f / 4 + 1];
        y[0] = fold_val(y[0], fw.a, st.acc[4][r], fw.b);
        y[1] = fold_val(y[1], fw.a, st.acc[5][r], fw.b);
        y[2] = fold_val(y[2], fw.a, st.acc[6][r], fw.b);
        y[3] = fold_val(y[3], fw.a, st.acc[7][r], fw.b);
        s_f[wave][f / 4 + 1] = y;
      }
      if (hi == 0) s_fml[wave][lo] = float2{fw.m, fold_val(ml.y, fw.a, st.l, fw.b)};
    }
  };
  // s_f -> workspace slot (lane t: floats 4t .. 4t+3 of each 256-float block).
  auto lds_to_slot = [&](int64_t slot) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rs = acc_rsrc(a, slot);
    for (int f0 = 4 * lane; f0 < G * kD; f0 += 256)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(q3::u32x4, s_f[wave][f0 / 4]), rs,
                                             f0 * 4, 0, kCpolDevice);
    if (lane < G) {
      const float2 ml = s_fml[wave][lane];
      const __amdgpu_buffer_rsrc_t rm = ml_rsrc(a, slot);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ml.x), rm, lane * 8, 0, kCpolDevice);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ml.y), rm, lane * 8 + 4, 0,
                                            kCpolDevice);
    }
  };
  // Folds slots j0 .. j1-1 of sequence-head seg into s_f in ascending order
  // (a fresh fold from slot j0 when `init`).  Loads run kAhead slots ahead.
  auto slots_to_lds = [&](int seg, int j0, int j1, bool init) __attribute__((always_inline)) {
    constexpr int kAhead = 4;
    const int64_t s0 = static_cast<int64_t>(seg) * a.max_parts;
    for (int f0 = 4 * lane; f0 < G * kD; f0 += 256) {
      const int g = f0 >> 7;
      q3::f32x4 x = s_f[wave][f0 / 4];
      float2 ml = s_fml[wave][g];
      for (int jb = j0; jb < j1; jb += kAhead) {
        q3::f32x4 p[kAhead];
        float pm[kAhead], pl[kAhead];
#pragma unroll
        for (int i = 0; i < kAhead; ++i) {
          const int j = jb + i < j1 ? jb + i : j1 - 1;
          p[i] = __builtin_bit_cast(q3::f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   acc_rsrc(a, s0 + j), f0 * 4, 0, kCpolDevice));
          pm[i] = __uint_as_float(
              __builtin_amdgcn_raw_buffer_load_b32(ml_rsrc(a, s0 + j), g * 8, 0, kCpolDevice));
          pl[i] = __uint_as_float(
              __builtin_amdgcn_raw_buffer_load_b32(ml_rsrc(a, s0 + j), g * 8 + 4, 0, kCpolDevice));
        }
#pragma unroll
        for (int i = 0; i < kAhead; ++i) {
          if (jb + i >= j1) break;
          if (init && jb + i == j0) {
            x = p[i];
            ml = float2{pm[i], pl[i]};
            continue;
          }
          const FoldW fw = fold_weights(ml.x, pm[i]);
          x[0] = fold_val(x[0], fw.a, p[i][0], fw.b);
          x[1] = fold_val(x[1], fw.a, p[i][1], fw.b);
          x[2] = fold_val(x[2], fw.a, p[i][2], fw.b);
          x[3] = fold_val(x[3], fw.a, p[i][3], fw.b);
          ml = float2{fw.m, fold_val(ml.y, fw.a, pl[i], fw.b)};
        }
      }
      s_f[wave][f0 / 4] = x;
      if ((f0 & (kD - 1)) == 0) s_fml[wave][g] = ml;
    }
  };
  // s_f, normalised -> the output rows of sequence-head seg.
  auto lds_to_out = [&](int seg) __attribute__((always_inline)) {
    const int b = seg / a.Hkv, hkv = seg % a.Hkv;
    for (int f0 = 4 * lane; f0 < G * kD; f0 += 256) {
      const int g = f0 >> 7, d = f0 & (kD - 1);
      const q3::f32x4 x = s_f[wave][f0 / 4];
      const float l = s_fml[wave][g].y;
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const q3::u32x2 v = {q3::pack_bf16x2(x[0] * inv, x[1] * inv),
                           q3::pack_bf16x2(x[2] * inv, x[3] * inv)};
      *reinterpret_cast<q3::u32x2*>(a.out + b * a.o_sb +
                                    (static_cast<int64_t>(hkv) * G + g) * a.o_sh + d) = v;
    }
  };
  auto ticket_of = [&](int seg) { return a.tickets + seg; };

  // At a partition's end: the state goes to its slot or into the fold; at
  // the segment's end the output is written or the part is handed on.
  // Runs after the batch's math, while its registers are free.
  auto end_batch = [&]() __attribute__((always_inline)) {
    if (ct_hi != seg_hi && ct_hi % cP != 0) return;
    st.l = q3::sum_xor32(q3::sum_xor16(st.l));
    const bool last = ct_hi == seg_hi;
    if (emit) {
      state_to_lds();
      lds_to_slot(static_cast<int64_t>(cseg) * a.max_parts + pstart / cP);
    } else if (!have_f) {
      if (last && complete) {  // a whole sequence-head of one partition
        const float inv = st.l > 0.f ? 1.f / st.l : 0.f;
        if (lo < G) store_out_bf16(a, cb, chkv * G + lo, st.acc, inv, hi);
      } else {
        state_to_lds();
        have_f = true;
      }
    } else {
      fold_state();
    }
    if (last) {
      if (complete && !emit) {
        if (have_f) lds_to_out(cseg);
        if (!own && lane == 0)  // caught up with the others' parts: the ticket is done
          __hip_atomic_store(ticket_of(cseg), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (!emit)  // the first part: its fold, in the slot of its last partition
          lds_to_slot(static_cast<int64_t>(cseg) * a.max_parts + sp.j1 - 1);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the slot stores are done
        uint32_t old = 0;
        if (lane == 0)
          old = __hip_atomic_fetch_add(ticket_of(cseg), 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old == static_cast<uint32_t>(sp.N - 1)) {  // the last part in merges
          if (nmerge == 0) mseg0 = cseg; else mseg1 = cseg;
          ++nmerge;
        }
      }
      cseg = -1;
    }
    pstart = ct_hi;
    reset(st);
  };

  // A segment's first batch starts at its first tile; the segment ends at
  // the sequence-head's end or, for the range's last segment, at g1.
  auto begin_segment = [&](const Chunk& c) __attribute__((always_inline)) {
    cseg = c.seg;
    cb = c.seg / a.Hkv;
    chkv = c.seg % a.Hkv;
    cn = c.ntiles;
    cP = part_tiles(cn);
    const int64_t cS = static_cast<int64_t>(a.Hkv) * pref(cb) + static_cast<int64_t>(chkv) * cn;
    seg_hi = g1 - cS < cn ? static_cast<int>(g1 - cS) : cn;
    own = c.t0 == 0;
    complete = seg_hi == cn;
    have_f = false;
    emit = false;
    pstart = c.t0;
    if (!(own && complete)) sp = split_of(cS, cn, pw);
    if (!own) {
      emit = true;
      const int ja = c.t0 / cP;  // this part's first partition
      if (complete && ja - sp.j1 + 1 <= kInlineSlots) {
        // the last part: when every other part is in, fold them first
        uint32_t t = 0;
        if (lane == 0)
          t = __hip_atomic_load(ticket_of(cseg), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        t = __builtin_amdgcn_readfirstlane(t);
        if (t == static_cast<uint32_t>(sp.N - 1)) {
          slots_to_lds(cseg, sp.j1 - 1, ja, true);
          have_f = true;
          emit = false;
        }
      }
    }
    load_q(qv, a, cb, chkv, lo, hi);
    // Wait for the query here, on this rare path: the wait the compiler
    // would place at its first use otherwise stands on every batch's path.
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  };

  auto process = [&](Chunk& c) {
    if (c.seg != cseg) begin_segment(c);
    compute_chunk(c, a.scale_log2, hi, qv, st);
    ct_hi = c.t0 + c.n;
    end_batch();
  };

  Chunk ca, cbuf;
  issue(ca);
  issue(cbuf);
  while (true) {
    if (ca.n == 0) break;
    process(ca);
    issue(ca);
    if (cbuf.n == 0) break;
    process(cbuf);
    issue(cbuf);
  }

  // Merges left to this wave (it took the last ticket): the first part's
  // fold, then every later partition, in order.
  for (int m = 0; m < nmerge; ++m) {
    const int seg = m == 0 ? mseg0 : mseg1;
    const int b = seg / a.Hkv, hkv = seg % a.Hkv;
    const int n = pref(b + 1) - pref(b);
    const int64_t S = static_cast<int64_t>(a.Hkv) * pref(b) + static_cast<int64_t>(hkv) * n;
    const Split s = split_of(S, n, pw);
    if (s.k - s.j1 + 1 > kInlineSlots) {  // long: the merge kernel's
      if (lane == 0)
        __hip_atomic_store(ticket_of(seg), kMergeLater, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    slots_to_lds(seg, s.j1 - 1, s.k, true);
    lds_to_out(seg);
    if (lane == 0) __hip_atomic_store(ticket_of(seg), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Grid path (batches above kStreamMaxB): one wave per partition, four
// partitions of one sequence-head per workgroup.

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void paged_decode_inv_grid_kernel(DecodeArgs a) {
  const int hkv = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lo = lane & 15;
  const int hi = lane >> 4;
  const int G = a.G;
  const int j = blockIdx.x * kWaves + wave;  // partition of this wave

  const int64_t row = row_of(a, b);
  const int L = static_cast<int>(row >= 0 ? clamp_len(a, a.seq_lens[row]) : 0);
  const int n_tiles = static_cast<int>(q3::cdiv(L, kTile));
  const int P = part_tiles(n_tiles);
  const int t0 = j * P;
  if (t0 >= n_tiles) {
    if (j == 0) {  // empty context: defined zero output
      for (int e = lane; e < G * kD; e += 64) {
        const int g = e / kD, d = e % kD;
        a.out[b * a.o_sb + (static_cast<int64_t>(hkv) * G + g) * a.o_sh + d] = 0;
      }
    }
    return;
  }
  const int t1 = min(n_tiles, t0 + P);
  // A partition spans at most kLongPartTiles * kTile / block_size <= kWin pages.
  const int base = (t0 * kTile) / a.bs;
  const int32_t pages = table_entry(a, row, base + lane);
  const uint16_t* kbase = a.k + static_cast<int64_t>(hkv) * a.k_sh;
  const uint16_t* vbase = a.v + static_cast<int64_t>(hkv) * a.v_sh;

  int t_next = t0;
  auto issue = [&](Chunk& c) {
    c.n = 0;
    if (t_next >= t1) return;
    const int n = min(kChunk, t1 - t_next);
    c.n = n;
    c.t0 = t_next;
    c.L = L;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      int64_t phys = -1;
      int sub = 0;
      if (i < n) {
        const int tok0 = (t_next + i) * kTile;
        phys = __builtin_amdgcn_readlane(pages, tok0 / a.bs - base);
        sub = tok0 % a.bs;
      }
      load_tile(c, i, a, kbase, vbase, phys, sub, lo, hi);
    }
    t_next += n;
  };

  Chunk ca, cbuf;
  issue(ca);
  issue(cbuf);
  q3::bf16x8 qv[4];
  load_q(qv, a, b, hkv, lo, hi);
  SoftmaxState st;
  reset(st);
  while (true) {
    if (ca.n == 0) break;
    compute_chunk(ca, a.scale_log2, hi, qv, st);
    issue(ca);
    if (cbuf.n == 0) break;
    compute_chunk(cbuf, a.scale_log2, hi, qv, st);
    issue(cbuf);
  }
  st.l = q3::sum_xor32(q3::sum_xor16(st.l));
  if (n_tiles <= P) {  // the only partition: the output itself
    const float inv = st.l > 0.f ? 1.f / st.l : 0.f;
    if (lo < G) store_out_bf16(a, b, hkv * G + lo, st.acc, inv, hi);
  } else {
    store_state(a, slot_of(a, b, hkv, j), lo, hi, st.acc, st.m, st.l);
  }
}

// ---------------------------------------------------------------------------
// Merge: the left fold of a sequence-head's partition states in ascending
// order, for the sequence-heads the attention pass left unfinished: on the
// grid path every one of more than one partition; on the stream path the
// long hand-offs marked kMergeLater (the first part's fold, then every later
// partition).  One workgroup per (KV head, batch entry) with one wave per
// query head of the group; every lane owns two output dims.  Loads run
// kBatch partitions ahead of the fold.
__global__ __launch_bounds__(kMaxG * 64) void paged_decode_inv_merge_kernel(DecodeArgs a) {
  constexpr int kBatch = 8;
  const int hkv = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;  // query head within the group (blockDim = 64 G)
  const int G = a.G;
  int n = 0, j1 = 1;
  bool todo;
  if (a.grid_mode) {
    const int64_t row = row_of(a, b);
    n = static_cast<int>(q3::cdiv(row >= 0 ? clamp_len(a, a.seq_lens[row]) : 0, kTile));
    todo = n > part_tiles(n);
  } else {
    todo = a.tickets[static_cast<int64_t>(b) * a.Hkv + hkv] == kMergeLater;
    if (todo) {
      const int64_t pref_b = a.s_pref[b];
      n = a.s_pref[b + 1] - static_cast<int32_t>(pref_b);
      const int64_t S = static_cast<int64_t>(a.Hkv) * pref_b + static_cast<int64_t>(hkv) * n;
      j1 = split_of(S, n, a.s_pw[0]).j1;
    }
  }
  if (todo) {
    const int k = static_cast<int>(q3::cdiv(n, part_tiles(n)));
    const int64_t hq = static_cast<int64_t>(hkv) * G + g;
    const int64_t s0 = slot_of(a, b, hkv, 0);
    auto acc_at = [&](int j) {
      return *reinterpret_cast<const float2*>(a.s_acc + ((s0 + j) * G + g) * kD + 2 * lane);
    };
    float2 ml = a.s_ml[(s0 + j1 - 1) * G + g];
    float2 o = acc_at(j1 - 1);
    float2 pm[2][kBatch], po[2][kBatch];
    auto fetch = [&](float2 (&m)[kBatch], float2 (&v)[kBatch], int j0) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int j = j0 + i < k ? j0 + i : k - 1;
        m[i] = a.s_ml[(s0 + j) * G + g];
        v[i] = acc_at(j);
      }
    };
    auto fold = [&](const float2 (&m)[kBatch], const float2 (&v)[kBatch], int j0) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (j0 + i < k) {
          const FoldW fw = fold_weights(ml.x, m[i].x);
          o.x = fold_val(o.x, fw.a, v[i].x, fw.b);
          o.y = fold_val(o.y, fw.a, v[i].y, fw.b);
          ml = float2{fw.m, fold_val(ml.y, fw.a, m[i].y, fw.b)};
        }
      }
    };
    if (j1 < k) {
      fetch(pm[0], po[0], j1);
      for (int j0 = j1; j0 < k; j0 += 2 * kBatch) {
        if (j0 + kBatch < k) fetch(pm[1], po[1], j0 + kBatch);
        fold(pm[0], po[0], j0);
        if (j0 + kBatch >= k) break;
        if (j0 + 2 * kBatch < k) fetch(pm[0], po[0], j0 + 2 * kBatch);
        fold(pm[1], po[1], j0 + kBatch);
      }
    }
    const float inv = ml.y > 0.f ? 1.f / ml.y : 0.f;
    *reinterpret_cast<uint32_t*>(a.out + b * a.o_sb + hq * a.o_sh + 2 * lane) =
        q3::pack_bf16x2(o.x * inv, o.y * inv);
  }
  if (!a.grid_mode) {
    __syncthreads();  // every wave has read the ticket
    if (todo && threadIdx.x == 0) a.tickets[static_cast<int64_t>(b) * a.Hkv + hkv] = 0u;
  }
}

// ---------------------------------------------------------------------------
// Host side.

// Partitions per sequence-head a table row of max_pages pages can hold.
int64_t max_parts_for(int64_t max_pages, int block_size) {
  return q3::cdiv(q3::cdiv(max_pages * block_size, kTile), kPartTiles);
}

struct Layout {
  int64_t acc, ml, pref, meta, tickets, total;
};

// Workspace layout: the stream path's tickets first (one per (b, hkv) for
// up to kStreamMaxB rows, so calls of any batch size that share a workspace
// find them at the same place: zero before the first call, and every call
// leaves them at zero), then the partition slots of every (b, hkv), the tile
// prefix and the tiles-per-wave word.  It depends on the launch shape only,
// never on the live lengths or the device.
Layout ws_layout(int B, int Hkv, int G, int64_t parts, int ticket_hkv) {
  const int64_t slots = static_cast<int64_t>(B) * Hkv * parts;
  Layout l;
  l.tickets = 0;
  l.acc = align256(static_cast<int64_t>(kStreamMaxB) * ticket_hkv * 4);
  l.ml = l.acc + align256(slots * G * kD * 4);
  l.pref = l.ml + align256(slots * G * 8);
  l.meta = l.pref + align256((static_cast<int64_t>(B) + 1) * 4);
  l.total = l.meta + 256;
  return l;
}

// The stream path's tile prefix is 32-bit: every sequence of the batch at
// the table's full length must fit it.
bool stream_fits(int B, int64_t max_pages, int block_size) {
  return B <= kStreamMaxB &&
         static_cast<int64_t>(B) * q3::cdiv(max_pages * block_size, kTile) <= 0x7fffffff;
}

// Launches the attention pass (stream or grid path) and the merge with the
// workspace at ws (ws_layout bytes, no initialisation needed).
int launch(DecodeArgs& a, char* ws, int ticket_hkv, hipStream_t s, const char* who) {
  const int64_t parts = max_parts_for(a.max_pages, a.bs);
  if (parts > 0x7fffffff / kWaves) return q3::fail(QWEN3_EINVAL, "%s: max_pages too large", who);
  a.max_parts = static_cast<int>(parts);
  const Layout L = ws_layout(a.B, a.Hkv, a.G, parts, ticket_hkv);
  a.s_acc = reinterpret_cast<float*>(ws + L.acc);
  a.s_ml = reinterpret_cast<float2*>(ws + L.ml);
  a.s_pref = reinterpret_cast<int32_t*>(ws + L.pref);
  a.s_pw = reinterpret_cast<int64_t*>(ws + L.meta);
  a.tickets = reinterpret_cast<uint32_t*>(ws + L.tickets);
  q3::clear_error();
  if (stream_fits(a.B, a.max_pages, a.bs)) {
    const int wgs = stream_workgroups();
    if (wgs <= 0) return q3::fail(QWEN3_EINVAL, "%s: cannot query the device's CU count", who);
    a.grid_mode = 0;
    hipLaunchKernelGGL(paged_decode_inv_stream_kernel, dim3(wgs), dim3(kWaves * 64), 0, s, a);
  } else {
    a.grid_mode = 1;
    hipLaunchKernelGGL(paged_decode_inv_grid_kernel,
                       dim3(static_cast<unsigned>(q3::cdiv(parts, kWaves)), a.Hkv, a.B),
                       dim3(kWaves * 64), 0, s, a);
  }
  int rc = q3::launch_status(who);
  // The merge runs when a sequence-head can need it: on the grid path when a
  // table row holds more than one partition, on the stream path when it can
  // hold a hand-off longer than the stream kernel folds itself.
  if (rc || parts <= (a.grid_mode ? 1 : kInlineSlots)) return rc;
  hipLaunchKernelGGL(paged_decode_inv_merge_kernel, dim3(a.Hkv, a.B), dim3(64 * a.G), 0, s, a);
  return q3::launch_status(who);
}

}  // namespace

extern "C" size_t qwen3_paged_decode_invariant_workspace_bytes(int B, int num_heads,
                                                               int num_kv_heads, int head_dim,
                                                               int64_t max_pages,
                                                               int block_size) {
  if (B <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > kMaxG || head_dim != kD || max_pages <= 0 ||
      block_size <= 0 || block_size % kTile != 0)
    return 0;
  // One slot per partition of every (b, hkv) at the table's full length:
  // the size depends on the launch shape only.
  const int64_t parts = max_parts_for(max_pages, block_size);
  if (static_cast<double>(B) * num_heads * parts * (kD + 2) * 4 > 0x1p60) return 0;
  return static_cast<size_t>(
      ws_layout(B, num_kv_heads, num_heads / num_kv_heads, parts, num_kv_heads).total);
}

extern "C" int qwen3_paged_decode_invariant_bf16(
    const void* q, const int64_t q_strides[2], const void* k_cache, const int64_t k_strides[3],
    const void* v_cache, const int64_t v_strides[3], int64_t num_blocks,
    const int32_t* block_table, int64_t bt_row_stride, int64_t max_rows, int64_t max_pages,
    const int32_t* seq_lens, int seq_len_bias, const int32_t* row_ids, void* out,
    const int64_t out_strides[2], int B, int num_heads, int num_kv_heads, int head_dim,
    int block_size, float scale, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "qwen3_paged_decode_invariant_bf16";
  DecodeArgs a;
  if (int rc = prepare(a, who, q, q_strides, k_cache, k_strides, v_cache, v_strides, num_blocks,
                       block_table, bt_row_stride, max_rows, max_pages, seq_lens,
                       seq_len_bias, row_ids, out, out_strides, B, num_heads, num_kv_heads,
                       head_dim, block_size, scale))
    return rc;
  if (B == 0) return QWEN3_OK;
  const size_t need = qwen3_paged_decode_invariant_workspace_bytes(
      B, num_heads, num_kv_heads, head_dim, max_pages, block_size);
  if (need == 0) return q3::fail(QWEN3_EINVAL, "%s: cannot size the workspace", who);
  if (!workspace || workspace_bytes < need)
    return q3::fail(QWEN3_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who,
                    need, workspace ? workspace_bytes : (size_t)0);
  if (!q3::aligned16(workspace))
    return q3::fail(QWEN3_EALIGN, "%s: workspace must be 16-byte aligned", who);
  return launch(a, static_cast<char*>(workspace), num_kv_heads, static_cast<hipStream_t>(stream),
                who);
}
