// Paged decode attention for gfx950 (GQA, one query token per sequence).
//
// Semantics follow paged_attn_decode_kernel
// (qwen3/kernels/paged_attention.py:27-129): for batch entry b and KV head
// hkv, the G = Hq/Hkv query heads hkv*G .. hkv*G+G-1 attend the first
// L = seq_lens[row] + bias tokens of the sequence, gathered page by page
// through block_table[row]; softmax in fp32, bf16 output.
//
// Design (MI355X-first, not a transcription of the Triton program):
//  * The work is the flat list of (sequence, KV head, 16-token tile) triples.
//    A persistent grid of two 256-thread workgroups per CU splits that list
//    into equal contiguous ranges, one per wave (stream-KV): every wave
//    streams the same number of tiles, so there is no tail imbalance and no
//    per-workgroup start-up cost beyond one prologue.  A sequence-head that
//    straddles two waves' ranges is finished by a small merge kernel
//    (log-sum-exp weights); at most two partials exist per wave.
//  * A tile of one KV head is 4 KiB of K plus 4 KiB of V, contiguous in the
//    pool.  Each lane issues 16-byte loads (4 for K, 4 for V); a wave keeps
//    two batches of kChunk tiles in flight while it computes the previous
//    batch (software pipeline), and prefetches the next 64 block-table
//    entries before it needs them.
//  * QK^T on the matrix cores: S^T(16 tok x 16 q) = K(16x128) Q^T(128x16)
//    as 4 x mfma_f32_16x16x32_bf16.  The G query heads fill G of the 16
//    columns (zero-padded Q); padding costs idle MFMA slots, not registers.
//  * The S^T accumulator layout (lane = q column + 16*(token/4)) is exactly
//    the B-operand layout of the PV product, so P goes to the matrix cores
//    with no cross-lane traffic: O^T(128 x 16) = V^T(128 x 16 tok) P^T as
//    8 x 2 mfma_f32_16x16x16_bf16 (P split into bf16 hi + lo terms), where
//    the V^T operand is built in-lane from the row-major 16-byte V loads
//    with byte permutes.
//  * Online softmax in the exp2 domain, one running max per query column,
//    updated once per batch of tiles.
//  * Batches above kStreamMaxB use a non-persistent grid variant (one
//    workgroup per partition of tiles) with the same tile math.
#include <mutex>

#include "paged_decode_tile.hpp"

namespace {

// Grid path (large batches).
constexpr int kGridTilesPerWave = 32;
constexpr int kGridTilesPerPart = kGridTilesPerWave * kWaves;
constexpr int kOStride = kD + 4;  // padded LDS row of a wave's partition output

// Completes the per-column denominator (lanes of one column hold disjoint
// token subsets) and returns 1/l (0 for an empty column).
__device__ __forceinline__ float finish_l(SoftmaxState& st) {
  st.l = q3::sum_xor32(q3::sum_xor16(st.l));
  return st.l > 0.f ? 1.f / st.l : 0.f;
}

// ---------------------------------------------------------------------------
// Stream path: persistent waves over the flat tile list.

// Load-side cursor of a wave: the next tile to fetch in the flat list.
struct Cursor {
  int64_t g, g1;   // global tile index of the next tile, end of the wave's range
  int b, hkv, t;   // its (sequence, KV head, tile)
  int n;           // tiles of sequence b
  int L;           // context length of sequence b
};

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void paged_decode_stream_kernel(DecodeArgs a) {
  __shared__ int32_t s_pref[kStreamMaxB + 1];
  __shared__ int32_t s_row[kStreamMaxB];
  __shared__ int32_t s_len[kStreamMaxB];
  __shared__ int32_t s_wsum[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lo = lane & 15;
  const int hi = lane >> 4;
  const int B = a.B;

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

  const int64_t T = static_cast<int64_t>(a.Hkv) * total;
  const int64_t W = static_cast<int64_t>(gridDim.x) * kWaves;
  int64_t pw = q3::cdiv(T, W);
  pw = pw < kMinTilesPerWave ? kMinTilesPerWave : pw;
  if (blockIdx.x == 0) {
    for (int b = tid; b <= B; b += kWaves * 64) a.s_pref[b] = s_pref[b];
    if (tid == 0) a.s_meta[0] = static_cast<int32_t>(pw);
  }
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  const int64_t g0 = w * pw;
  if (g0 >= T) return;

  // ---- locate the wave's first tile: largest b with Hkv * pref[b] <= g0 ----
  Cursor cur;
  {
    int lo_b = 0, hi_b = B - 1;
    while (lo_b < hi_b) {
      const int mid = (lo_b + hi_b + 1) >> 1;
      if (static_cast<int64_t>(a.Hkv) * s_pref[mid] <= g0) lo_b = mid; else hi_b = mid - 1;
    }
    cur.b = lo_b;
    cur.n = s_pref[lo_b + 1] - s_pref[lo_b];
    cur.L = s_len[lo_b];
    const int64_t off = g0 - static_cast<int64_t>(a.Hkv) * s_pref[lo_b];
    cur.hkv = static_cast<int>(off / cur.n);
    cur.t = static_cast<int>(off % cur.n);
    cur.g = g0;
    cur.g1 = g0 + pw < T ? g0 + pw : T;
  }
  TableWindow tw;
  window_load(tw, a, s_row[cur.b], (cur.t * kTile) / a.bs, lane);

  // Issues the next batch of at most kChunk tiles of the current sequence-head.
  auto issue = [&](Chunk& c) {
    c.n = 0;
    if (cur.g >= cur.g1) return;
    if (cur.t >= cur.n) {  // next sequence-head
      if (++cur.hkv == a.Hkv) {
        cur.hkv = 0;
        do {
          ++cur.b;
        } while (s_pref[cur.b + 1] == s_pref[cur.b]);
        cur.n = s_pref[cur.b + 1] - s_pref[cur.b];
        cur.L = s_len[cur.b];
      }
      cur.t = 0;
      tw.row = s_row[cur.b];
      window_load(tw, a, tw.row, 0, lane);
    }
    int64_t left = cur.g1 - cur.g;
    int n = cur.n - cur.t;
    n = n < kChunk ? n : kChunk;
    n = left < n ? static_cast<int>(left) : n;
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
    cur.g += n;
  };

  // Compute-side state: the sequence-head being accumulated.
  int cseg = -1, cb = 0, chkv = 0, ct_lo = 0, ct_hi = 0, cn = 0;
  bool cfirst = true;
  q3::bf16x8 qv[4];
  SoftmaxState st;
  reset(st);

  auto finalize = [&]() {
    const float inv = finish_l(st);
    const bool complete = ct_lo == 0 && ct_hi == cn;
    if (lo < a.G) {
      const int hq = chkv * a.G + lo;
      if (complete) {
        store_out_bf16(a, cb, hq, st.acc, inv, hi);
      } else {
        const int64_t slot = (w * 2 + (cfirst ? 0 : 1)) * a.G + lo;
        float* po = a.s_po + slot * kD + 32 * hi;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          q3::f32x4 v0 = {st.acc[0][r] * inv, st.acc[1][r] * inv, st.acc[2][r] * inv,
                          st.acc[3][r] * inv};
          q3::f32x4 v1 = {st.acc[4][r] * inv, st.acc[5][r] * inv, st.acc[6][r] * inv,
                          st.acc[7][r] * inv};
          *reinterpret_cast<q3::f32x4*>(po + 8 * r) = v0;
          *reinterpret_cast<q3::f32x4*>(po + 8 * r + 4) = v1;
        }
        if (hi == 0) a.s_plse[slot] = st.l > 0.f ? st.m + __builtin_log2f(st.l) : q3::kNegInf;
      }
    }
  };

  auto process = [&](Chunk& c) {
    if (c.seg != cseg) {
      if (cseg >= 0) {
        finalize();
        cfirst = false;
      }
      cseg = c.seg;
      cb = c.seg / a.Hkv;
      chkv = c.seg % a.Hkv;
      ct_lo = c.t0;
      cn = c.ntiles;
      load_q(qv, a, cb, chkv, lo, hi);
      reset(st);
    }
    compute_chunk(c, a.scale_log2, hi, qv, st);
    ct_hi = c.t0 + c.n;
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
  if (cseg >= 0) finalize();
}

// Combines the partials of every sequence-head split across waves and
// writes zeros for empty contexts.  One workgroup per (kv head, batch entry)
// with one wave per query head of the group: lanes first fetch the LSEs of up
// to 64 covering waves at once, then every lane owns two output dims and sums
// the weighted partials kBatch waves at a time.
__global__ __launch_bounds__(kMaxG * 64) void paged_decode_stream_merge_kernel(DecodeArgs a) {
  constexpr int kBatch = 8;
  const int hkv = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;  // query head within the group
  const int G = a.G;
  if (g >= G) return;
  const int64_t pref_b = a.s_pref[b];
  const int n = a.s_pref[b + 1] - static_cast<int32_t>(pref_b);
  const int64_t hq = static_cast<int64_t>(hkv) * G + g;
  uint32_t* op = reinterpret_cast<uint32_t*>(a.out + b * a.o_sb + hq * a.o_sh + 2 * lane);
  if (n == 0) {
    *op = 0u;
    return;
  }
  const int64_t pw = a.s_meta[0];
  const int64_t S = static_cast<int64_t>(a.Hkv) * pref_b + static_cast<int64_t>(hkv) * n;
  const int64_t E = S + n;
  const int64_t wf = S / pw, wl = (E - 1) / pw;
  if (wf == wl) return;  // written whole by its wave
  const int nw = static_cast<int>(wl - wf + 1);
  auto slot_of = [&](int i) -> int64_t {
    const int64_t wv = wf + i;
    const int half = (i == 0 && wv * pw != S) ? 1 : 0;
    return (wv * 2 + half) * G + g;
  };
  // Pass 1: global max of the partial LSEs.
  float M = q3::kNegInf;
  for (int i0 = 0; i0 < nw; i0 += 64)
    if (i0 + lane < nw) M = fmaxf(M, a.s_plse[slot_of(i0 + lane)]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, q3::shfl_xor(M, o));
  const float M_use = M == q3::kNegInf ? 0.f : M;
  // Pass 2: weighted sum of the partial outputs (lane owns dims 2*lane, 2*lane+1).
  float sw = 0.f, o0 = 0.f, o1 = 0.f;
  for (int i0 = 0; i0 < nw; i0 += 64) {
    const float wl_lane = (i0 + lane < nw) ? q3::fast_exp2(a.s_plse[slot_of(i0 + lane)] - M_use) : 0.f;
    float wsum = wl_lane;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) wsum += q3::shfl_xor(wsum, o);
    sw += wsum;
    const int cnt = nw - i0 < 64 ? nw - i0 : 64;
    for (int j0 = 0; j0 < cnt; j0 += kBatch) {
      float2 ov[kBatch];
      float wt[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const bool ok = j0 + j < cnt;
        wt[j] = __shfl(wl_lane, ok ? j0 + j : 0, 64);
        ov[j] = ok ? *reinterpret_cast<const float2*>(a.s_po + slot_of(i0 + j0 + j) * kD + 2 * lane)
                   : float2{0.f, 0.f};
        wt[j] = ok ? wt[j] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        o0 += wt[j] * ov[j].x;
        o1 += wt[j] * ov[j].y;
      }
    }
  }
  const float inv = sw > 0.f ? 1.f / sw : 0.f;
  *op = q3::pack_bf16x2(o0 * inv, o1 * inv);
}

// ---------------------------------------------------------------------------
// Grid path (batches above kStreamMaxB): one workgroup per partition of
// kGridTilesPerPart tiles of one sequence-head; waves combine through LDS.

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void paged_decode_grid_kernel(DecodeArgs a) {
  const int part = blockIdx.x;
  const int hkv = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lo = lane & 15;
  const int hi = lane >> 4;
  const int G = a.G;

  const int64_t row = row_of(a, b);
  const int tile0 = part * kGridTilesPerPart;
  const int w0 = tile0 + wave * kGridTilesPerWave;
  int32_t seq_len = 0;
  TableWindow tw;
  tw.row = row;
  tw.base = (w0 * kTile) / a.bs;
  tw.cur = -1;
  tw.next = -1;
  if (row >= 0) {
    seq_len = a.seq_lens[row];
    tw.cur = table_entry(a, row, tw.base + lane);
  }
  const int L = static_cast<int>(row >= 0 ? clamp_len(a, seq_len) : 0);
  const int n_tiles = static_cast<int>(q3::cdiv(L, kTile));
  if (tile0 >= n_tiles) {
    if (part == 0) {  // empty context: defined zero output
      for (int e = tid; e < G * kD; e += kWaves * 64) {
        const int g = e / kD, d = e % kD;
        a.out[b * a.o_sb + (static_cast<int64_t>(hkv) * G + g) * a.o_sh + d] = 0;
      }
    }
    return;
  }
  const int n_parts = static_cast<int>(q3::cdiv(n_tiles, kGridTilesPerPart));
  const int w1 = min(min(n_tiles, tile0 + kGridTilesPerPart), w0 + kGridTilesPerWave);
  const uint16_t* kbase = a.k + static_cast<int64_t>(hkv) * a.k_sh;
  const uint16_t* vbase = a.v + static_cast<int64_t>(hkv) * a.v_sh;

  int t_next = w0;
  auto issue = [&](Chunk& c) {
    c.n = 0;
    if (t_next >= w1) return;
    const int n = min(kChunk, w1 - t_next);
    c.n = n;
    c.t0 = t_next;
    c.L = L;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      int64_t phys = -1;
      int sub = 0;
      if (i < n) {
        const int tok0 = (t_next + i) * kTile;
        // kGridTilesPerWave tiles span at most kWin pages (block_size >= 16).
        phys = __builtin_amdgcn_readlane(tw.cur, tok0 / a.bs - tw.base);
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

  __shared__ float s_m[kWaves][kMaxG];
  __shared__ float s_l[kWaves][kMaxG];
  extern __shared__ float s_acc[];  // [kWaves][G][kOStride] per-wave partition outputs
  // Each wave stores its unnormalised output in its own slice; the writer
  // threads merge the slices in fixed wave order (bit-reproducible).
  if (hi == 0) {
    s_m[wave][lo] = st.m;
    s_l[wave][lo] = st.l;
  }
  if (lo < G) {
    float* dst = s_acc + (wave * G + lo) * kOStride + 32 * hi;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      q3::f32x4 v0 = {st.acc[0][r], st.acc[1][r], st.acc[2][r], st.acc[3][r]};
      q3::f32x4 v1 = {st.acc[4][r], st.acc[5][r], st.acc[6][r], st.acc[7][r]};
      *reinterpret_cast<q3::f32x4*>(dst + 8 * r) = v0;
      *reinterpret_cast<q3::f32x4*>(dst + 8 * r + 4) = v1;
    }
  }
  __syncthreads();
  for (int e = tid; e < G * (kD / 2); e += kWaves * 64) {
    const int g = e / (kD / 2);
    const int d = 2 * (e % (kD / 2));
    float Mg = q3::kNegInf;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) Mg = fmaxf(Mg, s_m[wv][g]);
    const float Mg_use = Mg == q3::kNegInf ? 0.f : Mg;
    float Lg = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) {
      const float wg = q3::fast_exp2(s_m[wv][g] - Mg_use);
      const float* src = s_acc + (wv * G + g) * kOStride + d;
      Lg += s_l[wv][g] * wg;
      o0 += src[0] * wg;
      o1 += src[1] * wg;
    }
    const float inv = Lg > 0.f ? 1.f / Lg : 0.f;
    o0 *= inv;
    o1 *= inv;
    const int64_t hq = static_cast<int64_t>(hkv) * G + g;
    if (n_parts == 1) {
      *reinterpret_cast<uint32_t*>(a.out + b * a.o_sb + hq * a.o_sh + d) = q3::pack_bf16x2(o0, o1);
    } else {
      const int64_t slot = (static_cast<int64_t>(b) * a.Hq + hq) * a.max_parts + part;
      float2 o2 = {o0, o1};
      *reinterpret_cast<float2*>(a.ws_o + slot * kD + d) = o2;
      if (d == 0) a.ws_lse[slot] = Lg > 0.f ? Mg + __builtin_log2f(Lg) : q3::kNegInf;
    }
  }
}

// Merges the partitions of every (b, query head) of the grid path whose
// context needed more than one.  Loads are batched kBatch partitions at a time.
__global__ __launch_bounds__(kD) void paged_decode_grid_merge_kernel(DecodeArgs a) {
  constexpr int kBatch = 8;
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int64_t row = row_of(a, b);
  if (row < 0) return;
  const int64_t L = clamp_len(a, a.seq_lens[row]);
  const int n_tiles = static_cast<int>(q3::cdiv(L, kTile));
  const int n_parts = static_cast<int>(q3::cdiv(n_tiles, kGridTilesPerPart));
  if (n_parts <= 1) return;
  const int64_t base = (static_cast<int64_t>(b) * a.Hq + hq) * a.max_parts;
  const float* lse = a.ws_lse + base;
  float M = q3::kNegInf;
  for (int p0 = 0; p0 < n_parts; p0 += kBatch) {
    float v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) v[i] = p0 + i < n_parts ? lse[p0 + i] : q3::kNegInf;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) M = fmaxf(M, v[i]);
  }
  const float M_use = M == q3::kNegInf ? 0.f : M;
  float sw = 0.f, o = 0.f;
  for (int p0 = 0; p0 < n_parts; p0 += kBatch) {
    float wv[kBatch], ov[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const bool ok = p0 + i < n_parts;
      wv[i] = ok ? lse[p0 + i] : q3::kNegInf;
      ov[i] = ok ? a.ws_o[(base + p0 + i) * kD + d] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const float wi = q3::fast_exp2(wv[i] - M_use);
      sw += wi;
      o += wi * ov[i];
    }
  }
  o = sw > 0.f ? o / sw : 0.f;
  a.out[b * a.o_sb + static_cast<int64_t>(hq) * a.o_sh + d] = q3::bf16_bits(o);
}

// ---------------------------------------------------------------------------
// Host side.

struct StreamLayout {
  int64_t po, plse, pref, meta, total;
};

// Workspace layout of the stream path for `waves` persistent waves and
// groups of G query heads.
StreamLayout stream_layout(int B, int64_t waves, int G) {
  StreamLayout s;
  s.po = 0;
  s.plse = s.po + align256(waves * 2 * G * kD * 4);
  s.pref = s.plse + align256(waves * 2 * G * 4);
  s.meta = s.pref + align256((static_cast<int64_t>(B) + 1) * 4);
  s.total = s.meta + 256;
  return s;
}

int64_t grid_parts(int64_t max_pages, int block_size) {
  return q3::cdiv(q3::cdiv(max_pages * block_size, kTile), kGridTilesPerPart);
}

int64_t grid_bytes(int B, int num_heads, int64_t max_pages, int block_size) {
  const int64_t slots = static_cast<int64_t>(B) * num_heads * grid_parts(max_pages, block_size);
  return align256(slots * kD * 4) + align256(slots * 4);
}

// Launches the stream path (attention pass + merge) with its workspace at ws.
int launch_stream(DecodeArgs& a, char* ws, int wgs, hipStream_t s, const char* who) {
  const StreamLayout L = stream_layout(a.B, int64_t(wgs) * kWaves, a.G);
  a.s_po = reinterpret_cast<float*>(ws + L.po);
  a.s_plse = reinterpret_cast<float*>(ws + L.plse);
  a.s_pref = reinterpret_cast<int32_t*>(ws + L.pref);
  a.s_meta = reinterpret_cast<int32_t*>(ws + L.meta);
  q3::clear_error();
  hipLaunchKernelGGL(paged_decode_stream_kernel, dim3(wgs), dim3(kWaves * 64), 0, s, a);
  int rc = q3::launch_status(who);
  if (rc) return rc;
  hipLaunchKernelGGL(paged_decode_stream_merge_kernel, dim3(a.Hkv, a.B), dim3(64 * a.G), 0, s,
                     a);
  return q3::launch_status(who);
}

// ---------------------------------------------------------------------------
// Static scratch of the allocation-free entry point.  Each device that runs
// the library holds one copy until the process ends; host code reaches a
// device's copy only through the address hipGetSymbolAddress returns for it
// (the array's name on the host is a stand-in, not a device address).
constexpr int64_t kStaticScratchBytes = int64_t(24) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) char scratch[kStaticScratchBytes];

// Device address of `scratch` on device `dev` (the current device), looked up
// once per device; nullptr if the runtime cannot resolve it.
char* scratch_on(int dev) {
  static std::mutex mu;
  static char* addr[kMaxDevices] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    addr[dev] = static_cast<char*>(p);
  }
  return addr[dev];
}

}  // namespace

extern "C" size_t qwen3_paged_decode_workspace_bytes(int B, int num_heads, int num_kv_heads,
                                                     int head_dim, int64_t max_pages,
                                                     int block_size) {
  if (B <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > kMaxG || head_dim != kD || max_pages <= 0 ||
      block_size <= 0 || block_size % kTile != 0)
    return 0;
  // Sized for the current device's persistent waves (the largest grid when
  // no device can be queried) and the shape's group size: it depends only
  // on the launch shape, never on the live lengths.
  if (B <= kStreamMaxB) {
    const int wgs = stream_workgroups();
    const int64_t waves = int64_t(wgs > 0 ? wgs : kStreamMaxWgs) * kWaves;
    return static_cast<size_t>(stream_layout(B, waves, num_heads / num_kv_heads).total);
  }
  return static_cast<size_t>(grid_bytes(B, num_heads, max_pages, block_size));
}

extern "C" int qwen3_paged_decode_bf16(
    const void* q, const int64_t q_strides[2], const void* k_cache, const int64_t k_strides[3],
    const void* v_cache, const int64_t v_strides[3], int64_t num_blocks,
    const int32_t* block_table, int64_t bt_row_stride, int64_t max_rows, int64_t max_pages,
    const int32_t* seq_lens, int seq_len_bias, const int32_t* row_ids, void* out,
    const int64_t out_strides[2], int B, int num_heads, int num_kv_heads, int head_dim,
    int block_size, float scale, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "qwen3_paged_decode_bf16";
  DecodeArgs a;
  if (int rc = prepare(a, who, q, q_strides, k_cache, k_strides, v_cache, v_strides, num_blocks,
                       block_table, bt_row_stride, max_rows, max_pages, seq_lens,
                       seq_len_bias, row_ids, out, out_strides, B, num_heads, num_kv_heads,
                       head_dim, block_size, scale))
    return rc;
  if (B == 0) return QWEN3_OK;
  const size_t need = qwen3_paged_decode_workspace_bytes(B, num_heads, num_kv_heads, head_dim,
                                                         max_pages, block_size);
  if (need == 0) return q3::fail(QWEN3_EINVAL, "%s: cannot size the workspace", who);
  if (!workspace || workspace_bytes < need)
    return q3::fail(QWEN3_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who,
                    need, workspace ? workspace_bytes : (size_t)0);
  if (!q3::aligned16(workspace))
    return q3::fail(QWEN3_EALIGN, "%s: workspace must be 16-byte aligned", who);
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B <= kStreamMaxB) {
    const int wgs = stream_workgroups();
    if (wgs <= 0) return q3::fail(QWEN3_EINVAL, "%s: cannot query the device's CU count", who);
    return launch_stream(a, ws, wgs, s, who);
  }
  const int64_t parts = grid_parts(max_pages, block_size);
  if (parts > 0x7fffffff) return q3::fail(QWEN3_EINVAL, "%s: max_pages too large", who);
  a.max_parts = static_cast<int>(parts);
  const int64_t slots = static_cast<int64_t>(B) * num_heads * parts;
  a.ws_o = reinterpret_cast<float*>(ws);
  a.ws_lse = reinterpret_cast<float*>(ws + align256(slots * kD * 4));
  const size_t lds = static_cast<size_t>(kWaves) * a.G * kOStride * sizeof(float);
  q3::clear_error();
  hipLaunchKernelGGL(paged_decode_grid_kernel, dim3(static_cast<unsigned>(parts), num_kv_heads, B),
                     dim3(kWaves * 64), lds, s, a);
  int rc = q3::launch_status(who);
  if (rc || parts == 1) return rc;
  hipLaunchKernelGGL(paged_decode_grid_merge_kernel, dim3(num_heads, B), dim3(kD), 0, s, a);
  return q3::launch_status(who);
}

extern "C" int qwen3_paged_decode_noalloc_bf16(
    const void* q, const int64_t q_strides[2], const void* k_cache, const int64_t k_strides[3],
    const void* v_cache, const int64_t v_strides[3], int64_t num_blocks,
    const int32_t* block_table, int64_t bt_row_stride, int64_t max_rows, int64_t max_pages,
    const int32_t* seq_lens, int seq_len_bias, const int32_t* row_ids, void* out,
    const int64_t out_strides[2], int B, int num_heads, int num_kv_heads, int head_dim,
    int block_size, float scale, void* stream) {
  const char* who = "qwen3_paged_decode_noalloc_bf16";
  DecodeArgs a;
  if (int rc = prepare(a, who, q, q_strides, k_cache, k_strides, v_cache, v_strides, num_blocks,
                       block_table, bt_row_stride, max_rows, max_pages, seq_lens,
                       seq_len_bias, row_ids, out, out_strides, B, num_heads, num_kv_heads,
                       head_dim, block_size, scale))
    return rc;
  if (B == 0) return QWEN3_OK;
  if (B > kStreamMaxB)
    return q3::fail(QWEN3_EWORKSPACE, "%s: batch %d exceeds the %d rows the static scratch "
                    "serves", who, B, kStreamMaxB);
  const int wgs = stream_workgroups();
  if (wgs <= 0) return q3::fail(QWEN3_EINVAL, "%s: cannot query the device's CU count", who);
  const int64_t need = stream_layout(B, int64_t(wgs) * kWaves, a.G).total;
  if (need > kStaticScratchBytes)
    return q3::fail(QWEN3_EWORKSPACE, "%s: needs %lld bytes of scratch (batch %d, %d query "
                    "heads per KV head); the static scratch holds %lld", who, (long long)need,
                    B, a.G, (long long)kStaticScratchBytes);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return q3::fail(QWEN3_EINVAL, "%s: cannot query the current device", who);
  char* ws = scratch_on(dev);
  if (!ws) return q3::fail(QWEN3_EINVAL, "%s: cannot resolve the static scratch", who);
  return launch_stream(a, ws, wgs, static_cast<hipStream_t>(stream), who);
}
