// Tile machinery shared by the paged decode's two implementations
// (paged_decode.hip, the default; paged_decode_invariant.hip, the
// batch-invariant one): arguments, the K/V tile loads, the MFMA tile math,
// the block-table window and argument validation.
#pragma once

#include "common.hpp"

namespace {

constexpr int kD = 128;        // head_dim
constexpr int kTile = 16;      // tokens per MFMA tile
constexpr int kWaves = 4;      // waves per workgroup
constexpr int kChunk = 2;      // tiles per load batch; two batches in flight per wave
constexpr int kMaxG = 16;      // query heads per KV head (MFMA columns)
constexpr int kWin = 64;       // block-table entries held per window (one per lane)
// Persistent (stream) path.
constexpr int kStreamMaxB = 2048;       // batch entries tabulated in LDS
constexpr int kStreamWgPerCu = 2;       // resident workgroups per CU (2 waves/SIMD)
constexpr int kStreamMaxWgs = 1024;     // persistent grid cap (512 CUs)
// Fewest tiles a wave streams: its two load batches, both issued before the
// first is computed, so a small batch costs one tile round trip per wave.
constexpr int kMinTilesPerWave = 2 * kChunk;

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  int64_t k_sblk, k_sh, k_sslot;
  const uint16_t* v;
  int64_t v_sblk, v_sh, v_sslot;
  int64_t num_blocks;
  const int32_t* bt;
  int64_t bt_stride, max_rows, max_pages;
  const int32_t* seq_lens;
  int bias;
  const int32_t* row_ids;
  uint16_t* out;
  int64_t o_sb, o_sh;
  int B, Hq, Hkv, G, bs;
  float scale_log2;  // softmax scale * log2(e)
  // default path workspace
  float* s_po;       // stream: [W][2][G][kD] normalised partial outputs
  float* s_plse;     // stream: [W][2][G] log2-sum-exp of each partial
  int32_t* s_pref;   // stream (both paths): [B + 1] exclusive prefix of tiles per sequence
  int32_t* s_meta;   // stream: [0] tiles per wave
  int max_parts;     // partitions per (b, hkv) (grid) or sequence-head (invariant) sized for
  float* ws_o;       // grid: [B][Hq][max_parts][kD] normalised partition outputs
  float* ws_lse;     // grid: [B][Hq][max_parts]
  // batch-invariant path workspace: one slot per (b, hkv, partition)
  float* s_acc;      // [B][Hkv][max_parts][G][kD] unnormalised partition / fold outputs
  float2* s_ml;      // [B][Hkv][max_parts][G] (running max, denominator) of each
  int64_t* s_pw;     // [0] tiles per wave (stream)
  uint32_t* tickets; // [2048][Hkv] parts in of each split sequence-head (stream)
  int grid_mode;     // the merge follows the grid path's partitions
};


// Row of batch entry b in the resident tables, or -1 if out of range.
__device__ __forceinline__ int64_t row_of(const DecodeArgs& a, int b) {
  const int64_t row = a.row_ids ? a.row_ids[b] : b;
  return (row >= 0 && row < a.max_rows) ? row : -1;
}

// Context length of a valid row, clamped to what one table row addresses.
__device__ __forceinline__ int64_t clamp_len(const DecodeArgs& a, int32_t seq_len) {
  int64_t L = static_cast<int64_t>(seq_len) + a.bias;
  const int64_t cap = a.max_pages * a.bs;
  L = L < cap ? L : cap;
  return L > 0 ? L : 0;
}

// ---------------------------------------------------------------------------
// Tile math shared by both paths.

// K/V registers of up to kChunk 16-token tiles of one KV head of one sequence.
//   k[i][c]: token lo of tile i, dims c*32 + 8*hi .. +7   (A operand of QK^T)
//   v[i][e]: token 4*hi + e of tile i, dims 8*lo .. +7    (row-major V rows)
struct Chunk {
  q3::u32x4 k[kChunk][4];
  q3::u32x4 v[kChunk][4];
  bool valid[kChunk];
  int n;       // tiles in this batch (0 = none)
  int t0;      // first tile (index within the sequence)
  int seg;     // b * Hkv + hkv
  int ntiles;  // tiles of the whole sequence
  int L;       // context length of the sequence
};

// K and V are read once per call: non-temporal loads (measured on the
// B=256 Qwen3-8B decode: 849 -> 767 us per call, the same output bits).
__device__ __forceinline__ void load_tile(Chunk& c, int i, const DecodeArgs& a,
                                          const uint16_t* kbase, const uint16_t* vbase,
                                          int64_t phys, int sub, int lo, int hi) {
  c.valid[i] = phys >= 0 && phys < a.num_blocks;
  if (c.valid[i]) {
    const uint16_t* kp = kbase + phys * a.k_sblk + (sub + lo) * a.k_sslot + hi * 8;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) c.k[i][cc] = q3::ld16_nt(kp + cc * 32);
    const uint16_t* vp = vbase + phys * a.v_sblk + (sub + 4 * hi) * a.v_sslot + lo * 8;
#pragma unroll
    for (int e = 0; e < 4; ++e) c.v[i][e] = q3::ld16_nt(vp + e * a.v_sslot);
  } else {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      c.k[i][cc] = q3::u32x4{0u, 0u, 0u, 0u};
      c.v[i][cc] = q3::u32x4{0u, 0u, 0u, 0u};
    }
  }
}

struct SoftmaxState {
  float m;           // running max (log2 domain) of column lo
  float l;           // this lane's share of the running denominator
  q3::f32x4 acc[8];  // acc[j][r] = O[lo][32*hi + 8*r + j] (unnormalised)
};

__device__ __forceinline__ void reset(SoftmaxState& st) {
  st.m = q3::kNegInf;
  st.l = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.acc[j] = q3::f32x4{0.f, 0.f, 0.f, 0.f};
}

// Q^T as the B operand: lane (column lo, k-group hi) holds, for chunk c of 32
// dims, the 8 dims c*32 + hi*8 .. +7 of query head hkv*G + lo (zero if lo >= G).
__device__ __forceinline__ void load_q(q3::bf16x8 (&qv)[4], const DecodeArgs& a, int b, int hkv,
                                       int lo, int hi) {
  q3::u32x4 z = {0u, 0u, 0u, 0u};
  if (lo < a.G) {
    const uint16_t* qp =
        a.q + b * a.q_sb + (static_cast<int64_t>(hkv) * a.G + lo) * a.q_sh + hi * 8;
#pragma unroll
    for (int c = 0; c < 4; ++c) qv[c] = q3::as_bf16x8(q3::ld16(qp + c * 32));
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) qv[c] = q3::as_bf16x8(z);
  }
}

// Folds c.n tiles (first tile c.t0) into the online softmax state.
__device__ __forceinline__ void compute_chunk(Chunk& c, float scale_log2, int hi,
                                              const q3::bf16x8 (&qv)[4], SoftmaxState& st) {
  // S^T = K Q^T: lane (column lo, k-group hi) receives tokens 4*hi + r.
  q3::f32x4 s[kChunk];
#pragma unroll
  for (int i = 0; i < kChunk; ++i) {
    s[i] = q3::f32x4{0.f, 0.f, 0.f, 0.f};
    if (i < c.n) {
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        s[i] = q3::mfma16x16x32(q3::as_bf16x8(c.k[i][cc]), qv[cc], s[i]);
    }
  }
  float mx = q3::kNegInf;
#pragma unroll
  for (int i = 0; i < kChunk; ++i) {
    const int tokb = (c.t0 + i) * kTile + 4 * hi;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = i < c.n && c.valid[i] && tokb + r < c.L;
      const float v = ok ? s[i][r] * scale_log2 : q3::kNegInf;
      s[i][r] = v;
      mx = fmaxf(mx, v);
      // A slot at or past L may hold anything (even NaN): its P is 0, but
      // 0 * NaN is not, so the V row of such a slot is zeroed.
      if (!ok) c.v[i][r] = q3::u32x4{0u, 0u, 0u, 0u};
    }
  }
  mx = q3::max_xor32(q3::max_xor16(mx));
  const float m_new = fmaxf(st.m, mx);
  const float m_use = m_new == q3::kNegInf ? 0.f : m_new;
  const float alpha = q3::fast_exp2(st.m - m_use);
  st.m = m_new;

  // P in fp32 as two bf16 terms, p = hi + lo (hi = bf16(p), lo = bf16(p -
  // hi)): 16 significant bits, so V^T P^T carries P at about the fp32
  // precision of the reference's product (the two MFMAs per step cost no
  // time in this memory-bound loop).
  q3::bf16x4 p[kChunk], pl[kChunk];
  float psum = 0.f;
#pragma unroll
  for (int i = 0; i < kChunk; ++i) {
    float e[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e[r] = q3::fast_exp2(s[i][r] - m_use);
      psum += e[r];
    }
    const q3::u32x2 pk = {q3::pack_bf16x2(e[0], e[1]), q3::pack_bf16x2(e[2], e[3])};
    p[i] = q3::as_bf16x4(pk);
    // the rounded terms back in fp32: a bf16's bits are the top half of a float's
    const float h0 = __uint_as_float(pk[0] << 16), h1 = __uint_as_float(pk[0] & 0xffff0000u);
    const float h2 = __uint_as_float(pk[1] << 16), h3 = __uint_as_float(pk[1] & 0xffff0000u);
    const q3::u32x2 lk = {q3::pack_bf16x2(e[0] - h0, e[1] - h1),
                          q3::pack_bf16x2(e[2] - h2, e[3] - h3)};
    pl[i] = q3::as_bf16x4(lk);
  }
  st.l = st.l * alpha + psum;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.acc[j] *= alpha;

  // O^T += V^T P^T.  For output slice j the A operand of lane (dim group lo,
  // k-group hi) is V[4*hi + e][8*lo + j], e = 0..3, gathered from the four
  // row-major 16-byte V loads of the lane.
#pragma unroll
  for (int i = 0; i < kChunk; ++i) {
    if (i < c.n) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int w = j >> 1, h = j & 1;
        q3::u32x2 av = {q3::pick_halves(c.v[i][0][w], c.v[i][1][w], h),
                        q3::pick_halves(c.v[i][2][w], c.v[i][3][w], h)};
        st.acc[j] = q3::mfma16x16x16(q3::as_bf16x4(av), p[i], st.acc[j]);
        st.acc[j] = q3::mfma16x16x16(q3::as_bf16x4(av), pl[i], st.acc[j]);
      }
    }
  }
}

// Writes the normalised output of column lo (a query head) as bf16: lane
// (lo, hi) owns dims 32*hi .. 32*hi + 31.
__device__ __forceinline__ void store_out_bf16(const DecodeArgs& a, int b, int hq,
                                               const q3::f32x4 (&acc)[8], float inv, int hi) {
  uint16_t* op = a.out + b * a.o_sb + static_cast<int64_t>(hq) * a.o_sh + 32 * hi;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    q3::u32x4 w = {q3::pack_bf16x2(acc[0][r] * inv, acc[1][r] * inv),
                   q3::pack_bf16x2(acc[2][r] * inv, acc[3][r] * inv),
                   q3::pack_bf16x2(acc[4][r] * inv, acc[5][r] * inv),
                   q3::pack_bf16x2(acc[6][r] * inv, acc[7][r] * inv)};
    q3::st16(op + 8 * r, w);
  }
}

// ---------------------------------------------------------------------------
// Block-table window (both paths).

// Wave-uniform window of kWin block-table entries of one row (lane i holds
// entry base + i) plus the prefetched next window.
struct TableWindow {
  int64_t row;
  int base;
  int32_t cur, next;
};

__device__ __forceinline__ int32_t table_entry(const DecodeArgs& a, int64_t row, int page) {
  return (row >= 0 && page < a.max_pages) ? a.bt[row * a.bt_stride + page] : -1;
}

__device__ __forceinline__ void window_load(TableWindow& tw, const DecodeArgs& a, int64_t row,
                                            int base, int lane) {
  tw.row = row;
  tw.base = base;
  tw.cur = table_entry(a, row, base + lane);
  tw.next = table_entry(a, row, base + kWin + lane);
}

// Physical block of `page` of row tw.row (wave-uniform).
__device__ __forceinline__ int64_t window_phys(TableWindow& tw, const DecodeArgs& a, int page,
                                               int lane) {
  if (page >= tw.base + kWin && page < tw.base + 2 * kWin) {
    tw.cur = tw.next;
    tw.base += kWin;
    tw.next = table_entry(a, tw.row, tw.base + kWin + lane);
  } else if (page < tw.base || page >= tw.base + kWin) {
    window_load(tw, a, tw.row, page, lane);
  }
  return __builtin_amdgcn_readlane(tw.cur, page - tw.base);
}

// ---------------------------------------------------------------------------
// Host side (both paths).

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Validates the arguments shared by both decode entry points and fills `a`
// (everything but the workspace pointers).
int prepare(DecodeArgs& a, const char* who, const void* q, const int64_t q_strides[2],
            const void* k_cache, const int64_t k_strides[3], const void* v_cache,
            const int64_t v_strides[3], int64_t num_blocks, const int32_t* block_table,
            int64_t bt_row_stride, int64_t max_rows, int64_t max_pages,
            const int32_t* seq_lens, int seq_len_bias, const int32_t* row_ids, void* out,
            const int64_t out_strides[2], int B, int num_heads, int num_kv_heads,
            int head_dim, int block_size, float scale) {
  if (!q || !k_cache || !v_cache || !block_table || !seq_lens || !out || !q_strides ||
      !k_strides || !v_strides || !out_strides)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (head_dim != kD)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: head_dim %d not supported (built for %d)", who,
                    head_dim, kD);
  if (block_size <= 0 || block_size % kTile != 0)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: block_size %d must be a multiple of %d", who,
                    block_size, kTile);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > kMaxG)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: num_heads %d / num_kv_heads %d unsupported", who,
                    num_heads, num_kv_heads);
  if (B < 0 || num_blocks <= 0 || max_rows <= 0 || max_pages <= 0 ||
      bt_row_stride < max_pages)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes (B=%d num_blocks=%lld max_rows=%lld "
                    "max_pages=%lld bt_row_stride=%lld)", who, B, (long long)num_blocks,
                    (long long)max_rows, (long long)max_pages, (long long)bt_row_stride);
  if (B > 65535 || num_kv_heads > 65535)
    return q3::fail(QWEN3_EINVAL, "%s: batch %d too large for one launch", who, B);
  if (max_pages * block_size > (int64_t(1) << 30))
    return q3::fail(QWEN3_EINVAL, "%s: max_pages * block_size too large", who);
  // 16-byte vector access of q/K/V/out rows.
  const int64_t vec_strides[] = {q_strides[0], q_strides[1], k_strides[0], k_strides[1],
                                 k_strides[2], v_strides[0], v_strides[1], v_strides[2],
                                 out_strides[0], out_strides[1]};
  bool ok = q3::aligned16(q) && q3::aligned16(k_cache) && q3::aligned16(v_cache) &&
            q3::aligned16(out);
  for (int64_t st : vec_strides) ok = ok && st % 8 == 0;
  if (!ok)
    return q3::fail(QWEN3_EALIGN, "%s: q/K/V/out need 16-byte aligned rows (strides multiple "
                    "of 8 elements)", who);
  a = DecodeArgs{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_strides[0];
  a.q_sh = q_strides[1];
  a.k = static_cast<const uint16_t*>(k_cache);
  a.k_sblk = k_strides[0];
  a.k_sh = k_strides[1];
  a.k_sslot = k_strides[2];
  a.v = static_cast<const uint16_t*>(v_cache);
  a.v_sblk = v_strides[0];
  a.v_sh = v_strides[1];
  a.v_sslot = v_strides[2];
  a.num_blocks = num_blocks;
  a.bt = block_table;
  a.bt_stride = bt_row_stride;
  a.max_rows = max_rows;
  a.max_pages = max_pages;
  a.seq_lens = seq_lens;
  a.bias = seq_len_bias;
  a.row_ids = row_ids;
  a.out = static_cast<uint16_t*>(out);
  a.o_sb = out_strides[0];
  a.o_sh = out_strides[1];
  a.B = B;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.G = num_heads / num_kv_heads;
  a.bs = block_size;
  a.scale_log2 = scale * q3::kLog2e;
  return QWEN3_OK;
}

// Persistent workgroups of the stream path on the current device (0: unknown).
int stream_workgroups() {
  const int wgs = cu_count() * kStreamWgPerCu;
  return wgs < kStreamMaxWgs ? wgs : kStreamMaxWgs;
}

}  // namespace
