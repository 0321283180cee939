// Paged decode attention for gfx950 (GQA, one query token per sequence).
//
// Semantics follow paged_attn_decode_kernel
// (qwen3/kernels/paged_attention.py:27-129): for batch entry b and KV head
// hkv, the G = Hq/Hkv query heads hkv*G .. hkv*G+G-1 attend the first
// L = seq_lens[row] + bias tokens of the sequence, gathered page by page
// through block_table[row]; softmax in fp32, bf16 output.
//
// Design (MI355X-first, not a transcription of the Triton program):
//  * Work unit = (partition of 16-token tiles, kv head, batch entry): one
//    256-thread workgroup (4 wave64s).  A partition covers TILES_PER_WAVE
//    tiles per wave; long contexts therefore split into many workgroups
//    (split-KV), and a second kernel merges partitions with log-sum-exp
//    weights.  Single-partition sequences are written directly.
//  * A 16-token tile of one KV head is 4 KiB of K and 4 KiB of V, contiguous
//    in the pool; every lane issues 16-byte loads (4 for K, 4 for V), all
//    loads of a chunk of tiles are issued before any math so a wave keeps
//    up to 32 KiB in flight.
//  * QK^T on the matrix cores: S^T(16 tok x 16 q) = K(16x128) Q^T(128x16)
//    as 4 x mfma_f32_16x16x32_bf16.  The G query heads fill G of the 16
//    columns (zero-padded Q); padding costs idle MFMA slots, not registers.
//  * The S^T accumulator layout (lane = q column + 16*(token/4)) is exactly
//    the B-operand layout of the PV product, so P goes to the matrix cores
//    with no cross-lane traffic: O^T(128 x 16) = V^T(128 x 16 tok) P^T as
//    8 x mfma_f32_16x16x16_bf16, where the V^T operand is built in-lane
//    from the row-major 16-byte V loads with byte permutes.
//  * Online softmax in the exp2 domain, one running max per query column,
//    updated once per chunk of tiles.
#include "common.hpp"

namespace {

constexpr int kD = 128;      // head_dim
constexpr int kTile = 16;    // tokens per MFMA tile
constexpr int kWaves = 4;    // waves per workgroup
constexpr int kChunk = 4;    // tiles whose loads are in flight together per wave
constexpr int kMaxG = 16;    // query heads per KV head (MFMA columns)
constexpr int kOStride = kD + 4;  // padded LDS row of the partition output

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
  int max_parts;     // partitions per (b, hkv) the workspace is sized for
  float* ws_o;       // [B][Hq][max_parts][kD] normalised partition outputs
  float* ws_lse;     // [B][Hq][max_parts] log2-sum-exp of each partition
};

// Context length (tokens) of batch entry b, clamped to what the table row can
// address; 0 for an out-of-range row id.
__device__ __forceinline__ int64_t context_len(const DecodeArgs& a, int b, int64_t* row_out) {
  const int64_t row = a.row_ids ? a.row_ids[b] : b;
  *row_out = row;
  if (row < 0 || row >= a.max_rows) return 0;
  int64_t L = static_cast<int64_t>(a.seq_lens[row]) + a.bias;
  const int64_t cap = a.max_pages * a.bs;
  L = L < cap ? L : cap;
  return L > 0 ? L : 0;
}

template <int TILES_PER_WAVE>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_part_kernel(DecodeArgs a) {
  constexpr int kTilesPerPart = TILES_PER_WAVE * kWaves;
  const int part = blockIdx.x;
  const int hkv = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lo = lane & 15;  // q column (QK/PV) or token row (K operand) or dim group (V)
  const int hi = lane >> 4;  // k-group

  int64_t row;
  const int64_t L = context_len(a, b, &row);
  const int n_tiles = static_cast<int>(q3::cdiv(L, kTile));
  const int tile0 = part * kTilesPerPart;
  const int G = a.G;

  if (tile0 >= n_tiles) {
    if (part == 0) {  // empty context: defined zero output
      for (int e = tid; e < G * kD; e += kWaves * 64) {
        const int g = e / kD, d = e % kD;
        a.out[b * a.o_sb + (static_cast<int64_t>(hkv) * G + g) * a.o_sh + d] = 0;
      }
    }
    return;
  }
  const int n_parts = static_cast<int>(q3::cdiv(n_tiles, kTilesPerPart));
  const int tile_end = min(n_tiles, tile0 + kTilesPerPart);

  __shared__ float s_m[kWaves][kMaxG];
  __shared__ float s_l[kWaves][kMaxG];
  __shared__ float s_o[kMaxG * kOStride];
  for (int e = tid; e < G * kOStride; e += kWaves * 64) s_o[e] = 0.f;

  // Q^T as the B operand: lane (column lo, k-group hi) holds, for chunk c of
  // 32 dims, the 8 dims c*32 + hi*8 .. +7 of query head hkv*G + lo.
  q3::bf16x8 qv[4];
  {
    q3::u32x4 z = {0u, 0u, 0u, 0u};
    if (lo < G) {
      const uint16_t* qp = a.q + b * a.q_sb + (static_cast<int64_t>(hkv) * G + lo) * a.q_sh + hi * 8;
#pragma unroll
      for (int c = 0; c < 4; ++c) qv[c] = q3::as_bf16x8(q3::ld16(qp + c * 32));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) qv[c] = q3::as_bf16x8(z);
    }
  }

  float m_run = q3::kNegInf;  // running max (log2 domain) of column lo
  float l_run = 0.f;          // this lane's share of the running denominator
  q3::f32x4 acc[8];           // acc[j][r] = O[lo][32*hi + 8*r + j] (unnormalised)
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = q3::f32x4{0.f, 0.f, 0.f, 0.f};

  const int w0 = tile0 + wave * TILES_PER_WAVE;
  const int w1 = min(tile_end, w0 + TILES_PER_WAVE);
  const uint16_t* kbase = a.k + static_cast<int64_t>(hkv) * a.k_sh;
  const uint16_t* vbase = a.v + static_cast<int64_t>(hkv) * a.v_sh;
  const int32_t* bt_row = a.bt + row * a.bt_stride;

  for (int t0 = w0; t0 < w1; t0 += kChunk) {
    q3::u32x4 kr[kChunk][4];
    q3::u32x4 vr[kChunk][4];
    bool tv[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const int t = t0 + i;
      int64_t phys = -1;
      int sub = 0;
      if (t < w1) {
        const int64_t tok0 = static_cast<int64_t>(t) * kTile;
        phys = bt_row[tok0 / a.bs];
        sub = static_cast<int>(tok0 % a.bs);
      }
      tv[i] = phys >= 0 && phys < a.num_blocks;
      if (tv[i]) {
        const uint16_t* kp = kbase + phys * a.k_sblk + (sub + lo) * a.k_sslot + hi * 8;
#pragma unroll
        for (int c = 0; c < 4; ++c) kr[i][c] = q3::ld16(kp + c * 32);
        const uint16_t* vp = vbase + phys * a.v_sblk + (sub + 4 * hi) * a.v_sslot + lo * 8;
#pragma unroll
        for (int e = 0; e < 4; ++e) vr[i][e] = q3::ld16(vp + e * a.v_sslot);
        // Slots at or past L in the last tile may hold anything (even NaN);
        // their P is 0 but 0 * NaN is not, so zero those V rows.
        const int64_t tok_e0 = static_cast<int64_t>(t) * kTile + 4 * hi;
        if (static_cast<int64_t>(t + 1) * kTile > L) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (tok_e0 + e >= L) vr[i][e] = q3::u32x4{0u, 0u, 0u, 0u};
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          kr[i][c] = q3::u32x4{0u, 0u, 0u, 0u};
          vr[i][c] = q3::u32x4{0u, 0u, 0u, 0u};
        }
      }
    }

    // S^T = K Q^T: lane (column lo, k-group hi) receives tokens 4*hi + r.
    q3::f32x4 s[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      s[i] = q3::f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) s[i] = q3::mfma16x16x32(q3::as_bf16x8(kr[i][c]), qv[c], s[i]);
    }

    float mx = q3::kNegInf;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const int64_t tokb = static_cast<int64_t>(t0 + i) * kTile + 4 * hi;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = (tv[i] && tokb + r < L) ? s[i][r] * a.scale_log2 : q3::kNegInf;
        s[i][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, q3::shfl_xor(mx, 16));
    mx = fmaxf(mx, q3::shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == q3::kNegInf ? 0.f : m_new;
    const float alpha = q3::fast_exp2(m_run - m_use);

    q3::bf16x4 p[kChunk];
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      float e[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        e[r] = q3::fast_exp2(s[i][r] - m_use);
        psum += e[r];
      }
      q3::u32x2 pk = {q3::pack_bf16x2(e[0], e[1]), q3::pack_bf16x2(e[2], e[3])};
      p[i] = q3::as_bf16x4(pk);
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] *= alpha;

    // O^T += V^T P^T.  For output slice j the A operand of lane (dim group lo,
    // k-group hi) is V[4*hi + e][8*lo + j], e = 0..3, gathered from the four
    // row-major 16-byte V loads of the lane.
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int w = j >> 1, h = j & 1;
        q3::u32x2 av = {q3::pick_halves(vr[i][0][w], vr[i][1][w], h),
                        q3::pick_halves(vr[i][2][w], vr[i][3][w], h)};
        acc[j] = q3::mfma16x16x16(q3::as_bf16x4(av), p[i], acc[j]);
      }
    }
  }

  // Lanes of one column hold disjoint token subsets of the denominator.
  l_run += q3::shfl_xor(l_run, 16);
  l_run += q3::shfl_xor(l_run, 32);

  // ---- combine the waves of the workgroup through LDS ----
  if (hi == 0) {
    s_m[wave][lo] = m_run;
    s_l[wave][lo] = l_run;
  }
  __syncthreads();
  float M = q3::kNegInf;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][lo]);
  const float M_use = M == q3::kNegInf ? 0.f : M;
  const float wgt = q3::fast_exp2(m_run - M_use);
  if (lo < G) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        atomicAdd(&s_o[lo * kOStride + 32 * hi + 8 * r + j], acc[j][r] * wgt);
  }
  __syncthreads();

  // ---- write: final bf16 output, or a normalised partial + its LSE ----
  for (int e = tid; e < G * (kD / 2); e += kWaves * 64) {
    const int g = e / (kD / 2);
    const int d = 2 * (e % (kD / 2));
    float Mg = q3::kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) Mg = fmaxf(Mg, s_m[w][g]);
    const float Mg_use = Mg == q3::kNegInf ? 0.f : Mg;
    float Lg = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) Lg += s_l[w][g] * q3::fast_exp2(s_m[w][g] - Mg_use);
    const float inv = Lg > 0.f ? 1.f / Lg : 0.f;
    const float o0 = s_o[g * kOStride + d] * inv;
    const float o1 = s_o[g * kOStride + d + 1] * inv;
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

// Merges the partitions of every (b, query head) whose context needed more
// than one: o = sum_p 2^(lse_p - lse_max) o_p / sum_p 2^(lse_p - lse_max).
template <int TILES_PER_WAVE>
__global__ __launch_bounds__(kD) void paged_decode_reduce_kernel(DecodeArgs a) {
  constexpr int kTilesPerPart = TILES_PER_WAVE * kWaves;
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  int64_t row;
  const int64_t L = context_len(a, b, &row);
  const int n_tiles = static_cast<int>(q3::cdiv(L, kTile));
  const int n_parts = static_cast<int>(q3::cdiv(n_tiles, kTilesPerPart));
  if (n_parts <= 1) return;
  const int64_t base = (static_cast<int64_t>(b) * a.Hq + hq) * a.max_parts;
  float M = q3::kNegInf;
  for (int p = 0; p < n_parts; ++p) M = fmaxf(M, a.ws_lse[base + p]);
  const float M_use = M == q3::kNegInf ? 0.f : M;
  float sw = 0.f, o = 0.f;
  for (int p = 0; p < n_parts; ++p) {
    const float w = q3::fast_exp2(a.ws_lse[base + p] - M_use);
    sw += w;
    o += w * a.ws_o[(base + p) * kD + d];
  }
  o = sw > 0.f ? o / sw : 0.f;
  a.out[b * a.o_sb + static_cast<int64_t>(hq) * a.o_sh + d] = q3::bf16_bits(o);
}

constexpr int kTilesPerWave = 4;
constexpr int kTilesPerPart = kTilesPerWave * kWaves;

int64_t max_parts_for(int64_t max_pages, int block_size) {
  const int64_t max_tiles = q3::cdiv(max_pages * block_size, kTile);
  return q3::cdiv(max_tiles, kTilesPerPart);
}

}  // namespace

extern "C" size_t qwen3_paged_decode_workspace_bytes(int B, int num_heads, int head_dim,
                                                     int64_t max_pages, int block_size) {
  if (B <= 0 || num_heads <= 0 || head_dim != kD || max_pages <= 0 || block_size <= 0 ||
      block_size % kTile != 0)
    return 0;
  const int64_t parts = max_parts_for(max_pages, block_size);
  const int64_t slots = static_cast<int64_t>(B) * num_heads * parts;
  // ws_o (slots x D fp32) followed by ws_lse (slots fp32), 256-byte aligned.
  const int64_t o_bytes = ((slots * kD * 4 + 255) / 256) * 256;
  return static_cast<size_t>(o_bytes + ((slots * 4 + 255) / 256) * 256);
}

extern "C" int qwen3_paged_decode_bf16(
    const void* q, const int64_t q_strides[2], const void* k_cache, const int64_t k_strides[3],
    const void* v_cache, const int64_t v_strides[3], int64_t num_blocks,
    const int32_t* block_table, int64_t bt_row_stride, int64_t max_rows, int64_t max_pages,
    const int32_t* seq_lens, int seq_len_bias, const int32_t* row_ids, void* out,
    const int64_t out_strides[2], int B, int num_heads, int num_kv_heads, int head_dim,
    int block_size, float scale, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "qwen3_paged_decode_bf16";
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
  if (B == 0) return QWEN3_OK;
  if (B > 65535 || num_kv_heads > 65535)
    return q3::fail(QWEN3_EINVAL, "%s: batch %d too large for one launch", who, B);
  // 16-byte vector access of q/K/V rows and 4-byte stores of output pairs.
  const int64_t vec_strides[] = {q_strides[0], q_strides[1], k_strides[0], k_strides[1],
                                 k_strides[2], v_strides[0], v_strides[1], v_strides[2]};
  bool ok = q3::aligned16(q) && q3::aligned16(k_cache) && q3::aligned16(v_cache) &&
            (reinterpret_cast<uintptr_t>(out) & 3u) == 0 && out_strides[0] % 2 == 0 &&
            out_strides[1] % 2 == 0;
  for (int64_t s : vec_strides) ok = ok && s % 8 == 0;
  if (!ok)
    return q3::fail(QWEN3_EALIGN, "%s: q/K/V need 16-byte aligned rows (strides multiple "
                    "of 8 elements), out needs 4-byte aligned element pairs", who);
  const int64_t parts = max_parts_for(max_pages, block_size);
  if (parts > 0x7fffffff) return q3::fail(QWEN3_EINVAL, "%s: max_pages too large", who);
  const size_t need = qwen3_paged_decode_workspace_bytes(B, num_heads, head_dim, max_pages,
                                                         block_size);
  if (parts > 1 && (!workspace || workspace_bytes < need))
    return q3::fail(QWEN3_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who,
                    need, workspace ? workspace_bytes : (size_t)0);

  DecodeArgs a{};
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
  a.max_parts = static_cast<int>(parts);
  if (parts > 1) {
    const int64_t slots = static_cast<int64_t>(B) * num_heads * parts;
    a.ws_o = static_cast<float*>(workspace);
    a.ws_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        ((slots * kD * 4 + 255) / 256) * 256);
  }

  q3::clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL((paged_decode_part_kernel<kTilesPerWave>),
                     dim3(static_cast<unsigned>(parts), num_kv_heads, B), dim3(kWaves * 64), 0,
                     s, a);
  int rc = q3::launch_status(who);
  if (rc || parts == 1) return rc;
  hipLaunchKernelGGL((paged_decode_reduce_kernel<kTilesPerWave>), dim3(num_heads, B), dim3(kD),
                     0, s, a);
  return q3::launch_status(who);
}
