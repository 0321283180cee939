// Decode-batch QKV projection fused with the pre-attention step: one launch
// computes, for up to 64 tokens,
//   qkv = RMSNorm(h) @ W_qkv^T                 (qwen3/attention.py:81, norm.py:22-26)
//   q, k = RMSNorm_head(q), RMSNorm_head(k)    (qwen3/attention.py:91-92)
//   q, k = RoPE(q, k) at each token's position (qwen3/rope.py:88-110)
// and stores q for the attention kernel and k, v into the paged pool at
// position seq_lens[row] through the resident block table, as the decode
// form of the pre-attention kernel does (qwen3/kernels/paged_attention.py:
// 292-350 for the write).
//
// Work split: one 1024-thread workgroup per (head, 16-token block).  Its 16
// waves are 8 column tiles of the head's 128 weight rows x 2 halves of K;
// each streams 16 weight rows from HBM as the B operand of
// mfma_f32_16x16x32_bf16 (loads coalesced per lane quad, redistributed with
// ds_bpermute).  The A operand, the block's 16 rows of the residual stream h
// after the input RMSNorm (rms from the producer's per-16-column partial
// sums of h^2), is staged once in LDS by the whole workgroup and read from
// there in the operand layout.  The head's 16 x 128 outputs meet in LDS, rounded to bf16 as the
// projection's output is, and 16 lanes per token finish the head with the
// arithmetic of the pre-attention kernel (same lane grouping, same
// summation order, so the same bits).  The 16-token blocks of one head run
// on one XCD (workgroups are dealt round-robin), so its weights come from
// HBM once.
#include "common.hpp"

namespace {

constexpr int kD = 128;
constexpr int kRowsPerBlock = 16;
constexpr int kColTiles = kD / 16;  // 8
constexpr int kKParts = 2;
constexpr int kWavesQ = kColTiles * kKParts;  // 16
constexpr int kThreadsQ = kWavesQ * 64;       // 1024
constexpr int kKStep = 32;
constexpr int kC = 8;  // k-steps per prefetch buffer (weights only)
constexpr int kMaxRows = 64;
constexpr int kMaxK = 4096;  // staged A rows: 16 x (K + 8) bf16 in LDS
constexpr int kXcds = 8;

struct QkvArgs {
  const uint16_t* h;  // residual stream (M x K)
  int64_t h_s;
  const float* ss_in;  // (M x ss_tiles) partial sums of h^2
  int ss_tiles;
  const uint16_t* norm_w;  // input RMSNorm weight (K)
  float eps;
  const uint16_t* w;  // fused qkv weight ((Hq + 2 Hkv) * 128 x K)
  int64_t w_s;
  int M, K, Hq, Hkv;
  const uint16_t* q_w;  // QK-norm weights (128)
  const uint16_t* k_w;
  float head_eps;
  const float* cos_t;
  const float* sin_t;
  int64_t tab_stride, tab_rows;
  const int64_t* positions;  // nullable: RoPE at seq_lens[row]
  uint16_t* q_out;
  int64_t qo_s0, qo_s1;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kc[4], vc[4];
  int64_t num_blocks;
  int layer;
  const int32_t* seq_lens;
  const int32_t* block_table;
  int64_t bt_stride, max_rows, max_pages;
  const int32_t* row_ids;  // nullable: identity
  int bs;
};

__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(static_cast<uint32_t>(q3::bf16_bits(x)) << 16);
}

__global__ __launch_bounds__(kThreadsQ) void qkv_rope_kernel(QkvArgs a) {
  // The block's 16 normalised A rows, staged once: row r at a_s + r * pitch.
  extern __shared__ uint16_t a_s[];
  __shared__ float rms_s[kRowsPerBlock];
  __shared__ float red[kColTiles][4][64];
  __shared__ uint16_t y_s[kRowsPerBlock][kD];
  __shared__ int64_t pos_s[kRowsPerBlock], phys_s[kRowsPerBlock];
  __shared__ int off_s[kRowsPerBlock];

  const int heads = a.Hq + 2 * a.Hkv;
  const int rbc = (a.M + 15) >> 4;
  const int b = blockIdx.x;
  const int slot = b >> 3;
  const int head = (slot / rbc) * kXcds + (b & (kXcds - 1));
  const int rb = slot % rbc;
  if (head >= heads) return;  // whole workgroup

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int ct = wave % kColTiles;  // column tile of the head
  const int kh = wave / kColTiles;  // half of K
  const int r16 = lane & 15;
  const int kg = 8 * (lane >> 4);
  const int kw = a.K / kKParts;
  const int k0 = kh * kw;
  const int steps = kw / kKStep;
  const int pitch = a.K + 8;  // bf16 elements per staged row (16-byte pad: no bank conflicts)

  // Weights: coalesced loads (lane l: row l / 4, k-group l % 4) moved into
  // the operand layout (lane L: row L % 16, k-group L / 16) by ds_bpermute.
  const int lrow = lane >> 2, lkg = 8 * (lane & 3);
  const int perm_addr = 4 * (4 * r16 + (lane >> 4));
  const uint16_t* wrow =
      a.w + static_cast<int64_t>(head * kD + ct * 16 + lrow) * a.w_s + lkg + k0;
  auto to_mfma = [&](q3::u32x4 v) {
    q3::u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(perm_addr, static_cast<int>(v[e])));
    return o;
  };
  struct Buf {
    q3::u32x4 b[kC];
  };
  auto load = [&](Buf& B, int s0) {
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      if (s0 + u >= steps) break;
      B.b[u] = q3::ld16(wrow + (s0 + u) * kKStep);
    }
  };
  Buf p, q;
  load(p, 0);
  load(q, kC);

  // A rows and norm weight for this thread's first staging chunks (16 rows x
  // K/8 chunks of 8), the rms of every row, and the position and pool slot
  // of every token of the block: all independent of the weights, so their
  // loads overlap them.
  const int cpr = a.K >> 3;  // chunks per row
  const int nchunks = kRowsPerBlock * cpr;
  constexpr int kPre = 2;  // chunks per thread loaded early (all of them for K <= 1024)
  q3::u32x4 hv[kPre], nv[kPre];
  auto chunk_src = [&](int c, q3::u32x4& h, q3::u32x4& n) {
    const int r = c / cpr, cc = c - r * cpr;
    const int row = min(rb * 16 + r, a.M - 1);
    h = q3::ld16(a.h + static_cast<int64_t>(row) * a.h_s + 8 * cc);
    n = q3::ld16(a.norm_w + 8 * cc);
  };
#pragma unroll
  for (int i = 0; i < kPre; ++i)
    if (tid + i * kThreadsQ < nchunks) chunk_src(tid + i * kThreadsQ, hv[i], nv[i]);
  if (wave == 0) {
    const int row = min(rb * 16 + (lane >> 2), a.M - 1);
    const int part = lane & 3;
    const float* sp = a.ss_in + static_cast<int64_t>(row) * a.ss_tiles;
    float s = 0.f;
    if (a.ss_tiles == 64) {
      float4 f[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) f[j] = reinterpret_cast<const float4*>(sp + 16 * part)[j];
#pragma unroll
      for (int j = 0; j < 4; ++j) s += ((f[j].x + f[j].y) + f[j].z) + f[j].w;
    } else {
      for (int t = part; t < a.ss_tiles; t += 4) s += sp[t];
    }
    s += q3::dpp_f32<q3::kDppXor1>(s);  // lane ^ 1
    s += q3::dpp_f32<q3::kDppXor2>(s);  // lane ^ 2
    if (part == 0) rms_s[lane >> 2] = 1.f / sqrtf(s / static_cast<float>(a.K) + a.eps);
  } else if (wave == 1 && lane < kRowsPerBlock) {
    const int t = rb * 16 + lane;
    int64_t pos = -1, phys = -1, off = 0;
    if (t < a.M) {
      const int64_t row = a.row_ids ? a.row_ids[t] : t;
      if (row >= 0 && row < a.max_rows) {
        const int64_t wpos = a.seq_lens[row];
        const int64_t pg = wpos >= 0 ? wpos / a.bs : -1;
        if (pg >= 0 && pg < a.max_pages) {
          phys = a.block_table[row * a.bt_stride + pg];
          off = wpos % a.bs;
        }
        pos = a.positions ? a.positions[t] : wpos;
      }
    }
    pos_s[lane] = pos;
    phys_s[lane] = phys;
    off_s[lane] = static_cast<int>(off);
  }
  __syncthreads();
  // a = bf16((h * rms) * w), the input RMSNorm (qwen3/norm.py:22-26)
  auto chunk_store = [&](int c, const q3::u32x4& h, const q3::u32x4& n) {
    const int r = c / cpr, cc = c - r * cpr;
    const float rr = rms_s[r];
    q3::u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = q3::pack_bf16x2((q3::bf16_lo(h[e]) * rr) * q3::bf16_lo(n[e]),
                             (q3::bf16_hi(h[e]) * rr) * q3::bf16_hi(n[e]));
    *reinterpret_cast<q3::u32x4*>(a_s + r * pitch + 8 * cc) = o;
  };
#pragma unroll
  for (int i = 0; i < kPre; ++i)
    if (tid + i * kThreadsQ < nchunks) chunk_store(tid + i * kThreadsQ, hv[i], nv[i]);
  for (int c = tid + kPre * kThreadsQ; c < nchunks; c += kThreadsQ) {
    q3::u32x4 h, n;
    chunk_src(c, h, n);
    chunk_store(c, h, n);
  }
  __syncthreads();

  // A fragment of step s: lane L reads row L % 16, k = k0 + 32 s + 8 (L / 16).
  const uint16_t* arow = a_s + r16 * pitch + k0 + kg;
  q3::f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Buf& B, int s0) {
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      if (s0 + u >= steps) break;
      const q3::u32x4 av = *reinterpret_cast<const q3::u32x4*>(arow + (s0 + u) * kKStep);
      acc = q3::mfma16x16x32(q3::as_bf16x8(av), q3::as_bf16x8(to_mfma(B.b[u])), acc);
    }
  };
  for (int s0 = 0; s0 < steps; s0 += 2 * kC) {
    compute(p, s0);
    load(p, s0 + 2 * kC);
    compute(q, s0 + kC);
    load(q, s0 + 3 * kC);
  }

  // Sum the two halves of K in order (first half + second half) and round to
  // bf16, the projection's output type: y_s[token][column].
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[ct][i][lane] = acc[i];
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      y_s[4 * (lane >> 4) + i][ct * 16 + r16] = q3::bf16_bits(acc[i] + red[ct][i][lane]);
  }
  __syncthreads();

  // Finish the head: 16 lanes per token, 8 dims per lane (lane j: dims
  // 8j .. 8j+7), the pre-attention kernel's grouping.
  if (tid >= kRowsPerBlock * 16) return;
  const int r = tid >> 4, j = tid & 15;
  const int t = rb * 16 + r;
  if (t >= a.M) return;  // whole 16-lane groups
  const q3::u32x4 xw = *reinterpret_cast<const q3::u32x4*>(&y_s[r][8 * j]);
  const int64_t pos = pos_s[r], phys = phys_s[r];
  const int off = off_s[r];
  const bool ok_pos = pos >= 0 && pos < a.tab_rows;
  const bool write_pool = ok_pos && phys >= 0 && phys < a.num_blocks;
  const int kv_base = a.Hq + a.Hkv;
  if (head >= kv_base) {  // v: a bit-exact copy into the pool
    if (write_pool)
      q3::st16(a.v_cache + phys * a.vc[0] + static_cast<int64_t>(a.layer) * a.vc[1] +
                   static_cast<int64_t>(head - kv_base) * a.vc[2] + off * a.vc[3] + 8 * j,
               xw);
    return;
  }
  const uint16_t* wn = head < a.Hq ? a.q_w : a.k_w;
  const q3::u32x4 ww = q3::ld16(wn + 8 * j);
  float x[8], w[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = q3::bf16_lo(xw[e]);
    x[2 * e + 1] = q3::bf16_hi(xw[e]);
    w[2 * e] = q3::bf16_lo(ww[e]);
    w[2 * e + 1] = q3::bf16_hi(ww[e]);
  }
  float cv[8], sv[8];
  if (ok_pos) {
    const float* cr = a.cos_t + pos * a.tab_stride + 8 * j;
    const float* sr = a.sin_t + pos * a.tab_stride + 8 * j;
    const float4 c0 = *reinterpret_cast<const float4*>(cr);
    const float4 c1 = *reinterpret_cast<const float4*>(cr + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(sr);
    const float4 s1 = *reinterpret_cast<const float4*>(sr + 4);
    const float cc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float ss_[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cv[e] = round_bf16(cc[e]);  // cos / sin .to(q.dtype)
      sv[e] = round_bf16(ss_[e]);
    }
  }
  // Squares rounded, then summed (no fused multiply-add), as x.pow(2).mean().
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = __fadd_rn(ss, __fmul_rn(x[e], x[e]));
  ss = q3::row16_sum(ss);
  const float rmsh = 1.f / sqrtf(ss / static_cast<float>(kD) + a.head_eps);
  uint32_t np[4], pp[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    np[e] = q3::pack_bf16x2((x[2 * e] * rmsh) * w[2 * e], (x[2 * e + 1] * rmsh) * w[2 * e + 1]);
#pragma unroll
  for (int e = 0; e < 4; ++e) pp[e] = q3::dpp_u32<q3::kDppRor8>(np[e]);  // lane j ^ 8
  const float sign = j < 8 ? -1.f : 1.f;  // rotate_half: (-x2, x1)
  q3::u32x4 out = {0u, 0u, 0u, 0u};
  if (ok_pos) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float o[2];
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) {
        const int el = 2 * e + hl;
        const float n = hl ? q3::bf16_hi(np[e]) : q3::bf16_lo(np[e]);
        const float rh = sign * (hl ? q3::bf16_hi(pp[e]) : q3::bf16_lo(pp[e]));
        o[hl] = round_bf16(n * cv[el]) + round_bf16(rh * sv[el]);
      }
      out[e] = q3::pack_bf16x2(o[0], o[1]);
    }
  }
  if (head < a.Hq) {
    q3::st16(a.q_out + static_cast<int64_t>(t) * a.qo_s0 + static_cast<int64_t>(head) * a.qo_s1 +
                 8 * j,
             out);
  } else if (write_pool) {
    q3::st16(a.k_cache + phys * a.kc[0] + static_cast<int64_t>(a.layer) * a.kc[1] +
                 static_cast<int64_t>(head - a.Hq) * a.kc[2] + off * a.kc[3] + 8 * j,
             out);
  }
}

}  // namespace

extern "C" int qwen3_decode_qkv_rope_bf16(
    const void* h, int64_t h_row_stride, const float* ss_in, int ss_in_tiles,
    const void* norm_weight, float eps, const void* qkv_weight, int64_t weight_row_stride, int M,
    int K, int num_heads, int num_kv_heads, int head_dim, const void* q_norm_weight,
    const void* k_norm_weight, float head_eps, const float* cos_table, const float* sin_table,
    int64_t table_row_stride, int64_t table_rows, const int64_t* positions, void* q_out,
    const int64_t q_out_strides[2], void* k_cache, const int64_t k_cache_strides[4],
    void* v_cache, const int64_t v_cache_strides[4], int64_t num_blocks, int layer_idx,
    int num_layers,
    const int32_t* seq_lens, const int32_t* block_table, int64_t bt_row_stride, int64_t max_rows,
    int64_t max_pages, const int32_t* row_ids, int block_size, void* stream) {
  const char* who = "qwen3_decode_qkv_rope_bf16";
  if (!h || !ss_in || !norm_weight || !qkv_weight || !q_norm_weight || !k_norm_weight ||
      !cos_table || !sin_table || !q_out || !q_out_strides || !k_cache || !k_cache_strides ||
      !v_cache || !v_cache_strides || !seq_lens || !block_table)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (head_dim != kD)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: head_dim %d not supported (built for %d)", who,
                    head_dim, kD);
  if (M < 0 || M > kMaxRows || K <= 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      ss_in_tiles <= 0 || block_size <= 0 || num_blocks <= 0 || layer_idx < 0 ||
      layer_idx >= num_layers ||
      table_rows < 0 || max_rows <= 0 || max_pages <= 0 || bt_row_stride < max_pages ||
      !(eps >= 0.f) || !(head_eps >= 0.f))
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes (M must be <= %d)", who, kMaxRows);
  if (K % (kKParts * kKStep) != 0 || K > kMaxK)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: K must be a multiple of %d and <= %d", who,
                    kKParts * kKStep, kMaxK);
  bool ok = q3::aligned16(h) && q3::aligned16(ss_in) && q3::aligned16(norm_weight) &&
            q3::aligned16(qkv_weight) && q3::aligned16(q_norm_weight) &&
            q3::aligned16(k_norm_weight) && q3::aligned16(cos_table) &&
            q3::aligned16(sin_table) && q3::aligned16(q_out) && q3::aligned16(k_cache) &&
            q3::aligned16(v_cache) && h_row_stride % 8 == 0 && weight_row_stride % 8 == 0 &&
            ss_in_tiles % 4 == 0 && table_row_stride % 4 == 0;
  const int64_t strides[] = {q_out_strides[0], q_out_strides[1], k_cache_strides[0],
                             k_cache_strides[1], k_cache_strides[2], k_cache_strides[3],
                             v_cache_strides[0], v_cache_strides[1], v_cache_strides[2],
                             v_cache_strides[3]};
  for (int64_t s : strides) ok = ok && s % 8 == 0;
  if (!ok)
    return q3::fail(QWEN3_EALIGN, "%s: tensors need 16-byte aligned rows", who);
  if (M == 0) return QWEN3_OK;
  QkvArgs a{};
  a.h = static_cast<const uint16_t*>(h);
  a.h_s = h_row_stride;
  a.ss_in = ss_in;
  a.ss_tiles = ss_in_tiles;
  a.norm_w = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(qkv_weight);
  a.w_s = weight_row_stride;
  a.M = M;
  a.K = K;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.q_w = static_cast<const uint16_t*>(q_norm_weight);
  a.k_w = static_cast<const uint16_t*>(k_norm_weight);
  a.head_eps = head_eps;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.tab_stride = table_row_stride;
  a.tab_rows = table_rows;
  a.positions = positions;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.qo_s0 = q_out_strides[0];
  a.qo_s1 = q_out_strides[1];
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  for (int i = 0; i < 4; ++i) {
    a.kc[i] = k_cache_strides[i];
    a.vc[i] = v_cache_strides[i];
  }
  a.num_blocks = num_blocks;
  a.layer = layer_idx;
  a.seq_lens = seq_lens;
  a.block_table = block_table;
  a.bt_stride = bt_row_stride;
  a.max_rows = max_rows;
  a.max_pages = max_pages;
  a.row_ids = row_ids;
  a.bs = block_size;
  const int heads = num_heads + 2 * num_kv_heads;
  const int64_t blocks = q3::cdiv(heads, kXcds) * kXcds * ((M + 15) / 16);
  q3::clear_error();
  const size_t lds = static_cast<size_t>(kRowsPerBlock) * (K + 8) * sizeof(uint16_t);
  hipLaunchKernelGGL(qkv_rope_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreadsQ), lds,
                     static_cast<hipStream_t>(stream), a);
  return q3::launch_status(who);
}
