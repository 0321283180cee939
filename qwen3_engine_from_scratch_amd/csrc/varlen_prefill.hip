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
//    sequence).  The head group holds HG query heads that share one KV
//    head (HG = the largest of 4, 2, 1 dividing G), so a K/V tile staged in
//    LDS serves every head of the group; each wave owns 32 query rows of one
//    head, and the tile covers 32 * 4 / HG rows.
//  * Query tiles are dispatched heaviest-first (the causal row tile with the
//    most keys is launched first) to shorten the ragged tail.
//  * Scores are computed transposed, S^T(32 keys x 32 queries) = K Q^T, with
//    mfma_f32_32x32x16_bf16, so each lane owns one query column and 16 of its
//    keys: the row max/sum needs one cross-lane step, and the S^T register
//    layout is directly the B operand (P^T) of O^T = V^T P^T.
//  * The V^T A-operand is assembled in-lane from 8-byte LDS reads of V rows
//    with byte permutes.  Causal blocks above the diagonal are skipped.
#include "common.hpp"

namespace {

constexpr int kD = 128;
constexpr int kBN = 64;             // keys per staged K/V tile
constexpr int kLds = kD + 8;        // padded LDS row (elements)
constexpr int kWaves = 4;

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
  int rows;      // query rows per head per workgroup (32 * kWaves / HG)
  int n_mtiles;  // grid.z
  float scale_log2;
  int causal;
};

__global__ __launch_bounds__(kWaves * 64) void varlen_prefill_kernel(PrefillArgs a) {
  const int seq = blockIdx.x;
  const int hg = blockIdx.y;
  const int mt = a.n_mtiles - 1 - static_cast<int>(blockIdx.z);  // heaviest first
  const int64_t start = a.cu[seq];
  const int64_t end = a.cu[seq + 1];
  if (start < 0 || end > a.total || end <= start) return;
  const int len = static_cast<int>(end - start);
  const int m0 = mt * a.rows;
  if (m0 >= len) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hl = lane >> 5;
  const int wph = kWaves / a.HG;  // waves per head
  const int head = hg * a.HG + wave / wph;
  const int kvh = (hg * a.HG) / a.G;
  const int q0 = m0 + (wave % wph) * 32;  // first query row of this wave
  const int qrow = q0 + l32;               // the query column this lane owns

  __shared__ uint16_t s_k[kBN * kLds];
  __shared__ uint16_t s_v[kBN * kLds];

  // Q^T as the B operand: lane (query l32, k-group hl), chunk c: dims
  // c*16 + 8*hl .. +7.
  q3::bf16x8 qv[8];
  {
    const bool ok = qrow < len;
    const uint16_t* qp = a.q + (start + qrow) * a.q_st + static_cast<int64_t>(head) * a.q_sh + 8 * hl;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      q3::u32x4 z = {0u, 0u, 0u, 0u};
      qv[c] = q3::as_bf16x8(ok ? q3::ld16(qp + c * 16) : z);
    }
  }

  float m_run = q3::kNegInf;
  float l_run = 0.f;
  q3::f32x16 acc[4];  // acc[db][r] = O[qrow][4*(8*(r/4) + 4*hl + r%4) + db]
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;

  const int kend = a.causal ? min(len, m0 + a.rows) : len;
  const int wave_last_q = min(q0 + 31, len - 1);
  const bool wave_active = q0 < len;

  for (int n0 = 0; n0 < kend; n0 += kBN) {
    // ---- stage K and V rows [n0, n0 + kBN) of KV head kvh into LDS ----
#pragma unroll
    for (int i = 0; i < (kBN * kD / 8) / (kWaves * 64); ++i) {
      const int idx = tid + i * kWaves * 64;
      const int r = idx / (kD / 8);
      const int c8 = (idx % (kD / 8)) * 8;
      q3::u32x4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
      if (n0 + r < len) {
        const int64_t t = start + n0 + r;
        kx = q3::ld16(a.k + t * a.k_st + static_cast<int64_t>(kvh) * a.k_sh + c8);
        vx = q3::ld16(a.v + t * a.v_st + static_cast<int64_t>(kvh) * a.v_sh + c8);
      }
      *reinterpret_cast<q3::u32x4*>(&s_k[r * kLds + c8]) = kx;
      *reinterpret_cast<q3::u32x4*>(&s_v[r * kLds + c8]) = vx;
    }
    __syncthreads();

    // Causal: the tile is entirely above this wave's last query row.
    const bool wave_skip = !wave_active || (a.causal && n0 > wave_last_q);
    if (!wave_skip) {
      // ---- S^T = K Q^T for two 32-key blocks ----
      q3::f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = 0.f;
        const uint16_t* kp = &s_k[(kb * 32 + l32) * kLds + 8 * hl];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const q3::bf16x8 kf = q3::as_bf16x8(*reinterpret_cast<const q3::u32x4*>(kp + c * 16));
          s[kb] = q3::mfma32x32x16(kf, qv[c], s[kb]);
        }
      }
      // ---- scale, mask, running max ----
      const bool need_mask = (n0 + kBN > len) || (a.causal && n0 + kBN - 1 > q0);
      float mx = q3::kNegInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[kb][r] * a.scale_log2;
          if (need_mask) {
            const int key = n0 + kb * 32 + 8 * (r / 4) + 4 * hl + (r % 4);
            const bool valid = key < len && (!a.causal || key <= qrow);
            x = valid ? x : q3::kNegInf;
          }
          s[kb][r] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, q3::shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == q3::kNegInf ? 0.f : m_new;
      const float alpha = q3::fast_exp2(m_run - m_use);
      m_run = m_new;
      float psum = 0.f;
      // P^T as B operands: chunk (kb, kc) takes registers 8*kc .. 8*kc+7.
      q3::bf16x8 p[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          float e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            e[i] = q3::fast_exp2(s[kb][8 * kc + i] - m_use);
            psum += e[i];
          }
          q3::u32x4 pk = {q3::pack_bf16x2(e[0], e[1]), q3::pack_bf16x2(e[2], e[3]),
                          q3::pack_bf16x2(e[4], e[5]), q3::pack_bf16x2(e[6], e[7])};
          p[kb][kc] = q3::as_bf16x8(pk);
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;

      // ---- O^T += V^T P^T ----
      // Chunk (kb, kc), element e pairs with key kb*32 + 16*kc + 8*(e/4) +
      // 4*hl + e%4; the A operand of dim block db is V[key][4*l32 + db].
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          q3::u32x2 vr[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int key = kb * 32 + 16 * kc + 8 * (e / 4) + 4 * hl + (e % 4);
            vr[e] = *reinterpret_cast<const q3::u32x2*>(&s_v[key * kLds + 4 * l32]);
          }
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const int w = db >> 1, h = db & 1;
            q3::u32x4 av = {q3::pick_halves(vr[0][w], vr[1][w], h),
                            q3::pick_halves(vr[2][w], vr[3][w], h),
                            q3::pick_halves(vr[4][w], vr[5][w], h),
                            q3::pick_halves(vr[6][w], vr[7][w], h)};
            acc[db] = q3::mfma32x32x16(q3::as_bf16x8(av), p[kb][kc], acc[db]);
          }
        }
    }
    __syncthreads();
  }

  if (!wave_active || qrow >= len) return;
  l_run += q3::shfl_xor(l_run, 32);
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  uint16_t* op = a.o + (start + qrow) * a.o_st + static_cast<int64_t>(head) * a.o_sh;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = 8 * (r / 4) + 4 * hl + (r % 4);
    q3::u32x2 w = {q3::pack_bf16x2(acc[0][r] * inv, acc[1][r] * inv),
                   q3::pack_bf16x2(acc[2][r] * inv, acc[3][r] * inv)};
    *reinterpret_cast<q3::u32x2*>(op + 4 * i) = w;
  }
}

}  // namespace

extern "C" int qwen3_varlen_prefill_bf16(const void* q, const int64_t q_strides[2],
                                         const void* k, const int64_t k_strides[2],
                                         const void* v, const int64_t v_strides[2], void* o,
                                         const int64_t o_strides[2], const int32_t* cu_seqlens,
                                         int num_seqs, int max_seqlen, int64_t total_tokens,
                                         int num_heads, int num_kv_heads, int head_dim,
                                         float scale, int causal, void* stream) {
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
  if (num_seqs > 0x7fffffff)
    return q3::fail(QWEN3_EINVAL, "%s: too many sequences", who);
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
  a.rows = 32 * kWaves / a.HG;
  a.n_mtiles = static_cast<int>(q3::cdiv(max_seqlen, a.rows));
  a.scale_log2 = scale * q3::kLog2e;
  a.causal = causal ? 1 : 0;
  const int groups = num_heads / a.HG;
  if (groups > 65535 || a.n_mtiles > 65535)
    return q3::fail(QWEN3_EINVAL, "%s: grid too large (heads %d, max_seqlen %d)", who,
                    num_heads, max_seqlen);

  q3::clear_error();
  hipLaunchKernelGGL(varlen_prefill_kernel, dim3(num_seqs, groups, a.n_mtiles),
                     dim3(kWaves * 64), 0, static_cast<hipStream_t>(stream), a);
  return q3::launch_status(who);
}
