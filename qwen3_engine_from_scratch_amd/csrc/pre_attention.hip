// Fused pre-attention step: per-head RMSNorm of q and k, rotary position
// embedding, and the K/V write into the paged pool — one kernel instead of
// the reference's q_norm, k_norm, apply_rotary_pos_emb and update_kv_batch
// (qwen3/attention.py:91-96 and qwen3/kernels/paged_attention.py:292-377).
//
// Arithmetic follows the reference step by step, with its roundings:
//   RMSNorm (qwen3/norm.py:22-26):  n = bf16((fp32(x) * rsqrt(mean(x^2) + eps)) * w)
//   RoPE (qwen3/rope.py:88-110):   c = bf16(cos[pos]), s = bf16(sin[pos]),
//                                   out = bf16(bf16(n * c) + bf16(rotate_half(n) * s))
//   rotate_half pairs element i with i + D/2 (qwen3/rope.py:72-85).
// The cos/sin tables are the caller's (the model's fp32 tables), so no
// transcendental is evaluated here.  Only the fp32 sum of squares may
// associate differently from the reference's reduction, which can move a
// value by one bf16 ulp.
//
// Layout: a 16-lane group handles up to four head rows of one token (D =
// 128: 8 bf16 per lane, one 16-byte load per row); the rotation partner of
// element e is e + 64, held by lane j ^ 8 at the same offset.  A token's rows
// are its q heads, k heads, then v heads (v rows are only copied into the
// pool).
#include "common.hpp"

namespace {

constexpr int kD = 128;
constexpr int kLanesPerRow = 16;
constexpr int kGroupsPerBlock = 256 / kLanesPerRow;

enum class Addr { Decode, Slots };

struct PreAttnArgs {
  const uint16_t* q;
  int64_t q_s0, q_s1;
  const uint16_t* k;
  int64_t k_s0, k_s1;
  const uint16_t* v;
  int64_t v_s0, v_s1;
  const uint16_t* q_w;
  const uint16_t* k_w;
  float eps;
  const float* cos_t;
  const float* sin_t;
  int64_t tab_stride, tab_rows;
  uint16_t* q_out;
  int64_t qo_s0, qo_s1;
  uint16_t* k_out;  // nullable
  int64_t ko_s0, ko_s1;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kc[4], vc[4];
  int64_t num_blocks;
  int layer, num_layers;
  // Decode addressing: position and slot from the resident tables.
  const int32_t* seq_lens;
  const int32_t* block_table;
  int64_t bt_stride, max_rows, max_pages;
  const int32_t* row_ids;  // nullable: identity
  const int64_t* rope_pos;  // nullable: RoPE at the write position seq_lens[row]
  // Slots addressing: explicit position and slot per token (slot < 0: no write).
  const int64_t* positions;
  const int64_t* slots;
  int64_t n_tokens;
  int Hq, Hkv, bs;
  int gpt_shift;  // log2 of the groups per token when a power of two, else -1
};

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(static_cast<uint32_t>(q3::bf16_bits(x)) << 16);
}

// Rows of one token handled by one 16-lane group: their loads are issued
// together, and the token's position, slot and cos/sin row are fetched
// once for all of them.
constexpr int kRowsPerGroup = 4;

template <Addr A>
__global__ __launch_bounds__(256) void pre_attention_kernel(PreAttnArgs a) {
  const int hr_count = a.Hq + 2 * a.Hkv;
  const int groups_per_token = (hr_count + kRowsPerGroup - 1) / kRowsPerGroup;
  // 32-bit group index (the host keeps tokens x groups below 2^31): a shift
  // or a 32-bit division instead of a 64-bit one.
  const uint32_t g = blockIdx.x * kGroupsPerBlock + (threadIdx.x >> 4);
  if (g >= static_cast<uint32_t>(a.n_tokens * groups_per_token)) return;  // whole groups leave
  const int j = threadIdx.x & (kLanesPerRow - 1);
  const uint32_t t32 = a.gpt_shift >= 0 ? g >> a.gpt_shift : g / groups_per_token;
  const int64_t t = t32;
  const int hr0 = static_cast<int>(g - t32 * groups_per_token) * kRowsPerGroup;
  const int nrows = min(kRowsPerGroup, hr_count - hr0);

  // This group's head rows first (independent of the position lookups).
  // The token's row bases are formed once; a row adds its head offset.
  const uint16_t* q_tok = a.q + t * a.q_s0;
  const uint16_t* k_tok = a.k + t * a.k_s0;
  const uint16_t* v_tok = a.v + t * a.v_s0;
  q3::u32x4 xw[kRowsPerGroup], ww[kRowsPerGroup];
#pragma unroll
  for (int i = 0; i < kRowsPerGroup; ++i) {
    const int hr = hr0 + i;
    if (i >= nrows) break;
    const uint16_t* src;
    if (hr < a.Hq) {
      src = q_tok + hr * a.q_s1;
      ww[i] = q3::ld16(a.q_w + 8 * j);
    } else if (hr < a.Hq + a.Hkv) {
      src = k_tok + (hr - a.Hq) * a.k_s1;
      ww[i] = q3::ld16(a.k_w + 8 * j);
    } else {
      src = v_tok + (hr - a.Hq - a.Hkv) * a.v_s1;
    }
    xw[i] = q3::ld16(src + 8 * j);
  }

  // Position (for RoPE) and pool slot of this token.
  int64_t pos = -1, phys = -1, off = 0;
  if constexpr (A == Addr::Decode) {
    const int64_t row = a.row_ids ? a.row_ids[t] : t;
    if (row >= 0 && row < a.max_rows) {
      const int64_t wpos = a.seq_lens[row];
      const int64_t pg = wpos >= 0 ? wpos / a.bs : -1;
      if (pg >= 0 && pg < a.max_pages) {
        phys = a.block_table[row * a.bt_stride + pg];
        off = wpos % a.bs;
      }
      pos = a.rope_pos ? a.rope_pos[t] : wpos;
    }
  } else {
    pos = a.positions[t];
    const int64_t slot = a.slots ? a.slots[t] : -1;
    if (slot >= 0) {
      phys = slot / a.bs;
      off = slot % a.bs;
    }
  }
  // A position outside the RoPE tables leaves the token's pool slot alone
  // (and its q/k rows zero).
  const bool ok_pos = pos >= 0 && pos < a.tab_rows;
  const bool write_pool = ok_pos && phys >= 0 && phys < a.num_blocks;
  const int64_t kc_tok = phys * a.kc[0] + static_cast<int64_t>(a.layer) * a.kc[1] + off * a.kc[3];
  const int64_t vc_tok = phys * a.vc[0] + static_cast<int64_t>(a.layer) * a.vc[1] + off * a.vc[3];

  float cv[8], sv[8];
  if (ok_pos && hr0 < a.Hq + a.Hkv) {
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
  // rotate_half: (-x2, x1).  The sign goes into this lane's sin values once
  // (sign * p * s == p * (sign * s) exactly).
  {
    const float sign = j < kLanesPerRow / 2 ? -1.f : 1.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sv[e] *= sign;
  }

#pragma unroll
  for (int i = 0; i < kRowsPerGroup; ++i) {
    if (i >= nrows) break;
    const int hr = hr0 + i;
    if (hr >= a.Hq + a.Hkv) {  // v row: bit-exact copy into the pool
      if (write_pool)
        q3::st16(a.v_cache + vc_tok + (hr - a.Hq - a.Hkv) * a.vc[2] + 8 * j, xw[i]);
      continue;
    }
    float x[8], w[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf_lo(xw[i][e]);
      x[2 * e + 1] = bf_hi(xw[i][e]);
      w[2 * e] = bf_lo(ww[i][e]);
      w[2 * e + 1] = bf_hi(ww[i][e]);
    }
    // Squares rounded, then summed (no fused multiply-add), as x.pow(2).mean().
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __fadd_rn(ss, __fmul_rn(x[e], x[e]));
    ss = q3::row16_sum(ss);
    // 1 / sqrt with IEEE sqrt and division: the hardware rsqrt's extra ulp
    // moves some outputs by two bf16 ulps from the reference's rsqrt.
    const float rms = 1.f / sqrtf(ss / static_cast<float>(kD) + a.eps);

    // n = bf16((x * rms) * w), packed as bf16 pairs for the partner exchange.
    uint32_t np[4], pp[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      np[e] = q3::pack_bf16x2((x[2 * e] * rms) * w[2 * e], (x[2 * e + 1] * rms) * w[2 * e + 1]);
#pragma unroll
    for (int e = 0; e < 4; ++e) pp[e] = q3::dpp_u32<q3::kDppRor8>(np[e]);  // lane j ^ 8

    q3::u32x4 out = {0u, 0u, 0u, 0u};
    if (ok_pos) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // bf16(n * c) and bf16(rotate_half(n) * s) for elements 2e, 2e + 1,
        // each pair rounded by one packed conversion
        const uint32_t nc = q3::pack_bf16x2(bf_lo(np[e]) * cv[2 * e], bf_hi(np[e]) * cv[2 * e + 1]);
        const uint32_t rs = q3::pack_bf16x2(bf_lo(pp[e]) * sv[2 * e], bf_hi(pp[e]) * sv[2 * e + 1]);
        out[e] = q3::pack_bf16x2(bf_lo(nc) + bf_lo(rs), bf_hi(nc) + bf_hi(rs));
      }
    }
    if (hr < a.Hq) {
      q3::st16(a.q_out + t * a.qo_s0 + hr * a.qo_s1 + 8 * j, out);
      continue;
    }
    const int h = hr - a.Hq;
    if (a.k_out) q3::st16(a.k_out + t * a.ko_s0 + h * a.ko_s1 + 8 * j, out);
    if (write_pool) q3::st16(a.k_cache + kc_tok + h * a.kc[2] + 8 * j, out);
  }
}

int check_args(const PreAttnArgs& a, int head_dim, const char* who) {
  if (!a.q || !a.k || !a.v || !a.q_w || !a.k_w || !a.cos_t || !a.sin_t || !a.q_out ||
      !a.k_cache || !a.v_cache)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (head_dim != kD)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: head_dim %d not supported (built for %d)", who,
                    head_dim, kD);
  if (a.Hq <= 0 || a.Hkv <= 0 || a.bs <= 0 || a.num_blocks <= 0 || a.layer < 0 ||
      a.layer >= a.num_layers || a.tab_rows < 0 || a.n_tokens < 0 || !(a.eps >= 0.f))
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  const void* ptrs[] = {a.q, a.k, a.v, a.q_w, a.k_w, a.cos_t, a.sin_t, a.q_out, a.k_cache,
                        a.v_cache};
  bool ok = true;
  for (const void* p : ptrs) ok = ok && q3::aligned16(p);
  if (a.k_out) ok = ok && q3::aligned16(a.k_out);
  const int64_t strides[] = {a.q_s0, a.q_s1, a.k_s0, a.k_s1, a.v_s0, a.v_s1, a.qo_s0, a.qo_s1,
                             a.ko_s0, a.ko_s1, a.kc[0], a.kc[1], a.kc[2], a.kc[3], a.vc[0],
                             a.vc[1], a.vc[2], a.vc[3]};
  for (int64_t s : strides) ok = ok && s % 8 == 0;
  ok = ok && a.tab_stride % 4 == 0;
  if (!ok)
    return q3::fail(QWEN3_EALIGN,
                    "%s: tensors need 16-byte aligned rows (bf16 strides multiple of 8, "
                    "cos/sin row stride multiple of 4)", who);
  return QWEN3_OK;
}

template <Addr A>
int launch(PreAttnArgs a, void* stream, const char* who) {
  if (a.n_tokens == 0) return QWEN3_OK;
  const int gpt = (a.Hq + 2 * a.Hkv + kRowsPerGroup - 1) / kRowsPerGroup;
  const int64_t groups = a.n_tokens * gpt;
  // The kernel indexes 16-lane groups with 32-bit integers.
  if (groups > 0x7fffffff - kGroupsPerBlock)
    return q3::fail(QWEN3_EINVAL, "%s: too many tokens", who);
  const int64_t blocks = q3::cdiv(groups, kGroupsPerBlock);
  a.gpt_shift = -1;
  for (int l = 0; l < 31; ++l)
    if ((1 << l) == gpt) a.gpt_shift = l;
  q3::clear_error();
  hipLaunchKernelGGL(pre_attention_kernel<A>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return q3::launch_status(who);
}

void fill_common(PreAttnArgs& a, const void* q, const int64_t q_strides[2], const void* k,
                 const int64_t k_strides[2], const void* v, const int64_t v_strides[2],
                 const void* q_weight, const void* k_weight, float eps, const float* cos_table,
                 const float* sin_table, int64_t table_row_stride, int64_t table_rows,
                 void* q_out, const int64_t q_out_strides[2], void* k_cache,
                 const int64_t k_cache_strides[4], void* v_cache,
                 const int64_t v_cache_strides[4], int64_t num_blocks, int layer_idx,
                 int num_layers, int num_heads, int num_kv_heads, int block_size) {
  a.q = static_cast<const uint16_t*>(q);
  a.q_s0 = q_strides[0];
  a.q_s1 = q_strides[1];
  a.k = static_cast<const uint16_t*>(k);
  a.k_s0 = k_strides[0];
  a.k_s1 = k_strides[1];
  a.v = static_cast<const uint16_t*>(v);
  a.v_s0 = v_strides[0];
  a.v_s1 = v_strides[1];
  a.q_w = static_cast<const uint16_t*>(q_weight);
  a.k_w = static_cast<const uint16_t*>(k_weight);
  a.eps = eps;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.tab_stride = table_row_stride;
  a.tab_rows = table_rows;
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
  a.num_layers = num_layers;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.bs = block_size;
}

}  // namespace

extern "C" int qwen3_qk_norm_rope_decode_bf16(
    const void* q, const int64_t q_strides[2], const void* k, const int64_t k_strides[2],
    const void* v, const int64_t v_strides[2], const void* q_weight, const void* k_weight,
    float eps, const float* cos_table, const float* sin_table, int64_t table_row_stride,
    int64_t table_rows, void* q_out, const int64_t q_out_strides[2], void* k_cache,
    const int64_t k_cache_strides[4], void* v_cache, const int64_t v_cache_strides[4],
    int64_t num_blocks, int layer_idx, int num_layers, const int32_t* seq_lens,
    const int32_t* block_table,
    int64_t bt_row_stride, int64_t max_rows, int64_t max_pages, const int32_t* row_ids,
    const int64_t* positions, int B, int num_heads, int num_kv_heads, int head_dim,
    int block_size, void* stream) {
  const char* who = "qwen3_qk_norm_rope_decode_bf16";
  if (!q_strides || !k_strides || !v_strides || !q_out_strides || !k_cache_strides ||
      !v_cache_strides || !seq_lens || !block_table)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (B < 0 || max_rows <= 0 || max_pages <= 0 || bt_row_stride < max_pages)
    return q3::fail(QWEN3_EINVAL, "%s: bad table sizes", who);
  PreAttnArgs a{};
  fill_common(a, q, q_strides, k, k_strides, v, v_strides, q_weight, k_weight, eps, cos_table,
              sin_table, table_row_stride, table_rows, q_out, q_out_strides, k_cache,
              k_cache_strides, v_cache, v_cache_strides, num_blocks, layer_idx, num_layers,
              num_heads, num_kv_heads, block_size);
  a.seq_lens = seq_lens;
  a.block_table = block_table;
  a.bt_stride = bt_row_stride;
  a.max_rows = max_rows;
  a.max_pages = max_pages;
  a.row_ids = row_ids;
  a.rope_pos = positions;
  a.n_tokens = B;
  if (int rc = check_args(a, head_dim, who)) return rc;
  return launch<Addr::Decode>(a, stream, who);
}

extern "C" int qwen3_qk_norm_rope_slots_bf16(
    const void* q, const int64_t q_strides[2], const void* k, const int64_t k_strides[2],
    const void* v, const int64_t v_strides[2], const void* q_weight, const void* k_weight,
    float eps, const float* cos_table, const float* sin_table, int64_t table_row_stride,
    int64_t table_rows, const int64_t* positions, const int64_t* slot_mapping, void* q_out,
    const int64_t q_out_strides[2], void* k_out, const int64_t k_out_strides[2], void* k_cache,
    const int64_t k_cache_strides[4], void* v_cache, const int64_t v_cache_strides[4],
    int64_t num_blocks, int layer_idx, int num_layers, int64_t num_tokens, int num_heads,
    int num_kv_heads, int head_dim, int block_size, void* stream) {
  const char* who = "qwen3_qk_norm_rope_slots_bf16";
  if (!q_strides || !k_strides || !v_strides || !q_out_strides || !k_cache_strides ||
      !v_cache_strides || !positions || (k_out && !k_out_strides))
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  PreAttnArgs a{};
  fill_common(a, q, q_strides, k, k_strides, v, v_strides, q_weight, k_weight, eps, cos_table,
              sin_table, table_row_stride, table_rows, q_out, q_out_strides, k_cache,
              k_cache_strides, v_cache, v_cache_strides, num_blocks, layer_idx, num_layers,
              num_heads, num_kv_heads, block_size);
  a.positions = positions;
  a.slots = slot_mapping;
  a.k_out = static_cast<uint16_t*>(k_out);
  if (k_out) {
    a.ko_s0 = k_out_strides[0];
    a.ko_s1 = k_out_strides[1];
  }
  a.n_tokens = num_tokens;
  if (int rc = check_args(a, head_dim, who)) return rc;
  return launch<Addr::Slots>(a, stream, who);
}
