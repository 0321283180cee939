// Paged KV-cache slot writes: a bit-exact copy of new K/V head rows into the
// pool (num_blocks, num_layers, num_kv_heads, block_size, head_dim).
//
// One thread moves one 16-byte chunk (8 bf16) of one head row of K or V, so
// 16 consecutive lanes cover a 256-byte head row and every global access is a
// full dwordx4.  Three addressing forms share the kernel:
//   Decode — position from the resident seq_lens/block_table rows
//            (update_kv_batch_kernel, qwen3/kernels/paged_attention.py:324-350)
//   Range  — consecutive positions of one request through one block-table row
//            (PagedKVCache.update, qwen3/PagedKVcache.py:197-214)
//   Slots  — an explicit slot per token, negative = skip (batched prefill)
#include "common.hpp"

namespace {

enum class Form { Decode, Range, Slots };

struct KvWriteArgs {
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t kn_s0, kn_s1, vn_s0, vn_s1;  // item (batch/token) and head strides
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kc[4], vc[4];  // block, layer, head, slot strides
  int64_t num_blocks;
  int layer, num_layers;
  const int32_t* seq_lens;     // Decode
  const int32_t* block_table;  // Decode: full table; Range: one row
  int64_t bt_stride;           // Decode
  int64_t max_rows;            // Decode
  int64_t max_pages;           // pages addressable through one table row
  const int32_t* row_ids;      // Decode (nullable: identity)
  int64_t start_pos;           // Range
  const int64_t* slots;        // Slots
  int64_t n_items;             // B (Decode) or tokens (Range, Slots)
  int H, D, bs;
};

template <Form F, int VEC>
__global__ __launch_bounds__(256) void kv_write_kernel(KvWriteArgs a) {
  const int chunks = a.D / VEC;
  const int64_t per_item = static_cast<int64_t>(a.H) * 2 * chunks;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= a.n_items * per_item) return;
  const int64_t item = gid / per_item;
  int rem = static_cast<int>(gid - item * per_item);
  const int c = rem % chunks;
  rem /= chunks;
  const int is_v = rem & 1;
  const int h = rem >> 1;

  int64_t phys, off;
  if constexpr (F == Form::Decode) {
    const int64_t row = a.row_ids ? a.row_ids[item] : item;
    if (row < 0 || row >= a.max_rows) return;
    const int64_t pos = a.seq_lens[row];
    if (pos < 0) return;
    const int64_t pg = pos / a.bs;
    if (pg >= a.max_pages) return;
    phys = a.block_table[row * a.bt_stride + pg];
    off = pos % a.bs;
  } else if constexpr (F == Form::Range) {
    const int64_t pos = a.start_pos + item;
    const int64_t pg = pos / a.bs;
    if (pos < 0 || pg >= a.max_pages) return;
    phys = a.block_table[pg];
    off = pos % a.bs;
  } else {
    const int64_t slot = a.slots[item];
    if (slot < 0) return;
    phys = slot / a.bs;
    off = slot % a.bs;
  }
  if (phys < 0 || phys >= a.num_blocks) return;

  const uint16_t* src = is_v ? a.v_new + item * a.vn_s0 + h * a.vn_s1
                             : a.k_new + item * a.kn_s0 + h * a.kn_s1;
  const int64_t* cs = is_v ? a.vc : a.kc;
  uint16_t* dst = (is_v ? a.v_cache : a.k_cache) + phys * cs[0] +
                  static_cast<int64_t>(a.layer) * cs[1] + h * cs[2] + off * cs[3];
  src += c * VEC;
  dst += c * VEC;
  if constexpr (VEC == 8) {
    q3::st16(dst, q3::ld16(src));
  } else {
    *dst = *src;
  }
}

// The same copy when a head row is 2^lc 16-byte chunks and one item (2 H
// rows) is 2^li <= 256 chunks: a 256-thread workgroup moves 256 >> li whole
// items and every index is a shift instead of the general kernel's 64-bit
// division per chunk (the 66.5 MB write of an 8,115-token prefill: 13.9 ->
// 13.4 us back to back).
template <Form F>
__global__ __launch_bounds__(256) void kv_write_pow2_kernel(KvWriteArgs a, int lc, int li) {
  const int tid = threadIdx.x;
  const int64_t item = (static_cast<int64_t>(blockIdx.x) << (8 - li)) + (tid >> li);
  if (item >= a.n_items) return;
  const int rem = tid & ((1 << li) - 1);
  const int c = rem & ((1 << lc) - 1);
  const int is_v = (rem >> lc) & 1;
  const int h = rem >> (lc + 1);

  int64_t phys, off;
  if constexpr (F == Form::Decode) {
    const int64_t row = a.row_ids ? a.row_ids[item] : item;
    if (row < 0 || row >= a.max_rows) return;
    const int64_t pos = a.seq_lens[row];
    if (pos < 0) return;
    const int64_t pg = pos / a.bs;
    if (pg >= a.max_pages) return;
    phys = a.block_table[row * a.bt_stride + pg];
    off = pos % a.bs;
  } else if constexpr (F == Form::Range) {
    const int64_t pos = a.start_pos + item;
    const int64_t pg = pos / a.bs;
    if (pos < 0 || pg >= a.max_pages) return;
    phys = a.block_table[pg];
    off = pos % a.bs;
  } else {
    const int64_t slot = a.slots[item];
    if (slot < 0) return;
    phys = slot / a.bs;
    off = slot % a.bs;
  }
  if (phys < 0 || phys >= a.num_blocks) return;
  const uint16_t* src = is_v ? a.v_new + item * a.vn_s0 + h * a.vn_s1
                             : a.k_new + item * a.kn_s0 + h * a.kn_s1;
  const int64_t* cs = is_v ? a.vc : a.kc;
  uint16_t* dst = (is_v ? a.v_cache : a.k_cache) + phys * cs[0] +
                  static_cast<int64_t>(a.layer) * cs[1] + h * cs[2] + off * cs[3];
  q3::st16(dst + c * 8, q3::ld16(src + c * 8));
}

// One wave per item when an item is 64 x NPL chunks (NPL = 1, 2, 4, 8): the
// item's slot is looked up once, and each lane issues its NPL loads before
// its NPL stores, so a lane keeps NPL loads in flight (after a cache flush
// the copy is bound by load latency, not by bandwidth).
template <Form F, int NPL>
__global__ __launch_bounds__(256) void kv_write_wave_kernel(KvWriteArgs a, int lc) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= a.n_items) return;

  int64_t phys, off;
  if constexpr (F == Form::Decode) {
    const int64_t row = a.row_ids ? a.row_ids[item] : item;
    if (row < 0 || row >= a.max_rows) return;
    const int64_t pos = a.seq_lens[row];
    if (pos < 0) return;
    const int64_t pg = pos / a.bs;
    if (pg >= a.max_pages) return;
    phys = a.block_table[row * a.bt_stride + pg];
    off = pos % a.bs;
  } else if constexpr (F == Form::Range) {
    const int64_t pos = a.start_pos + item;
    const int64_t pg = pos / a.bs;
    if (pos < 0 || pg >= a.max_pages) return;
    phys = a.block_table[pg];
    off = pos % a.bs;
  } else {
    const int64_t slot = a.slots[item];
    if (slot < 0) return;
    phys = slot / a.bs;
    off = slot % a.bs;
  }
  if (phys < 0 || phys >= a.num_blocks) return;
  const uint16_t* k_src = a.k_new + item * a.kn_s0;
  const uint16_t* v_src = a.v_new + item * a.vn_s0;
  uint16_t* k_dst = a.k_cache + phys * a.kc[0] + static_cast<int64_t>(a.layer) * a.kc[1] + off * a.kc[3];
  uint16_t* v_dst = a.v_cache + phys * a.vc[0] + static_cast<int64_t>(a.layer) * a.vc[1] + off * a.vc[3];
  q3::u32x4 val[NPL];
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int cc = lane + 64 * k;  // chunk of the item: (head, k/v, 16-byte chunk)
    const int c = cc & ((1 << lc) - 1), is_v = (cc >> lc) & 1, h = cc >> (lc + 1);
    val[k] = q3::ld16((is_v ? v_src + h * a.vn_s1 : k_src + h * a.kn_s1) + c * 8);
  }
#pragma unroll
  for (int k = 0; k < NPL; ++k) {
    const int cc = lane + 64 * k;
    const int c = cc & ((1 << lc) - 1), is_v = (cc >> lc) & 1, h = cc >> (lc + 1);
    q3::st16((is_v ? v_dst + h * a.vc[2] : k_dst + h * a.kc[2]) + c * 8, val[k]);
  }
}

int log2_exact(int64_t x) {  // -1 unless x is a power of two
  if (x <= 0 || (x & (x - 1))) return -1;
  int l = 0;
  while ((int64_t{1} << l) < x) ++l;
  return l;
}

// Validates the arguments shared by the three forms and picks the vector
// width: 16-byte chunks when every base pointer and stride keeps 16-byte
// alignment, element copies otherwise.
int check_common(const KvWriteArgs& a, const char* who, bool* vec16) {
  if (!a.k_new || !a.v_new || !a.k_cache || !a.v_cache)
    return q3::fail(QWEN3_EINVAL, "%s: null tensor pointer", who);
  if (a.H <= 0 || a.D <= 0 || a.bs <= 0 || a.num_blocks <= 0 || a.layer < 0 ||
      a.layer >= a.num_layers)
    return q3::fail(QWEN3_EINVAL,
                    "%s: bad sizes (num_kv_heads=%d head_dim=%d block_size=%d "
                    "num_blocks=%lld layer=%d num_layers=%d)",
                    who, a.H, a.D, a.bs, (long long)a.num_blocks, a.layer, a.num_layers);
  bool ok = a.D % 8 == 0 && q3::aligned16(a.k_new) && q3::aligned16(a.v_new) &&
            q3::aligned16(a.k_cache) && q3::aligned16(a.v_cache);
  const int64_t strides[] = {a.kn_s0, a.kn_s1, a.vn_s0, a.vn_s1, a.kc[0], a.kc[1],
                             a.kc[2], a.kc[3], a.vc[0], a.vc[1], a.vc[2], a.vc[3]};
  for (int64_t s : strides) ok = ok && (s % 8 == 0);
  *vec16 = ok;
  return QWEN3_OK;
}

template <Form F>
int launch(const KvWriteArgs& a, void* stream, const char* who) {
  bool vec16 = false;
  int rc = check_common(a, who, &vec16);
  if (rc) return rc;
  if (a.n_items <= 0) return QWEN3_OK;
  const int chunks = vec16 ? a.D / 8 : a.D;
  const int64_t threads = a.n_items * a.H * 2 * chunks;
  const int64_t blocks = q3::cdiv(threads, 256);
  if (blocks > 0x7fffffff) return q3::fail(QWEN3_EINVAL, "%s: too many tokens", who);
  q3::clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int lc = log2_exact(a.D / 8), li = log2_exact(2 * static_cast<int64_t>(a.H) * (a.D / 8));
  if (vec16 && lc >= 0 && li >= 6 && li <= 9) {
    const int64_t wgs = q3::cdiv(a.n_items, int64_t{4});
    if (wgs > 0x7fffffff) return q3::fail(QWEN3_EINVAL, "%s: too many tokens", who);
    switch (li) {
      case 6: hipLaunchKernelGGL((kv_write_wave_kernel<F, 1>), dim3(wgs), dim3(256), 0, s, a, lc); break;
      case 7: hipLaunchKernelGGL((kv_write_wave_kernel<F, 2>), dim3(wgs), dim3(256), 0, s, a, lc); break;
      case 8: hipLaunchKernelGGL((kv_write_wave_kernel<F, 4>), dim3(wgs), dim3(256), 0, s, a, lc); break;
      default: hipLaunchKernelGGL((kv_write_wave_kernel<F, 8>), dim3(wgs), dim3(256), 0, s, a, lc); break;
    }
  } else if (vec16 && lc >= 0 && li >= 0 && li <= 8) {
    const int64_t wgs = q3::cdiv(a.n_items, int64_t{1} << (8 - li));
    hipLaunchKernelGGL((kv_write_pow2_kernel<F>), dim3(wgs), dim3(256), 0, s, a, lc, li);
  } else if (vec16)
    hipLaunchKernelGGL((kv_write_kernel<F, 8>), dim3(blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((kv_write_kernel<F, 1>), dim3(blocks), dim3(256), 0, s, a);
  return q3::launch_status(who);
}

void fill_cache(KvWriteArgs& a, const void* k_new, const int64_t* kns, const void* v_new,
                const int64_t* vns, void* k_cache, const int64_t* kcs, void* v_cache,
                const int64_t* vcs) {
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.kn_s0 = kns[0];
  a.kn_s1 = kns[1];
  a.vn_s0 = vns[0];
  a.vn_s1 = vns[1];
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  for (int i = 0; i < 4; ++i) {
    a.kc[i] = kcs[i];
    a.vc[i] = vcs[i];
  }
}

}  // namespace

extern "C" int qwen3_kv_write_decode_bf16(
    const void* k_new, const int64_t k_new_strides[2], const void* v_new,
    const int64_t v_new_strides[2], void* k_cache, const int64_t k_cache_strides[4],
    void* v_cache, const int64_t v_cache_strides[4], int64_t num_blocks, int layer_idx,
    int num_layers,
    const int32_t* seq_lens, const int32_t* block_table, int64_t bt_row_stride,
    int64_t max_rows, int64_t max_pages, const int32_t* row_ids, int B, int num_kv_heads,
    int head_dim, int block_size, void* stream) {
  const char* who = "qwen3_kv_write_decode_bf16";
  if (!k_new_strides || !v_new_strides || !k_cache_strides || !v_cache_strides)
    return q3::fail(QWEN3_EINVAL, "%s: null stride array", who);
  if (!seq_lens || !block_table)
    return q3::fail(QWEN3_EINVAL, "%s: null seq_lens/block_table", who);
  if (B < 0 || max_rows <= 0 || max_pages <= 0 || bt_row_stride < max_pages)
    return q3::fail(QWEN3_EINVAL,
                    "%s: bad table sizes (B=%d max_rows=%lld max_pages=%lld "
                    "bt_row_stride=%lld)",
                    who, B, (long long)max_rows, (long long)max_pages,
                    (long long)bt_row_stride);
  KvWriteArgs a{};
  fill_cache(a, k_new, k_new_strides, v_new, v_new_strides, k_cache, k_cache_strides,
             v_cache, v_cache_strides);
  a.num_blocks = num_blocks;
  a.layer = layer_idx;
  a.num_layers = num_layers;
  a.seq_lens = seq_lens;
  a.block_table = block_table;
  a.bt_stride = bt_row_stride;
  a.max_rows = max_rows;
  a.max_pages = max_pages;
  a.row_ids = row_ids;
  a.n_items = B;
  a.H = num_kv_heads;
  a.D = head_dim;
  a.bs = block_size;
  return launch<Form::Decode>(a, stream, who);
}

extern "C" int qwen3_kv_write_range_bf16(
    const void* k_new, const int64_t k_new_strides[2], const void* v_new,
    const int64_t v_new_strides[2], void* k_cache, const int64_t k_cache_strides[4],
    void* v_cache, const int64_t v_cache_strides[4], int64_t num_blocks, int layer_idx,
    int num_layers,
    const int32_t* block_table_row, int64_t row_pages, int64_t start_pos,
    int64_t num_tokens, int num_kv_heads, int head_dim, int block_size, void* stream) {
  const char* who = "qwen3_kv_write_range_bf16";
  if (!k_new_strides || !v_new_strides || !k_cache_strides || !v_cache_strides)
    return q3::fail(QWEN3_EINVAL, "%s: null stride array", who);
  if (!block_table_row || row_pages <= 0 || start_pos < 0 || num_tokens < 0)
    return q3::fail(QWEN3_EINVAL, "%s: bad table row (row_pages=%lld start=%lld n=%lld)",
                    who, (long long)row_pages, (long long)start_pos,
                    (long long)num_tokens);
  if (block_size > 0 && q3::cdiv(start_pos + num_tokens, block_size) > row_pages)
    return q3::fail(QWEN3_EINVAL,
                    "%s: positions [%lld, %lld) exceed the %lld pages of the row", who,
                    (long long)start_pos, (long long)(start_pos + num_tokens),
                    (long long)row_pages);
  KvWriteArgs a{};
  fill_cache(a, k_new, k_new_strides, v_new, v_new_strides, k_cache, k_cache_strides,
             v_cache, v_cache_strides);
  a.num_blocks = num_blocks;
  a.layer = layer_idx;
  a.num_layers = num_layers;
  a.block_table = block_table_row;
  a.max_pages = row_pages;
  a.start_pos = start_pos;
  a.n_items = num_tokens;
  a.H = num_kv_heads;
  a.D = head_dim;
  a.bs = block_size;
  return launch<Form::Range>(a, stream, who);
}

extern "C" int qwen3_kv_write_slots_bf16(
    const void* k_new, const int64_t k_new_strides[2], const void* v_new,
    const int64_t v_new_strides[2], void* k_cache, const int64_t k_cache_strides[4],
    void* v_cache, const int64_t v_cache_strides[4], int64_t num_blocks, int layer_idx,
    int num_layers,
    const int64_t* slot_mapping, int64_t num_tokens, int num_kv_heads, int head_dim,
    int block_size, void* stream) {
  const char* who = "qwen3_kv_write_slots_bf16";
  if (!k_new_strides || !v_new_strides || !k_cache_strides || !v_cache_strides)
    return q3::fail(QWEN3_EINVAL, "%s: null stride array", who);
  if (!slot_mapping || num_tokens < 0)
    return q3::fail(QWEN3_EINVAL, "%s: bad slot mapping", who);
  KvWriteArgs a{};
  fill_cache(a, k_new, k_new_strides, v_new, v_new_strides, k_cache, k_cache_strides,
             v_cache, v_cache_strides);
  a.num_blocks = num_blocks;
  a.layer = layer_idx;
  a.num_layers = num_layers;
  a.slots = slot_mapping;
  a.n_items = num_tokens;
  a.H = num_kv_heads;
  a.D = head_dim;
  a.bs = block_size;
  return launch<Form::Slots>(a, stream, who);
}
