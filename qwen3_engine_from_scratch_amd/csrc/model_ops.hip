// Row-wise model kernels around the attention path of a Qwen3 decoder step:
// fused residual add + RMSNorm (also the embedding lookup and the final-norm
// row selection), SiLU * up of the MLP, greedy (argmax) token selection, the
// device-side advance of the resident sequence lengths, and the batched
// page-in (table entries + zeroing) of newly allocated pool blocks.
//
// Arithmetic and roundings follow the reference modules:
//   residual add (qwen3/decoder.py:49,55):   h = bf16(residual + x)
//   RMSNorm (qwen3/norm.py:22-26):            n = bf16((fp32(h) * rsqrt(mean(h^2) + eps)) * w)
//   SwiGLU (qwen3/mlp.py:31-36):              y = bf16(bf16(silu(gate)) * up)
//   greedy sampling (qwen3/sampling.py:256-258): argmax, first index on ties
#include "common.hpp"

namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(static_cast<uint32_t>(q3::bf16_bits(x)) << 16);
}

// ---------------------------------------------------------------------------
// Residual add + RMSNorm: one wave per output row, 16-byte chunks, CPL chunks
// per lane (hidden <= 512 * CPL).
struct NormArgs {
  const uint16_t* x;      // nullable: no add
  int64_t x_s;
  const uint16_t* res;    // residual stream (or the embedding table)
  int64_t res_s;
  uint16_t* res_out;      // nullable: h is not stored
  int64_t res_out_s;
  const uint16_t* w;
  float eps;
  uint16_t* out;
  int64_t out_s;
  const int64_t* row_index;  // nullable: row i reads row i
  int64_t src_rows;          // rows addressable through row_index
  int64_t rows;
  int hidden;
};

template <int CPL>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(NormArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (i >= a.rows) return;  // whole waves leave together
  const int lane = threadIdx.x & (kWave - 1);
  int64_t r = i;
  bool valid = true;
  if (a.row_index) {
    r = a.row_index[i];
    valid = r >= 0 && r < a.src_rows;
  }
  const int nchunk = a.hidden >> 3;
  q3::u32x4 hv[CPL];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + kWave * c;
    hv[c] = q3::u32x4{0u, 0u, 0u, 0u};
    if (!valid || ch >= nchunk) continue;
    q3::u32x4 rv = q3::ld16(a.res + r * a.res_s + 8 * ch);
    if (a.x) {
      const q3::u32x4 xv = q3::ld16(a.x + r * a.x_s + 8 * ch);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        rv[e] = q3::pack_bf16x2(q3::bf16_lo(rv[e]) + q3::bf16_lo(xv[e]),
                                q3::bf16_hi(rv[e]) + q3::bf16_hi(xv[e]));
    }
    hv[c] = rv;
    // Squares rounded, then summed (no fused multiply-add), as h.pow(2).mean().
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = q3::bf16_lo(rv[e]), hi = q3::bf16_hi(rv[e]);
      ss = __fadd_rn(ss, __fmul_rn(lo, lo));
      ss = __fadd_rn(ss, __fmul_rn(hi, hi));
    }
  }
  // the xor butterfly over the wave's 64 lanes, with the same pairings (and
  // bits) from DPP and permlane swaps instead of LDS permutes
  ss = q3::sum_xor32(q3::sum_xor16(q3::row16_sum(ss)));
  const float rms = 1.f / sqrtf(ss / static_cast<float>(a.hidden) + a.eps);
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + kWave * c;
    if (ch >= nchunk) continue;
    const q3::u32x4 wv = q3::ld16(a.w + 8 * ch);
    q3::u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = q3::pack_bf16x2((q3::bf16_lo(hv[c][e]) * rms) * q3::bf16_lo(wv[e]),
                             (q3::bf16_hi(hv[c][e]) * rms) * q3::bf16_hi(wv[e]));
    q3::st16(a.out + i * a.out_s + 8 * ch, o);
    if (a.res_out) q3::st16(a.res_out + i * a.res_out_s + 8 * ch, hv[c]);
  }
}

// ---------------------------------------------------------------------------
// SwiGLU activation: out[r, j] = bf16(bf16(silu(g)) * u), g = gu[r, j],
// u = gu[r, inter + j].  One thread per 8 output elements.
struct SiluArgs {
  const uint16_t* gu;
  int64_t gu_s;
  uint16_t* out;
  int64_t out_s;
  int64_t rows;
  int inter;
};

__device__ __forceinline__ float silu(float g) { return g / (1.f + expf(-g)); }

__global__ __launch_bounds__(256) void silu_mul_kernel(SiluArgs a) {
  const int64_t chunks = a.inter >> 3;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= a.rows * chunks) return;
  const int64_t r = t / chunks;
  const int64_t ch = t - r * chunks;
  const q3::u32x4 g = q3::ld16(a.gu + r * a.gu_s + 8 * ch);
  const q3::u32x4 u = q3::ld16(a.gu + r * a.gu_s + a.inter + 8 * ch);
  q3::u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = q3::pack_bf16x2(round_bf16(silu(q3::bf16_lo(g[e]))) * q3::bf16_lo(u[e]),
                           round_bf16(silu(q3::bf16_hi(g[e]))) * q3::bf16_hi(u[e]));
  q3::st16(a.out + r * a.out_s + 8 * ch, o);
}

// ---------------------------------------------------------------------------
// Greedy selection: per row the index of the largest bf16 logit, the first
// one on ties, NaN ranking above every number (torch.argmax's order).  The
// comparison runs on a 64-bit key: the value's order-preserving integer in
// the high word, the complemented index in the low word, so the maximum key
// is the maximum value with the smallest index.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ uint64_t argmax_key(uint32_t bits16, uint32_t idx) {
  int32_t k;
  if ((bits16 & 0x7F80u) == 0x7F80u && (bits16 & 0x7Fu))
    k = 0x10000;  // NaN
  else
    k = (bits16 & 0x8000u) ? -static_cast<int32_t>(bits16 & 0x7FFFu)
                           : static_cast<int32_t>(bits16 & 0x7FFFu);
  return (static_cast<uint64_t>(static_cast<uint32_t>(k + 0x8000)) << 32) | (~idx);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max64(uint64_t v) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
    v = umax64(v, (static_cast<uint64_t>(hi) << 32) | lo);
  }
  return v;
}

template <bool kVec>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const uint16_t* logits,
                                                                int64_t row_s, int64_t vocab,
                                                                int64_t* out) {
  const int64_t row = blockIdx.x;
  const uint16_t* p = logits + row * row_s;
  uint64_t best = 0;  // below every real key
  if constexpr (kVec) {
    // eight 16-byte loads in flight per thread before any is used
    constexpr int kBatch = 8;
    const int64_t nvec = vocab >> 3;
    for (int64_t c0 = threadIdx.x; c0 < nvec; c0 += kArgmaxThreads * kBatch) {
      q3::u32x4 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t c = c0 + u * kArgmaxThreads;
        if (c < nvec) v[u] = q3::ld16(p + 8 * c);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t c = c0 + u * kArgmaxThreads;
        if (c >= nvec) break;
        const uint32_t base = static_cast<uint32_t>(8 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          best = umax64(best, argmax_key(v[u][e] & 0xFFFFu, base + 2 * e));
          best = umax64(best, argmax_key(v[u][e] >> 16, base + 2 * e + 1));
        }
      }
    }
  } else {
    for (int64_t c = threadIdx.x; c < vocab; c += kArgmaxThreads)
      best = umax64(best, argmax_key(p[c], static_cast<uint32_t>(c)));
  }
  best = wave_max64(best);
  __shared__ uint64_t part[kArgmaxThreads / kWave];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & (kWave - 1)) == 0) part[wave] = best;
  __syncthreads();
  if (wave == 0) {
    uint64_t v = (threadIdx.x < kArgmaxThreads / kWave) ? part[threadIdx.x] : 0;
    v = wave_max64(v);
    if (threadIdx.x == 0) out[row] = static_cast<int64_t>(~static_cast<uint32_t>(v));
  }
}

// ---------------------------------------------------------------------------
// seq_lens[row_ids[i]] += delta for every listed row except `skip_row` (the
// padding row of a captured batch, whose length stays put).  Listed rows
// other than skip_row must be distinct.
__global__ void advance_kernel(int32_t* seq_lens, int64_t max_rows, const int32_t* row_ids,
                               int n, int skip_row, int delta) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int r = row_ids[i];
  if (r == skip_row || r < 0 || r >= max_rows) return;
  seq_lens[r] += delta;
}

// Page-in of newly allocated pool blocks: entry i (rows[i], cols[i],
// blocks[i]) maps page cols[i] of resident-table row rows[i] to block
// blocks[i], whose K and V contents (every layer and head) are zeroed.
// Grid: (chunks of a block, entries, K/V).
constexpr int kPageThreads = 256;

__global__ __launch_bounds__(kPageThreads) void page_in_kernel(
    int32_t* table, int64_t stride, int64_t max_rows, int64_t max_pages,
    const int32_t* entries, int n, uint16_t* k_cache, uint16_t* v_cache, int64_t block_elems,
    int64_t num_blocks) {
  const int i = blockIdx.y;
  const int64_t row = entries[i], col = entries[n + i], blk = entries[2 * n + i];
  if (blk < 0 || blk >= num_blocks) return;
  if (blockIdx.x == 0 && blockIdx.z == 0 && threadIdx.x == 0 && row >= 0 && row < max_rows &&
      col >= 0 && col < max_pages)
    table[row * stride + col] = static_cast<int32_t>(blk);
  uint16_t* base = (blockIdx.z == 0 ? k_cache : v_cache) + blk * block_elems;
  const int64_t chunks = block_elems / 8;
  const q3::u32x4 z = {0u, 0u, 0u, 0u};
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kPageThreads + threadIdx.x; c < chunks;
       c += static_cast<int64_t>(gridDim.x) * kPageThreads)
    q3::st16(base + 8 * c, z);
}

}  // namespace

extern "C" int qwen3_page_in_bf16(int32_t* block_table, int64_t bt_row_stride, int64_t max_rows,
                                  int64_t max_pages, const int32_t* entries, int n,
                                  void* k_cache, void* v_cache, int64_t block_elems,
                                  int64_t num_blocks, void* stream) {
  const char* who = "qwen3_page_in_bf16";
  if (!block_table || !entries || !k_cache || !v_cache)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (n < 0 || n > 65535 || max_rows <= 0 || max_pages <= 0 || bt_row_stride < max_pages ||
      block_elems <= 0 || num_blocks <= 0)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (block_elems % 8 != 0 || !q3::aligned16(k_cache) || !q3::aligned16(v_cache))
    return q3::fail(QWEN3_EALIGN, "%s: blocks must be whole 16-byte chunks", who);
  if (n == 0) return QWEN3_OK;
  const int64_t chunks = block_elems / 8;
  const unsigned gx = static_cast<unsigned>(
      q3::cdiv(chunks, kPageThreads) < 64 ? q3::cdiv(chunks, kPageThreads) : 64);
  q3::clear_error();
  hipLaunchKernelGGL(page_in_kernel, dim3(gx, static_cast<unsigned>(n), 2), dim3(kPageThreads), 0,
                     static_cast<hipStream_t>(stream), block_table, bt_row_stride, max_rows,
                     max_pages, entries, n, static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), block_elems, num_blocks);
  return q3::launch_status(who);
}

extern "C" int qwen3_add_rms_norm_bf16(const void* x, int64_t x_row_stride, const void* residual,
                                       int64_t residual_row_stride, void* residual_out,
                                       int64_t residual_out_row_stride, const void* weight,
                                       float eps, void* out, int64_t out_row_stride,
                                       const int64_t* row_index, int64_t src_rows, int64_t rows,
                                       int hidden, void* stream) {
  const char* who = "qwen3_add_rms_norm_bf16";
  if (!residual || !weight || !out) return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (rows < 0 || hidden <= 0 || !(eps >= 0.f) || (row_index && src_rows <= 0))
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (hidden % 8 != 0 || hidden > 8 * kWave * 16)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: hidden %d must be a multiple of 8 and <= %d", who,
                    hidden, 8 * kWave * 16);
  bool ok = q3::aligned16(residual) && q3::aligned16(weight) && q3::aligned16(out) &&
            residual_row_stride % 8 == 0 && out_row_stride % 8 == 0;
  if (x) ok = ok && q3::aligned16(x) && x_row_stride % 8 == 0;
  if (residual_out) ok = ok && q3::aligned16(residual_out) && residual_out_row_stride % 8 == 0;
  if (!ok)
    return q3::fail(QWEN3_EALIGN, "%s: rows must be 16-byte aligned (strides multiple of 8)", who);
  if (rows == 0) return QWEN3_OK;
  NormArgs a{static_cast<const uint16_t*>(x),  x_row_stride,
             static_cast<const uint16_t*>(residual), residual_row_stride,
             static_cast<uint16_t*>(residual_out), residual_out_row_stride,
             static_cast<const uint16_t*>(weight), eps,
             static_cast<uint16_t*>(out), out_row_stride,
             row_index, src_rows, rows, hidden};
  const int64_t blocks = q3::cdiv(rows, 4);
  if (blocks > 0x7fffffff) return q3::fail(QWEN3_EINVAL, "%s: too many rows", who);
  const int cpl = static_cast<int>(q3::cdiv(hidden / 8, kWave));
  q3::clear_error();
  auto s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  if (cpl <= 1)
    hipLaunchKernelGGL(add_rms_norm_kernel<1>, grid, block, 0, s, a);
  else if (cpl <= 2)
    hipLaunchKernelGGL(add_rms_norm_kernel<2>, grid, block, 0, s, a);
  else if (cpl <= 4)
    hipLaunchKernelGGL(add_rms_norm_kernel<4>, grid, block, 0, s, a);
  else if (cpl <= 8)
    hipLaunchKernelGGL(add_rms_norm_kernel<8>, grid, block, 0, s, a);
  else
    hipLaunchKernelGGL(add_rms_norm_kernel<16>, grid, block, 0, s, a);
  return q3::launch_status(who);
}

extern "C" int qwen3_silu_mul_bf16(const void* gate_up, int64_t gate_up_row_stride, void* out,
                                   int64_t out_row_stride, int64_t rows, int intermediate,
                                   void* stream) {
  const char* who = "qwen3_silu_mul_bf16";
  if (!gate_up || !out) return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (rows < 0 || intermediate <= 0) return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (intermediate % 8 != 0)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: intermediate %d must be a multiple of 8", who,
                    intermediate);
  if (!q3::aligned16(gate_up) || !q3::aligned16(out) || gate_up_row_stride % 8 != 0 ||
      out_row_stride % 8 != 0)
    return q3::fail(QWEN3_EALIGN, "%s: rows must be 16-byte aligned (strides multiple of 8)", who);
  if (rows == 0) return QWEN3_OK;
  SiluArgs a{static_cast<const uint16_t*>(gate_up), gate_up_row_stride,
             static_cast<uint16_t*>(out), out_row_stride, rows, intermediate};
  const int64_t blocks = q3::cdiv(rows * (intermediate / 8), 256);
  if (blocks > 0x7fffffff) return q3::fail(QWEN3_EINVAL, "%s: too many rows", who);
  q3::clear_error();
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return q3::launch_status(who);
}

extern "C" int qwen3_argmax_bf16(const void* logits, int64_t row_stride, int64_t rows,
                                 int64_t vocab, int64_t* out, void* stream) {
  const char* who = "qwen3_argmax_bf16";
  if (!logits || !out) return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (rows < 0 || vocab <= 0 || vocab > 0xFFFFFFFFll || row_stride < vocab)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (rows > 0x7fffffff) return q3::fail(QWEN3_EINVAL, "%s: too many rows", who);
  if (rows == 0) return QWEN3_OK;
  q3::clear_error();
  auto s = static_cast<hipStream_t>(stream);
  const auto lg = static_cast<const uint16_t*>(logits);
  if (q3::aligned16(logits) && row_stride % 8 == 0 && vocab % 8 == 0)
    hipLaunchKernelGGL(argmax_kernel<true>, dim3(static_cast<unsigned>(rows)),
                       dim3(kArgmaxThreads), 0, s, lg, row_stride, vocab, out);
  else
    hipLaunchKernelGGL(argmax_kernel<false>, dim3(static_cast<unsigned>(rows)),
                       dim3(kArgmaxThreads), 0, s, lg, row_stride, vocab, out);
  return q3::launch_status(who);
}

extern "C" int qwen3_advance_seq_lens(int32_t* seq_lens, int64_t max_rows, const int32_t* row_ids,
                                      int n, int skip_row, int delta, void* stream) {
  const char* who = "qwen3_advance_seq_lens";
  if (!seq_lens || (!row_ids && n > 0))
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (n < 0 || max_rows <= 0) return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (n == 0) return QWEN3_OK;
  q3::clear_error();
  hipLaunchKernelGGL(advance_kernel, dim3(static_cast<unsigned>(q3::cdiv(n, 256))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), seq_lens, max_rows, row_ids, n, skip_row,
                     delta);
  return q3::launch_status(who);
}
