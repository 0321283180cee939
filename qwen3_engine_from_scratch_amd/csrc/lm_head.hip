// Greedy decode head: for up to 64 rows, the final RMSNorm of the residual
// stream, the lm_head projection over the whole vocabulary and each row's
// argmax, without writing the logits:
//   a = bf16((h * rsqrt(mean(h^2) + eps)) * w)      (qwen3/norm.py:22-26,
//                                                    rms from the producer's
//                                                    per-16-column sums)
//   logit[r][v] = bf16(a[r] . W[v])                 (qwen3/model.py:226-230)
//   token[r] = first v of the largest logit[r][v]   (torch.argmax; NaN ranks
//                                                    highest, as the argmax kernel)
//
// Work split: one 512-thread workgroup per CU.  It normalises the rows once
// into LDS, then its eight waves take vocabulary tiles of 16 rows of W in
// turn (tile t goes to wave t % (8 P) of the grid, so neighbouring tiles
// stream on different CUs and XCDs) and run each tile's whole K through
// mfma_f32_16x16x32_bf16 (A from LDS, B streamed from HBM with coalesced
// loads moved into the operand layout by ds_bpermute).  A tile's logits are
// rounded to bf16 and folded into (value, index) maxima that each lane keeps
// for the columns it computes; after the last tile the lanes and waves of a
// workgroup combine them into 64 row maxima in the workspace, and a
// one-workgroup pass reduces those per row.
#include "common.hpp"

namespace {

constexpr int kMaxRows = 64;
constexpr int kRowBlocks = kMaxRows / 16;
constexpr int kWavesH = 8;
constexpr int kThreadsH = kWavesH * 64;
constexpr int kKStep = 32;
constexpr int kC = 8;           // k-steps per load buffer
constexpr int kMaxK = 1024;     // staged rows: 64 x (K + 8) bf16 in LDS
constexpr int kMaxParts = 1024;  // workgroups the workspace holds maxima for

struct HeadArgs {
  const uint16_t* h;
  int64_t h_s;
  const float* ss;
  int ss_tiles;
  const uint16_t* norm_w;
  float eps;
  const uint16_t* w;
  int64_t w_s;
  int M, V, K;
  unsigned long long* part;  // [64][kMaxParts] row maxima of each workgroup
  int64_t* out;
};

// Argmax key of a bf16 value at column c: larger value, larger key; ties go
// to the smaller column; NaN above everything.
__device__ __forceinline__ unsigned long long head_key(uint32_t b, uint32_t col) {
  const bool nan = (b & 0x7F80u) == 0x7F80u && (b & 0x7Fu);
  const uint32_t k = nan ? 0x10000u : ((b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u));
  return (static_cast<unsigned long long>(k + 1) << 32) | (~col);
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

// Maximum over the 16 lanes of a DPP row (a maximum does not depend on
// the pairing; each step moves both halves of the key with DPP).
template <int kCtrl>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const uint32_t lo = q3::dpp_u32<kCtrl>(static_cast<uint32_t>(v));
  const uint32_t hi = q3::dpp_u32<kCtrl>(static_cast<uint32_t>(v >> 32));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}
__device__ __forceinline__ unsigned long long row16_max64(unsigned long long v) {
  v = umax64(v, dpp_u64<q3::kDppXor1>(v));
  v = umax64(v, dpp_u64<q3::kDppXor2>(v));
  v = umax64(v, dpp_u64<q3::kDppHalfMirror>(v));
  return umax64(v, dpp_u64<q3::kDppMirror>(v));
}

__global__ __launch_bounds__(kThreadsH) void lm_head_argmax_kernel(HeadArgs a) {
  extern __shared__ uint16_t a_s[];  // row r at a_s + r * pitch
  __shared__ float rms_s[kMaxRows];
  __shared__ unsigned long long red[kWavesH][kMaxRows];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int kg = 8 * (lane >> 4);
  const int pitch = a.K + 8;
  const int steps = a.K / kKStep;

  // The wave's first weight tile is requested before anything else: it does
  // not depend on the rows.
  const int lrow = lane >> 2, lkg = 8 * (lane & 3);
  const int tiles = (a.V + 15) >> 4;
  const int stride = gridDim.x * kWavesH;
  // Weight row of this lane for tile t (rows past V repeat the last, masked
  // in the epilogue).
  auto tile_row = [&](int t) {
    const int vrow = min(t * 16 + lrow, a.V - 1);
    return a.w + static_cast<int64_t>(vrow) * a.w_s + lkg;
  };
  q3::u32x4 bp[kC], bq[kC];
  auto load = [&](q3::u32x4 (&B)[kC], const uint16_t* wrow, int s0) {
#pragma unroll
    for (int u = 0; u < kC; ++u)
      if (s0 + u < steps) B[u] = q3::ld16(wrow + (s0 + u) * kKStep);
  };
  int t = blockIdx.x * kWavesH + wave;
  const uint16_t* wrow = tile_row(t < tiles ? t : 0);
  if (t < tiles) {
    load(bp, wrow, 0);
    load(bq, wrow, kC);
  }

  // The rows of h, all loads in flight before the rms is known: chunk c =
  // tid + i * threads of the 64 x K/8 16-byte chunks (at most 16 per thread
  // for K <= 1024).  When the thread count is a multiple of the chunks per
  // row, a thread's chunks share one column and so one norm-weight chunk.
  constexpr int kChunksPerThread = 16;
  const int cpr = a.K >> 3;
  const int nch = kMaxRows * cpr;
  const bool one_col = (kThreadsH) % cpr == 0;
  q3::u32x4 hv[kChunksPerThread];
  q3::u32x4 nv0 = {0u, 0u, 0u, 0u};
  if (one_col) nv0 = q3::ld16(a.norm_w + 8 * (tid % cpr));
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int c = tid + i * (kThreadsH);
    if (c >= nch) break;
    const int r = c / cpr, cc = c - r * cpr;
    hv[i] = q3::ld16(a.h + static_cast<int64_t>(min(r, a.M - 1)) * a.h_s + 8 * cc);
  }
  // ---- rms of every row (four lanes per row, as the decode linears) ----
  if (tid < 4 * kMaxRows) {
    const int row = min(tid >> 2, a.M - 1);
    const int part = tid & 3;
    const float* sp = a.ss + static_cast<int64_t>(row) * a.ss_tiles;
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
    if (part == 0) rms_s[tid >> 2] = 1.f / sqrtf(s / static_cast<float>(a.K) + a.eps);
  }
  __syncthreads();
  // a = bf16((h * rms) * w) for 64 rows (rows past M repeat M - 1)
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int c = tid + i * (kThreadsH);
    if (c >= nch) break;
    const int r = c / cpr, cc = c - r * cpr;
    const q3::u32x4 nv = one_col ? nv0 : q3::ld16(a.norm_w + 8 * cc);
    const float rr = rms_s[r];
    q3::u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = q3::pack_bf16x2((q3::bf16_lo(hv[i][e]) * rr) * q3::bf16_lo(nv[e]),
                             (q3::bf16_hi(hv[i][e]) * rr) * q3::bf16_hi(nv[e]));
    *reinterpret_cast<q3::u32x4*>(a_s + r * pitch + 8 * cc) = o;
  }
  __syncthreads();

  // ---- vocabulary tiles ----
  const int perm_addr = 4 * (4 * r16 + (lane >> 4));
  auto to_mfma = [&](q3::u32x4 v) {
    q3::u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(perm_addr, static_cast<int>(v[e])));
    return o;
  };
  unsigned long long best[kRowBlocks][4];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) best[rb][i] = 0ull;

  for (; t < tiles; t += stride) {
    // The loads run one tile ahead: the last steps of a tile issue the
    // first steps of the wave's next tile, so the stream never drains.
    const bool more = t + stride < tiles;
    const uint16_t* wnext = tile_row(more ? t + stride : t);
    q3::f32x4 acc[kRowBlocks];
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) acc[rb] = q3::f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const q3::u32x4 (&B)[kC], int s0) {
#pragma unroll
      for (int u = 0; u < kC; ++u) {
        if (s0 + u >= steps) break;
        const q3::bf16x8 bv = q3::as_bf16x8(to_mfma(B[u]));
        const int k = (s0 + u) * kKStep + kg;
#pragma unroll
        for (int rb = 0; rb < kRowBlocks; ++rb) {
          const q3::u32x4 av =
              *reinterpret_cast<const q3::u32x4*>(a_s + (16 * rb + r16) * pitch + k);
          acc[rb] = q3::mfma16x16x32(q3::as_bf16x8(av), bv, acc[rb]);
        }
      }
    };
    for (int s0 = 0; s0 < steps; s0 += 2 * kC) {
      const bool last = s0 + 2 * kC >= steps;  // steps is a multiple of 2 kC
      compute(bp, s0);
      if (!last) load(bp, wrow, s0 + 2 * kC);
      else if (more) load(bp, wnext, 0);
      compute(bq, s0 + kC);
      if (!last) load(bq, wrow, s0 + 3 * kC);
      else if (more) load(bq, wnext, kC);
    }
    const int v0 = t * 16;
    // D layout: lane holds column r16 of rows 4 (lane >> 4) + i of each block
    const uint32_t col = static_cast<uint32_t>(v0 + r16);
    const bool live = static_cast<int>(col) < a.V;
    // each lane keeps the best of the columns it computes; the 16 columns
    // of a tile meet only once, after the last tile
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned long long key = live ? head_key(q3::bf16_bits(acc[rb][i]), col) : 0ull;
        best[rb][i] = umax64(best[rb][i], key);
      }
    wrow = wnext;
  }

  // ---- the workgroup's row maxima ----
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      best[rb][i] = row16_max64(best[rb][i]);
  if (r16 == 0) {
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][16 * rb + 4 * (lane >> 4) + i] = best[rb][i];
  }
  __syncthreads();
  if (tid < kMaxRows) {
    unsigned long long b = red[0][tid];
#pragma unroll
    for (int w = 1; w < kWavesH; ++w) b = umax64(b, red[w][tid]);
    a.part[static_cast<int64_t>(tid) * kMaxParts + blockIdx.x] = b;
  }
}

// Reduces the per-workgroup maxima of every row (row-major in the
// workspace): one workgroup per row, one entry per thread.
constexpr int kFinishThreads = 256;
__global__ __launch_bounds__(kFinishThreads) void lm_head_argmax_finish_kernel(
    const unsigned long long* part, int parts, int64_t* out) {
  __shared__ unsigned long long wbest[kFinishThreads / 64];
  const int row = blockIdx.x;
  const unsigned long long* rp = part + static_cast<int64_t>(row) * kMaxParts;
  unsigned long long b = 0ull;
  for (int p = threadIdx.x; p < parts; p += kFinishThreads) b = umax64(b, rp[p]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) b = umax64(b, __shfl_xor(b, m, 64));
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kFinishThreads / 64; ++w) b = umax64(b, wbest[w]);
    out[row] = b ? static_cast<int64_t>(~static_cast<uint32_t>(b)) : 0;
  }
}

int cu_count_head() {
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

}  // namespace

extern "C" size_t qwen3_lm_head_argmax_workspace_bytes(void) {
  return static_cast<size_t>(kMaxParts) * kMaxRows * sizeof(unsigned long long);
}

extern "C" int qwen3_lm_head_argmax_bf16(const void* h, int64_t h_row_stride, const float* ss_in,
                                         int ss_in_tiles, const void* norm_weight, float eps,
                                         const void* weight, int64_t weight_row_stride, int M,
                                         int vocab, int K, void* workspace,
                                         size_t workspace_bytes, int64_t* out, void* stream) {
  const char* who = "qwen3_lm_head_argmax_bf16";
  if (!h || !ss_in || !norm_weight || !weight || !out || !workspace)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (M < 0 || M > kMaxRows || vocab <= 0 || K <= 0 || ss_in_tiles <= 0 || !(eps >= 0.f))
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes (M must be <= %d)", who, kMaxRows);
  if (K % (2 * kC * kKStep) != 0 || K > kMaxK)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: K must be a multiple of %d and <= %d", who,
                    2 * kC * kKStep, kMaxK);
  if (workspace_bytes < qwen3_lm_head_argmax_workspace_bytes())
    return q3::fail(QWEN3_EWORKSPACE, "%s: workspace of %zu bytes needed, %zu given", who,
                    qwen3_lm_head_argmax_workspace_bytes(), workspace_bytes);
  const bool ok = q3::aligned16(h) && q3::aligned16(ss_in) && q3::aligned16(norm_weight) &&
                  q3::aligned16(weight) && q3::aligned16(workspace) && h_row_stride % 8 == 0 &&
                  weight_row_stride % 8 == 0 && ss_in_tiles % 4 == 0;
  if (!ok) return q3::fail(QWEN3_EALIGN, "%s: tensors need 16-byte aligned rows", who);
  if (M == 0) return QWEN3_OK;
  int parts = cu_count_head();
  if (parts <= 0) return q3::fail(QWEN3_EINVAL, "%s: cannot query the device's CU count", who);
  parts = parts < kMaxParts ? parts : kMaxParts;
  HeadArgs a{};
  a.h = static_cast<const uint16_t*>(h);
  a.h_s = h_row_stride;
  a.ss = ss_in;
  a.ss_tiles = ss_in_tiles;
  a.norm_w = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(weight);
  a.w_s = weight_row_stride;
  a.M = M;
  a.V = vocab;
  a.K = K;
  a.part = static_cast<unsigned long long*>(workspace);
  a.out = out;
  q3::clear_error();
  auto s = static_cast<hipStream_t>(stream);
  const size_t lds = static_cast<size_t>(kMaxRows) * (K + 8) * sizeof(uint16_t);
  hipLaunchKernelGGL(lm_head_argmax_kernel, dim3(parts), dim3(kThreadsH), lds, s, a);
  const int rc = q3::launch_status(who);
  if (rc) return rc;
  hipLaunchKernelGGL(lm_head_argmax_finish_kernel, dim3(M), dim3(kFinishThreads), 0, s,
                     static_cast<const unsigned long long*>(workspace), parts, out);
  return q3::launch_status(who);
}
