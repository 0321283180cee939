// Decode-batch linear layers (M <= 64 rows) with the row-wise work around
// them folded in, so a decoder layer needs fewer launches:
//   prologue (optional)  A = RMSNorm(h): the residual stream h normalised
//                        with the row's rms, taken from per-16-column
//                        partial sums of squares written by the kernel that
//                        produced h, and the norm weight:
//                        a = bf16((h * rsqrt(mean(h^2) + eps)) * w)   (qwen3/norm.py:22-26)
//   epilogue             kStore:   y = bf16(acc)
//                        kResidual: o = bf16(acc); h' = bf16(res + o) stored to
//                                  res_out, plus h'^2 summed per 16-column tile
//                                  (qwen3/decoder.py:49,55)
//                        kSilu:    y = bf16(bf16(silu(bf16(gate))) * bf16(up)), gate
//                                  and up the two halves of the fused projection
//                                  (qwen3/mlp.py:31-36)
// Weights are nn.Linear's (N x K) row-major matrices, y = a @ W^T.
//
// Work split: one workgroup per (16 output columns, 16 rows) block (32
// columns for kSilu: the gate and up tiles of the same columns).  Its four
// waves (eight when K >= 2048) take an equal share of K each and stream
// their weight rows straight from HBM as the B operand of
// mfma_f32_16x16x32_bf16, with two register buffers of loads in flight.
// Loads are coalesced (a lane quad reads one row's 64-byte k-step) and
// redistributed into the operand layout with ds_bpermute.  The partial tiles
// are summed through LDS in wave order, so results are reproducible bit for
// bit.  The row blocks of one column tile are placed on the same XCD
// (workgroups are dealt to the 8 XCDs round-robin), so the tile's weights
// come from HBM once and from that XCD's L2 for the other row blocks.
#include "common.hpp"

namespace {

constexpr int kMaxRows = 64;
constexpr int kTile = 16;         // output columns per tile
constexpr int kKStep = 32;        // k per MFMA
constexpr int kMaxNormK = 8192;  // widest input a norm prologue stages in LDS
constexpr int kXcds = 8;          // XCDs of an MI355X; workgroup b runs on XCD b % 8

enum Epi : int { kStore = 0, kResidual = 1, kSilu = 2 };

struct LinArgs {
  const uint16_t* x;  // A rows (M x K): activations, or the residual stream h with a norm
  int64_t x_s;
  const float* ss_in;  // nullable: no norm; else (M x ss_in_tiles) partial sums of h^2
  int ss_in_tiles;
  const uint16_t* norm_w;
  float eps;
  const uint16_t* w;  // (N_w x K) weights
  int64_t w_s;
  uint16_t* y;  // kStore / kSilu output (M x N)
  int64_t y_s;
  const uint16_t* res;  // kResidual
  int64_t res_s;
  uint16_t* res_out;
  int64_t res_out_s;
  float* ss_out;  // kResidual: (M x N/16)
  int M, N, K;
  int up_row;  // kSilu: first weight row of the up half
};

__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(static_cast<uint32_t>(q3::bf16_bits(x)) << 16);
}
__device__ __forceinline__ uint16_t to_bf16(float x) { return q3::bf16_bits(x); }

template <bool kNorm, int kEpi, int kWaves>
__global__ __launch_bounds__(kWaves * 64) void decode_linear_kernel(LinArgs a) {
  constexpr int kCols = kEpi == kSilu ? 2 : 1;  // B tiles per workgroup
  constexpr int kC = 4;                         // k-steps per prefetch buffer
  __shared__ float rms_s[16];
  __shared__ float red[kWaves][kCols][4][64];
  __shared__ q3::u32x4 nw_s[kNorm ? kMaxNormK / 8 : 1];  // norm weight, staged once

  // (tile, row block) of this workgroup: the rbc row blocks of a tile share
  // one XCD (block b runs on XCD b % 8).
  const int rbc = (a.M + 15) >> 4;
  const int b = blockIdx.x;
  const int slot = b >> 3;
  const int tile = (slot / rbc) * kXcds + (b & (kXcds - 1));
  const int rb = slot % rbc;
  if (tile >= a.N / kTile) return;  // whole workgroup

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n0 = tile * kTile;
  const int r16 = lane & 15;
  const int kg = 8 * (lane >> 4);  // this lane's 8-element k-group within a step
  const int kw = a.K / kWaves;
  const int k0 = wave * kw;
  const int steps = kw / kKStep;

  // Loads are coalesced: the four lanes of a quad read one row's 64 bytes of
  // a k-step (lane l: row l / 4, k-group l % 4).  The MFMA operands want
  // lane L to hold row L % 16, k-group L / 16, so every loaded vector is
  // redistributed with ds_bpermute: lane L takes lane 4 * (L % 16) + L / 16.
  const int lrow = lane >> 2, lkg = 8 * (lane & 3);
  const int perm_addr = 4 * (4 * r16 + (lane >> 4));
  const uint16_t* wrow[kCols];
  wrow[0] = a.w + static_cast<int64_t>(n0 + lrow) * a.w_s + lkg + k0;
  if constexpr (kCols == 2)
    wrow[1] = a.w + static_cast<int64_t>(a.up_row + n0 + lrow) * a.w_s + lkg + k0;
  const int xr = min(rb * 16 + lrow, a.M - 1);  // rows past M repeat the last row
  const uint16_t* xrow = a.x + static_cast<int64_t>(xr) * a.x_s + lkg + k0;
  auto to_mfma = [&](q3::u32x4 v) {
    q3::u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(perm_addr, static_cast<int>(v[e])));
    return o;
  };

  // Two register buffers of kC k-steps: the loads of one are in flight while
  // the other feeds the MFMAs.
  struct Buf {
    q3::u32x4 b[kC][kCols];
    q3::u32x4 x[kC];
  };
  auto load = [&](Buf& B, int s0) {
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      if (s0 + u >= steps) break;
      const int k = (s0 + u) * kKStep;
#pragma unroll
      for (int c = 0; c < kCols; ++c) B.b[u][c] = q3::ld16(wrow[c] + k);
      B.x[u] = q3::ld16(xrow + k);
    }
  };
  Buf p, q;
  load(p, 0);
  load(q, kC);
  // The residual this lane's outputs add to (wave 0 runs the epilogue),
  // loaded now so its latency hides under the weight stream.
  uint32_t res_pre[4] = {0u, 0u, 0u, 0u};
  if constexpr (kEpi == kResidual) {
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rb * 16 + 4 * (lane >> 4) + i;
        if (row < a.M) res_pre[i] = a.res[static_cast<int64_t>(row) * a.res_s + n0 + r16];
      }
    }
  }
  if constexpr (kNorm) {
    for (int i = threadIdx.x; i < a.K / 8; i += kWaves * 64) nw_s[i] = q3::ld16(a.norm_w + 8 * i);
  }

  float rms = 0.f;
  if constexpr (kNorm) {
    // rms of this block's rows from the producer's per-tile partial sums:
    // four threads per row take every fourth tile, then a fixed butterfly,
    // so every workgroup gets the same value for a row.
    if (threadIdx.x < 64) {
      const int row = min(rb * 16 + static_cast<int>(threadIdx.x >> 2), a.M - 1);
      const int part = threadIdx.x & 3;
      const float* sp = a.ss_in + static_cast<int64_t>(row) * a.ss_in_tiles;
      float s = 0.f;
      if (a.ss_in_tiles == 64) {
        // hidden 1024: 16 tiles per thread as four float4 loads, all in flight
        float4 f[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) f[j] = reinterpret_cast<const float4*>(sp + 16 * part)[j];
#pragma unroll
        for (int j = 0; j < 4; ++j) s += ((f[j].x + f[j].y) + f[j].z) + f[j].w;
      } else {
        for (int t = part; t < a.ss_in_tiles; t += 4) s += sp[t];
      }
      s += q3::dpp_f32<q3::kDppXor1>(s);  // lane ^ 1
      s += q3::dpp_f32<q3::kDppXor2>(s);  // lane ^ 2
      if (part == 0) rms_s[threadIdx.x >> 2] = 1.f / sqrtf(s / static_cast<float>(a.K) + a.eps);
    }
    __syncthreads();
    rms = rms_s[r16];
  }

  q3::f32x4 acc[kCols];
#pragma unroll
  for (int c = 0; c < kCols; ++c) acc[c] = q3::f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Buf& B, int s0) {
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      if (s0 + u >= steps) break;
      q3::u32x4 av = to_mfma(B.x[u]);
      if constexpr (kNorm) {
        const q3::u32x4 nw = nw_s[(k0 + kg + (s0 + u) * kKStep) >> 3];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          av[e] = q3::pack_bf16x2((q3::bf16_lo(av[e]) * rms) * q3::bf16_lo(nw[e]),
                                  (q3::bf16_hi(av[e]) * rms) * q3::bf16_hi(nw[e]));
      }
#pragma unroll
      for (int c = 0; c < kCols; ++c)
        acc[c] = q3::mfma16x16x32(q3::as_bf16x8(av), q3::as_bf16x8(to_mfma(B.b[u][c])), acc[c]);
    }
  };
  for (int s0 = 0; s0 < steps; s0 += 2 * kC) {
    compute(p, s0);
    load(p, s0 + 2 * kC);
    compute(q, s0 + kC);
    load(q, s0 + 3 * kC);
  }

  // Cross-wave sum in wave order; wave 0 runs the epilogue.
#pragma unroll
  for (int c = 0; c < kCols; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][c][i][lane] = acc[c][i];
  __syncthreads();
  if (wave != 0) return;
  float v[kCols][4];
#pragma unroll
  for (int c = 0; c < kCols; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float t = red[0][c][i][lane];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) t += red[w][c][i][lane];
      v[c][i] = t;
    }

  // D layout: lane holds column r16, rows 4 * (lane >> 4) + i of the block.
  const int col = n0 + r16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = rb * 16 + 4 * (lane >> 4) + i;
    const bool live = row < a.M;
    if constexpr (kEpi == kStore) {
      if (live) a.y[static_cast<int64_t>(row) * a.y_s + col] = to_bf16(v[0][i]);
    } else if constexpr (kEpi == kSilu) {
      const float g = round_bf16(v[0][i]);
      const float u = round_bf16(v[1][i]);
      const float sg = round_bf16(g / (1.f + expf(-g)));
      if (live) a.y[static_cast<int64_t>(row) * a.y_s + col] = to_bf16(sg * u);
    } else {
      float h = 0.f;
      if (live) {
        const float o = round_bf16(v[0][i]);
        const float r = __uint_as_float(res_pre[i] << 16);
        h = round_bf16(r + o);
        a.res_out[static_cast<int64_t>(row) * a.res_out_s + col] = to_bf16(h);
      }
      float sq = __fmul_rn(h, h);
      sq = q3::row16_sum(sq);
      if (live && r16 == 0) a.ss_out[static_cast<int64_t>(row) * (a.N / kTile) + tile] = sq;
    }
  }
}

// The SwiGLU linear with its RMSNorm prologue for 17..64 rows: one
// 512-thread workgroup per 16 output columns holding every row.  The rows
// are normalised once into LDS (the row-block split above fetches the
// normalised activations once per (row block, column tile) pair: 3x the
// weight bytes of traffic per CU at 64 rows), the eight waves split K and
// stream the gate and up weight tiles, and their partial tiles meet in the
// same LDS space once the rows are no longer read.
constexpr int kWaves64 = 8;
constexpr int kMaxK64 = 1024;  // 64 x (K + 8) bf16 rows in LDS

__global__ __launch_bounds__(kWaves64 * 64) void gate_up64_kernel(LinArgs a) {
  extern __shared__ uint16_t a_s[];  // rows, then the cross-wave partial tiles
  __shared__ float rms_s[64];
  const int tile = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r16 = lane & 15;
  const int kg = 8 * (lane >> 4);
  const int pitch = a.K + 8;
  const int kw = a.K / kWaves64;
  const int k0 = wave * kw;
  const int steps = kw / kKStep;  // at most kMaxK64 / (8 x 32) = 4
  const int n0 = tile * kTile;

  // This wave's weight loads first: they do not depend on the rows.
  const int lrow = lane >> 2, lkg = 8 * (lane & 3);
  const int perm_addr = 4 * (4 * r16 + (lane >> 4));
  const uint16_t* wg = a.w + static_cast<int64_t>(n0 + lrow) * a.w_s + lkg + k0;
  const uint16_t* wu = a.w + static_cast<int64_t>(a.up_row + n0 + lrow) * a.w_s + lkg + k0;
  constexpr int kMaxSteps = kMaxK64 / (kWaves64 * kKStep);
  q3::u32x4 bg[kMaxSteps], bu[kMaxSteps];
#pragma unroll
  for (int u = 0; u < kMaxSteps; ++u) {
    if (u >= steps) break;
    bg[u] = q3::ld16(wg + u * kKStep);
    bu[u] = q3::ld16(wu + u * kKStep);
  }
  // The rows of h, all loads in flight before the rms is known: chunk c =
  // tid + i * threads of the 64 x K/8 16-byte chunks (at most 16 per thread
  // for K <= 1024).  When the thread count is a multiple of the chunks per
  // row, a thread's chunks share one column and so one norm-weight chunk.
  constexpr int kChunksPerThread = 16;
  const int cpr = a.K >> 3;
  const int nch = 64 * cpr;
  const bool one_col = (kWaves64 * 64) % cpr == 0;
  q3::u32x4 hv[kChunksPerThread];
  q3::u32x4 nv0 = {0u, 0u, 0u, 0u};
  if (one_col) nv0 = q3::ld16(a.norm_w + 8 * (tid % cpr));
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int c = tid + i * (kWaves64 * 64);
    if (c >= nch) break;
    const int r = c / cpr, cc = c - r * cpr;
    hv[i] = q3::ld16(a.x + static_cast<int64_t>(min(r, a.M - 1)) * a.x_s + 8 * cc);
  }
  // rms of every row from the producer's partial sums (as the kernel above)
  if (tid < 256) {
    const int row = min(tid >> 2, a.M - 1);
    const int part = tid & 3;
    const float* sp = a.ss_in + static_cast<int64_t>(row) * a.ss_in_tiles;
    float s = 0.f;
    if (a.ss_in_tiles == 64) {
      float4 f[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) f[j] = reinterpret_cast<const float4*>(sp + 16 * part)[j];
#pragma unroll
      for (int j = 0; j < 4; ++j) s += ((f[j].x + f[j].y) + f[j].z) + f[j].w;
    } else {
      for (int t = part; t < a.ss_in_tiles; t += 4) s += sp[t];
    }
    s += q3::dpp_f32<q3::kDppXor1>(s);  // lane ^ 1
    s += q3::dpp_f32<q3::kDppXor2>(s);  // lane ^ 2
    if (part == 0) rms_s[tid >> 2] = 1.f / sqrtf(s / static_cast<float>(a.K) + a.eps);
  }
  __syncthreads();
  // a = bf16((h * rms) * w) for 64 rows (rows past M repeat M - 1)
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int c = tid + i * (kWaves64 * 64);
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

  q3::f32x4 acc[4][2];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) acc[rb][0] = acc[rb][1] = q3::f32x4{0.f, 0.f, 0.f, 0.f};
  auto to_mfma = [&](q3::u32x4 v) {
    q3::u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(perm_addr, static_cast<int>(v[e])));
    return o;
  };
#pragma unroll
  for (int u = 0; u < kMaxSteps; ++u) {
    if (u >= steps) break;
    const q3::bf16x8 g = q3::as_bf16x8(to_mfma(bg[u]));
    const q3::bf16x8 up = q3::as_bf16x8(to_mfma(bu[u]));
    const int k = k0 + u * kKStep + kg;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const q3::bf16x8 av =
          q3::as_bf16x8(*reinterpret_cast<const q3::u32x4*>(a_s + (16 * rb + r16) * pitch + k));
      acc[rb][0] = q3::mfma16x16x32(av, g, acc[rb][0]);
      acc[rb][1] = q3::mfma16x16x32(av, up, acc[rb][1]);
    }
  }
  __syncthreads();  // the rows are no longer read: their space takes the partial tiles
  float* red = reinterpret_cast<float*>(a_s);  // [wave][rb][gate/up][4][64]
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(((wave * 4 + rb) * 2 + c) * 4 + i) * 64 + lane] = acc[rb][c][i];
  __syncthreads();
  // wave rb < 4 finishes row block rb: sum the eight partials in wave order
  if (wave >= 4) return;
  const int rb = wave;
  const int col = n0 + r16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float gsum = red[(((0 * 4 + rb) * 2 + 0) * 4 + i) * 64 + lane];
    float usum = red[(((0 * 4 + rb) * 2 + 1) * 4 + i) * 64 + lane];
#pragma unroll
    for (int w = 1; w < kWaves64; ++w) {
      gsum += red[(((w * 4 + rb) * 2 + 0) * 4 + i) * 64 + lane];
      usum += red[(((w * 4 + rb) * 2 + 1) * 4 + i) * 64 + lane];
    }
    const int row = 16 * rb + 4 * (lane >> 4) + i;
    if (row < a.M) {
      const float g = round_bf16(gsum);
      const float u = round_bf16(usum);
      const float sg = round_bf16(g / (1.f + expf(-g)));
      a.y[static_cast<int64_t>(row) * a.y_s + col] = to_bf16(sg * u);
    }
  }
}

// Embedding rows into the residual stream, with the per-16-column partial
// sums of squares the first layer's norm needs.  One wave per row; an id
// outside [0, vocab) gives a zero row.
__global__ __launch_bounds__(256) void embed_ss_kernel(const int64_t* ids, const uint16_t* emb,
                                                       int64_t emb_s, int64_t vocab, int hidden,
                                                       int M, uint16_t* h, int64_t h_s,
                                                       float* ss) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int lane = threadIdx.x & 63;
  const int64_t id = ids[row];
  const bool ok = id >= 0 && id < vocab;
  const int tiles = hidden / kTile;
  for (int t = lane; t < tiles; t += 64) {
    q3::u32x4 v0 = {0u, 0u, 0u, 0u}, v1 = {0u, 0u, 0u, 0u};
    if (ok) {
      v0 = q3::ld16(emb + id * emb_s + kTile * t);
      v1 = q3::ld16(emb + id * emb_s + kTile * t + 8);
    }
    q3::st16(h + static_cast<int64_t>(row) * h_s + kTile * t, v0);
    q3::st16(h + static_cast<int64_t>(row) * h_s + kTile * t + 8, v1);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = q3::bf16_lo(v0[e]), a1 = q3::bf16_hi(v0[e]);
      const float b0 = q3::bf16_lo(v1[e]), b1 = q3::bf16_hi(v1[e]);
      s = __fadd_rn(s, __fmul_rn(a0, a0));
      s = __fadd_rn(s, __fmul_rn(a1, a1));
      s = __fadd_rn(s, __fmul_rn(b0, b0));
      s = __fadd_rn(s, __fmul_rn(b1, b1));
    }
    ss[static_cast<int64_t>(row) * tiles + t] = s;
  }
}

}  // namespace

extern "C" int qwen3_decode_linear_bf16(const void* x, int64_t x_row_stride, const float* ss_in,
                                        int ss_in_tiles, const void* norm_weight, float eps,
                                        const void* weight, int64_t weight_row_stride, int M,
                                        int N, int K, int epilogue, void* y, int64_t y_row_stride,
                                        const void* residual, int64_t residual_row_stride,
                                        void* residual_out, int64_t residual_out_row_stride,
                                        float* ss_out, int up_row, void* stream) {
  const char* who = "qwen3_decode_linear_bf16";
  if (!x || !weight) return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (M < 0 || M > kMaxRows || N <= 0 || K <= 0)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes (M must be <= %d)", who, kMaxRows);
  if (N % kTile != 0 || K % (4 * kKStep) != 0)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: N must be a multiple of %d and K of %d", who, kTile,
                    4 * kKStep);
  if (epilogue < kStore || epilogue > kSilu)
    return q3::fail(QWEN3_EINVAL, "%s: unknown epilogue %d", who, epilogue);
  const bool norm = ss_in != nullptr;
  if (norm && (!norm_weight || ss_in_tiles <= 0 || !(eps >= 0.f)))
    return q3::fail(QWEN3_EINVAL, "%s: the norm prologue needs its weight and partial sums", who);
  if (norm && K > kMaxNormK)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: a norm prologue supports K <= %d", who, kMaxNormK);
  if ((epilogue != kResidual && !y) ||
      (epilogue == kResidual && (!residual || !residual_out || !ss_out)))
    return q3::fail(QWEN3_EINVAL, "%s: null output for this epilogue", who);
  if (epilogue == kSilu && up_row < N)
    return q3::fail(QWEN3_EINVAL, "%s: up half must start at or after row N", who);
  bool ok = q3::aligned16(x) && q3::aligned16(weight) && x_row_stride % 8 == 0 &&
            weight_row_stride % 8 == 0;
  if (norm) ok = ok && q3::aligned16(norm_weight) && q3::aligned16(ss_in) && ss_in_tiles % 4 == 0;
  if (!ok)
    return q3::fail(QWEN3_EALIGN, "%s: x / weight rows must be 16-byte aligned", who);
  const int tiles = N / kTile;
  if (M == 0) return QWEN3_OK;
  LinArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_s = x_row_stride;
  a.ss_in = ss_in;
  a.ss_in_tiles = ss_in_tiles;
  a.norm_w = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(weight);
  a.w_s = weight_row_stride;
  a.y = static_cast<uint16_t*>(y);
  a.y_s = y_row_stride;
  a.res = static_cast<const uint16_t*>(residual);
  a.res_s = residual_row_stride;
  a.res_out = static_cast<uint16_t*>(residual_out);
  a.res_out_s = residual_out_row_stride;
  a.ss_out = ss_out;
  a.M = M;
  a.N = N;
  a.K = K;
  a.up_row = up_row;
  q3::clear_error();
  auto s = static_cast<hipStream_t>(stream);
  if (epilogue == kSilu && norm && M > 16 && K <= kMaxK64 && K % (kWaves64 * kKStep) == 0) {
    // every row in one workgroup per column tile; the cross-wave partials
    // (8 x 4 x 2 x 4 x 64 floats) reuse the rows' LDS
    const size_t rows_lds = static_cast<size_t>(64) * (K + 8) * sizeof(uint16_t);
    const size_t red_lds = static_cast<size_t>(kWaves64) * 4 * 2 * 4 * 64 * sizeof(float);
    hipLaunchKernelGGL(gate_up64_kernel, dim3(static_cast<unsigned>(tiles)),
                       dim3(kWaves64 * 64), rows_lds > red_lds ? rows_lds : red_lds, s, a);
    return q3::launch_status(who);
  }
  // (tile, row block) pairs, tiles rounded up to a multiple of the XCD count
  const int64_t blocks = q3::cdiv(tiles, kXcds) * kXcds * ((M + 15) / 16);
  // Eight waves (each an eighth of K) once K reaches 2048, so no wave runs
  // more than three rounds of its double-buffered loads.
  const bool wide = K % (8 * kKStep) == 0 && K >= 2048;
  const dim3 grid(static_cast<unsigned>(blocks));
#define Q3_LAUNCH(NORM, EPI)                                                                  \
  do {                                                                                        \
    if (wide)                                                                                 \
      hipLaunchKernelGGL((decode_linear_kernel<NORM, EPI, 8>), grid, dim3(512), 0, s, a);     \
    else                                                                                      \
      hipLaunchKernelGGL((decode_linear_kernel<NORM, EPI, 4>), grid, dim3(256), 0, s, a);     \
  } while (0)
  if (norm) {
    if (epilogue == kStore) Q3_LAUNCH(true, kStore);
    else if (epilogue == kResidual) Q3_LAUNCH(true, kResidual);
    else Q3_LAUNCH(true, kSilu);
  } else {
    if (epilogue == kStore) Q3_LAUNCH(false, kStore);
    else if (epilogue == kResidual) Q3_LAUNCH(false, kResidual);
    else Q3_LAUNCH(false, kSilu);
  }
#undef Q3_LAUNCH
  return q3::launch_status(who);
}

extern "C" int qwen3_embed_ss_bf16(const int64_t* ids, const void* embedding,
                                   int64_t embedding_row_stride, int64_t vocab, int hidden, int M,
                                   void* h_out, int64_t h_row_stride, float* ss_out,
                                   void* stream) {
  const char* who = "qwen3_embed_ss_bf16";
  if (!ids || !embedding || !h_out || !ss_out)
    return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (M < 0 || vocab <= 0 || hidden <= 0) return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (hidden % kTile != 0)
    return q3::fail(QWEN3_EUNSUPPORTED, "%s: hidden must be a multiple of %d", who, kTile);
  if (!q3::aligned16(embedding) || !q3::aligned16(h_out) || embedding_row_stride % 8 != 0 ||
      h_row_stride % 8 != 0)
    return q3::fail(QWEN3_EALIGN, "%s: rows must be 16-byte aligned", who);
  if (M == 0) return QWEN3_OK;
  q3::clear_error();
  hipLaunchKernelGGL(embed_ss_kernel, dim3(static_cast<unsigned>(q3::cdiv(M, 4))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), ids,
                     static_cast<const uint16_t*>(embedding), embedding_row_stride, vocab, hidden,
                     M, static_cast<uint16_t*>(h_out), h_row_stride, ss_out);
  return q3::launch_status(who);
}
