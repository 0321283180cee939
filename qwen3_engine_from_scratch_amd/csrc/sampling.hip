// Token sampling on the GPU: temperature, top-k, top-p and a categorical
// draw per row of bf16 logits, the rule of sample_tokens
// (qwen3/sampling.py:112-178, 234-270):
//   temperature <= 0     greedy: the first index of the largest logit
//   otherwise            x = logit / temperature over the k largest logits
//                        (k = top_k, or all when top_k <= 0), sorted
//                        descending; position j is kept while the softmax
//                        mass before it is <= top_p (position 0 always);
//                        the token is argmax over kept positions of
//                        x + Gumbel noise, i.e. a draw from softmax(x)
//                        restricted to them.
// Ties in value are ordered by token index (lower first).  The random
// stream is this file's own (Philox4x32-10 keyed by seed and row, counter =
// token index / 4, one 32-bit draw per token), so draws are reproducible for
// a seed but are not the reference's stream; the distribution is the same.
//
// One 1024-thread workgroup per row, passes over the row (L2-resident after
// the first):
//   A  count histogram of the high 12 bits of the 16-bit order-preserving
//      key, and the maximum key
//   B  count histogram of the low 4 bits inside the top-k boundary bin ->
//      the exact k-th largest key and how many of its ties are kept
//   C  softmax mass histogram (high 12 bits) of the top-k set, and its total
//   D  low-4-bit mass histogram inside the top-p boundary bin -> the exact
//      top-p cut
//   E  Gumbel-max over the kept tokens
// 4096 high bins keep the LDS atomics of a wave mostly on distinct
// addresses (logits crowd into a few binades: 256 bins of sign + exponent
// would serialise them), and the boundary bins are found by a block-wide
// scan over four bins per thread.  A pass over the row costs far more than
// the work on it (one workgroup streams the whole row), so as soon as the
// tokens that can still be kept fit in LDS (the bins at or above the top-k
// boundary after A, or above the top-p boundary after C) the pass that finds
// the boundary also appends them to a candidate list, and the later passes
// and the draw run over that list; ranks among the ties at a partial cut come
// from the tie indices themselves.
// Masses are summed as 64-bit fixed point (2^40 per unit), so every
// histogram and the cut are independent of summation order.
#include "common.hpp"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr double kFix = 1099511627776.0;  // 2^40

// Order-preserving 16-bit key of a bf16 value (larger value, larger key);
// NaN maps below every number, so it is never sampled.
__device__ __forceinline__ uint32_t okey(uint32_t b) {
  if ((b & 0x7F80u) == 0x7F80u && (b & 0x7Fu)) return 0u;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}
__device__ __forceinline__ float key_value(uint32_t key) {
  const uint32_t b = (key & 0x8000u) ? (key & 0x7FFFu) : (~key & 0xFFFFu);
  return __uint_as_float(b << 16);
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC 2011): 10 rounds of the published multipliers and
// Weyl key increments.
__device__ __forceinline__ uint32_t mulhilo(uint32_t a, uint32_t b, uint32_t& hi) {
  const uint64_t p = static_cast<uint64_t>(a) * b;
  hi = static_cast<uint32_t>(p >> 32);
  return static_cast<uint32_t>(p);
}
__device__ __forceinline__ q3::u32x4 philox4(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                              uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0, hi1;
    const uint32_t lo0 = mulhilo(0xD2511F53u, c0, hi0);
    const uint32_t lo1 = mulhilo(0xCD9E8D57u, c2, hi1);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0, c1 = n1, c2 = n2, c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return q3::u32x4{c0, c1, c2, c3};
}
// The four 32-bit draws of tokens 4n .. 4n+3 of a row: one Philox block,
// counter (n, row, constant), key = seed.
__device__ __forceinline__ q3::u32x4 draws4(uint64_t seed, int64_t row, int64_t n) {
  return philox4(static_cast<uint32_t>(n), static_cast<uint32_t>(n >> 32),
                 static_cast<uint32_t>(row), 0x5EED5EEDu, static_cast<uint32_t>(seed),
                 static_cast<uint32_t>(seed >> 32));
}
// Standard Gumbel noise of a 32-bit draw: u in (0, 1), g = -log(-log u).
__device__ __forceinline__ float gumbel_of(uint32_t r) {
  const float u = (static_cast<float>(r >> 8) + 0.5f) * (1.f / 16777216.f);
  return -__logf(-__logf(u));
}

constexpr int kLoBits = 4;
constexpr int kLoBins = 1 << kLoBits;              // 16
constexpr int kHiBins = 1 << (16 - kLoBits);       // 4096
constexpr int kBinsPerThread = kHiBins / kThreads;  // 4
constexpr int kCap = 4096;  // candidate list entries

struct Shared {
  uint32_t cnt[kHiBins];
  unsigned long long mass[kHiBins];
  uint32_t lo_cnt[kLoBins];
  unsigned long long lo_mass[kLoBins];
  int wsum[kWaves];
  unsigned long long wmass[kWaves];
  uint32_t wmax[kWaves];
  unsigned long long best[kWaves];
  int sel_bin;
  unsigned long long sel_run;
  unsigned long long cand[kCap];  // candidate list: (key << 32) | token index
  uint32_t ties[kThreads];        // indices of the ties at the cut
  int ncand, nties;
  uint32_t idx_cut;
};

// Block-wide sums; every thread gets the result.
__device__ __forceinline__ int block_sum_int(int v, Shared& sh) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wsum[threadIdx.x >> 6] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += sh.wsum[w];
  return t;
}

// Exclusive block scan of per-thread counts in thread order; also returns
// the total.
__device__ __forceinline__ int block_scan_int(int v, int& total, Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  __syncthreads();
  if (lane == 63) sh.wsum[wave] = incl;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) before += sh.wsum[w];
    total += sh.wsum[w];
  }
  return before + incl - v;
}

// The same scan over 64-bit values.
__device__ __forceinline__ unsigned long long block_scan_u64(unsigned long long v,
                                                             unsigned long long& total,
                                                             Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  __syncthreads();
  if (lane == 63) sh.wmass[wave] = incl;
  __syncthreads();
  unsigned long long before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) before += sh.wmass[w];
    total += sh.wmass[w];
  }
  return before + incl - v;
}

// Visits the row in rounds of kThreads * 8 tokens: thread t gets tokens
// base + 8t .. base + 8t + 7 of each round (16-byte loads when aligned).  The
// loads of kBatch rounds are issued before any is used, so a pass over the
// row waits for memory once per batch rather than once per round.
template <bool kVec, typename F>
__device__ __forceinline__ void for_each_round(const uint16_t* p, int64_t vocab, F&& f) {
  constexpr int kBatch = kVec ? 8 : 2;  // element loads hold more registers
  const int64_t per_round = static_cast<int64_t>(kThreads) * 8;
  for (int64_t base = 0; base < vocab; base += per_round * kBatch) {
    q3::u32x4 v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t i0 = base + u * per_round + 8 * static_cast<int64_t>(threadIdx.x);
      if (kVec && i0 + 8 <= vocab) {
        v[u] = q3::ld16(p + i0);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = i0 + 2 * e < vocab ? p[i0 + 2 * e] : 0x7FC1u;  // NaN pad
          const uint32_t hi = i0 + 2 * e + 1 < vocab ? p[i0 + 2 * e + 1] : 0x7FC1u;
          v[u][e] = lo | (hi << 16);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t i0 = base + u * per_round + 8 * static_cast<int64_t>(threadIdx.x);
      if (base + u * per_round >= vocab) break;  // uniform: the round is past the row
      uint32_t b[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        b[2 * e] = v[u][e] & 0xFFFFu;
        b[2 * e + 1] = v[u][e] >> 16;
      }
      f(i0, b);
    }
  }
}

// Scans the low-bit count histogram from the top: returns the bin where the
// running count (starting at `above`) first reaches `need`, and the count
// strictly above that bin.
__device__ __forceinline__ int find_count_bin(const uint32_t* h, int64_t need, int64_t& above) {
  int64_t run = above;
  for (int bin = kLoBins - 1; bin >= 0; --bin) {
    if (run + h[bin] >= need) {
      above = run;
      return bin;
    }
    run += h[bin];
  }
  above = run;
  return 0;
}

// The same over the 4096 high bins, by the whole block: thread t sums bins
// 4095 - 4t .. 4092 - 4t, an exclusive scan gives the count above them, and
// the one thread whose range holds the crossing walks its four bins.  Every
// thread returns the bin and sets `above`; the histogram must hold at least
// `need` counts.
__device__ __forceinline__ int find_count_bin_block(const uint32_t* h, int64_t need,
                                                    int64_t& above, Shared& sh) {
  const int top = kHiBins - 1 - kBinsPerThread * static_cast<int>(threadIdx.x);
  int mine = 0;
#pragma unroll
  for (int j = 0; j < kBinsPerThread; ++j) mine += static_cast<int>(h[top - j]);
  int total;
  const int before = block_scan_int(mine, total, sh);
  int64_t run = before;
  if (run < need && need <= run + mine) {
#pragma unroll
    for (int j = 0; j < kBinsPerThread; ++j) {
      if (run + h[top - j] >= need) {
        sh.sel_bin = top - j;
        sh.sel_run = static_cast<unsigned long long>(run);
        break;
      }
      run += h[top - j];
    }
  }
  __syncthreads();
  above = static_cast<int64_t>(sh.sel_run);
  return sh.sel_bin;
}

// The top-p boundary over the 4096 high mass bins: limit = top_p x total
// (top_p clamped at 0), and the first bin from the top whose inclusive mass,
// converted to double, exceeds it (there is one when top_p < 1 and the total
// is positive).  Returns the bin, or -1, and sets `run` to the mass above
// it.  The same block-wide scan as find_count_bin_block; the caller has
// passed a barrier since the last read of sh.sel_bin.
__device__ __forceinline__ int find_mass_bin_block(const unsigned long long* m, float top_p,
                                                   double& limit, unsigned long long& run,
                                                   Shared& sh) {
  const int top = kHiBins - 1 - kBinsPerThread * static_cast<int>(threadIdx.x);
  unsigned long long mine = 0;
#pragma unroll
  for (int j = 0; j < kBinsPerThread; ++j) mine += m[top - j];
  if (threadIdx.x == 0) sh.sel_bin = -1;  // before the scan's barriers
  unsigned long long total;
  unsigned long long r = block_scan_u64(mine, total, sh);
  limit = static_cast<double>(fmaxf(top_p, 0.f)) * static_cast<double>(total);
  if (static_cast<double>(r) <= limit && static_cast<double>(r + mine) > limit) {
#pragma unroll
    for (int j = 0; j < kBinsPerThread; ++j) {
      if (static_cast<double>(r + m[top - j]) > limit) {
        sh.sel_bin = top - j;
        sh.sel_run = r;
        break;
      }
      r += m[top - j];
    }
  }
  __syncthreads();
  run = sh.sel_run;
  return sh.sel_bin;
}

template <bool kVec>
__global__ __launch_bounds__(kThreads) void sample_kernel(const uint16_t* logits, int64_t row_s,
                                                          int64_t vocab, const float* temperature,
                                                          const int32_t* top_k,
                                                          const float* top_p, uint64_t seed,
                                                          int64_t* out) {
  __shared__ Shared sh;
  const int64_t row = blockIdx.x;
  const uint16_t* p = logits + row * row_s;
  const float temp = temperature ? temperature[row] : 0.f;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;

  // ---- greedy -----------------------------------------------------------
  if (!(temp > 0.f)) {
    // first index of the largest value; NaN ranks highest, as torch.argmax
    unsigned long long bestk = 0;
    for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (i0 + e >= vocab) break;
        const uint32_t bb = b[e];
        const bool nan = (bb & 0x7F80u) == 0x7F80u && (bb & 0x7Fu);
        const uint32_t k = nan ? 0x10000u : okey(bb);
        const unsigned long long key =
            (static_cast<unsigned long long>(k + 1) << 32) | (~static_cast<uint32_t>(i0 + e));
        bestk = key > bestk ? key : bestk;
      }
    });
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const unsigned long long o = __shfl_xor(bestk, m, 64);
      bestk = o > bestk ? o : bestk;
    }
    if (lane == 0) sh.best[wave] = bestk;
    __syncthreads();
    if (tid == 0) {
      unsigned long long b = 0;
      for (int w = 0; w < kWaves; ++w) b = sh.best[w] > b ? sh.best[w] : b;
      out[row] = static_cast<int64_t>(~static_cast<uint32_t>(b));
    }
    return;
  }

  const int64_t kreq = top_k ? top_k[row] : 0;
  const int64_t k = (kreq <= 0 || kreq > vocab) ? vocab : kreq;
  const float pcut = top_p ? top_p[row] : 1.f;
  const bool use_p = pcut < 1.f;
  const float inv_t = 1.f / temp;

  // Appends (key, index) of the lanes where q holds to the candidate list:
  // one LDS atomic per wave.  Called by every lane of the wave.
  auto compact = [&](bool q, uint32_t key, int64_t idx) {
    const unsigned long long m = __ballot(q);
    if (m == 0ull) return;
    const int leader = __ffsll(static_cast<long long>(m)) - 1;
    int base = 0;
    if (lane == leader) base = atomicAdd(&sh.ncand, __popcll(m));
    base = __shfl(base, leader, 64);
    if (q) {
      const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
      if (pos < kCap)
        sh.cand[pos] = (static_cast<unsigned long long>(key) << 32) | static_cast<uint32_t>(idx);
    }
  };
  // Once the candidate list holds every token that can still be kept
  // (ncand >= 0), the later passes visit it instead of the row.
  int ncand = -1;
  auto visit = [&](auto&& f) {
    if (ncand >= 0) {
      for (int i = tid; i < ncand; i += kThreads) {
        const unsigned long long c = sh.cand[i];
        f(static_cast<uint32_t>(c >> 32), static_cast<int64_t>(static_cast<uint32_t>(c)));
      }
    } else {
      for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (i0 + e < vocab) f(okey(b[e]), i0 + e);
      });
    }
  };
  // Tokens of the high bins >= hb, from the pass-A histogram (every thread
  // gets the sum).
  auto count_from = [&](int hb) {
    const int top = kHiBins - 1 - kBinsPerThread * tid;
    int c = 0;
#pragma unroll
    for (int j = 0; j < kBinsPerThread; ++j) c += top - j >= hb ? static_cast<int>(sh.cnt[top - j]) : 0;
    return block_sum_int(c, sh);
  };
  auto finish_compaction = [&]() {
    __syncthreads();
    const int n = sh.ncand;
    ncand = n <= kCap ? n : -1;
  };

  // ---- A: high-bin counts and the maximum key ----------------------------
  for (int i = tid; i < kHiBins; i += kThreads) sh.cnt[i] = 0;
  if (tid < kLoBins) sh.lo_cnt[tid] = 0;
  if (tid == 0) sh.ncand = 0;
  __syncthreads();
  uint32_t kmax = 0;
  for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (i0 + e >= vocab) break;
      const uint32_t key = okey(b[e]);
      kmax = key > kmax ? key : kmax;
      atomicAdd(&sh.cnt[key >> kLoBits], 1u);
    }
  });
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint32_t o = __shfl_xor(kmax, m, 64);
    kmax = o > kmax ? o : kmax;
  }
  if (lane == 0) sh.wmax[wave] = kmax;
  __syncthreads();
  kmax = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) kmax = sh.wmax[w] > kmax ? sh.wmax[w] : kmax;
  const float xmax = key_value(kmax) * inv_t;

  // ---- B: exact k-th largest key (kk) and the ties of it kept (tk) ------
  uint32_t kk = 0;  // every key >= 0: with k == vocab nothing is cut
  int64_t tk = 0, kties = 0;
  if (k < vocab) {
    int64_t above = 0;
    const int hb = find_count_bin_block(sh.cnt, k, above, sh);
    // the tokens of bins >= hb hold the top-k list: keep them when they fit
    const bool keep_list = above + static_cast<int64_t>(sh.cnt[hb]) <= kCap;
    for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool valid = i0 + e < vocab;
        const uint32_t key = okey(b[e]);
        const int kb = static_cast<int>(key >> kLoBits);
        if (valid && kb == hb) atomicAdd(&sh.lo_cnt[key & (kLoBins - 1)], 1u);
        if (keep_list) compact(valid && kb >= hb, key, i0 + e);
      }
    });
    if (keep_list) finish_compaction();
    __syncthreads();
    const int lb = find_count_bin(sh.lo_cnt, k, above);
    kk = (static_cast<uint32_t>(hb) << kLoBits) | static_cast<uint32_t>(lb);
    kties = sh.lo_cnt[lb];
    tk = k - above;  // 1 <= tk <= kties
  }
  // membership in the top-k list before tie ranks: key > kk, or key == kk
  // with rank < tk (ranks in token order)

  // ---- C, D: the top-p cut over the top-k list ---------------------------
  // kc / tc: the final cut (key and ties kept at it); the kept list is the
  // first min(k, n_p) positions of the sorted top-k list.
  uint32_t kc = kk;
  int64_t tc = tk, cties = kties;
  if (use_p) {
    // masses of the top-k list; the ties at kk count only up to tk of them
    __syncthreads();
    for (int i = tid; i < kHiBins; i += kThreads) sh.mass[i] = 0ull;
    if (tid < kLoBins) {
      sh.lo_mass[tid] = 0ull;
      sh.lo_cnt[tid] = 0;
    }
    __syncthreads();
    const bool partial_k = k < vocab && tk < kties;
    const float wk = __expf(key_value(kk) * inv_t - xmax);
    visit([&](uint32_t key, int64_t) {
      if (key < kk || (partial_k && key == kk)) return;
      const float w = __expf(key_value(key) * inv_t - xmax);
      atomicAdd(&sh.mass[key >> kLoBits],
                static_cast<unsigned long long>(static_cast<double>(w) * kFix + 0.5));
    });
    __syncthreads();
    const unsigned long long wk_fix =
        static_cast<unsigned long long>(static_cast<double>(wk) * kFix + 0.5);
    if (partial_k && tid == 0) sh.mass[kk >> kLoBits] += wk_fix * static_cast<unsigned long long>(tk);
    __syncthreads();
    // high bins of the cut: the bin holding the first position whose mass
    // before it exceeds the limit
    double limit;
    unsigned long long above_hi;
    const int hb = find_mass_bin_block(sh.mass, pcut, limit, above_hi, sh);
    if (hb >= 0) {  // else a row without mass (all NaN): no cut
      auto lo_hist = [&](uint32_t key, int64_t) {
        if (static_cast<int>(key >> kLoBits) != hb || key < kk) return;
        atomicAdd(&sh.lo_cnt[key & (kLoBins - 1)], 1u);
        if (partial_k && key == kk) return;
        const float w = __expf(key_value(key) * inv_t - xmax);
        atomicAdd(&sh.lo_mass[key & (kLoBins - 1)],
                  static_cast<unsigned long long>(static_cast<double>(w) * kFix + 0.5));
      };
      if (ncand >= 0) {
        visit(lo_hist);
      } else {
        // the tokens that can be kept lie in bins >= hb: keep them when they fit
        const bool keep_list = count_from(hb) <= kCap;
        for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const bool valid = i0 + e < vocab;
            const uint32_t key = okey(b[e]);
            if (valid) lo_hist(key, i0 + e);
            if (keep_list)
              compact(valid && static_cast<int>(key >> kLoBits) >= hb && key >= kk, key, i0 + e);
          }
        });
        if (keep_list) finish_compaction();
      }
      __syncthreads();
      if (partial_k && static_cast<int>(kk >> kLoBits) == hb && tid == 0) {
        sh.lo_mass[kk & (kLoBins - 1)] += wk_fix * static_cast<unsigned long long>(tk);
        sh.lo_cnt[kk & (kLoBins - 1)] = static_cast<uint32_t>(tk);
      }
      __syncthreads();
      unsigned long long r2 = above_hi;
      for (int bin = kLoBins - 1; bin >= 0; --bin) {
        const unsigned long long m = sh.lo_mass[bin];
        if (sh.lo_cnt[bin] == 0) continue;
        if (static_cast<double>(r2 + m) > limit) {
          // ties at this key: keep rank r while the mass before it, r2 +
          // r * w, is within the limit (rank 0 of the list's first key is
          // always kept since r2 is then 0)
          const uint32_t key = (static_cast<uint32_t>(hb) << kLoBits) | static_cast<uint32_t>(bin);
          const unsigned long long w = m / sh.lo_cnt[bin];
          int64_t keep = 0;
          while (keep < static_cast<int64_t>(sh.lo_cnt[bin]) &&
                 static_cast<double>(r2 + w * static_cast<unsigned long long>(keep)) <= limit)
            ++keep;
          if (keep == 0) keep = 1;  // cannot happen unless rounding: keep the first
          // the top-p cut is inside the top-k list (its key >= kk)
          kc = key;
          cties = key == kk ? kties : sh.lo_cnt[bin];
          tc = key == kk ? (keep < tk ? keep : tk) : keep;
          break;
        }
        r2 += m;
      }
    }
  }

  // ---- E: Gumbel-max over the kept tokens ---------------------------------
  // kept: key > kc, or key == kc with tie rank < tc (no rank needed when all
  // ties are kept, or when the cut is at a key nothing ties with)
  const bool need_rank = tc < cties;
  unsigned long long bestk = 0;  // (ordered score, complemented index)
  auto offer = [&](uint32_t key, int64_t idx, uint32_t draw) {
    const float sc = key_value(key) * inv_t + gumbel_of(draw);
    const uint32_t sb = __float_as_uint(sc);
    const uint32_t so = (sb & 0x80000000u) ? ~sb : (sb | 0x80000000u);
    const unsigned long long c =
        (static_cast<unsigned long long>(so) << 32) | (~static_cast<uint32_t>(idx));
    bestk = c > bestk ? c : bestk;
  };
  if (ncand >= 0 && (!need_rank || cties <= kThreads)) {
    // from the candidate list; with a partial tie, the tc-th smallest index
    // of the ties at kc bounds the kept ones
    uint32_t idx_cut = 0xFFFFFFFFu;
    if (need_rank) {
      if (tid == 0) {
        sh.nties = 0;
        sh.idx_cut = 0xFFFFFFFFu;
      }
      __syncthreads();
      for (int i0 = 0; i0 < ncand; i0 += kThreads) {
        const int i = i0 + tid;
        const unsigned long long c = i < ncand ? sh.cand[i] : 0ull;
        const bool q = i < ncand && static_cast<uint32_t>(c >> 32) == kc;
        const unsigned long long m = __ballot(q);
        if (m == 0ull) continue;
        const int leader = __ffsll(static_cast<long long>(m)) - 1;
        int base = 0;
        if (lane == leader) base = atomicAdd(&sh.nties, __popcll(m));
        base = __shfl(base, leader, 64);
        if (q) {
          const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
          if (pos < kThreads) sh.ties[pos] = static_cast<uint32_t>(c);
        }
      }
      __syncthreads();
      const int nt = sh.nties < kThreads ? sh.nties : kThreads;
      if (tid < nt) {
        const uint32_t mine = sh.ties[tid];
        int rank = 0;
        for (int j = 0; j < nt; ++j) rank += sh.ties[j] < mine ? 1 : 0;
        if (rank == tc - 1) sh.idx_cut = mine;
      }
      __syncthreads();
      idx_cut = sh.idx_cut;
    }
    for (int i = tid; i < ncand; i += kThreads) {
      const unsigned long long c = sh.cand[i];
      const uint32_t key = static_cast<uint32_t>(c >> 32);
      const uint32_t idx = static_cast<uint32_t>(c);
      const bool kept = key > kc || (key == kc && idx <= idx_cut);
      if (!kept || key == 0) continue;
      offer(key, idx, draws4(seed, row, idx >> 2)[idx & 3]);
    }
  } else {
    int64_t ties_before = 0;
    for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b) {
      int rank0 = 0;
      if (need_rank) {
        int c = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) c += (i0 + e < vocab && okey(b[e]) == kc) ? 1 : 0;
        int total;
        rank0 = block_scan_int(c, total, sh);
        rank0 += static_cast<int>(ties_before);
        ties_before += total;
      }
      int r = rank0;
      bool kept[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t key = okey(b[e]);
        bool kp = key > kc;
        if (key == kc && i0 + e < vocab) {
          kp = !need_rank || r < tc;
          ++r;
        }
        kept[e] = kp && key != 0 && i0 + e < vocab;
      }
      // one Philox block per four tokens (i0 is a multiple of 8)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (!(kept[4 * h] || kept[4 * h + 1] || kept[4 * h + 2] || kept[4 * h + 3])) continue;
        const q3::u32x4 d = draws4(seed, row, (i0 >> 2) + h);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kept[4 * h + j]) offer(okey(b[4 * h + j]), i0 + 4 * h + j, d[j]);
      }
    });
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const unsigned long long o = __shfl_xor(bestk, m, 64);
    bestk = o > bestk ? o : bestk;
  }
  __syncthreads();
  if (lane == 0) sh.best[wave] = bestk;
  __syncthreads();
  if (tid == 0) {
    unsigned long long bb = 0;
    for (int w = 0; w < kWaves; ++w) bb = sh.best[w] > bb ? sh.best[w] : bb;
    out[row] = bb ? static_cast<int64_t>(~static_cast<uint32_t>(bb)) : 0;
  }
}

}  // namespace

extern "C" int qwen3_sample_bf16(const void* logits, int64_t row_stride, int64_t rows,
                                 int64_t vocab, const float* temperature, const int32_t* top_k,
                                 const float* top_p, uint64_t seed, int64_t* out, void* stream) {
  const char* who = "qwen3_sample_bf16";
  if (!logits || !out) return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (rows < 0 || rows > 0x7fffffff || vocab <= 0 || vocab > 0x7fffffff || row_stride < vocab)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (rows == 0) return QWEN3_OK;
  q3::clear_error();
  auto s = static_cast<hipStream_t>(stream);
  const auto lg = static_cast<const uint16_t*>(logits);
  if (q3::aligned16(logits) && row_stride % 8 == 0)
    hipLaunchKernelGGL(sample_kernel<true>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0,
                       s, lg, row_stride, vocab, temperature, top_k, top_p, seed, out);
  else
    hipLaunchKernelGGL(sample_kernel<false>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0,
                       s, lg, row_stride, vocab, temperature, top_k, top_p, seed, out);
  return q3::launch_status(who);
}
