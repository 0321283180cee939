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
//
// With a workspace (qwen3_sample_ws_bf16) and at most 128 rows, the row is
// first cut into P parts (P = 2..8, so rows x P workgroups fill the CUs),
// and each part's workgroup keeps its tokens at or above a key that k of
// them reach (the k-th largest of its threads' own maxima; the k-th
// largest token's high bin when k is above the thread count).  Every token
// at or above the row's k-th largest key is then kept: a part holding one
// below its own threshold holds k tokens above it, more than the row has.
// One workgroup per row then runs passes A to E over the concatenated lists
// instead of the row (or over the row when a list overflowed or top-k cuts
// nothing).  The lists hold the whole top-k list and every tie at its
// boundary, and no step depends on the order of the candidates, so the
// draws are the single workgroup's.  Greedy rows take each part's first
// maximum and then the first among the parts.
//
// The VALU is the limit of every pass (a wave64 instruction occupies its
// SIMD four cycles), so the per-token work is kept small: whole rounds of
// a thread's 8 tokens are tested without per-token bounds checks, a part's
// first pass takes only per-thread maxima on packed 16-bit keys (two tokens
// per instruction), and the list pass skips a round on its packed maximum.
#include <type_traits>

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
// The keys of a pair of bf16 (low and high half of x) without the NaN
// test: a number's key, NaN above +inf (positive sign) or below -inf
// (negative sign).  Two instructions for two tokens (a packed 16-bit
// arithmetic shift gives each negative half its flip mask).
typedef int16_t i16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t raw_keys2(uint32_t x) {
  const i16x2 sign = __builtin_bit_cast(i16x2, x) >> static_cast<int16_t>(15);
  return x ^ (__builtin_bit_cast(uint32_t, sign) | 0x80008000u);
}
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}
// The largest raw key of a whole round's 8 tokens (b as unpacked by the
// visitor).  Equal to the largest key unless the round holds a NaN: then it
// is above 0xFF80 (a positive NaN) or, with only negative NaNs above -inf's
// key 0x7F, below 0x7F.
__device__ __forceinline__ uint32_t round_raw_max(const uint32_t* b) {
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) m = max_u16x2(m, raw_keys2(b[2 * j] | (b[2 * j + 1] << 16)));
  return (m & 0xFFFFu) > (m >> 16) ? (m & 0xFFFFu) : (m >> 16);
}

// Greedy order: the same key with every NaN above every number (0xFFFF,
// which no number maps to), as torch.argmax ranks them.
__device__ __forceinline__ uint32_t gkey(uint32_t b) {
  return (b & 0x7FFFu) > 0x7F80u ? 0xFFFFu : ((b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u));
}
// One thread's greedy candidate among its 8 tokens i0 .. i0 + 7 of a round
// (those below n when the round is partial): (gkey + 1) << 32 | ~index of
// the first largest, 0 when none is valid.  The 8 are ranked on 19-bit
// packed keys (gkey << 3 | 7 - e: the lower e wins a tie) without a branch.
template <typename Full>
__device__ __forceinline__ unsigned long long greedy_round(int64_t i0, const uint32_t* b,
                                                          int64_t n, Full full) {
  uint32_t m = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t pk = (gkey(b[e]) << 3) | (7u - e);
    if (full || i0 + e < n) m = pk > m ? pk : m;
  }
  const uint32_t idx = static_cast<uint32_t>(i0) + (7u - (m & 7u));
  const unsigned long long c = (static_cast<unsigned long long>((m >> 3) + 1) << 32) | ~idx;
  return m ? c : 0ull;
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

// One part's results of the parallel passes (one per row and part, in the
// workspace).
struct alignas(16) PartOut {
  uint32_t kmax;                  // the part's largest key (kmax, ncand: one 8-byte load)
  int32_t ncand;                  // candidates written, -1 none
  unsigned long long best;        // greedy rows: (key + 1) << 32 | ~index, the first maximum
  unsigned long long cand[kCap];  // (key << 32) | token index
};

// Parts per row of the parallel form: about one workgroup per CU over the
// batch (four parts for 64 rows measured best on 256 CUs: 44 us against
// 55 for two and 65 for eight), each part at least one round (kThreads * 8
// tokens); 1 means the single-workgroup form.
constexpr int kMaxParts = 8;
__host__ __device__ inline int parts_for(int64_t rows, int64_t vocab) {
  int p = rows <= 32 ? kMaxParts : rows <= 64 ? 4 : rows <= 128 ? 2 : 1;
  const int64_t rounds = (vocab + kThreads * 8 - 1) / (kThreads * 8);
  return static_cast<int>(p < rounds ? p : rounds);
}
// Tokens [lo, hi) of part c: whole rounds, the last part takes the rest.
__device__ __forceinline__ void part_range(int64_t vocab, int P, int c, int64_t& lo, int64_t& hi) {
  const int64_t per = kThreads * 8;
  const int64_t rounds = (vocab + per - 1) / per;
  const int64_t rp = (rounds + P - 1) / P;
  lo = c * rp * per;
  hi = lo + rp * per < vocab ? lo + rp * per : vocab;
  if (lo > vocab) lo = vocab;
}

// Block-wide maximum; every thread gets the result.
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, Shared& sh) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const unsigned long long o = __shfl_xor(v, m, 64);
    v = o > v ? o : v;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.best[threadIdx.x >> 6] = v;
  __syncthreads();
  // lane w of every wave takes wave w's maximum: four steps instead of a
  // sixteen-entry loop in every thread
  const int lane = threadIdx.x & 63;
  v = lane < kWaves ? sh.best[lane] : 0ull;
#pragma unroll
  for (int m = 1; m < kWaves; m <<= 1) {
    const unsigned long long o = __shfl_xor(v, m, 64);
    v = o > v ? o : v;
  }
  return __shfl(v, 0, 64);
}

// Appends (key, index) of the lanes where q holds to the block's candidate
// list (sh.cand, sh.ncand; entries past kCap are counted, not stored): one
// LDS atomic per wave.  Called by every lane of the wave.
__device__ __forceinline__ void append_candidate(bool q, uint32_t key, int64_t idx, Shared& sh) {
  const int lane = threadIdx.x & 63;
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
}

// The same for the tokens i0 + e of a thread's round where q[e] holds
// (keys[e] their keys): a wave prefix sum places them, one LDS atomic per
// wave.  Called by every lane of the wave.
__device__ __forceinline__ void append_round(const bool (&q)[8], const uint32_t (&keys)[8],
                                             int64_t i0, Shared& sh) {
  const int lane = threadIdx.x & 63;
  int c = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) c += q[e] ? 1 : 0;
  int incl = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  int base = 0;
  if (lane == 63) base = atomicAdd(&sh.ncand, incl);
  int pos = __shfl(base, 63, 64) + incl - c;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (!q[e]) continue;
    if (pos < kCap)
      sh.cand[pos] = (static_cast<unsigned long long>(keys[e]) << 32) | static_cast<uint32_t>(i0 + e);
    ++pos;
  }
}

// The waves' partials (part[w] of wave w, in LDS) combined in one wave:
// lane w takes part[w], a four-step scan gives every wave the sum of the
// waves before it and the total (instead of a sixteen-entry loop in every
// thread).
template <typename T>
__device__ __forceinline__ void scan_waves(const T* part, T& before, T& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const T x = lane < kWaves ? part[lane] : T(0);
  T incl = x;
#pragma unroll
  for (int o = 1; o < kWaves; o <<= 1) {
    const T y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  total = __shfl(incl, kWaves - 1, 64);
  before = __shfl(incl - x, wave, 64);
}

// Block-wide sums; every thread gets the result.
__device__ __forceinline__ int block_sum_int(int v, Shared& sh) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wsum[threadIdx.x >> 6] = v;
  __syncthreads();
  int before, t;
  scan_waves(sh.wsum, before, t);
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
  int before;
  scan_waves(sh.wsum, before, total);
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
  unsigned long long before;
  scan_waves(sh.wmass, before, total);
  return before + incl - v;
}

// Visits the row in rounds of kThreads * 8 tokens: thread t gets tokens
// base + 8t .. base + 8t + 7 of each round (16-byte loads when aligned), as
// f(i0, b, full) with `full` a compile-time true when the whole round lies
// inside the row (no token needs a bounds test) and false for the row's
// last, partial round.  The
// loads of kBatch rounds are issued before any is used, so a pass over the
// row waits for memory once per batch rather than once per round.  The
// 16-byte loads sit in no branch (a lane whose 8 tokens pass the row's end
// loads the row's first 8 instead and patches its tokens afterwards): a
// load under a divergent branch makes the compiler wait for it at the
// branch's end, one memory round trip per round.
template <bool kVec>
constexpr int batch_rounds() {
  return kVec ? 8 : 2;  // element loads hold more registers
}
constexpr int64_t kPerRound = static_cast<int64_t>(kThreads) * 8;

// Loads the rounds base .. base + kBatch - 1 of the row into v.
template <bool kVec, int kBatch>
__device__ __forceinline__ void load_rounds(const uint16_t* p, int64_t vocab, int64_t base,
                                            q3::u32x4 (&v)[kBatch]) {
  const int64_t lane0 = 8 * static_cast<int64_t>(threadIdx.x);
  if (kVec && vocab >= 8) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (base + u * kPerRound >= vocab) break;  // uniform: the round is past the row
      const int64_t i0 = base + u * kPerRound + lane0;
      v[u] = q3::ld16(p + (i0 + 8 <= vocab ? i0 : 0));
    }
  }
  if (!kVec || vocab < 8 || base + kPerRound * kBatch > vocab) {  // uniform: the row ends here
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (base + u * kPerRound >= vocab) break;
      const int64_t i0 = base + u * kPerRound + lane0;
      if (kVec && vocab >= 8 && i0 + 8 <= vocab) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = i0 + 2 * e < vocab ? p[i0 + 2 * e] : 0x7FC1u;  // NaN pad
        const uint32_t hi = i0 + 2 * e + 1 < vocab ? p[i0 + 2 * e + 1] : 0x7FC1u;
        v[u][e] = lo | (hi << 16);
      }
    }
  }
}

// Calls f(i0, b, full) for the loaded rounds that lie in the row.
template <int kBatch, typename F>
__device__ __forceinline__ void visit_rounds(int64_t vocab, int64_t base,
                                             const q3::u32x4 (&v)[kBatch], F&& f) {
  const int64_t lane0 = 8 * static_cast<int64_t>(threadIdx.x);
#pragma unroll
  for (int u = 0; u < kBatch; ++u) {
    const int64_t i0 = base + u * kPerRound + lane0;
    if (base + u * kPerRound >= vocab) break;  // uniform: the round is past the row
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b[2 * e] = v[u][e] & 0xFFFFu;
      b[2 * e + 1] = v[u][e] >> 16;
    }
    if (base + (u + 1) * kPerRound <= vocab)  // uniform
      f(i0, b, std::true_type{});
    else
      f(i0, b, std::false_type{});
  }
}

template <bool kVec, typename F>
__device__ __forceinline__ void for_each_round(const uint16_t* p, int64_t vocab, F&& f) {
  constexpr int kBatch = batch_rounds<kVec>();
  for (int64_t base = 0; base < vocab; base += kPerRound * kBatch) {
    q3::u32x4 v[kBatch];
    load_rounds<kVec, kBatch>(p, vocab, base, v);
    visit_rounds<kBatch>(vocab, base, v, f);
  }
}

// The same over tokens [lo, hi) of the row (lo a multiple of 8): f gets the
// row index of the first of its 8 tokens.
template <bool kVec, typename F>
__device__ __forceinline__ void for_each_round_in(const uint16_t* p, int64_t lo, int64_t hi,
                                                  F&& f) {
  if (hi <= lo) return;
  for_each_round<kVec>(p + lo, hi - lo, [&](int64_t i0, const uint32_t* b, auto full) {
    f(lo + i0, b, full);
  });
}

// Scans the low-bit count histogram from the top: returns the bin where the
// running count (starting at `above`) first reaches `need`, and the count
// strictly above that bin.
// Every lane of a wave gets the result: lane i < 16 takes bin 15 - i, a
// four-step scan gives the counts from the top, a ballot the crossing.
__device__ __forceinline__ int find_count_bin(const uint32_t* h, int64_t need, int64_t& above) {
  const int lane = threadIdx.x & 63;
  const int64_t c = lane < kLoBins ? static_cast<int64_t>(h[kLoBins - 1 - lane]) : 0;
  int64_t incl = c;
#pragma unroll
  for (int o = 1; o < kLoBins; o <<= 1) {
    const int64_t y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  const unsigned long long m = __ballot(lane < kLoBins && above + incl >= need);
  if (m == 0ull) {  // not reached: every count is above, bin 0
    above += __shfl(incl, kLoBins - 1, 64);
    return 0;
  }
  const int i = __ffsll(static_cast<long long>(m)) - 1;
  above += __shfl(incl - c, i, 64);
  return kLoBins - 1 - i;
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

// A value of each of a row's P parts, all loads issued before any is used
// (a loop over a runtime part count would wait for each in turn); parts
// past P read part 0 and count as `none`.
template <typename T, typename F>
__device__ __forceinline__ void part_values(int P, T none, F&& get, T (&v)[kMaxParts]) {
  T raw[kMaxParts];
#pragma unroll
  for (int c = 0; c < kMaxParts; ++c) raw[c] = get(c < P ? c : 0);
#pragma unroll
  for (int c = 0; c < kMaxParts; ++c) v[c] = c < P ? raw[c] : none;
}

// The parallel form's first kernel, workgroup (row, part): for a greedy row
// the part's first maximum; for a row that top-k cuts, the part's largest
// key and its tokens at or above its own threshold (a list of -1 entries:
// more than kCap, or nothing cut by top-k).  A part of at most 8 rounds is
// held in registers for both of its passes.
template <bool kVec>
__global__ __launch_bounds__(kThreads) void sample_part_kernel(const uint16_t* logits,
                                                               int64_t row_s, int64_t vocab,
                                                               const float* temperature,
                                                               const int32_t* top_k, int P,
                                                               PartOut* parts) {
  __shared__ Shared sh;
  const int64_t row = blockIdx.x / P;
  const int c = static_cast<int>(blockIdx.x % P);
  const uint16_t* p = logits + row * row_s;
  const bool greedy = !((temperature ? temperature[row] : 0.f) > 0.f);
  const int64_t kreq = top_k ? top_k[row] : 0;
  const int tid = threadIdx.x;
  int64_t lo, hi;
  part_range(vocab, P, c, lo, hi);
  PartOut& po = parts[row * P + c];
  if (!greedy && (kreq <= 0 || kreq >= vocab)) {  // top-k cuts nothing: no list
    if (tid == 0) po.ncand = -1;
    return;
  }
  if (!greedy) {
    for (int i = tid; i < kHiBins; i += kThreads) sh.cnt[i] = 0;
    if (tid == 0) sh.ncand = 0;
    __syncthreads();
  }
  if (greedy) {  // the part's first largest value, as the single-workgroup greedy path
    unsigned long long best = 0;
    for_each_round_in<kVec>(p, lo, hi, [&](int64_t i0, const uint32_t* b, auto full) {
      const unsigned long long cb = greedy_round(i0, b, hi, full);
      best = cb > best ? cb : best;
    });
    best = block_max_u64(best, sh);
    if (tid == 0) po.best = best;
    return;
  }
  // The part keeps every token whose key is >= t_lo, a key that at least
  // kreq of the part's tokens reach: then a part token below t_lo has kreq
  // tokens of the row strictly above it, so the list holds every token at
  // or above the row's k-th largest key.  t_lo is the kreq-th largest of the
  // threads' own largest keys (kreq threads reaching it are kreq distinct
  // tokens), found on a histogram of those, one LDS atomic per thread; a
  // kreq above the thread count takes the high bin of the kreq-th largest
  // token from a histogram of every token instead.
  const int64_t n_part = hi - lo;
  auto passes = [&](auto&& visit) {
    // each thread's largest key: whole rounds on raw keys, a NaN seen there
    // sends the thread through its tokens again on exact keys
    uint32_t tmax = 0, rmax = 0;
    visit([&](int64_t i0, const uint32_t* b, auto full) {
      if constexpr (decltype(full)::value) {
        const uint32_t m = round_raw_max(b);
        rmax = m > rmax ? m : rmax;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t key = okey(b[e]);
          if (i0 + e < hi) tmax = key > tmax ? key : tmax;
        }
      }
    });
    if (rmax > 0xFF80u) {  // a positive NaN in a whole round: exact keys
      tmax = 0;
      visit([&](int64_t i0, const uint32_t* b, auto full) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t key = okey(b[e]);
          if (full || i0 + e < hi) tmax = key > tmax ? key : tmax;
        }
      });
    } else if (rmax >= 0x7Fu) {  // else no whole round, or only negative NaNs (key 0)
      tmax = rmax > tmax ? rmax : tmax;
    }
    const bool has = 8 * static_cast<int64_t>(tid) < n_part;  // the thread holds tokens
    if (has) atomicAdd(&sh.cnt[tmax >> kLoBits], 1u);
    if (tid < kLoBins) sh.lo_cnt[tid] = 0;
    const uint32_t kmax = static_cast<uint32_t>(block_max_u64(tmax, sh));  // syncs the counts
    const int64_t n_thr = n_part < 8 * kThreads ? (n_part + 7) / 8 : kThreads;
    uint32_t t_lo = 0;  // keys kept: >= t_lo (a part of at most kreq tokens keeps them all)
    if (n_part > kreq && kreq <= n_thr) {
      // the kreq-th largest thread maximum: its high bin, then its low bits
      int64_t above = 0;
      const int hb = find_count_bin_block(sh.cnt, kreq, above, sh);
      if (has && static_cast<int>(tmax >> kLoBits) == hb)
        atomicAdd(&sh.lo_cnt[tmax & (kLoBins - 1)], 1u);
      __syncthreads();
      const int lb = find_count_bin(sh.lo_cnt, kreq, above);
      t_lo = (static_cast<uint32_t>(hb) << kLoBits) | static_cast<uint32_t>(lb);
    } else if (n_part > kreq) {
      for (int i = tid; i < kHiBins; i += kThreads) sh.cnt[i] = 0;
      __syncthreads();
      visit([&](int64_t i0, const uint32_t* b, auto full) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (!full && i0 + e >= hi) break;
          atomicAdd(&sh.cnt[okey(b[e]) >> kLoBits], 1u);
        }
      });
      __syncthreads();
      int64_t above = 0;
      t_lo = static_cast<uint32_t>(find_count_bin_block(sh.cnt, kreq, above, sh)) << kLoBits;
    }
    visit([&](int64_t i0, const uint32_t* b, auto full) {
      bool q[8], any = false;
      uint32_t keys[8];
      bool exact = true;
      if constexpr (decltype(full)::value) {
        // most rounds keep nothing of the wave: a whole round is passed
        // over on its raw maximum; without a positive NaN in the thread's
        // round (and with t_lo above every negative NaN's raw key) the raw
        // keys are the keys for the test
        uint32_t r2[4], m = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          r2[j] = raw_keys2(b[2 * j] | (b[2 * j + 1] << 16));
          m = max_u16x2(m, r2[j]);
        }
        const uint32_t rmx = (m & 0xFFFFu) > (m >> 16) ? (m & 0xFFFFu) : (m >> 16);
        if (__ballot(rmx >= t_lo) == 0ull) return;
        if (rmx <= 0xFF80u && t_lo > 0x7Eu) {
          exact = false;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            keys[2 * j] = r2[j] & 0xFFFFu;
            keys[2 * j + 1] = r2[j] >> 16;
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            q[e] = keys[e] >= t_lo;
            any = any || q[e];
          }
        }
      }
      if (exact) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          keys[e] = okey(b[e]);
          q[e] = (full || i0 + e < hi) && keys[e] >= t_lo;
          any = any || q[e];
        }
      }
      if (__ballot(any) == 0ull) return;
      append_round(q, keys, i0, sh);
    });
    __syncthreads();
    const int n = sh.ncand;
    const bool ok = n <= kCap;
    if (tid == 0) {
      po.kmax = kmax;
      po.ncand = ok ? n : -1;
    }
    if (ok)
      for (int i = tid; i < n; i += kThreads) po.cand[i] = sh.cand[i];
  };
  constexpr int kB = batch_rounds<kVec>();
  if (n_part <= kB * kPerRound) {  // one batch: both passes over registers
    q3::u32x4 v[kB];
    load_rounds<kVec, kB>(p + lo, n_part, 0, v);
    passes([&](auto&& f) {
      visit_rounds<kB>(n_part, 0, v, [&](int64_t i0, const uint32_t* b, auto full) {
        f(lo + i0, b, full);
      });
    });
  } else {
    passes([&](auto&& f) { for_each_round_in<kVec>(p, lo, hi, f); });
  }
}

// One workgroup per row.  kPre: greedy rows and, when every part kept its
// list, passes A and B run over the parts' lists instead of the row;
// otherwise the workgroup streams the row for them itself.
template <bool kVec, bool kPre>
__global__ __launch_bounds__(kThreads) void sample_kernel(const uint16_t* logits, int64_t row_s,
                                                          int64_t vocab, const float* temperature,
                                                          const int32_t* top_k,
                                                          const float* top_p, uint64_t seed,
                                                          int64_t* out, int P,
                                                          const PartOut* parts) {
  __shared__ Shared sh;
  const int64_t row = blockIdx.x;
  const uint16_t* p = logits + row * row_s;
  const float temp = temperature ? temperature[row] : 0.f;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const PartOut* rp = kPre ? parts + row * P : nullptr;

  // ---- greedy -----------------------------------------------------------
  if (kPre && !(temp > 0.f)) {
    if (tid == 0) {
      unsigned long long v[kMaxParts];
      part_values(P, 0ull, [&](int c) { return rp[c].best; }, v);
      unsigned long long b = 0;
#pragma unroll
      for (int c = 0; c < kMaxParts; ++c) b = v[c] > b ? v[c] : b;
      out[row] = static_cast<int64_t>(~static_cast<uint32_t>(b));
    }
    return;
  }
  if (!(temp > 0.f)) {
    // first index of the largest value; NaN ranks highest, as torch.argmax
    unsigned long long bestk = 0;
    for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b, auto full) {
      const unsigned long long cb = greedy_round(i0, b, vocab, full);
      bestk = cb > bestk ? cb : bestk;
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
  auto compact = [&](bool q, uint32_t key, int64_t idx) { append_candidate(q, key, idx, sh); };
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
      for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b, auto full) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (full || i0 + e < vocab) f(okey(b[e]), i0 + e);
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
  uint32_t kmax = 0;
  bool from_list = false;  // the parts' lists stand for the row in passes A, B
  if constexpr (kPre) {
    // One round trip: every part's (kmax, ncand) and, ahead of knowing the
    // counts, entry tid % L of part tid / L (L = kThreads / P entries per
    // part: all of a short list).
    const int L = kThreads / P;
    const int cpart = tid / L < P ? tid / L : P - 1;
    const int coff = tid - (tid / L) * L;
    const unsigned long long spec = rp[cpart].cand[coff];
    unsigned long long hdr[kMaxParts];
    part_values(P, 0ull, [&](int c) {
      return *reinterpret_cast<const unsigned long long*>(&rp[c].kmax);
    }, hdr);
    // the entry's load stays here, in flight with the counts (the compiler
    // would otherwise move it into the branch that uses it, after them)
    asm volatile("" ::"v"(spec));
    int nc[kMaxParts];
    int total = 0;
    from_list = true;
    bool short_list = true;
#pragma unroll
    for (int c = 0; c < kMaxParts; ++c) {
      nc[c] = static_cast<int>(hdr[c] >> 32);
      const uint32_t km = static_cast<uint32_t>(hdr[c]);
      from_list = from_list && nc[c] >= 0;
      short_list = short_list && nc[c] <= L;
      total += nc[c] > 0 ? nc[c] : 0;
      kmax = km > kmax ? km : kmax;
    }
    from_list = from_list && total <= kCap;
    if (from_list && short_list) {  // uniform
      // A short union (the usual case: k plus a few per part): one entry
      // per thread, sorted by key (descending) and token index (ascending)
      // with a bitonic network; the top-k list is then its first k
      // positions and the top-p cut a prefix sum over them.  The same
      // masses, limit and comparisons as passes C and D (a position is
      // kept while the mass before it is within the limit; ties share one
      // mass, so this is their rank rule), so the draw is the same.
      // Sort keys: key << 32 | ~index (0 pads, below every entry).
      int start_c = 0;  // the entries of the parts before this thread's
#pragma unroll
      for (int j = 0; j < kMaxParts; ++j) start_c += j < cpart ? nc[j] : 0;
      if (tid / L < P && coff < nc[cpart])
        sh.cand[start_c + coff] = (spec & 0xFFFFFFFF00000000ull) | (~static_cast<uint32_t>(spec));
      if (tid < kThreads / 4) sh.cnt[tid] = 0;
      __syncthreads();
      unsigned long long x = tid < total ? sh.cand[tid] : 0ull;
      if (total <= kThreads / 4) {  // uniform
        // up to 256 entries: each entry's rank (the entries above it) from
        // four threads that each compare it with a quarter of the list (LDS
        // broadcast reads, no dependent chain), then a scatter to its rank
        const int e = tid & (kThreads / 4 - 1), q = tid / (kThreads / 4);
        const int j0 = (total * q) / 4, j1 = (total * (q + 1)) / 4;
        if (e < total) {
          const unsigned long long me = sh.cand[e];
          int above = 0;
          for (int j = j0; j < j1; j += 8) {  // eight reads in flight
            unsigned long long v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = sh.cand[j + u < j1 ? j + u : j0];
#pragma unroll
            for (int u = 0; u < 8; ++u) above += (j + u < j1 && v[u] > me) ? 1 : 0;
          }
          atomicAdd(&sh.cnt[e], static_cast<uint32_t>(above));
        }
        __syncthreads();
        if (tid < total) sh.cand[kThreads + sh.cnt[tid]] = x;
        __syncthreads();
        x = tid < total ? sh.cand[kThreads + tid] : 0ull;
      }
      int n2 = 64;  // longer lists: a bitonic network over the next power of two
      while (n2 < total) n2 <<= 1;
      if (total <= kThreads / 4) n2 = 1;  // sorted already
      for (int kb = 2; kb <= n2; kb <<= 1) {
        for (int jb = kb >> 1; jb > 0; jb >>= 1) {
          unsigned long long y;
          if (jb >= 64) {  // uniform: across waves, through LDS
            __syncthreads();
            sh.cand[tid] = x;
            __syncthreads();
            y = sh.cand[tid ^ jb];
          } else {
            y = __shfl_xor(x, jb, 64);
          }
          const bool keep_max = ((tid & jb) == 0) == ((tid & kb) == 0);
          x = keep_max ? (x > y ? x : y) : (x < y ? x : y);
        }
      }
      const uint32_t key = static_cast<uint32_t>(x >> 32);
      const uint32_t idx = ~static_cast<uint32_t>(x);
      const bool in_k = tid < k && tid < total;
      bool kept = in_k;
      if (use_p) {
        const float xmax = key_value(kmax) * inv_t;
        unsigned long long wf = 0;
        if (in_k) {
          const float w = __expf(key_value(key) * inv_t - xmax);
          wf = static_cast<unsigned long long>(static_cast<double>(w) * kFix + 0.5);
        }
        unsigned long long mass;
        const unsigned long long before = block_scan_u64(wf, mass, sh);
        const double limit = static_cast<double>(fmaxf(pcut, 0.f)) * static_cast<double>(mass);
        kept = in_k && static_cast<double>(before) <= limit;
      }
      unsigned long long best = 0;
      if (kept && key != 0) {  // as pass E's offer
        const float sc = key_value(key) * inv_t + gumbel_of(draws4(seed, row, idx >> 2)[idx & 3]);
        const uint32_t sb = __float_as_uint(sc);
        const uint32_t so = (sb & 0x80000000u) ? ~sb : (sb | 0x80000000u);
        best = (static_cast<unsigned long long>(so) << 32) | (~idx);
      }
      best = block_max_u64(best, sh);
      if (tid == 0) out[row] = best ? static_cast<int64_t>(~static_cast<uint32_t>(best)) : 0;
      return;
    }
    if (from_list) {
      for (int i = tid; i < kHiBins; i += kThreads) sh.cnt[i] = 0;
      if (tid < kLoBins) sh.lo_cnt[tid] = 0;
      __syncthreads();
      // entry e of the concatenated lists: part c's run starts at the sum
      // of the runs before it
      for (int e = tid; e < total; e += kThreads) {
        int c = 0, before = 0, start = 0;  // the last part whose run starts at or before e
#pragma unroll
        for (int j = 0; j < kMaxParts; ++j) {
          if (e >= start) {
            c = j;
            before = start;
          }
          start += nc[j];
        }
        const unsigned long long cd = rp[c].cand[e - before];
        sh.cand[e] = cd;
        atomicAdd(&sh.cnt[static_cast<uint32_t>(cd >> 32) >> kLoBits], 1u);
      }
      ncand = total;
      __syncthreads();
    } else {
      kmax = 0;
    }
  }
  if (!from_list) {
    for (int i = tid; i < kHiBins; i += kThreads) sh.cnt[i] = 0;
    if (tid < kLoBins) sh.lo_cnt[tid] = 0;
    if (tid == 0) sh.ncand = 0;
    __syncthreads();
    for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b, auto full) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (!full && i0 + e >= vocab) break;
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
  }
  const float xmax = key_value(kmax) * inv_t;

  // ---- B: exact k-th largest key (kk) and the ties of it kept (tk) ------
  uint32_t kk = 0;  // every key >= 0: with k == vocab nothing is cut
  int64_t tk = 0, kties = 0;
  if (k < vocab) {
    int64_t above = 0;
    const int hb = find_count_bin_block(sh.cnt, k, above, sh);
    // the tokens of bins >= hb hold the top-k list: keep them when they fit
    const bool keep_list = above + static_cast<int64_t>(sh.cnt[hb]) <= kCap;
    if (from_list) {
      // the low-bin counts inside bin hb, over the list (which holds every
      // token at or above the k-th largest key: those counts are the row's)
      for (int i = tid; i < ncand; i += kThreads) {
        const uint32_t key = static_cast<uint32_t>(sh.cand[i] >> 32);
        if (static_cast<int>(key >> kLoBits) == hb) atomicAdd(&sh.lo_cnt[key & (kLoBins - 1)], 1u);
      }
    } else {
      for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b, auto full) {
        bool q[8], any = false;  // tokens at or above the boundary bin
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          q[e] = (full || i0 + e < vocab) && static_cast<int>(okey(b[e]) >> kLoBits) >= hb;
          any = any || q[e];
        }
        if (__ballot(any) == 0ull) return;  // most rounds: none in the wave
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t key = okey(b[e]);
          if (q[e] && static_cast<int>(key >> kLoBits) == hb)
            atomicAdd(&sh.lo_cnt[key & (kLoBins - 1)], 1u);
          if (keep_list) compact(q[e], key, i0 + e);
        }
      });
      if (keep_list) finish_compaction();
    }
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
        for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b, auto full) {
          bool q[8], any = false;  // tokens that can still be kept
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t key = okey(b[e]);
            q[e] = (full || i0 + e < vocab) && static_cast<int>(key >> kLoBits) >= hb &&
                   key >= kk;
            any = any || q[e];
          }
          if (__ballot(any) == 0ull) return;  // most rounds: none in the wave
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t key = okey(b[e]);
            if (q[e]) lo_hist(key, i0 + e);
            if (keep_list) compact(q[e], key, i0 + e);
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
    for_each_round<kVec>(p, vocab, [&](int64_t i0, const uint32_t* b, auto) {
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
    hipLaunchKernelGGL((sample_kernel<true, false>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, s, lg, row_stride, vocab, temperature, top_k, top_p,
                       seed, out, 0, nullptr);
  else
    hipLaunchKernelGGL((sample_kernel<false, false>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, s, lg, row_stride, vocab, temperature, top_k, top_p,
                       seed, out, 0, nullptr);
  return q3::launch_status(who);
}

extern "C" size_t qwen3_sample_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  const int P = parts_for(rows, vocab);
  return P > 1 ? static_cast<size_t>(rows) * P * sizeof(PartOut) : 0;
}

namespace {
template <bool kVec>
void launch_parts(const uint16_t* lg, int64_t row_stride, int64_t rows, int64_t vocab,
                  const float* temperature, const int32_t* top_k, const float* top_p,
                  uint64_t seed, int64_t* out, int P, PartOut* parts, hipStream_t s) {
  hipLaunchKernelGGL(sample_part_kernel<kVec>, dim3(static_cast<unsigned>(rows * P)),
                     dim3(kThreads), 0, s, lg, row_stride, vocab, temperature, top_k, P, parts);
  hipLaunchKernelGGL((sample_kernel<kVec, true>), dim3(static_cast<unsigned>(rows)),
                     dim3(kThreads), 0, s, lg, row_stride, vocab, temperature, top_k, top_p, seed,
                     out, P, parts);
}
}  // namespace

extern "C" int qwen3_sample_ws_bf16(const void* logits, int64_t row_stride, int64_t rows,
                                    int64_t vocab, const float* temperature,
                                    const int32_t* top_k, const float* top_p, uint64_t seed,
                                    int64_t* out, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  const char* who = "qwen3_sample_ws_bf16";
  // no workspace, or a batch that fills the CUs with one workgroup per row:
  // the single-workgroup form
  if (!workspace || parts_for(rows, vocab) <= 1)
    return qwen3_sample_bf16(logits, row_stride, rows, vocab, temperature, top_k, top_p, seed,
                             out, stream);
  if (!logits || !out) return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (rows < 0 || rows > 0x7fffffff || vocab <= 0 || vocab > 0x7fffffff || row_stride < vocab)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  if (rows == 0) return QWEN3_OK;
  const int P = parts_for(rows, vocab);
  if (static_cast<int64_t>(rows) * P > 0x7fffffff)
    return q3::fail(QWEN3_EINVAL, "%s: bad sizes", who);
  const size_t need = qwen3_sample_workspace_bytes(rows, vocab);
  if (workspace_bytes < need)
    return q3::fail(QWEN3_EWORKSPACE, "%s: workspace of %zu bytes, %zu needed", who,
                    workspace_bytes, need);
  if (!q3::aligned16(workspace))
    return q3::fail(QWEN3_EALIGN, "%s: workspace must be 16-byte aligned", who);
  q3::clear_error();
  auto s = static_cast<hipStream_t>(stream);
  const auto lg = static_cast<const uint16_t*>(logits);
  auto parts = static_cast<PartOut*>(workspace);
  if (q3::aligned16(logits) && row_stride % 8 == 0)
    launch_parts<true>(lg, row_stride, rows, vocab, temperature, top_k, top_p, seed, out, P,
                       parts, s);
  else
    launch_parts<false>(lg, row_stride, rows, vocab, temperature, top_k, top_p, seed, out, P,
                        parts, s);
  return q3::launch_status(who);
}
