// Streaming HBM read reference: the rate at which the device reads a buffer
// with 16-byte loads across a persistent grid (no counterpart in the
// reference engine).  It is the ceiling the HBM-bound kernels of the
// library are measured against: it reads the same bytes as a kernel under
// test, with the same non-temporal (or plain) load type, and does nothing
// else with them.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWgPerCu = 2;  // eight waves per CU, as the decode stream runs
constexpr int kUnroll = 8;   // 16-byte loads in flight per lane

template <bool NT>
__global__ __launch_bounds__(kThreads) void hbm_read_kernel(const q3::u32x4* src, int64_t n16,
                                                            uint32_t* sink) {
  // Wave w reads one contiguous range of 16-byte chunks, as the decode's
  // waves stream contiguous K/V tiles: each load instruction covers 1 KiB
  // (64 lanes), kUnroll of them (kUnroll KiB) in flight per step.
  constexpr int64_t kStep = 64 * kUnroll;
  const int lane = threadIdx.x & 63;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kThreads / 64);
  const int64_t w = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t per = (n16 + waves * kStep - 1) / (waves * kStep) * kStep;
  const int64_t lo = w * per;
  const int64_t hi = lo + per < n16 ? lo + per : n16;
  uint32_t acc = 0;
  for (int64_t base = lo; base < hi; base += kStep) {
    q3::u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * 64 + lane;
      const q3::u32x4 z = {0u, 0u, 0u, 0u};
      v[u] = i < hi ? (NT ? q3::ld16_nt(src + i) : q3::ld16(src + i)) : z;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc += v[u][0] + v[u][1] + v[u][2] + v[u][3];
  }
  // A data-dependent store keeps the loads; it almost never happens.
  if (acc == 0x9e3779b9u) *sink = acc;
}

}  // namespace

extern "C" int qwen3_hbm_read_reference(const void* src, int64_t bytes, int nontemporal,
                                        void* sink, void* stream) {
  const char* who = "qwen3_hbm_read_reference";
  if (!src || !sink) return q3::fail(QWEN3_EINVAL, "%s: null pointer argument", who);
  if (bytes < 0 || bytes % 16 != 0)
    return q3::fail(QWEN3_EINVAL, "%s: bytes %lld must be a non-negative multiple of 16", who,
                    static_cast<long long>(bytes));
  if (!q3::aligned16(src) || !q3::aligned16(sink))
    return q3::fail(QWEN3_EALIGN, "%s: src and sink must be 16-byte aligned", who);
  if (bytes == 0) return QWEN3_OK;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return q3::fail(QWEN3_EINVAL, "%s: no current HIP device", who);
  q3::clear_error();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* p = static_cast<const q3::u32x4*>(src);
  auto* out = static_cast<uint32_t*>(sink);
  if (nontemporal)
    hipLaunchKernelGGL(hbm_read_kernel<true>, dim3(cus * kWgPerCu), dim3(kThreads), 0, s, p,
                       bytes / 16, out);
  else
    hipLaunchKernelGGL(hbm_read_kernel<false>, dim3(cus * kWgPerCu), dim3(kThreads), 0, s, p,
                       bytes / 16, out);
  return q3::launch_status(who);
}
