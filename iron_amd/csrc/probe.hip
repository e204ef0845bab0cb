// Measurement probes for the floors that bound the kernels: an empty kernel
// (what one launch, or one node of a replayed hipGraph, costs with no work),
// a pure streaming read of n bytes (what the memory system delivers to one
// launch of that size, with no arithmetic and no stores beyond one word per
// workgroup), and an MFMA-only loop with clock stamps (the matrix cores' issue
// rate and the shader clock under that load). bench.py --mode floor and
// --mode mfma run them under the same graph protocol as the kernels they
// bound.
#include "iron_common.hpp"
#include "../../include/iron_hip.h"

#include <mutex>

namespace iron {
namespace {

constexpr int kProbeThreads = 256;

__global__ __launch_bounds__(kProbeThreads) void empty_kernel(int) {}

// Workgroup b reads 16-byte chunks b * U * 256 + u * 256 + tid (u < U), every
// load issued before the first use, and stores the XOR of its data to
// sink[b] so that the loads are live. Chunks past the end re-read the last
// chunk (an unconditional clamped load) and are dropped by a select.
template <int U>
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const uint4* __restrict__ src, long long n16,
                                                                      uint32_t* __restrict__ sink) {
  const long long base = static_cast<long long>(blockIdx.x) * U * kProbeThreads + threadIdx.x;
  uint4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) v[u] = ld_stream16(src + min(base + u * kProbeThreads, n16 - 1));
  uint32_t acc = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t w = v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    acc ^= (base + u * kProbeThreads < n16) ? w : 0u;
  }
  // fold the workgroup's words into one (wave shuffles, then the 4 waves through LDS)
  __shared__ uint32_t red[kProbeThreads / kWave];
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, kWave);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kProbeThreads / kWave; ++w) t ^= red[w];
    sink[blockIdx.x] = t;
  }
}

// The XCD each workgroup runs on (hardware register XCC_ID, low 4 bits),
// one word per workgroup.
__global__ __launch_bounds__(kProbeThreads) void xcc_id_kernel(int* __restrict__ ids) {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  if (threadIdx.x == 0) ids[blockIdx.x] = static_cast<int>(x & 15u);
}

typedef __bf16 probe_bf16x8 __attribute__((ext_vector_type(8)));
typedef float probe_f32x16 __attribute__((ext_vector_type(16)));

// MFMA issue probe: every wave issues n_mfma v_mfma_f32_32x32x16_bf16 over
// CHAINS independent accumulators (register operands only: no loads, no LDS),
// as the GEMM's wave tile does per K step, and lane 0 records the shader clock
// (s_memtime) and the 100 MHz real-time counter (s_memrealtime) before and
// after, so the host reads the cycles per MFMA and the clock the SIMDs ran at.
// The accumulators are summed into sink[wave] so that the MFMAs are live.
template <int CHAINS>
__global__ void mfma_probe_kernel(int n_mfma, float* __restrict__ sink, unsigned long long* __restrict__ clocks) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  probe_bf16x8 av, bv;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    av[e] = static_cast<__bf16>(static_cast<float>((lane + e) % 7) * 0.125f);
    bv[e] = static_cast<__bf16>(static_cast<float>((lane * 3 + e) % 5) * 0.25f);
  }
  probe_f32x16 acc[CHAINS];
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.f;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < n_mfma; i += CHAINS) {
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc[c], 0, 0, 0);
  }
  float t = 0.f;
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) t += acc[c][v];
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  t = wave_sum(t);
  if (lane == 0) {
    sink[wave] = t;
    clocks[4 * wave] = t0;
    clocks[4 * wave + 1] = t1;
    clocks[4 * wave + 2] = r0;
    clocks[4 * wave + 3] = r1;
  }
}

}  // namespace
}  // namespace iron

using namespace iron;

extern "C" int iron_probe_mfma(int workgroups, int waves_per_workgroup, int mfma_per_wave, int chains, void* sink,
                               void* clocks, long long waves_capacity, void* stream) {
  IRON_REQUIRE(sink && clocks, "iron_probe_mfma: null pointer");
  IRON_REQUIRE(workgroups > 0 && workgroups <= 65536 && waves_per_workgroup > 0 && waves_per_workgroup <= 16,
               "iron_probe_mfma: workgroups=%d (1..65536), waves_per_workgroup=%d (1..16)", workgroups,
               waves_per_workgroup);
  IRON_REQUIRE(chains == 1 || chains == 2 || chains == 4 || chains == 8, "iron_probe_mfma: chains=%d not in {1,2,4,8}",
               chains);
  IRON_REQUIRE(mfma_per_wave > 0 && mfma_per_wave % chains == 0,
               "iron_probe_mfma: mfma_per_wave=%d must be a positive multiple of chains", mfma_per_wave);
  IRON_REQUIRE(static_cast<long long>(workgroups) * waves_per_workgroup <= waves_capacity,
               "iron_probe_mfma: sink/clocks hold %lld waves, %lld needed", waves_capacity,
               static_cast<long long>(workgroups) * waves_per_workgroup);
  const dim3 grid(workgroups), block(waves_per_workgroup * kWave);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* sk = static_cast<float*>(sink);
  unsigned long long* ck = static_cast<unsigned long long*>(clocks);
  switch (chains) {
    case 1: IRON_LAUNCH(mfma_probe_kernel<1>, grid, block, 0, s, mfma_per_wave, sk, ck); break;
    case 2: IRON_LAUNCH(mfma_probe_kernel<2>, grid, block, 0, s, mfma_per_wave, sk, ck); break;
    case 4: IRON_LAUNCH(mfma_probe_kernel<4>, grid, block, 0, s, mfma_per_wave, sk, ck); break;
    default: IRON_LAUNCH(mfma_probe_kernel<8>, grid, block, 0, s, mfma_per_wave, sk, ck); break;
  }
  return check_launch("probe_mfma");
}

extern "C" int iron_probe_empty(int workgroups, void* stream) {
  IRON_REQUIRE(workgroups > 0 && workgroups <= (1 << 20), "iron_probe_empty: workgroups=%d outside [1, 2^20]",
               workgroups);
  IRON_LAUNCH(empty_kernel, dim3(workgroups), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream), 0);
  return check_launch("probe_empty");
}

extern "C" long long iron_probe_read_workgroups(long long nbytes, int loads_per_lane) {
  if (nbytes <= 0 || nbytes % 16 || !(loads_per_lane == 1 || loads_per_lane == 2 || loads_per_lane == 4 ||
                                      loads_per_lane == 8))
    return -1;
  const long long per_wg = static_cast<long long>(loads_per_lane) * kProbeThreads;
  return (nbytes / 16 + per_wg - 1) / per_wg;
}

extern "C" int iron_probe_read(const void* src, long long nbytes, void* sink, long long sink_words,
                               int loads_per_lane, void* stream) {
  IRON_REQUIRE(src && sink, "iron_probe_read: null pointer");
  IRON_REQUIRE(aligned16(src), "iron_probe_read: src must be 16-byte aligned");
  const long long wgs = iron_probe_read_workgroups(nbytes, loads_per_lane);
  IRON_REQUIRE(wgs > 0, "iron_probe_read: nbytes=%lld must be a positive multiple of 16 and loads_per_lane=%d one "
               "of 1, 2, 4, 8", nbytes, loads_per_lane);
  IRON_REQUIRE(wgs < (1LL << 31), "iron_probe_read: nbytes=%lld too large", nbytes);
  IRON_REQUIRE(sink_words >= wgs, "iron_probe_read: sink holds %lld words, %lld needed", sink_words, wgs);
  const uint4* s4 = static_cast<const uint4*>(src);
  uint32_t* out = static_cast<uint32_t*>(sink);
  const long long n16 = nbytes / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(wgs)), block(kProbeThreads);
  switch (loads_per_lane) {
    case 1: IRON_LAUNCH(stream_read_kernel<1>, grid, block, 0, s, s4, n16, out); break;
    case 2: IRON_LAUNCH(stream_read_kernel<2>, grid, block, 0, s, s4, n16, out); break;
    case 4: IRON_LAUNCH(stream_read_kernel<4>, grid, block, 0, s, s4, n16, out); break;
    default: IRON_LAUNCH(stream_read_kernel<8>, grid, block, 0, s, s4, n16, out); break;
  }
  return check_launch("probe_read");
}

extern "C" int iron_probe_xcc_ids(int workgroups, void* ids, void* stream) {
  IRON_REQUIRE(ids, "iron_probe_xcc_ids: null pointer");
  IRON_REQUIRE(workgroups > 0 && workgroups <= (1 << 20), "iron_probe_xcc_ids: workgroups=%d outside [1, 2^20]",
               workgroups);
  IRON_LAUNCH(xcc_id_kernel, dim3(workgroups), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream),
              static_cast<int*>(ids));
  return check_launch("probe_xcc_ids");
}

// ---------------------------------------------------------------------------
// The XCD dispatch mapping the one-launch attention merge relies on: workgroup
// ids that agree mod 8 run on one XCD. Checked once per device with the probe
// kernel above (64 workgroups; the ids land in a file-scope device array, so
// nothing is allocated) and cached; not checked while `stream` is being
// captured (the check reads its result back on the host), in which case the
// answer is 0 for now and the callers take their paths that do not need it.
// ---------------------------------------------------------------------------
static constexpr int kXccProbeWgs = 64;
static __device__ int g_xcc_ids[kXccProbeWgs];

int iron::xcd_round_robin(hipStream_t stream) {
  static std::mutex m;
  static int state[64];  // per device: 0 unknown, 1 holds, -1 does not
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(m);
  if (state[dev]) return state[dev] > 0 ? 1 : 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return 0;
  int nx = 0;
  if (hipDeviceGetAttribute(&nx, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || nx != 8) {
    state[dev] = -1;
    return 0;
  }
  void* ids_dev = nullptr;
  if (hipGetSymbolAddress(&ids_dev, HIP_SYMBOL(g_xcc_ids)) != hipSuccess || !ids_dev) return 0;
  hipLaunchKernelGGL(xcc_id_kernel, dim3(kXccProbeWgs), dim3(kProbeThreads), 0, stream, static_cast<int*>(ids_dev));
  int ids[kXccProbeWgs];
  if (hipGetLastError() != hipSuccess ||
      hipMemcpyAsync(ids, ids_dev, sizeof(ids), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return 0;
  bool ok = true, seen[16] = {};
  for (int b = 0; b < kXccProbeWgs; ++b) ok &= ids[b] == ids[b % 8];
  for (int b = 0; b < 8 && ok; ++b) {
    ok &= ids[b] >= 0 && ids[b] < 16 && !seen[ids[b]];
    if (ok) seen[ids[b]] = true;
  }
  state[dev] = ok ? 1 : -1;
  return ok ? 1 : 0;
}

extern "C" int iron_xcd_round_robin(void* stream) { return xcd_round_robin(static_cast<hipStream_t>(stream)); }
