// SwiGLU feed-forward block of one decode token in ONE launch, int4 group-32
// weights (hidden E = 2048, FFN F = 8192: the Llama-3.2-1B shape):
//
//   h = bf16(silu(Wg xn) * (Wu xn))      xn: x as given, RMS-normalised with a
//                                        weight, or with the norm weight folded
//                                        into Wg/Wu and the outputs scaled
//   y = bf16(Wd h + residual)
//
// The separate form is two launches (the gate/up pair GEMV, then the down
// GEMV), and the down projection cannot start before the whole of h exists.
// Here the grid is 256 workgroups of 8 waves (one per CU), all resident at
// once, and each does both halves: wave w of workgroup b computes FFN units
// 32 b + 4 w + [0, 4) and down row 8 b + w. Every wave issues its loads at
// the start in the order they are used (x, the gate/up rows, then the down
// row), so the down weights stream while the gate/up products are computed;
// each wave then publishes its four h values as tagged pairs (exchange.hpp),
// and every workgroup gathers all 8192 h values into LDS before its down row.
// Loads retire in order, so that gather returns once the down row's weights
// are in; the handoff costs what the last producer's h needs to become
// visible beyond that.
//
// Tags. The workspace holds a status word (offset 0), an epoch word (offset
// 128) and the exchange pairs (from offset 256). A call tags its pairs with
// epoch + 1, read by every workgroup at its start; workgroup 0 advances the
// epoch (skipping the value whose successor is 0) once its gather has seen
// every pair of the call, i.e. once every workgroup has read the old value
// (not after a give-up, which the caller resolves by zero-filling the
// workspace).
// Pairs left by an earlier call carry an older tag and are never accepted.
//
// Bounded waits: a gather that does not see its pairs within wait_us, or sees
// a nonzero status word (read with every round of its loads), gives up; it
// sets status bit 1, its workgroup skips its output rows, and every later wait
// (this call or the next) sees the status and gives up at once. The caller checks the word and, after a
// give-up, zero-fills the workspace before the next call.
//
// Arithmetic. The per-row sums are those of the two separate GEMVs
// (gemv_i4_fast: the SwiGLU pair with one 32-element group per lane, and the
// down projection with lane l owning groups l + 64 j, j = 0..3, accumulated in
// j order, then the DPP wave total), so y is bit-identical to the two-launch
// form.
#include "iron_common.hpp"
#include "i4_dot.hpp"
#include "exchange.hpp"
#include "trace.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

constexpr int kSwE = 2048;                           // hidden size (K of gate/up, rows of down)
constexpr int kSwF = 8192;                           // FFN size (rows of gate/up, K of down)
constexpr int kSwGrid = 256;                         // workgroups: one per CU
constexpr int kSwWaves = 8;                          // waves per workgroup
constexpr int kSwUnits = kSwF / kSwGrid / kSwWaves;  // FFN units per wave: 4
constexpr int kSwDownGpl = kSwF / 32 / kWave;        // down groups per lane: 4
static_assert(kSwE / kSwGrid == kSwWaves, "one down row per wave");
static_assert(kSwE == 32 * kWave, "one gate/up group per lane");

constexpr int kSwStatusOff = 0;
constexpr int kSwEpochOff = 128;
constexpr int kSwPairsOff = 256;
constexpr int kSwPairs = kSwF / 2;  // two h values per pair
constexpr long long kSwWorkspace = kSwPairsOff + 8LL * kSwPairs;
constexpr int kSwGatherLoads = kSwPairs / 2 / (kSwWaves * kWave);  // 16-byte loads per thread: 4

enum : int { SW_NORM_NONE = 0, SW_NORM_WEIGHT = 1, SW_NORM_SCALE = 2 };

struct SwArgs {
  const uint8_t* gc;       // gate codes (F, E/2)
  const uint16_t* gs;      // gate scales (F, E/32)
  const uint8_t* uc;       // up
  const uint16_t* us;
  const uint8_t* dc;       // down codes (E, F/2)
  const uint16_t* ds;      // down scales (E, F/32)
  const uint16_t* x;       // (E,)
  const uint16_t* norm_w;  // (E,) for SW_NORM_WEIGHT
  const uint16_t* resid;   // (E,) or null
  uint16_t* y;             // (E,)
  unsigned char* ws;
  float eps;
  uint32_t magic;  // i4_dot.hpp: signed or unsigned codes
  float offset;
  unsigned wait_ticks;  // 100 MHz
  void* trace;          // phase trace records (trace.hpp), or null
};

template <int NM>
__global__ __launch_bounds__(kSwWaves * kWave) void swiglu_decode_i4_kernel(SwArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t h_s[kSwPairs];  // h as bf16 pairs
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  // trace points: 0 start, 1 x ready, 2 h published, 3 h gathered, 4 down row done
  const unsigned long long t_start = trace_clock();
  const int blk = xcd_block(1);  // each XCD owns a contiguous eighth of the units and rows
  unsigned* status = reinterpret_cast<unsigned*>(a.ws + kSwStatusOff);
  unsigned* epoch = reinterpret_cast<unsigned*>(a.ws + kSwEpochOff);
  const __amdgpu_buffer_rsrc_t xr = xch_rsrc(a.ws + kSwPairsOff);
  const unsigned e = *epoch;
  const unsigned tag = e + 1u;

  // Loads, in the order of use: x (and the norm weight), the gate/up rows and
  // scales, then the down row, its scales and residual.
  const int u0 = blk * (kSwUnits * kSwWaves) + wave * kSwUnits;
  const int dr = blk * kSwWaves + wave;
  uint4 xq[4], nq[4];
  {
    const uint4* xv = reinterpret_cast<const uint4*>(a.x);
#pragma unroll
    for (int q = 0; q < 4; ++q) xq[q] = xv[lane * 4 + q];
    if (NM == SW_NORM_WEIGHT) {
      const uint4* nv = reinterpret_cast<const uint4*>(a.norm_w);
#pragma unroll
      for (int q = 0; q < 4; ++q) nq[q] = nv[lane * 4 + q];
    }
  }
  uint4 cg[kSwUnits], cu[kSwUnits], cd[kSwDownGpl];
  uint16_t sg[kSwUnits], su[kSwUnits], sd[kSwDownGpl];
#pragma unroll
  for (int i = 0; i < kSwUnits; ++i) {
    const size_t off = static_cast<size_t>(u0 + i) * (kSwE / 2) + lane * 16;
    cg[i] = ld_stream16(a.gc + off);
    cu[i] = ld_stream16(a.uc + off);
  }
#pragma unroll
  for (int i = 0; i < kSwUnits; ++i) {
    sg[i] = a.gs[(u0 + i) * (kSwE / 32) + lane];
    su[i] = a.us[(u0 + i) * (kSwE / 32) + lane];
  }
  // the down row's loads go after these: the products wait only for what they use
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < kSwDownGpl; ++j)
    cd[j] = ld_stream16(a.dc + static_cast<size_t>(dr) * (kSwF / 2) + (lane + j * kWave) * 16);
#pragma unroll
  for (int j = 0; j < kSwDownGpl; ++j) sd[j] = a.ds[dr * (kSwF / 32) + lane + j * kWave];
  const float rres = bf16_to_f32(a.resid ? a.resid[dr] : a.x[0]);  // unconditional load
  // keeps the scheduler from sinking any of these loads below the products
  __builtin_amdgcn_sched_barrier(0);
  trace_write(a.trace, kTraceSwigluDecode, blockIdx.x, 0, t_start);

  // The wave's four FFN units (the pair GEMV's arithmetic, one group per lane).
  float inv = 1.f;
  if (NM != SW_NORM_NONE) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) ss = sumsq_chunk(xq[q], ss);
    inv = inv_rms(wave_sum(ss), kSwE, a.eps);
  }
  trace_stamp(a.trace, kTraceSwigluDecode, blockIdx.x, 1);
  if (NM == SW_NORM_WEIGHT) {
#pragma unroll
    for (int q = 0; q < 4; ++q) xq[q] = normalize_chunk(xq[q], nq[q], inv);
  }
  XGroup xg;
  build_xgroup(xq, xg);
  __builtin_amdgcn_sched_barrier(0);
  uint32_t hv[kSwUnits / 2];
#pragma unroll
  for (int i = 0; i < kSwUnits; ++i) {
    float t = wave_sum(fmaf(bf16_to_f32(sg[i]), i4_group_total(cg[i], xg, a.magic, a.offset), 0.f));
    float t2 = wave_sum(fmaf(bf16_to_f32(su[i]), i4_group_total(cu[i], xg, a.magic, a.offset), 0.f));
    if (NM == SW_NORM_SCALE) {
      t *= inv;
      t2 *= inv;
    }
    const uint32_t h = f32_to_bf16(silu_f32(t) * t2);
    if (i & 1)
      hv[i >> 1] |= h << 16;
    else
      hv[i >> 1] = h;
  }
  if (lane == 0) st_pairs2(xr, u0 / 2, hv[0], hv[1], tag);
  trace_stamp(a.trace, kTraceSwigluDecode, blockIdx.x, 2);

  // Gather every h value (4096 pairs: four 16-byte loads per thread) into LDS.
  // One round trip per retry: the pairs still missing are loaded again
  // together with the status word (lane 0 of each wave), and the wave retries
  // until every lane holds its pairs, the status is nonzero, or wait_us passes.
  bool ok = true;  // wave-uniform
  {
    u32x4_v v[kSwGatherLoads];
#pragma unroll
    for (int k = 0; k < kSwGatherLoads; ++k) v[k] = ld_pairs2(xr, 2 * (tid + kSwWaves * kWave * k));
    unsigned st = lane == 0 ? read_status(status) : 0u;
    const unsigned long long t0 = now_ticks();
    unsigned got = 0;  // bit k: the pairs of load k are in LDS
    for (;;) {
#pragma unroll
      for (int k = 0; k < kSwGatherLoads; ++k)
        if (!(got & (1u << k)) && v[k][1] == tag && v[k][3] == tag) {
          *reinterpret_cast<uint2*>(&h_s[2 * (tid + kSwWaves * kWave * k)]) = make_uint2(v[k][0], v[k][2]);
          got |= 1u << k;
        }
      if (__builtin_amdgcn_ballot_w64(st != 0u)) {
        ok = false;
        break;
      }
      if (!__builtin_amdgcn_ballot_w64(got != (1u << kSwGatherLoads) - 1)) break;
      if (now_ticks() - t0 > a.wait_ticks) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int k = 0; k < kSwGatherLoads; ++k)
        if (!(got & (1u << k))) v[k] = ld_pairs2(xr, 2 * (tid + kSwWaves * kWave * k));
      if (lane == 0) st = read_status(status);
    }
  }
  if (!ok && lane == 0) give_up(status, 1u);
  const int failed = __syncthreads_or(!ok);
  // Once this gather has seen every pair, every workgroup has read the epoch
  // (each published its pairs after doing so). After a give-up the status word
  // is set and the caller zero-fills the workspace, epoch included.
  if (blockIdx.x == 0 && tid == 0 && !failed) *epoch = (e + 1u == 0xffffffffu) ? 0u : e + 1u;
  if (failed) return;
  trace_stamp(a.trace, kTraceSwigluDecode, blockIdx.x, 3);

  // The wave's down row against h (the down GEMV's arithmetic).
  const uint4* hq = reinterpret_cast<const uint4*>(h_s);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < kSwDownGpl; ++j) {
    uint4 hc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) hc[q] = hq[(lane + j * kWave) * 4 + q];
    XGroup g;
    build_xgroup(hc, g);
    acc = fmaf(bf16_to_f32(sd[j]), i4_group_total(cd[j], g, a.magic, a.offset), acc);
  }
  const float t = wave_sum(acc);
  if (lane == 0) a.y[dr] = f32_to_bf16(a.resid ? t + rres : t);
  trace_stamp(a.trace, kTraceSwigluDecode, blockIdx.x, 4);
}

}  // namespace
}  // namespace iron

using namespace iron;

#include <mutex>

// The 256 workgroups wait for each other: all of them must be resident at
// once. Checked once per device and norm variant from the occupancy query.
static int sw_check_residency(const char* who, int nm) {
  static std::mutex m;
  static int known[64][3];  // 0 unknown, 1 fits, -1 does not
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail_einval("%s: no current device", who);
  std::lock_guard<std::mutex> lock(m);
  int& k = known[dev][nm];
  if (k == 0) {
    int cus = 0, per_cu = 0;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int threads = kSwWaves * kWave;
    hipError_t e = hipErrorInvalidValue;
    switch (nm) {
      case SW_NORM_WEIGHT:
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, swiglu_decode_i4_kernel<SW_NORM_WEIGHT>, threads, 0);
        break;
      case SW_NORM_SCALE:
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, swiglu_decode_i4_kernel<SW_NORM_SCALE>, threads, 0);
        break;
      default:
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, swiglu_decode_i4_kernel<SW_NORM_NONE>, threads, 0);
        break;
    }
    k = (e == hipSuccess && static_cast<long long>(cus) * per_cu >= kSwGrid) ? 1 : -1;
    if (k < 0)
      return fail_einval("%s: the device holds %d x %d workgroups of this kernel at once, fewer than its %d", who, cus,
                         per_cu, kSwGrid);
  }
  return k > 0 ? 0 : fail_einval("%s: the device cannot hold the %d workgroups of this kernel at once", who, kSwGrid);
}

extern "C" long long iron_swiglu_decode_i4g32_workspace_bytes(int E, int F) {
  return (E == kSwE && F == kSwF) ? kSwWorkspace : -1;
}

extern "C" int iron_swiglu_decode_i4g32(const void* gate_codes, const void* gate_scales, const void* up_codes,
                                        const void* up_scales, const void* down_codes, const void* down_scales,
                                        const void* x, void* y, int E, int F, int is_signed, int norm_mode,
                                        const void* norm_w, float eps, const void* residual, void* workspace,
                                        unsigned wait_us, void* stream) {
  const char* who = "iron_swiglu_decode_i4g32";
  IRON_REQUIRE(E == kSwE && F == kSwF, "%s: E=%d F=%d (this kernel takes E=%d, F=%d)", who, E, F, kSwE, kSwF);
  IRON_REQUIRE(gate_codes && gate_scales && up_codes && up_scales && down_codes && down_scales && x && y && workspace,
               "%s: null pointer", who);
  IRON_REQUIRE(norm_mode >= SW_NORM_NONE && norm_mode <= SW_NORM_SCALE, "%s: norm_mode=%d", who, norm_mode);
  IRON_REQUIRE(norm_mode != SW_NORM_WEIGHT || norm_w, "%s: norm_mode 1 needs norm_w", who);
  IRON_REQUIRE(wait_us >= 1 && wait_us <= 10000000u, "%s: wait_us=%u outside [1, 1e7]", who, wait_us);
  auto a2 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; };
  IRON_REQUIRE(aligned16(gate_codes) && aligned16(up_codes) && aligned16(down_codes) && aligned16(x) &&
                   (norm_mode != SW_NORM_WEIGHT || aligned16(norm_w)) && a2(gate_scales) && a2(up_scales) &&
                   a2(down_scales) && a2(y) && (!residual || a2(residual)) &&
                   (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
               "%s: codes, x and norm_w must be 16-byte, scales, y and residual 2-byte, workspace 256-byte aligned",
               who);
  if (int rc = sw_check_residency(who, norm_mode)) return rc;
  SwArgs a;
  a.gc = static_cast<const uint8_t*>(gate_codes);
  a.gs = static_cast<const uint16_t*>(gate_scales);
  a.uc = static_cast<const uint8_t*>(up_codes);
  a.us = static_cast<const uint16_t*>(up_scales);
  a.dc = static_cast<const uint8_t*>(down_codes);
  a.ds = static_cast<const uint16_t*>(down_scales);
  a.x = static_cast<const uint16_t*>(x);
  a.norm_w = static_cast<const uint16_t*>(norm_w);
  a.resid = static_cast<const uint16_t*>(residual);
  a.y = static_cast<uint16_t*>(y);
  a.ws = static_cast<unsigned char*>(workspace);
  a.eps = eps;
  a.magic = is_signed ? 0x43084308u : 0x43004300u;
  a.offset = is_signed ? 136.f : 128.f;
  a.wait_ticks = wait_us * 100u;
  if (int rc = take_trace(who, kSwGrid, &a.trace)) return rc;
  const dim3 g(kSwGrid), blk(kSwWaves * kWave);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (norm_mode) {
    case SW_NORM_WEIGHT: IRON_LAUNCH(swiglu_decode_i4_kernel<SW_NORM_WEIGHT>, g, blk, 0, s, a); break;
    case SW_NORM_SCALE: IRON_LAUNCH(swiglu_decode_i4_kernel<SW_NORM_SCALE>, g, blk, 0, s, a); break;
    default: IRON_LAUNCH(swiglu_decode_i4_kernel<SW_NORM_NONE>, g, blk, 0, s, a); break;
  }
  return check_launch(who);
}
