// Shared device helpers for the gfx950 kernels of libiron_hip.
//
// bf16 values travel as raw uint16 bit patterns so that every rounding step is
// explicit: widening is a 16-bit shift, narrowing is round-to-nearest-even
// written out below (torch's CPU bf16 conversion rounds the same way, which is
// what makes the int4 dequant bit-exact against the test oracle).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iron {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;  // CDNA4 wavefront width

// a b - c d and a b + c d with each product and the sum rounded to fp32 on
// their own (no fused multiply-add, which HIP forms by default): the RoPE
// rotation as the fp32 reference computes it, the same in every kernel.
__device__ __forceinline__ float rot_sub(float a, float b, float c, float d) {
#pragma clang fp contract(off)
  return a * b - c * d;
}
__device__ __forceinline__ float rot_add(float a, float b, float c, float d) {
#pragma clang fp contract(off)
  return a * b + c * d;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even narrowing of two floats in one v_cvt_pk_bf16_f32
// (NaN stays a quiet NaN); `lo` lands in bits 0..15.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(cvt_pk_bf16(f, 0.f) & 0xffffu);
}

// One output element of a split-K GEMM from its fp32 partial sums (range kb at
// p[kb * stride]): summed in range order starting from 0 and rounded once to
// bf16, which is the split-K merge of the GEMMs with no epilogue.
__device__ __forceinline__ float merged_bf16(const float* p, size_t stride, int splits) {
  float x = 0.f;
  for (int kb = 0; kb < splits; ++kb) x += p[kb * stride];
  return bf16_to_f32(f32_to_bf16(x));
}

// Low / high bf16 of a packed 32-bit word, widened to fp32.
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) { return cvt_pk_bf16(lo, hi); }

// Word 3 of a raw buffer resource on gfx9 (32-bit data format, no swizzle).
constexpr int kBufferFlags = 0x00020000;

typedef int i32x4v __attribute__((ext_vector_type(4)));

// Raw buffer resource (V#) over the bytes from `base`: 32-bit offsets, no stride,
// no range check beyond 2^31 - 1 bytes.
__device__ __forceinline__ i32x4v buffer_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4v r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32));
  r[2] = 0x7fffffff;
  r[3] = kBufferFlags;
  return r;
}

// buffer_load_dwordx4 ... lds: 16 bytes per lane from rsrc + voffset into LDS at
// lds (the wave's base; lane l lands at lds + 16 l). Written as assembly: while a
// global_load_lds it issued is in flight, the compiler can only wait for every
// outstanding LDS read at once (lgkmcnt(0)) before using any of them; with loads
// it does not see, it keeps exact counts (lgkmcnt(N)), so LDS reads issued ahead
// overlap the work before their use. The caller orders completion with its own
// s_waitcnt vmcnt and barriers. M0 is written behind the compiler's back (it
// does not preserve a reserved register named as clobbered), so the calling
// kernel must be one in which the compiler itself never uses M0: no LDS-direct
// builtins and no M0-indexed instructions (checked in the kernels' assembly).
// An LDS-DMA instruction must not directly follow the scalar write of M0 it
// reads (one wait state on GFX9, which the compiler inserts for its own code
// but not inside assembly): the s_nop 0 provides it.
__device__ __forceinline__ void load_lds16(const i32x4v& rsrc, unsigned voffset, const void* lds) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voffset),
               "s"(rsrc)
               : "memory", "m0");
}

// Argmax key: unsigned order of (value, -index), so the largest key is the
// largest value and, among equal values, the smallest index.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<unsigned long long>(ord) << 32) | (0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t argmax_key_index(unsigned long long k) {
  return 0xffffffffu - static_cast<uint32_t>(k & 0xffffffffu);
}

// acc + a.lo*b.lo + a.hi*b.hi with fp32 accumulation (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// v + (v moved across lanes by DPP control CTRL); lanes outside ROWMASK add 0.
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float add_dpp(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                    ROWMASK, 0xf, false));
}

// Full-wave sum with DPP row operations (no LDS round trip): pairs, quads,
// half-row mirror, row mirror, then row_bcast:15 / row_bcast:31 fold the four
// 16-lane rows into lane 63, which is broadcast through an SGPR. Every lane
// returns the total. All 64 lanes must be active.
__device__ __forceinline__ float wave_sum(float v) {
  v = add_dpp<0xB1>(v);        // quad_perm [1,0,3,2]
  v = add_dpp<0x4E>(v);        // quad_perm [2,3,0,1]
  v = add_dpp<0x141>(v);       // row_half_mirror
  v = add_dpp<0x140>(v);       // row_mirror: every lane holds its row's sum
  v = add_dpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v = add_dpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float max_dpp(float v) {
  // lanes outside ROWMASK keep `old` = -inf, so the max leaves them unchanged
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                      static_cast<int>(0xff800000u), __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xf, false)));
}

// Full-wave max, same DPP pattern as wave_sum. All 64 lanes must be active.
__device__ __forceinline__ float wave_max(float v) {
  v = max_dpp<0xB1>(v);
  v = max_dpp<0x4E>(v);
  v = max_dpp<0x141>(v);
  v = max_dpp<0x140>(v);
  v = max_dpp<0x142, 0xA>(v);
  v = max_dpp<0x143, 0xC>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Streaming 16-byte load that bypasses cache retention (weights are read once).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 1 / sqrt(ss / n + eps) by one v_rsq_f32 (relative error ~1 ulp), the RMS
// scale of the GEMVs' fused norms: one instruction instead of a square root
// and a full division, and the same bits in every kernel variant whatever
// its compile flags.
__device__ __forceinline__ float inv_rms(float ss, int n, float eps) {
  return __builtin_amdgcn_rsqf(ss / static_cast<float>(n) + eps);
}

// Normalises the 8 bf16 values of an x chunk: bf16(x * inv * w).
__device__ __forceinline__ uint4 normalize_chunk(uint4 xv, uint4 wv, float inv) {
  uint4 r;
  r.x = pack_bf16x2(lo_bf16(xv.x) * inv * lo_bf16(wv.x), hi_bf16(xv.x) * inv * hi_bf16(wv.x));
  r.y = pack_bf16x2(lo_bf16(xv.y) * inv * lo_bf16(wv.y), hi_bf16(xv.y) * inv * hi_bf16(wv.y));
  r.z = pack_bf16x2(lo_bf16(xv.z) * inv * lo_bf16(wv.z), hi_bf16(xv.z) * inv * hi_bf16(wv.z));
  r.w = pack_bf16x2(lo_bf16(xv.w) * inv * lo_bf16(wv.w), hi_bf16(xv.w) * inv * hi_bf16(wv.w));
  return r;
}

// Workgroup index -> logical tile. With `enable` (and a grid that is a
// multiple of 8), each XCD (workgroup b runs on XCD b % 8) owns one
// contiguous eighth of the rows: its weight rows are adjacent in HBM and every
// 64-byte line of y is written from one L2 only.
__device__ __forceinline__ int xcd_block(int enable) {
  const int nb = gridDim.x, b = blockIdx.x;
  return (!enable || (nb & 7)) ? b : (b & 7) * (nb >> 3) + (b >> 3);
}

// xcd_block(1) for a kernel that knows its grid size nb (== gridDim.x) from its
// own arguments: gridDim.x is read from the dispatch packet, a scalar load
// that every address computation behind it would wait for.
__device__ __forceinline__ int xcd_tile(int nb) {
  const int b = blockIdx.x;
  return (nb & 7) ? b : (b & 7) * (nb >> 3) + (b >> 3);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ float gelu_tanh_f32(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), tanh via exp.
  const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
  const float t = 1.0f - 2.0f / (1.0f + __expf(2.0f * inner));
  return 0.5f * x * (1.0f + t);
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Epilogue selectors shared by GEMV and GEMM entry points.
enum Epilogue : int { EPI_NONE = 0, EPI_GELU_TANH = 1, EPI_SILU = 2, EPI_SIGMOID = 3, EPI_GELU_SIGMOID = 4 };

__device__ __forceinline__ float apply_epilogue(float v, int epi) {
  switch (epi) {
    case EPI_GELU_TANH: return gelu_tanh_f32(v);
    case EPI_SILU: return v * sigmoid_f32(v);
    case EPI_SIGMOID: return sigmoid_f32(v);
    case EPI_GELU_SIGMOID: return v * sigmoid_f32(1.702f * v);
    default: return v;
  }
}

}  // namespace iron

// ---------------------------------------------------------------------------
// Host-side error plumbing shared by every entry point.
// ---------------------------------------------------------------------------
namespace iron {
void set_error(const char* fmt, ...);
int fail_einval(const char* fmt, ...);
int check_launch(const char* what);
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Events armed by iron_time_next_launch() for this thread's next entry-point
// call: `start` is recorded at the start of its first kernel, `stop` at the
// end of every kernel it launches (so at the end of the last one).
struct TimingEvents {
  hipEvent_t start;
  hipEvent_t stop;
};
TimingEvents take_timing_events();  // events for this launch (start only on the first)
void disarm_timing();               // end of an entry point (called by check_launch)
// Device phase trace armed by iron_trace_next_launch() for this thread's next
// entry-point call. An entry point whose kernel carries trace points asks for
// `records` 64-byte records (one per workgroup): *buffer receives the armed
// buffer (nullptr when tracing is off), and the trace is disarmed. Returns
// IRON_EINVAL (error set) when the armed buffer is too small.
int take_trace(const char* who, long long records, void** buffer);
void disarm_trace();  // end of an entry point (check_launch, fail_einval)
// 1 when workgroups whose linear ids agree mod 8 run on one XCD of the current
// device (checked once per device, then cached); 0 when they do not, or when
// it cannot be checked now (`stream` is being captured).
int xcd_round_robin(hipStream_t stream);
}  // namespace iron

// Every kernel launch goes through here: with timing events armed, the launch
// records them at the kernel's own start and end (hipExtLaunchKernelGGL).
#define IRON_LAUNCH(kernel, grid, block, shmem, stream, ...)                                          \
  do {                                                                                                \
    const ::iron::TimingEvents _te = ::iron::take_timing_events();                                  \
    if (_te.stop)                                                                                     \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, _te.start, _te.stop, 0, __VA_ARGS__); \
    else                                                                                              \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                            \
  } while (0)

#define IRON_EINVAL 22
#define IRON_REQUIRE(cond, ...)                         \
  do {                                                  \
    if (!(cond)) return ::iron::fail_einval(__VA_ARGS__); \
  } while (0)
