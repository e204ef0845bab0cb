// Device phase trace (iron_trace_next_launch): kernels with trace points write
// one 64-byte record per workgroup into the armed buffer, from thread 0:
//   32-bit words 0-3: kernel id (TraceKernel), workgroup index, XCC_ID, HW_ID
//   bytes 16 + 8 k:   stamp k (s_memrealtime: the 100 MHz constant clock
//                     shared by every XCD), k < kTraceStamps
// Stamp k is the moment the workgroup's wave 0 passed the kernel's k-th trace
// point; a point the workgroup never reaches stays as the caller zero-filled
// it. The GEMV, decode attention and bf16 GEMM kernels have a separate traced instance, launched
// only while a buffer is armed (their untraced instance holds no trace code: a
// clock read at entry measured 0.1 us on the int4 GEMV). In a kernel without
// one, each trace point is a uniform branch on the trace pointer, and the
// start clock is read unconditionally at entry (trace_clock) and recorded
// later (trace_write): a test of the trace pointer at entry would make the
// kernel wait for that argument before it issues its other argument loads.
#pragma once

#include "iron_common.hpp"

namespace iron {
namespace {

enum TraceKernel : unsigned { kTraceGqaDecode = 1, kTraceGemvI4 = 2, kTraceSwigluDecode = 3, kTraceGemm = 4 };
constexpr int kTraceStamps = 6;
constexpr int kTraceRecordBytes = 64;

// The constant clock, read where this statement stands (volatile assembly is
// not moved across other volatile assembly); its value is ready after the next
// wait for scalar loads, which trace_write performs before it reads it.
__device__ __forceinline__ unsigned long long trace_clock() {
  unsigned long long t;
  asm volatile("s_memrealtime %0" : "=s"(t));
  return t;
}

__device__ __forceinline__ void trace_write(void* trace, unsigned kernel, unsigned wg, int k, unsigned long long t) {
  if (trace == nullptr) return;
  asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(t));
  if (threadIdx.x != 0) return;
  unsigned char* rec = static_cast<unsigned char*>(trace) + static_cast<size_t>(wg) * kTraceRecordBytes;
  if (k == 0) {
    unsigned xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    *reinterpret_cast<uint4*>(rec) = make_uint4(kernel, wg, xcc & 0xfu, hw);
  }
  *reinterpret_cast<unsigned long long*>(rec + 16 + 8 * k) = t;
}

// A trace point after the start: the clock is read only when tracing.
__device__ __forceinline__ void trace_stamp(void* trace, unsigned kernel, unsigned wg, int k) {
  if (trace == nullptr) return;
  trace_write(trace, kernel, wg, k, trace_clock());
}

}  // namespace
}  // namespace iron
