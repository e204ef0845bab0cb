// Data-movement kernels behind the reference's Repeat, StridedCopy and
// Transpose operators (pure copies: HBM-bound, one read and one write of each
// moved element).
#include "iron_common.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

// out[(r * repeat + k) * row_bytes + b] = x[r * row_bytes + b]. One thread
// moves one 16-byte chunk (rows whose byte length is a multiple of 16) or one
// byte (any other row length).
__global__ __launch_bounds__(256) void repeat_rows16_kernel(const uint4* __restrict__ x, uint4* __restrict__ out,
                                                            long long rows, long long chunks, int repeat) {
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= rows * chunks) return;
  const long long r = t / chunks, c = t % chunks;
  const uint4 v = x[t];
  for (int k = 0; k < repeat; ++k) out[(r * repeat + k) * chunks + c] = v;
}

__global__ __launch_bounds__(256) void repeat_rows1_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ out,
                                                           long long rows, long long row_bytes, int repeat) {
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= rows * row_bytes) return;
  const long long r = t / row_bytes, c = t % row_bytes;
  const uint8_t v = x[t];
  for (int k = 0; k < repeat; ++k) out[(r * repeat + k) * row_bytes + c] = v;
}

// A 4-D access pattern split into channels: element i of channel c sits at
//   base + addend + c * chan_step + sum_d idx_d(i) * stride_d
// with idx the row-major decomposition of i over sizes[0..3].
struct Pattern {
  long long size[4];
  long long stride[4];
  long long base;
  long long chan_step;
  const int* addend;  // optional device-resident element addend (runtime parameter)
};

__device__ __forceinline__ long long pattern_offset(const Pattern& p, long long i, int c) {
  long long off = p.base + c * p.chan_step + (p.addend ? *p.addend : 0);
#pragma unroll
  for (int d = 3; d >= 0; --d) {
    const long long q = i % p.size[d];
    i /= p.size[d];
    off += q * p.stride[d];
  }
  return off;
}

// Element k of the copy (channel k / per_channel, index k % per_channel):
// out[dst(k)] = in[src(k)]. Offsets outside either buffer (possible only
// through a runtime addend) are skipped.
template <typename T>
__global__ __launch_bounds__(256) void strided_copy_kernel(const T* __restrict__ in, T* __restrict__ out, Pattern src,
                                                           Pattern dst, long long per_channel, int channels,
                                                           long long in_len, long long out_len) {
  const long long k = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (k >= per_channel * channels) return;
  const int c = static_cast<int>(k / per_channel);
  const long long i = k % per_channel;
  const long long s = pattern_offset(src, i, c), d = pattern_offset(dst, i, c);
  if (s < 0 || s >= in_len || d < 0 || d >= out_len) return;
  out[d] = in[s];
}

// Batched 64x64-tiled transpose: out[b] (cols, rows) = in[b] (rows, cols)^T.
__global__ __launch_bounds__(256) void transpose_batched_kernel(const uint16_t* __restrict__ in,
                                                                uint16_t* __restrict__ out, int rows, int cols) {
  __shared__ uint16_t tile[64][65];
  const size_t mat = static_cast<size_t>(rows) * cols;
  in += blockIdx.z * mat;
  out += blockIdx.z * mat;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e / 64, c = e % 64;
    if (r0 + r < rows && c0 + c < cols) tile[r][c] = in[static_cast<size_t>(r0 + r) * cols + c0 + c];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int c = e / 64, r = e % 64;
    if (r0 + r < rows && c0 + c < cols) out[static_cast<size_t>(c0 + c) * rows + r0 + r] = tile[r][c];
  }
}

// Split a pattern (sizes/strides padded in front to 4-D with size 1, stride 0)
// across channels along its last dimension of size >= 1, channel c starting
// c * (size / channels) * stride further on; the per-channel size is the
// floor of that division (the reference's access-pattern split,
// strided_copy/reference.py:9-37). Returns the elements per channel.
long long split_pattern(const long long* sizes, const long long* strides, int ndim, long long base, int channels,
                        Pattern& p) {
  for (int d = 0; d < 4; ++d) {
    const int s = d - (4 - ndim);
    p.size[d] = s >= 0 ? sizes[s] : 1;
    p.stride[d] = s >= 0 ? strides[s] : 0;
  }
  int highest = -1;
  for (int d = 0; d < 4; ++d)
    if (p.size[d] >= 1) highest = d;
  long long per = 1;
  if (highest < 0) {
    per = 0;
    p.chan_step = 0;
  } else {
    p.size[highest] /= channels;
    p.chan_step = p.size[highest] * p.stride[highest];
    for (int d = 0; d < 4; ++d) per *= p.size[d];
  }
  p.base = base;
  return per;
}

}  // namespace
}  // namespace iron

using namespace iron;

extern "C" int iron_repeat_rows(const void* x, void* out, long long rows, long long row_bytes, int repeat,
                                void* stream) {
  IRON_REQUIRE(x && out && x != out, "iron_repeat_rows: null or aliased pointers");
  IRON_REQUIRE(rows > 0 && row_bytes > 0 && repeat > 0, "iron_repeat_rows: rows, row_bytes and repeat must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (row_bytes % 16 == 0 && aligned16(x) && aligned16(out)) {
    const long long n = rows * (row_bytes / 16);
    IRON_LAUNCH(repeat_rows16_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                static_cast<const uint4*>(x), static_cast<uint4*>(out), rows, row_bytes / 16, repeat);
  } else {
    const long long n = rows * row_bytes;
    IRON_LAUNCH(repeat_rows1_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                static_cast<const uint8_t*>(x), static_cast<uint8_t*>(out), rows, row_bytes, repeat);
  }
  return check_launch("repeat_rows");
}

extern "C" int iron_strided_copy(const void* in, void* out, int elem_bytes, long long in_len, long long out_len,
                                 int ndim_in, const long long* in_sizes, const long long* in_strides,
                                 long long in_offset, const int* in_addend_dev, int ndim_out,
                                 const long long* out_sizes, const long long* out_strides, long long out_offset,
                                 const int* out_addend_dev, int channels, void* stream) {
  IRON_REQUIRE(in && out && in_sizes && in_strides && out_sizes && out_strides, "iron_strided_copy: null pointer");
  IRON_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
               "iron_strided_copy: elem_bytes=%d not in {1,2,4,8}", elem_bytes);
  IRON_REQUIRE(ndim_in >= 1 && ndim_in <= 4 && ndim_out >= 1 && ndim_out <= 4,
               "iron_strided_copy: patterns have 1 to 4 dimensions");
  IRON_REQUIRE(channels >= 1, "iron_strided_copy: channels must be >= 1");
  for (int d = 0; d < ndim_in; ++d) IRON_REQUIRE(in_sizes[d] >= 0, "iron_strided_copy: negative input size");
  for (int d = 0; d < ndim_out; ++d) IRON_REQUIRE(out_sizes[d] >= 0, "iron_strided_copy: negative output size");
  Pattern src, dst;
  const long long per = split_pattern(in_sizes, in_strides, ndim_in, in_offset, channels, src);
  const long long per_out = split_pattern(out_sizes, out_strides, ndim_out, out_offset, channels, dst);
  IRON_REQUIRE(per == per_out, "iron_strided_copy: tap element counts differ (%lld vs %lld per channel); the input "
               "and output access patterns must move the same number of elements", per, per_out);
  if (per == 0) return 0;
  src.addend = in_addend_dev;
  dst.addend = out_addend_dev;
  // with no runtime addend, every offset must be inside its buffer (checked at the extremes)
  auto extent = [](const Pattern& p, int ch, long long& lo, long long& hi) {
    lo = hi = p.base;
    for (int d = 0; d < 4; ++d) {
      const long long span = (p.size[d] - 1) * p.stride[d];
      (span < 0 ? lo : hi) += span;
    }
    const long long cspan = (ch - 1) * p.chan_step;
    (cspan < 0 ? lo : hi) += cspan;
  };
  long long lo, hi;
  extent(src, channels, lo, hi);
  IRON_REQUIRE(in_addend_dev || (lo >= 0 && hi < in_len), "iron_strided_copy: input pattern reaches [%lld, %lld], "
               "outside the %lld-element input", lo, hi, in_len);
  extent(dst, channels, lo, hi);
  IRON_REQUIRE(out_addend_dev || (lo >= 0 && hi < out_len), "iron_strided_copy: output pattern reaches [%lld, %lld], "
               "outside the %lld-element output", lo, hi, out_len);
  const long long n = per * channels;
  IRON_REQUIRE(n < (1LL << 40), "iron_strided_copy: pattern too large");
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (elem_bytes) {
    case 1: IRON_LAUNCH(strided_copy_kernel<uint8_t>, grid, block, 0, s, static_cast<const uint8_t*>(in), static_cast<uint8_t*>(out), src, dst, per, channels, in_len, out_len); break;
    case 2: IRON_LAUNCH(strided_copy_kernel<uint16_t>, grid, block, 0, s, static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), src, dst, per, channels, in_len, out_len); break;
    case 4: IRON_LAUNCH(strided_copy_kernel<uint32_t>, grid, block, 0, s, static_cast<const uint32_t*>(in), static_cast<uint32_t*>(out), src, dst, per, channels, in_len, out_len); break;
    default: IRON_LAUNCH(strided_copy_kernel<unsigned long long>, grid, block, 0, s, static_cast<const unsigned long long*>(in), static_cast<unsigned long long*>(out), src, dst, per, channels, in_len, out_len); break;
  }
  return check_launch("strided_copy");
}

extern "C" int iron_transpose_batched_bf16(const void* in, void* out, int rows, int cols, int batches, void* stream) {
  IRON_REQUIRE(in && out && in != out, "iron_transpose_batched_bf16: null or aliased pointers");
  IRON_REQUIRE(rows > 0 && cols > 0 && batches > 0, "iron_transpose_batched_bf16: empty input");
  dim3 grid((cols + 63) / 64, (rows + 63) / 64, batches);
  IRON_REQUIRE(grid.y < 65536 && grid.z < 65536, "iron_transpose_batched_bf16: too many rows or batches");
  IRON_LAUNCH(transpose_batched_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
              static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), rows, cols);
  return check_launch("transpose_batched_bf16");
}
