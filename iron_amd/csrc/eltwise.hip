// Bandwidth-bound elementwise, normalisation, softmax and RoPE kernels.
//
// Every kernel moves 16 bytes (8 bf16) per lane per access and does its math
// in fp32 with a single bf16 rounding on the way out. Row-wise kernels
// (RMSNorm, softmax) give one 256-thread workgroup to a row; the row stays in
// registers between the reduction and the output pass, so each input byte is
// read from HBM once.
#include "iron_common.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxChunksPerThread = 8;  // rows up to 256*8*8 = 16384 stay in registers

// Block-wide sum/max through LDS (one partial per wave). All threads return it.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* smem) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  v = MAX ? wave_max(v) : wave_sum(v);
  __syncthreads();  // smem may still be read by a previous reduction
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  float r = smem[0];
  for (int w = 1; w < kBlock / kWave; ++w) r = MAX ? fmaxf(r, smem[w]) : r + smem[w];
  return r;
}

// ------------------------------------------------------------------ RMSNorm
// s = x (+ residual); sum_out = s (when requested); out = s * rsqrt(mean(s^2)+eps) [* w]
// PART: the residual is a split-K GEMM output given as its fp32 partial sums
// (splits ranges of rows*cols floats each), merged here as the GEMM's own merge
// does (range order from 0, one bf16 rounding) before the add.
template <int CPT, bool PART = false>
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ resid,
                                                         const uint16_t* __restrict__ w, uint16_t* out,
                                                         uint16_t* sum_out, int cols, float eps,
                                                         const float* __restrict__ part, int splits) {
  __shared__ float smem[kBlock / kWave];
  const size_t row = blockIdx.x;
  const int nch = cols >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * cols);
  const uint4* rr = resid ? reinterpret_cast<const uint4*>(resid + row * cols) : nullptr;
  float v[CPT][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * kBlock;
    if (c < nch) {
      const uint4 a = xr[c];
      const uint32_t wa[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[i][2 * e] = lo_bf16(wa[e]);
        v[i][2 * e + 1] = hi_bf16(wa[e]);
      }
      if (PART) {
        const size_t range4 = static_cast<size_t>(gridDim.x) * cols / 4;  // float4s per K range
        const float4* pp = reinterpret_cast<const float4*>(part + row * cols) + 2 * c;
        float r[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int kb = 0; kb < splits; ++kb) {
          const float4 u = pp[kb * range4], q = pp[kb * range4 + 1];
          r[0] += u.x; r[1] += u.y; r[2] += u.z; r[3] += u.w;
          r[4] += q.x; r[5] += q.y; r[6] += q.z; r[7] += q.w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[i][e] = bf16_to_f32(f32_to_bf16(v[i][e] + bf16_to_f32(f32_to_bf16(r[e]))));
      } else if (rr) {
        const uint4 b = rr[c];
        const uint32_t wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // the sum is rounded to bf16 (it is the new residual stream)
          v[i][2 * e] = bf16_to_f32(f32_to_bf16(v[i][2 * e] + lo_bf16(wb[e])));
          v[i][2 * e + 1] = bf16_to_f32(f32_to_bf16(v[i][2 * e + 1] + hi_bf16(wb[e])));
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[i][e], v[i][e], ss);
    }
  }
  ss = block_reduce<false>(ss, smem);
  const float inv = rsqrtf(ss / static_cast<float>(cols) + eps);
  uint4* orow = reinterpret_cast<uint4*>(out + row * cols);
  uint4* srow = sum_out ? reinterpret_cast<uint4*>(sum_out + row * cols) : nullptr;
  const uint4* wv = reinterpret_cast<const uint4*>(w);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * kBlock;
    if (c < nch) {
      float g[8];
      if (w) {
        const uint4 q = wv[c];
        const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g[2 * e] = lo_bf16(wq[e]);
          g[2 * e + 1] = hi_bf16(wq[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] = 1.f;
      }
      if (srow)
        srow[c] = make_uint4(pack_bf16x2(v[i][0], v[i][1]), pack_bf16x2(v[i][2], v[i][3]),
                             pack_bf16x2(v[i][4], v[i][5]), pack_bf16x2(v[i][6], v[i][7]));
      orow[c] = make_uint4(pack_bf16x2(v[i][0] * inv * g[0], v[i][1] * inv * g[1]),
                           pack_bf16x2(v[i][2] * inv * g[2], v[i][3] * inv * g[3]),
                           pack_bf16x2(v[i][4] * inv * g[4], v[i][5] * inv * g[5]),
                           pack_bf16x2(v[i][6] * inv * g[6], v[i][7] * inv * g[7]));
    }
  }
}

// --------------------------------------------------------------- elementwise
enum EwOp : int { EW_ADD = 0, EW_MUL = 1, EW_SILU = 2, EW_SILU_MUL = 3, EW_GELU_TANH = 4 };

__device__ __forceinline__ float ew_apply(int op, float a, float b) {
  switch (op) {
    case EW_ADD: return a + b;
    case EW_MUL: return a * b;
    case EW_SILU: return silu_f32(a);
    case EW_SILU_MUL: return silu_f32(a) * b;
    default: return gelu_tanh_f32(a);
  }
}

template <int OP>
__global__ __launch_bounds__(kBlock) void eltwise_kernel(const uint16_t* __restrict__ a,
                                                         const uint16_t* __restrict__ b, uint16_t* out,
                                                         long long n) {
  const long long stride = static_cast<long long>(gridDim.x) * kBlock;
  const long long nvec = n >> 3;
  for (long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x; i < nvec; i += stride) {
    const uint4 va = reinterpret_cast<const uint4*>(a)[i];
    const uint4 vb = (OP == EW_ADD || OP == EW_MUL || OP == EW_SILU_MUL) ? reinterpret_cast<const uint4*>(b)[i]
                                                                          : make_uint4(0, 0, 0, 0);
    const uint32_t wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(ew_apply(OP, lo_bf16(wa[e]), lo_bf16(wb[e])), ew_apply(OP, hi_bf16(wa[e]), hi_bf16(wb[e])));
    reinterpret_cast<uint4*>(out)[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  // tail (n % 8 elements), handled by the first block
  if (blockIdx.x == 0) {
    const long long t = (nvec << 3) + threadIdx.x;
    if (t < n) {
      const float bv = (OP == EW_ADD || OP == EW_MUL || OP == EW_SILU_MUL) ? bf16_to_f32(b[t]) : 0.f;
      out[t] = f32_to_bf16(ew_apply(OP, bf16_to_f32(a[t]), bv));
    }
  }
}

// ------------------------------------------------------------------ softmax
// Row softmax over `cols`; columns >= valid are treated as -inf (output 0).
// valid_ptr (device int32, may be NULL) overrides `valid` at run time so a
// captured graph can change the context length between replays.
template <int CPT>
__global__ __launch_bounds__(kBlock) void softmax_kernel(const uint16_t* __restrict__ x, uint16_t* out,
                                                         int cols, int valid, const int* valid_ptr) {
  __shared__ float smem[kBlock / kWave];
  const size_t row = blockIdx.x;
  if (valid_ptr) valid = *valid_ptr;
  valid = valid < 0 ? 0 : (valid > cols ? cols : valid);
  const int nch = cols >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * cols);
  float v[CPT][8];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * kBlock;
    if (c < nch) {
      const uint4 q = xr[c];
      const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[i][2 * e] = (c * 8 + 2 * e < valid) ? lo_bf16(wq[e]) : -INFINITY;
        v[i][2 * e + 1] = (c * 8 + 2 * e + 1 < valid) ? hi_bf16(wq[e]) : -INFINITY;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) m = fmaxf(m, v[i][e]);
    }
  }
  m = block_reduce<true>(m, smem);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * kBlock;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[i][e] = (v[i][e] == -INFINITY) ? 0.f : __expf(v[i][e] - m);
        s += v[i][e];
      }
    }
  }
  s = block_reduce<false>(s, smem);
  const float inv = s > 0.f ? 1.f / s : 0.f;
  uint4* orow = reinterpret_cast<uint4*>(out + row * cols);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * kBlock;
    if (c < nch)
      orow[c] = make_uint4(pack_bf16x2(v[i][0] * inv, v[i][1] * inv), pack_bf16x2(v[i][2] * inv, v[i][3] * inv),
                           pack_bf16x2(v[i][4] * inv, v[i][5] * inv), pack_bf16x2(v[i][6] * inv, v[i][7] * inv));
  }
}

// --------------------------------------------------------------------- RoPE
// x (rows, cols); angles (angle_rows, cols) interleaved [cos0, sin0, cos1, ...]
// (bf16 or fp32); row r uses angle row r / (rows / angle_rows).
// method 0: rotate halves (x1, x2) -> (x1 c - x2 s, x2 c + x1 s)
// method 1: rotate interleaved pairs (xe, xo) -> (xe c - xo s, xe s + xo c)
// One thread per rotated pair.
__global__ __launch_bounds__(kBlock) void rope_kernel(const uint16_t* __restrict__ x, const void* angles,
                                                      int angles_fp32, uint16_t* out, int rows, int cols,
                                                      int angle_rows, int method) {
  const long long t = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
  const int half = cols >> 1;
  if (t >= static_cast<long long>(rows) * half) return;
  const int r = static_cast<int>(t / half), i = static_cast<int>(t % half);
  const int ar = r / (rows / angle_rows);
  float c, s;
  if (angles_fp32) {
    const float* ap = static_cast<const float*>(angles) + static_cast<size_t>(ar) * cols;
    c = ap[2 * i];
    s = ap[2 * i + 1];
  } else {
    const uint16_t* ap = static_cast<const uint16_t*>(angles) + static_cast<size_t>(ar) * cols;
    c = bf16_to_f32(ap[2 * i]);
    s = bf16_to_f32(ap[2 * i + 1]);
  }
  const uint16_t* xr = x + static_cast<size_t>(r) * cols;
  uint16_t* orow = out + static_cast<size_t>(r) * cols;
  if (method == 0) {
    const float x1 = bf16_to_f32(xr[i]), x2 = bf16_to_f32(xr[i + half]);
    orow[i] = f32_to_bf16(rot_sub(x1, c, x2, s));
    orow[i + half] = f32_to_bf16(rot_add(x2, c, x1, s));
  } else {
    const float xe = bf16_to_f32(xr[2 * i]), xo = bf16_to_f32(xr[2 * i + 1]);
    orow[2 * i] = f32_to_bf16(rot_sub(xe, c, xo, s));
    orow[2 * i + 1] = f32_to_bf16(rot_add(xe, s, xo, c));
  }
}

int ew_launch(int op, const void* a, const void* b, void* out, long long n, hipStream_t s) {
  IRON_REQUIRE(a && out && n > 0, "eltwise: null pointer or empty size");
  IRON_REQUIRE(aligned16(a) && aligned16(out) && (!b || aligned16(b)), "eltwise: operands must be 16-byte aligned");
  const long long nvec = n >> 3;
  long long blocks = (nvec + kBlock - 1) / kBlock;
  if (blocks < 1) blocks = 1;
  if (blocks > 65535) blocks = 65535;
  const auto* A = static_cast<const uint16_t*>(a);
  const auto* B = static_cast<const uint16_t*>(b);
  auto* O = static_cast<uint16_t*>(out);
  dim3 g(static_cast<unsigned>(blocks)), blk(kBlock);
  switch (op) {
    case EW_ADD: IRON_LAUNCH((eltwise_kernel<EW_ADD>), g, blk, 0, s, A, B, O, n); break;
    case EW_MUL: IRON_LAUNCH((eltwise_kernel<EW_MUL>), g, blk, 0, s, A, B, O, n); break;
    case EW_SILU: IRON_LAUNCH((eltwise_kernel<EW_SILU>), g, blk, 0, s, A, B, O, n); break;
    case EW_SILU_MUL: IRON_LAUNCH((eltwise_kernel<EW_SILU_MUL>), g, blk, 0, s, A, B, O, n); break;
    default: IRON_LAUNCH((eltwise_kernel<EW_GELU_TANH>), g, blk, 0, s, A, B, O, n); break;
  }
  return check_launch("eltwise");
}

}  // namespace
}  // namespace iron

using namespace iron;

extern "C" int iron_rmsnorm(const void* x, const void* residual, const void* w, void* out, void* sum_out,
                            int rows, int cols, float eps, void* stream) {
  IRON_REQUIRE(x && out, "iron_rmsnorm: null pointer");
  IRON_REQUIRE(rows > 0 && cols > 0 && cols % 8 == 0, "iron_rmsnorm: rows=%d cols=%d (cols must be a multiple of 8)",
               rows, cols);
  IRON_REQUIRE(cols <= kBlock * kMaxChunksPerThread * 8, "iron_rmsnorm: cols=%d exceeds %d", cols,
               kBlock * kMaxChunksPerThread * 8);
  IRON_REQUIRE(aligned16(x) && aligned16(out) && (!w || aligned16(w)) && (!residual || aligned16(residual)) &&
                   (!sum_out || aligned16(sum_out)),
               "iron_rmsnorm: operands must be 16-byte aligned");
  IRON_REQUIRE(!(sum_out && !residual), "iron_rmsnorm: sum_out needs a residual");
  const int nch = cols / 8;
  const int cpt = (nch + kBlock - 1) / kBlock;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  auto R = static_cast<const uint16_t*>(residual);
  auto W = static_cast<const uint16_t*>(w);
  auto O = static_cast<uint16_t*>(out);
  auto S = static_cast<uint16_t*>(sum_out);
  dim3 g(rows), b(kBlock);
  if (cpt <= 1) IRON_LAUNCH((rmsnorm_kernel<1>), g, b, 0, s, X, R, W, O, S, cols, eps, nullptr, 0);
  else if (cpt <= 2) IRON_LAUNCH((rmsnorm_kernel<2>), g, b, 0, s, X, R, W, O, S, cols, eps, nullptr, 0);
  else if (cpt <= 4) IRON_LAUNCH((rmsnorm_kernel<4>), g, b, 0, s, X, R, W, O, S, cols, eps, nullptr, 0);
  else IRON_LAUNCH((rmsnorm_kernel<8>), g, b, 0, s, X, R, W, O, S, cols, eps, nullptr, 0);
  return check_launch("rmsnorm");
}

extern "C" int iron_rmsnorm_splitk(const void* x, const float* partial, int splits, const void* w, void* out,
                                   void* sum_out, int rows, int cols, float eps, void* stream) {
  IRON_REQUIRE(x && partial && out, "iron_rmsnorm_splitk: null pointer");
  IRON_REQUIRE(splits >= 1 && splits <= 64, "iron_rmsnorm_splitk: splits=%d outside [1, 64]", splits);
  IRON_REQUIRE(rows > 0 && cols > 0 && cols % 8 == 0,
               "iron_rmsnorm_splitk: rows=%d cols=%d (cols must be a multiple of 8)", rows, cols);
  IRON_REQUIRE(cols <= kBlock * kMaxChunksPerThread * 8, "iron_rmsnorm_splitk: cols=%d exceeds %d", cols,
               kBlock * kMaxChunksPerThread * 8);
  IRON_REQUIRE(aligned16(x) && aligned16(out) && aligned16(partial) && (!w || aligned16(w)) &&
                   (!sum_out || aligned16(sum_out)),
               "iron_rmsnorm_splitk: operands must be 16-byte aligned");
  const int cpt = (cols / 8 + kBlock - 1) / kBlock;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  auto W = static_cast<const uint16_t*>(w);
  auto O = static_cast<uint16_t*>(out);
  auto S = static_cast<uint16_t*>(sum_out);
  dim3 g(rows), b(kBlock);
  if (cpt <= 1) IRON_LAUNCH((rmsnorm_kernel<1, true>), g, b, 0, s, X, nullptr, W, O, S, cols, eps, partial, splits);
  else if (cpt <= 2) IRON_LAUNCH((rmsnorm_kernel<2, true>), g, b, 0, s, X, nullptr, W, O, S, cols, eps, partial, splits);
  else if (cpt <= 4) IRON_LAUNCH((rmsnorm_kernel<4, true>), g, b, 0, s, X, nullptr, W, O, S, cols, eps, partial, splits);
  else IRON_LAUNCH((rmsnorm_kernel<8, true>), g, b, 0, s, X, nullptr, W, O, S, cols, eps, partial, splits);
  return check_launch("rmsnorm_splitk");
}

extern "C" int iron_add(const void* a, const void* b, void* out, long long n, void* stream) {
  IRON_REQUIRE(b, "iron_add: null pointer");
  return ew_launch(EW_ADD, a, b, out, n, static_cast<hipStream_t>(stream));
}

extern "C" int iron_mul(const void* a, const void* b, void* out, long long n, void* stream) {
  IRON_REQUIRE(b, "iron_mul: null pointer");
  return ew_launch(EW_MUL, a, b, out, n, static_cast<hipStream_t>(stream));
}

extern "C" int iron_silu(const void* x, void* out, long long n, void* stream) {
  return ew_launch(EW_SILU, x, nullptr, out, n, static_cast<hipStream_t>(stream));
}

extern "C" int iron_silu_mul(const void* gate, const void* up, void* out, long long n, void* stream) {
  IRON_REQUIRE(up, "iron_silu_mul: null pointer");
  return ew_launch(EW_SILU_MUL, gate, up, out, n, static_cast<hipStream_t>(stream));
}

extern "C" int iron_gelu(const void* x, void* out, long long n, void* stream) {
  return ew_launch(EW_GELU_TANH, x, nullptr, out, n, static_cast<hipStream_t>(stream));
}

extern "C" int iron_softmax(const void* x, void* out, int rows, int cols, int valid_cols,
                            const int* valid_cols_dev, void* stream) {
  IRON_REQUIRE(x && out, "iron_softmax: null pointer");
  IRON_REQUIRE(rows > 0 && cols > 0 && cols % 8 == 0, "iron_softmax: rows=%d cols=%d (cols must be a multiple of 8)",
               rows, cols);
  IRON_REQUIRE(cols <= kBlock * kMaxChunksPerThread * 8, "iron_softmax: cols=%d exceeds %d", cols,
               kBlock * kMaxChunksPerThread * 8);
  IRON_REQUIRE(aligned16(x) && aligned16(out), "iron_softmax: operands must be 16-byte aligned");
  const int cpt = (cols / 8 + kBlock - 1) / kBlock;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  auto O = static_cast<uint16_t*>(out);
  dim3 g(rows), b(kBlock);
  if (cpt <= 1) IRON_LAUNCH((softmax_kernel<1>), g, b, 0, s, X, O, cols, valid_cols, valid_cols_dev);
  else if (cpt <= 2) IRON_LAUNCH((softmax_kernel<2>), g, b, 0, s, X, O, cols, valid_cols, valid_cols_dev);
  else if (cpt <= 4) IRON_LAUNCH((softmax_kernel<4>), g, b, 0, s, X, O, cols, valid_cols, valid_cols_dev);
  else IRON_LAUNCH((softmax_kernel<8>), g, b, 0, s, X, O, cols, valid_cols, valid_cols_dev);
  return check_launch("softmax");
}

extern "C" int iron_rope(const void* x, const void* angles, int angles_fp32, void* out, int rows, int cols,
                         int angle_rows, int method, void* stream) {
  IRON_REQUIRE(x && angles && out, "iron_rope: null pointer");
  IRON_REQUIRE(rows > 0 && cols > 0 && cols % 2 == 0, "iron_rope: rows=%d cols=%d (cols must be even)", rows, cols);
  IRON_REQUIRE(angle_rows > 0 && angle_rows <= rows && rows % angle_rows == 0,
               "iron_rope: angle_rows=%d must divide rows=%d", angle_rows, rows);
  IRON_REQUIRE(method == 0 || method == 1, "iron_rope: method_type must be 0 or 1, got %d", method);
  IRON_REQUIRE(out != x || method == 0 || method == 1, "iron_rope: bad aliasing");
  const long long pairs = static_cast<long long>(rows) * (cols / 2);
  IRON_LAUNCH(rope_kernel, dim3(static_cast<unsigned>((pairs + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), angles, angles_fp32,
                     static_cast<uint16_t*>(out), rows, cols, angle_rows, method);
  return check_launch("rope");
}
