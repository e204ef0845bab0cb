// bf16 GEMM on MFMA for prefill: C[M][N] = epilogue(sum_k A[m][k] * B[n][k]).
//
// "NT" form: A (M, K) and B (N, K) are both K-contiguous, which is how
// nn.Linear weights are stored (out_features, in_features) and what the MFMA
// operands want: with v_mfma_f32_32x32x16_bf16 every lane feeds 8 consecutive
// k of one row (lane l -> row l%32, k (l/32)*8..+8), so each operand fragment
// is a single 16-byte LDS read. Other layouts are reduced to this one on the
// host (B row-major (K, N) through a transpose, C column-major by swapping the
// operands: C^T = B A^T).
//
// Tiling: 128x128 output tile per 256-thread workgroup, 4 waves in 2x2, each
// wave owns 64x64 = 2x2 MFMA tiles (64 fp32 accumulators per lane). K advances
// 64 per step through a double-buffered LDS ring (one barrier per step).
// Global loads run two steps ahead through two register stages: with one
// workgroup per CU (the prefill shapes) a single step of look-ahead leaves the
// MFMAs waiting on L2 latency. LDS rows are 128 B (64 bf16); the 16-byte chunk
// c of row r lives at slot c ^ ((r / 2) % 8) (see swz).
// Tile order is XCD-aware: workgroup b runs on XCD b % 8, and consecutive
// tiles along M (which share one B column block) go to the same XCD, so a
// weight block is fetched from HBM into one L2 only.
// Epilogue: round to bf16, then activation and clamp (the flm.GEMM order),
// staged through LDS so global stores are 16-byte and row-contiguous.
#include "iron_common.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int kChunks = BK / 8;  // 16-byte chunks per LDS row

struct GemmArgs {
  const uint16_t* A;  // (M, K)
  const uint16_t* B;  // (N, K)
  uint16_t* C;        // (M, N), row stride ldc
  int M, N, K;
  long long ldc;
  int epi;
  int clamp;
  float lo, hi;
  float* partial;  // split-K: fp32 (splits, M, N) partial sums instead of C
  int splits;      // K ranges (1 = no split)
};

// A 16-byte LDS access of 16 lanes covers all 64 banks once when their 16
// consecutive rows use 16 distinct (row parity, slot) pairs: the slot is
// chunk ^ ((row / 2) % 8). (chunk ^ (row % 8) repeats every 8 rows, which put
// rows r and r + 8 on the same banks: a 2-way conflict on every fragment read.)
__device__ __forceinline__ int swz(int row, int chunk) { return row * kChunks + (chunk ^ ((row >> 1) & 7)); }

typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

// One step's global loads into register stage r (4 A + 4 B chunks per
// thread). GUARD zero-fills rows past M / N; steps past the end reload the
// last step (never stored).
#define IRON_GEMM_LOAD_CHUNK(r, i, k0)                                                                   \
  {                                                                                                      \
    const int id_ = tid + (i) * kThreads, row_ = id_ >> 3, c_ = id_ & 7;                                 \
    const int gm_ = m0 + row_, gn_ = n0 + row_;                                                          \
    r[i] = (!GUARD || gm_ < a.M) ? *reinterpret_cast<const u32x4v*>(Ag + static_cast<size_t>(gm_) * a.K +   \
                                                                     (k0) + c_ * 8)                       \
                                 : u32x4v{0, 0, 0, 0};                                                   \
    r[4 + (i)] = (!GUARD || gn_ < a.N) ? *reinterpret_cast<const u32x4v*>(Bg + static_cast<size_t>(gn_) *  \
                                                                          a.K + (k0) + c_ * 8)           \
                                       : u32x4v{0, 0, 0, 0};                                             \
  }
#define IRON_GEMM_LOAD(r, step)                                                                          \
  {                                                                                                      \
    const int k0_ = min(step, nk - 1) * BK;                                                              \
    IRON_GEMM_LOAD_CHUNK(r, 0, k0_) IRON_GEMM_LOAD_CHUNK(r, 1, k0_)                                      \
    IRON_GEMM_LOAD_CHUNK(r, 2, k0_) IRON_GEMM_LOAD_CHUNK(r, 3, k0_)                                      \
  }
#define IRON_GEMM_STORE_CHUNK(r, i, As_, Bs_)                                                            \
  {                                                                                                      \
    const int id_ = tid + (i) * kThreads, row_ = id_ >> 3, c_ = id_ & 7;                                 \
    As_[swz(row_, c_)] = r[i];                                                                           \
    Bs_[swz(row_, c_)] = r[4 + (i)];                                                                     \
  }
#define IRON_GEMM_STORE(r, buf)                                                                          \
  {                                                                                                      \
    u32x4v* As_ = reinterpret_cast<u32x4v*>(smem + (buf) * 2 * BM * kChunks);                            \
    u32x4v* Bs_ = As_ + BM * kChunks;                                                                    \
    IRON_GEMM_STORE_CHUNK(r, 0, As_, Bs_) IRON_GEMM_STORE_CHUNK(r, 1, As_, Bs_)                          \
    IRON_GEMM_STORE_CHUNK(r, 2, As_, Bs_) IRON_GEMM_STORE_CHUNK(r, 3, As_, Bs_)                          \
  }
// 4 k-slices of 16: per slice each wave reads 2 A and 2 B fragments (one
// 16-byte LDS read each) and issues its 2x2 MFMAs.
#define IRON_GEMM_COMPUTE(buf)                                                                           \
  {                                                                                                      \
    const uint4* As_ = smem + (buf) * 2 * BM * kChunks;                                                  \
    const uint4* Bs_ = As_ + BM * kChunks;                                                               \
    _Pragma("unroll") for (int kk = 0; kk < BK / 16; ++kk) {                                             \
      const int c_ = kk * 2 + (lane >> 5);                                                               \
      bf16x8_t fa[2], fb[2];                                                                             \
      _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                                    \
        fa[i] = __builtin_bit_cast(bf16x8_t, As_[swz(wm * 64 + i * 32 + (lane & 31), c_)]);              \
        fb[i] = __builtin_bit_cast(bf16x8_t, Bs_[swz(wn * 64 + i * 32 + (lane & 31), c_)]);              \
      }                                                                                                  \
      _Pragma("unroll") for (int i = 0; i < 2; ++i)                                                      \
      _Pragma("unroll") for (int j = 0; j < 2; ++j)                                                      \
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);           \
    }                                                                                                    \
  }

template <bool GUARD>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(GemmArgs a) {
  __shared__ uint4 smem[2 * 2 * BM * kChunks];  // [buf][A|B][row][chunk] = 64 KiB
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware tile order (over tiles x K ranges)
  const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
  const int T = tiles_m * tiles_n * a.splits;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;
  const int kb = t / (tiles_m * tiles_n);
  t %= tiles_m * tiles_n;
  const int tm = t % tiles_m, tn = t / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = a.K / BK / a.splits;  // steps in this workgroup's K range
  const uint16_t* Ag = a.A + static_cast<size_t>(kb) * nk * BK;
  const uint16_t* Bg = a.B + static_cast<size_t>(kb) * nk * BK;

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // two register stages: steps s+1 and s+2 are in flight while step s computes
  u32x4v st0[8], st1[8];
  IRON_GEMM_LOAD(st0, 0);
  IRON_GEMM_LOAD(st1, 1);
  IRON_GEMM_STORE(st0, 0);
  __syncthreads();
  for (int it = 0; it < nk; it += 2) {
    IRON_GEMM_LOAD(st0, it + 2);
    IRON_GEMM_COMPUTE(0);  // step it
    if (it + 1 < nk) IRON_GEMM_STORE(st1, 1);
    __syncthreads();
    if (it + 1 < nk) {
      IRON_GEMM_LOAD(st1, it + 3);
      IRON_GEMM_COMPUTE(1);  // step it + 1
      if (it + 2 < nk) IRON_GEMM_STORE(st0, 0);
      __syncthreads();
    }
  }

  if (a.partial) {  // split-K: raw fp32 sums straight from the accumulators
    float* P = a.partial + static_cast<size_t>(kb) * a.M * a.N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int gm = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          const int gn = n0 + wn * 64 + j * 32 + (lane & 31);
          if (!GUARD || (gm < a.M && gn < a.N)) P[static_cast<size_t>(gm) * a.N + gn] = acc[i][j][v];
        }
    return;
  }

  // epilogue through LDS: C tile as bf16 [128][128] (32 KiB)
  uint16_t* Cs = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = wn * 64 + j * 32 + (lane & 31);
        float x = acc[i][j][v];
        if (a.epi != EPI_NONE || a.clamp) {
          x = bf16_to_f32(f32_to_bf16(x));
          x = apply_epilogue(x, a.epi);
          if (a.clamp) x = fminf(fmaxf(x, a.lo), a.hi);
        }
        Cs[row * BN + col] = f32_to_bf16(x);
      }
  __syncthreads();
  const bool full_n = (n0 + BN <= a.N) && (a.ldc % 8 == 0);
#pragma unroll
  for (int i = 0; i < (BM * BN / 8) / kThreads; ++i) {
    const int id = tid + i * kThreads, row = id >> 4, c = id & 15;
    const int gm = m0 + row, gn = n0 + c * 8;
    if (gm >= a.M) continue;
    const uint4 v = reinterpret_cast<const uint4*>(Cs)[row * (BN / 8) + c];
    uint16_t* dst = a.C + static_cast<size_t>(gm) * a.ldc + gn;
    if (full_n) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
      for (int q = 0; q < 8; ++q)
        if (gn + q < a.N) dst[q] = e[q];
    }
  }
}

#undef IRON_GEMM_LOAD_CHUNK
#undef IRON_GEMM_LOAD
#undef IRON_GEMM_STORE_CHUNK
#undef IRON_GEMM_STORE
#undef IRON_GEMM_COMPUTE

// Split-K merge: C = clamp(act(bf16(sum_kb partial[kb]))), the same epilogue
// order as the single-pass kernel. One thread per output element.
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmArgs a) {
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  const long long mn = static_cast<long long>(a.M) * a.N;
  if (t >= mn) return;
  float x = 0.f;
  for (int kb = 0; kb < a.splits; ++kb) x += a.partial[kb * mn + t];
  if (a.epi != EPI_NONE || a.clamp) {
    x = bf16_to_f32(f32_to_bf16(x));
    x = apply_epilogue(x, a.epi);
    if (a.clamp) x = fminf(fmaxf(x, a.lo), a.hi);
  }
  const long long m = t / a.N, n = t % a.N;
  a.C[m * a.ldc + n] = f32_to_bf16(x);
}

// 64x64 tiled transpose through LDS: out (cols, rows) = in (rows, cols)^T.
__global__ __launch_bounds__(256) void transpose_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                        int rows, int cols) {
  __shared__ uint16_t tile[64][65];
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

}  // namespace
}  // namespace iron

using namespace iron;

static int gemm_check(const char* fn, const void* A, const void* B, const void* C, int M, int N, int K,
                      long long ldc, int epilogue, int has_clamp, float clamp_lo, float clamp_hi) {
  IRON_REQUIRE(A && B && C, "%s: null pointer", fn);
  IRON_REQUIRE(M > 0 && N > 0 && K > 0, "%s: M=%d N=%d K=%d must be positive", fn, M, N, K);
  IRON_REQUIRE(K % BK == 0, "%s: K=%d must be a multiple of %d", fn, K, BK);
  IRON_REQUIRE(aligned16(A) && aligned16(B), "%s: A and B must be 16-byte aligned", fn);
  IRON_REQUIRE(ldc >= N, "%s: ldc=%lld < N=%d", fn, ldc, N);
  IRON_REQUIRE(epilogue >= EPI_NONE && epilogue <= EPI_GELU_SIGMOID, "%s: bad epilogue %d", fn, epilogue);
  IRON_REQUIRE(!has_clamp || clamp_lo <= clamp_hi, "%s: clamp min > max", fn);
  if ((ldc % 8 == 0) && !aligned16(C)) return fail_einval("%s: C must be 16-byte aligned", fn);
  return 0;
}

static void gemm_launch(const GemmArgs& a, hipStream_t s) {
  const long long tiles = static_cast<long long>((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN) * a.splits;
  if (a.M % BM == 0 && a.N % BN == 0)
    IRON_LAUNCH(gemm_nt_kernel<false>, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, s, a);
  else
    IRON_LAUNCH(gemm_nt_kernel<true>, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, s, a);
}

extern "C" int iron_gemm_bf16_nt(const void* A, const void* B, void* C, int M, int N, int K, long long ldc,
                                 int epilogue, int has_clamp, float clamp_lo, float clamp_hi, void* stream) {
  if (int rc = gemm_check("iron_gemm_bf16_nt", A, B, C, M, N, K, ldc, epilogue, has_clamp, clamp_lo, clamp_hi))
    return rc;
  const long long tiles = static_cast<long long>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  IRON_REQUIRE(tiles < (1LL << 31), "iron_gemm_bf16_nt: problem too large");
  GemmArgs a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), static_cast<uint16_t*>(C), M, N, K,
             ldc, epilogue, has_clamp, clamp_lo, clamp_hi, nullptr, 1};
  gemm_launch(a, static_cast<hipStream_t>(stream));
  return check_launch("gemm_bf16_nt");
}

extern "C" int iron_gemm_splitk_choose(int M, int N, int K) {
  // Split K while the workgroups stay within 1.25x the 256 CUs and every K range
  // keeps >= 8 steps of 64; at most 8 ranges.
  if (M <= 0 || N <= 0 || K <= 0 || K % BK) return 1;
  const long long tiles = static_cast<long long>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  int s = 1;
  while (s < 8 && tiles * s * 2 <= 320 && (K / BK) % (s * 2) == 0 && K / BK / (s * 2) >= 8) s *= 2;
  return s;
}

extern "C" long long iron_gemm_splitk_workspace_bytes(int M, int N, int splits) {
  if (M <= 0 || N <= 0 || splits <= 0) return -1;
  return splits > 1 ? static_cast<long long>(splits) * M * N * 4 : 0;
}

extern "C" int iron_gemm_bf16_nt_splitk(const void* A, const void* B, void* C, int M, int N, int K, long long ldc,
                                        int epilogue, int has_clamp, float clamp_lo, float clamp_hi, int splits,
                                        void* workspace, long long workspace_bytes, void* stream) {
  if (int rc = gemm_check("iron_gemm_bf16_nt_splitk", A, B, C, M, N, K, ldc, epilogue, has_clamp, clamp_lo,
                          clamp_hi))
    return rc;
  IRON_REQUIRE(splits >= 1 && (K / BK) % splits == 0,
               "iron_gemm_bf16_nt_splitk: splits=%d must divide the %d K steps of 64", splits, K / BK);
  if (splits == 1)
    return iron_gemm_bf16_nt(A, B, C, M, N, K, ldc, epilogue, has_clamp, clamp_lo, clamp_hi, stream);
  const long long need = static_cast<long long>(splits) * M * N * 4;
  IRON_REQUIRE(workspace && workspace_bytes >= need, "iron_gemm_bf16_nt_splitk: workspace of %lld bytes < %lld",
               workspace_bytes, need);
  IRON_REQUIRE(aligned16(workspace), "iron_gemm_bf16_nt_splitk: workspace must be 16-byte aligned");
  const long long tiles = static_cast<long long>((M + BM - 1) / BM) * ((N + BN - 1) / BN) * splits;
  IRON_REQUIRE(tiles < (1LL << 31) && static_cast<long long>(M) * N < (1LL << 38),
               "iron_gemm_bf16_nt_splitk: problem too large");
  GemmArgs a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), static_cast<uint16_t*>(C), M, N, K,
             ldc, epilogue, has_clamp, clamp_lo, clamp_hi, static_cast<float*>(workspace), splits};
  hipStream_t s = static_cast<hipStream_t>(stream);
  gemm_launch(a, s);
  const long long mn = static_cast<long long>(M) * N;
  IRON_LAUNCH(gemm_splitk_reduce_kernel, dim3(static_cast<unsigned>((mn + 255) / 256)), dim3(256), 0, s, a);
  return check_launch("gemm_bf16_nt_splitk");
}

extern "C" int iron_transpose_bf16(const void* in, void* out, int rows, int cols, void* stream) {
  IRON_REQUIRE(in && out && in != out, "iron_transpose_bf16: null or aliased pointers");
  IRON_REQUIRE(rows > 0 && cols > 0, "iron_transpose_bf16: empty matrix");
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  IRON_REQUIRE(grid.y < 65536, "iron_transpose_bf16: too many rows");
  IRON_LAUNCH(transpose_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), rows, cols);
  return check_launch("transpose_bf16");
}
