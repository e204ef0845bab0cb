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
// 64 per step through a double-buffered LDS ring (one barrier per step); the
// next step's global loads are in flight while MFMAs run. LDS rows are 128 B
// (64 bf16); the 16-byte chunk c of row r lives at c ^ (r & 7), so the 32 rows
// read by one fragment load spread over all banks.
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
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * kChunks + (chunk ^ (row & 7)); }

__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(GemmArgs a) {
  __shared__ uint4 smem[2 * 2 * BM * kChunks];  // [buf][A|B][row][chunk] = 64 KiB
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware tile order
  const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;
  const int tm = t % tiles_m, tn = t / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  // global -> register staging: 4 A chunks + 4 B chunks per thread per step
  uint4 ra[4], rb[4];
  auto load_step = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = tid + i * kThreads, row = id >> 3, c = id & 7;
      const int gm = m0 + row, gn = n0 + row;
      ra[i] = gm < a.M ? *reinterpret_cast<const uint4*>(a.A + static_cast<size_t>(gm) * a.K + k0 + c * 8)
                       : make_uint4(0, 0, 0, 0);
      rb[i] = gn < a.N ? *reinterpret_cast<const uint4*>(a.B + static_cast<size_t>(gn) * a.K + k0 + c * 8)
                       : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_step = [&](int buf) {
    uint4* As = smem + buf * 2 * BM * kChunks;
    uint4* Bs = As + BM * kChunks;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = tid + i * kThreads, row = id >> 3, c = id & 7;
      As[swz(row, c)] = ra[i];
      Bs[swz(row, c)] = rb[i];
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = a.K / BK;
  load_step(0);
  store_step(0);
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const int buf = it & 1;
    if (it + 1 < nk) load_step((it + 1) * BK);
    const uint4* As = smem + buf * 2 * BM * kChunks;
    const uint4* Bs = As + BM * kChunks;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      bf16x8_t fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int ra_row = wm * 64 + i * 32 + (lane & 31);
        fa[i] = __builtin_bit_cast(bf16x8_t, As[swz(ra_row, c)]);
        const int rb_row = wn * 64 + i * 32 + (lane & 31);
        fb[i] = __builtin_bit_cast(bf16x8_t, Bs[swz(rb_row, c)]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (it + 1 < nk) store_step(buf ^ 1);
    __syncthreads();
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

extern "C" int iron_gemm_bf16_nt(const void* A, const void* B, void* C, int M, int N, int K, long long ldc,
                                 int epilogue, int has_clamp, float clamp_lo, float clamp_hi, void* stream) {
  IRON_REQUIRE(A && B && C, "iron_gemm_bf16_nt: null pointer");
  IRON_REQUIRE(M > 0 && N > 0 && K > 0, "iron_gemm_bf16_nt: M=%d N=%d K=%d must be positive", M, N, K);
  IRON_REQUIRE(K % BK == 0, "iron_gemm_bf16_nt: K=%d must be a multiple of %d", K, BK);
  IRON_REQUIRE(aligned16(A) && aligned16(B), "iron_gemm_bf16_nt: A and B must be 16-byte aligned");
  IRON_REQUIRE(ldc >= N, "iron_gemm_bf16_nt: ldc=%lld < N=%d", ldc, N);
  IRON_REQUIRE(epilogue >= EPI_NONE && epilogue <= EPI_GELU_SIGMOID, "iron_gemm_bf16_nt: bad epilogue %d", epilogue);
  IRON_REQUIRE(!has_clamp || clamp_lo <= clamp_hi, "iron_gemm_bf16_nt: clamp min > max");
  if ((ldc % 8 == 0) && !aligned16(C)) return fail_einval("iron_gemm_bf16_nt: C must be 16-byte aligned");
  GemmArgs a{static_cast<const uint16_t*>(A), static_cast<const uint16_t*>(B), static_cast<uint16_t*>(C), M, N, K,
             ldc, epilogue, has_clamp, clamp_lo, clamp_hi};
  const long long tiles = static_cast<long long>((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  IRON_REQUIRE(tiles < (1LL << 31), "iron_gemm_bf16_nt: problem too large");
  IRON_LAUNCH(gemm_nt_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("gemm_bf16_nt");
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
