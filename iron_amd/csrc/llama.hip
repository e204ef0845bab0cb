// Glue kernels of the Llama decode/prefill step that keep the whole token loop
// on the GPU: embedding lookup from a device token id, greedy argmax that
// advances the device-resident position (so a captured decode graph can be
// replayed token after token with no host round trip), and the prefill
// scatter that rotates q/k and writes k/v into the caches.
#include "iron_common.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

// out[i, :] = table[ids[i], :] (zeros for an out-of-range id). One 16-byte
// chunk per thread.
__global__ __launch_bounds__(256) void embedding_kernel(const uint16_t* __restrict__ table, const int* __restrict__ ids,
                                                        uint16_t* __restrict__ out, int n, int dim, int vocab) {
  const int per_row = dim >> 3;
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= static_cast<long long>(n) * per_row) return;
  const int i = static_cast<int>(t / per_row), c = static_cast<int>(t % per_row);
  const int id = ids[i];
  uint4 v = make_uint4(0, 0, 0, 0);
  if (id >= 0 && id < vocab) v = reinterpret_cast<const uint4*>(table + static_cast<size_t>(id) * dim)[c];
  reinterpret_cast<uint4*>(out + static_cast<size_t>(i) * dim)[c] = v;
}

// Greedy argmax over bf16 logits (first index on ties, like torch.argmax),
// one 1024-thread workgroup. Writes token_out[0]; when pos is given, records
// history[pos] = token (if pos < history_cap) and advances *pos by one.
__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* __restrict__ x, int n, int* token_out, int* pos,
                                                      int* history, int history_cap) {
  __shared__ float sv[16];
  __shared__ int si[16];
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float v = bf16_to_f32(x[i]);
    if (v > best) {  // strided scan visits indices in increasing order: keeps the first maximum
      best = v;
      bi = i;
    }
  }
  // wave reduction on (value, index)
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int idx = si[0];
    for (int w = 1; w < 16; ++w)
      if (sv[w] > b || (sv[w] == b && si[w] < idx)) {
        b = sv[w];
        idx = si[w];
      }
    if (idx == 0x7fffffff) idx = 0;  // all NaN
    token_out[0] = idx;
    if (pos) {
      const int p = *pos;
      if (history && p >= 0 && p < history_cap) history[p] = idx;
      *pos = p + 1;
    }
  }
}

// Greedy token selection from the per-workgroup argmax keys of the LM-head
// GEMV, fused with the bookkeeping and the next token's embedding (one
// 1024-thread workgroup): token_out = argmax; history[*pos] = token;
// *pos += 1; x_out = table[token] (skipped when table is NULL).
__global__ __launch_bounds__(1024) void select_embed_kernel(const unsigned long long* __restrict__ keys, int n_keys,
                                                            const uint16_t* __restrict__ table, int dim, int vocab,
                                                            uint16_t* __restrict__ x_out, int* token_out, int* pos,
                                                            int* history, int history_cap) {
  __shared__ unsigned long long ks[16];
  __shared__ int tok_s;
  const int p = pos ? *pos : 0;  // independent of the keys: in flight with them
  // 32 keys per thread per step, all loads issued before the first compare
  // (one step covers the 32064 keys of a 128256-row head)
  constexpr int U = 32;
  unsigned long long best = 0;
  for (int base = 0; base < n_keys; base += 1024 * U) {
    unsigned long long k[U];
    // unconditional loads of a clamped index (a repeated key cannot change the
    // maximum): a guarded load became a branch with its own wait per key
#pragma unroll
    for (int u = 0; u < U; ++u) k[u] = keys[min(base + u * 1024 + static_cast<int>(threadIdx.x), n_keys - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u) best = k[u] > best ? k[u] : best;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, kWave);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) ks[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = ks[0];
    for (int w = 1; w < 16; ++w) b = ks[w] > b ? ks[w] : b;
    int tok = static_cast<int>(argmax_key_index(b));
    if (tok < 0 || tok >= vocab) tok = 0;
    tok_s = tok;
    token_out[0] = tok;
    if (pos) {
      if (history && p >= 0 && p < history_cap) history[p] = tok;
      *pos = p + 1;
    }
  }
  __syncthreads();
  if (table) {
    const uint4* src = reinterpret_cast<const uint4*>(table + static_cast<size_t>(tok_s) * dim);
    for (int c = threadIdx.x; c < (dim >> 3); c += 1024) reinterpret_cast<uint4*>(x_out)[c] = src[c];
  }
}

// Prefill: qkv (S, (H + 2*Hkv) * 64) rows -> q_out (S, H*64) rotated,
// k_cache[:, pos0+s] rotated, v_cache[:, pos0+s] copied. One thread per
// rotated pair (q and k heads) or per v element pair. PART: qkv is a split-K
// GEMM output given as its fp32 partial sums (splits ranges of S*(H+2Hkv)*64
// floats), merged here exactly as the GEMM's own merge.
template <bool PART>
__global__ __launch_bounds__(256) void qkv_scatter_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ angles,
                                                          uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
                                                          uint16_t* __restrict__ v_cache, int S, int H, int Hkv,
                                                          int max_len, int pos0, const float* __restrict__ part,
                                                          int splits) {
  constexpr int D = 64;
  const int heads = H + 2 * Hkv;
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= static_cast<long long>(S) * heads * 32) return;
  const int s = static_cast<int>(t / (heads * 32));
  const int rem = static_cast<int>(t % (heads * 32));
  const int h = rem / 32, i = rem % 32;
  const int p = pos0 + s;
  const size_t off = static_cast<size_t>(s) * heads * D + h * D;
  const uint16_t* row = PART ? nullptr : qkv + off;
  const size_t range = static_cast<size_t>(S) * heads * D;
  auto val = [&](int col) { return PART ? merged_bf16(part + off + col, range, splits) : bf16_to_f32(row[col]); };
  if (h < H + Hkv) {
    const float c = angles[static_cast<size_t>(p) * D + 2 * i], sn = angles[static_cast<size_t>(p) * D + 2 * i + 1];
    const float x1 = val(i), x2 = val(i + 32);
    const uint16_t y1 = f32_to_bf16(rot_sub(x1, c, x2, sn)), y2 = f32_to_bf16(rot_add(x2, c, x1, sn));
    uint16_t* dst = h < H ? q_out + static_cast<size_t>(s) * H * D + h * D
                          : k_cache + (static_cast<size_t>(h - H) * max_len + p) * D;
    dst[i] = y1;
    dst[i + 32] = y2;
  } else {
    uint16_t* dst = v_cache + (static_cast<size_t>(h - H - Hkv) * max_len + p) * D;
    dst[i] = PART ? f32_to_bf16(val(i)) : row[i];
    dst[i + 32] = PART ? f32_to_bf16(val(i + 32)) : row[i + 32];
  }
}

// The same scatter with 16-byte accesses: one thread per 8 rotated pairs,
// dims 8 g .. 8 g + 7 and 32 + the same of one head of one row (g = 0..3),
// the table's 16 floats [cos, sin] x 8 of those pairs in four 16-byte loads.
// Every element takes the arithmetic of qkv_scatter_kernel (the split-K sum
// in range order, rot_sub / rot_add, one bf16 rounding), so the two kernels
// write identical bits. Used when every operand is 16-byte aligned.
template <bool PART>
__global__ __launch_bounds__(256) void qkv_scatter8_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ angles,
                                                           uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
                                                           uint16_t* __restrict__ v_cache, int S, int H, int Hkv,
                                                           int max_len, int pos0, const float* __restrict__ part,
                                                           int splits) {
  constexpr int D = 64;
  const int heads = H + 2 * Hkv;
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= static_cast<long long>(S) * heads * 4) return;
  const int s = static_cast<int>(t / (heads * 4));
  const int rem = static_cast<int>(t % (heads * 4));
  const int h = rem >> 2, i0 = (rem & 3) * 8;
  const int p = pos0 + s;
  const size_t off = static_cast<size_t>(s) * heads * D + h * D;
  float x1[8], x2[8];  // dims i0 + e and i0 + 32 + e
  if (PART) {
    const size_t range = static_cast<size_t>(S) * heads * D;
    float r1[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, r2[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < splits; ++kb) {
      const float4* pa = reinterpret_cast<const float4*>(part + kb * range + off + i0);
      const float4* pb = reinterpret_cast<const float4*>(part + kb * range + off + i0 + 32);
      const float4 a0 = pa[0], a1 = pa[1], b0 = pb[0], b1 = pb[1];
      r1[0] += a0.x; r1[1] += a0.y; r1[2] += a0.z; r1[3] += a0.w;
      r1[4] += a1.x; r1[5] += a1.y; r1[6] += a1.z; r1[7] += a1.w;
      r2[0] += b0.x; r2[1] += b0.y; r2[2] += b0.z; r2[3] += b0.w;
      r2[4] += b1.x; r2[5] += b1.y; r2[6] += b1.z; r2[7] += b1.w;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x1[e] = bf16_to_f32(f32_to_bf16(r1[e]));
      x2[e] = bf16_to_f32(f32_to_bf16(r2[e]));
    }
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(qkv + off + i0);
    const uint4 b = *reinterpret_cast<const uint4*>(qkv + off + i0 + 32);
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x1[2 * e] = lo_bf16(wa[e]);
      x1[2 * e + 1] = hi_bf16(wa[e]);
      x2[2 * e] = lo_bf16(wb[e]);
      x2[2 * e + 1] = hi_bf16(wb[e]);
    }
  }
  uint32_t y1[4], y2[4];
  uint16_t* dst;
  if (h < H + Hkv) {
    const float4* ap = reinterpret_cast<const float4*>(angles + static_cast<size_t>(p) * D + 2 * i0);
    float ang[16];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float4 q = ap[u];
      ang[4 * u] = q.x;
      ang[4 * u + 1] = q.y;
      ang[4 * u + 2] = q.z;
      ang[4 * u + 3] = q.w;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c0 = ang[4 * e], s0 = ang[4 * e + 1], c1 = ang[4 * e + 2], s1 = ang[4 * e + 3];
      y1[e] = pack_bf16x2(rot_sub(x1[2 * e], c0, x2[2 * e], s0), rot_sub(x1[2 * e + 1], c1, x2[2 * e + 1], s1));
      y2[e] = pack_bf16x2(rot_add(x2[2 * e], c0, x1[2 * e], s0), rot_add(x2[2 * e + 1], c1, x1[2 * e + 1], s1));
    }
    dst = h < H ? q_out + static_cast<size_t>(s) * H * D + h * D
                : k_cache + (static_cast<size_t>(h - H) * max_len + p) * D;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {  // exact: bf16 values (or the partial sums rounded once above)
      y1[e] = pack_bf16x2(x1[2 * e], x1[2 * e + 1]);
      y2[e] = pack_bf16x2(x2[2 * e], x2[2 * e + 1]);
    }
    dst = v_cache + (static_cast<size_t>(h - H - Hkv) * max_len + p) * D;
  }
  *reinterpret_cast<uint4*>(dst + i0) = make_uint4(y1[0], y1[1], y1[2], y1[3]);
  *reinterpret_cast<uint4*>(dst + i0 + 32) = make_uint4(y2[0], y2[1], y2[2], y2[3]);
}

}  // namespace
}  // namespace iron

using namespace iron;

extern "C" int iron_embedding(const void* table, const int* ids, void* out, int n, int dim, int vocab, void* stream) {
  IRON_REQUIRE(table && ids && out, "iron_embedding: null pointer");
  IRON_REQUIRE(n > 0 && dim > 0 && dim % 8 == 0 && vocab > 0, "iron_embedding: n=%d dim=%d vocab=%d", n, dim, vocab);
  IRON_REQUIRE(aligned16(table) && aligned16(out), "iron_embedding: table and out must be 16-byte aligned");
  const long long threads = static_cast<long long>(n) * (dim / 8);
  IRON_LAUNCH(embedding_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(table), ids,
                     static_cast<uint16_t*>(out), n, dim, vocab);
  return check_launch("embedding");
}

extern "C" int iron_argmax_bf16(const void* x, int n, int* token_out, int* pos, int* history, int history_cap,
                                void* stream) {
  IRON_REQUIRE(x && token_out, "iron_argmax_bf16: null pointer");
  IRON_REQUIRE(n > 0, "iron_argmax_bf16: empty input");
  IRON_REQUIRE(!history || pos, "iron_argmax_bf16: history needs a position counter");
  IRON_LAUNCH(argmax_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), n, token_out, pos, history, history_cap);
  return check_launch("argmax");
}

extern "C" int iron_argmax_select(const void* keys, int n_keys, const void* table, int dim, int vocab, void* x_out,
                                  int* token_out, int* pos, int* history, int history_cap, void* stream) {
  IRON_REQUIRE(keys && token_out && n_keys > 0, "iron_argmax_select: null pointer or no keys");
  IRON_REQUIRE(vocab > 0, "iron_argmax_select: vocab must be positive");
  IRON_REQUIRE(!table || (x_out && dim > 0 && dim % 8 == 0 && aligned16(table) && aligned16(x_out)),
               "iron_argmax_select: embedding needs x_out, dim %% 8 == 0 and 16-byte alignment");
  IRON_REQUIRE(!history || pos, "iron_argmax_select: history needs a position counter");
  IRON_LAUNCH(select_embed_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
              static_cast<const unsigned long long*>(keys), n_keys, static_cast<const uint16_t*>(table), dim, vocab,
              static_cast<uint16_t*>(x_out), token_out, pos, history, history_cap);
  return check_launch("argmax_select");
}

extern "C" int iron_qkv_rope_scatter(const void* qkv, const float* angles, int angle_rows, void* q_out, void* k_cache,
                                     void* v_cache, int seq, int n_heads, int n_kv_heads, int head_dim, int max_len,
                                     int pos0, void* stream) {
  IRON_REQUIRE(qkv && angles && q_out && k_cache && v_cache, "iron_qkv_rope_scatter: null pointer");
  IRON_REQUIRE(head_dim == 64, "iron_qkv_rope_scatter: head_dim=%d (only 64 is supported)", head_dim);
  IRON_REQUIRE(seq > 0 && n_heads > 0 && n_kv_heads > 0, "iron_qkv_rope_scatter: empty shape");
  IRON_REQUIRE(pos0 >= 0 && pos0 + seq <= max_len && pos0 + seq <= angle_rows,
               "iron_qkv_rope_scatter: positions [%d, %d) exceed the cache (%d) or angle table (%d)", pos0,
               pos0 + seq, max_len, angle_rows);
  const long long pairs = static_cast<long long>(seq) * (n_heads + 2 * n_kv_heads) * 32;
  if (aligned16(qkv) && aligned16(angles) && aligned16(q_out) && aligned16(k_cache) && aligned16(v_cache)) {
    IRON_LAUNCH(qkv_scatter8_kernel<false>, dim3(static_cast<unsigned>((pairs / 8 + 255) / 256)), dim3(256), 0,
                static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv), angles,
                static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), seq,
                n_heads, n_kv_heads, max_len, pos0, nullptr, 0);
  } else {
    IRON_LAUNCH(qkv_scatter_kernel<false>, dim3(static_cast<unsigned>((pairs + 255) / 256)), dim3(256), 0,
                static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv), angles,
                static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), seq,
                n_heads, n_kv_heads, max_len, pos0, nullptr, 0);
  }
  return check_launch("qkv_rope_scatter");
}

extern "C" int iron_qkv_rope_scatter_splitk(const float* partial, int splits, const float* angles, int angle_rows,
                                            void* q_out, void* k_cache, void* v_cache, int seq, int n_heads,
                                            int n_kv_heads, int head_dim, int max_len, int pos0, void* stream) {
  IRON_REQUIRE(partial && angles && q_out && k_cache && v_cache, "iron_qkv_rope_scatter_splitk: null pointer");
  IRON_REQUIRE(splits >= 1 && splits <= 64, "iron_qkv_rope_scatter_splitk: splits=%d outside [1, 64]", splits);
  IRON_REQUIRE(head_dim == 64, "iron_qkv_rope_scatter_splitk: head_dim=%d (only 64 is supported)", head_dim);
  IRON_REQUIRE(seq > 0 && n_heads > 0 && n_kv_heads > 0, "iron_qkv_rope_scatter_splitk: empty shape");
  IRON_REQUIRE(pos0 >= 0 && pos0 + seq <= max_len && pos0 + seq <= angle_rows,
               "iron_qkv_rope_scatter_splitk: positions [%d, %d) exceed the cache (%d) or angle table (%d)", pos0,
               pos0 + seq, max_len, angle_rows);
  const long long pairs = static_cast<long long>(seq) * (n_heads + 2 * n_kv_heads) * 32;
  if (aligned16(partial) && aligned16(angles) && aligned16(q_out) && aligned16(k_cache) && aligned16(v_cache)) {
    IRON_LAUNCH(qkv_scatter8_kernel<true>, dim3(static_cast<unsigned>((pairs / 8 + 255) / 256)), dim3(256), 0,
                static_cast<hipStream_t>(stream), nullptr, angles, static_cast<uint16_t*>(q_out),
                static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), seq, n_heads, n_kv_heads, max_len,
                pos0, partial, splits);
  } else {
    IRON_LAUNCH(qkv_scatter_kernel<true>, dim3(static_cast<unsigned>((pairs + 255) / 256)), dim3(256), 0,
                static_cast<hipStream_t>(stream), nullptr, angles, static_cast<uint16_t*>(q_out),
                static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), seq, n_heads, n_kv_heads, max_len,
                pos0, partial, splits);
  }
  return check_launch("qkv_rope_scatter_splitk");
}
