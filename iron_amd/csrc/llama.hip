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
  const long long threads = static_cast<long long>(seq) * (n_heads + 2 * n_kv_heads) * 32;
  IRON_LAUNCH(qkv_scatter_kernel<false>, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv), angles,
                     static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                     seq, n_heads, n_kv_heads, max_len, pos0, nullptr, 0);
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
  const long long threads = static_cast<long long>(seq) * (n_heads + 2 * n_kv_heads) * 32;
  IRON_LAUNCH(qkv_scatter_kernel<true>, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
              static_cast<hipStream_t>(stream), nullptr, angles, static_cast<uint16_t*>(q_out),
              static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), seq, n_heads, n_kv_heads, max_len, pos0,
              partial, splits);
  return check_launch("qkv_rope_scatter_splitk");
}
