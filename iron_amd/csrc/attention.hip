// GQA attention for decode (split-K flash-decode) and causal prefill.
//
// Decode: one new token. A workgroup owns (KV head j, a chunk of 64 cache
// positions) and serves the G = H/Hkv query heads that share KV head j, so
// every K/V byte is read from HBM once for all of them. Inside the chunk the
// softmax is exact in fp32 (scores scaled by log2(e)/sqrt(D), exp2); the
// chunk's unnormalised output, maximum and sum go to a workspace, and a second
// small kernel merges the chunks. (Merging in the last-arriving workgroup
// would need an agent-scope fence per workgroup, which on this GPU writes back
// and invalidates the whole per-XCD L2: far dearer than one more launch.)
// RoPE for q and the new k is applied on load (two-halves rotation, row `pos`
// of an fp32 [cos, sin] interleaved table, result rounded to bf16 as the RoPE
// operator does), and the new k/v are written into the caches at `pos` by the
// workgroup whose chunk holds `pos`.
//
// Cache layout: (Hkv, max_len, D) bf16, position-major within a head, so a
// chunk of one head is one contiguous 8 KiB block.
#include "iron_common.hpp"
#include "../../include/iron_hip.h"

namespace iron {
namespace {

constexpr int kDecChunk = 64;  // cache positions per workgroup
constexpr int kDecThreads = 256;
constexpr int kD = 64;         // head dim (the reference MHA supports d = 64 only)

struct DecodeArgs {
  const uint16_t* q;      // (H, D) un-rotated
  const uint16_t* k_new;  // (Hkv, D) un-rotated
  const uint16_t* v_new;  // (Hkv, D)
  uint16_t* k_cache;      // (Hkv, max_len, D)
  uint16_t* v_cache;      // (Hkv, max_len, D)
  const float* angles;    // (angle_rows, D) [cos0, sin0, cos1, sin1, ...]
  uint16_t* out;          // (H, D)
  float* part;            // (Hkv, nsplit, G*D + 2G) partials
  const int* pos_dev;     // optional device-resident position (overrides pos)
  int pos;
  int max_len;
  int angle_rows;
  int nsplit;             // gridDim.x
  float scale_log2;       // log2(e) * scale
};

template <int G>
constexpr int part_stride() {
  return G * kD + 2 * G;
}

// Loads of one 16-byte chunk as 8 floats.
__device__ __forceinline__ void unpack8(const uint4 v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = lo_bf16(w[e]);
    f[2 * e + 1] = hi_bf16(w[e]);
  }
}

// Two-halves RoPE of the 8 dims of chunk c of a 64-vector, given that chunk
// (own) and chunk c ^ 4 (pair), and the 16 table floats [cos, sin] x 8 of dims
// (c & 3) * 8 + e. Lower half: x1 c - x2 s; upper half: x2 c + x1 s. Rounded
// to bf16, as the RoPE operator stores it.
__device__ __forceinline__ void rope_chunk(const uint4 own, const uint4 pair, const float* ang, bool lower, float* out) {
  float xo[8], xp[8];
  unpack8(own, xo);
  unpack8(pair, xp);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = ang[2 * e], s = ang[2 * e + 1];
    const float r = lower ? xo[e] * c - xp[e] * s : xo[e] * c + xp[e] * s;
    out[e] = bf16_to_f32(f32_to_bf16(r));
  }
}

// Partials of one 64-position chunk of KV head j for its G query heads.
// Thread -> (position rows r and r + 32 of the chunk, dims 8c..8c+7). Every
// global load the workgroup needs (K/V rows, q and its RoPE partner chunks,
// the table row, the new k/v) is issued right after `pos` is known, before
// any barrier, so the kernel pays one memory round trip after the position.
template <int G>
__global__ __launch_bounds__(kDecThreads) void gqa_decode_kernel(DecodeArgs a) {
  constexpr int D = kD;
  constexpr int NW = kDecThreads / kWave;
  constexpr int PS = part_stride<G>();
  __shared__ float max_s[NW][G];
  __shared__ float sum_s[NW][G];
  // per (head, position row, dim); rows padded to 65 floats so the 8x8 (row, chunk) lanes of a
  // wave writing one dim spread over the banks (a 64-float row would put 16 lanes on one bank)
  __shared__ float o_s[G][kDecThreads / 8][D + 1];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int s = blockIdx.x, j = blockIdx.y;
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) return;  // rejected on the host when pos is known
  const int L = pos + 1;
  const int p0 = s * kDecChunk;
  if (p0 >= L) return;
  const int c = tid & 7, r = tid >> 3;
  const bool lower = c < 4;
  const bool owner = pos >= p0 && pos < p0 + kDecChunk;

  uint4 kraw[2], vraw[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = p0 + r + 32 * h;
    kraw[h] = vraw[h] = make_uint4(0, 0, 0, 0);
    if (p < pos) {
      const size_t off = (static_cast<size_t>(j) * a.max_len + p) * D + c * 8;
      kraw[h] = ld_stream16(a.k_cache + off);
      vraw[h] = ld_stream16(a.v_cache + off);
    }
  }
  const uint16_t* qh = a.q + static_cast<size_t>(j) * G * D;
  uint4 qa[G], qb[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qa[g] = *reinterpret_cast<const uint4*>(qh + g * D + c * 8);
    qb[g] = *reinterpret_cast<const uint4*>(qh + g * D + (c ^ 4) * 8);
  }
  float ang[16];
  {
    const float4* ap = reinterpret_cast<const float4*>(a.angles + static_cast<size_t>(pos) * D + (c & 3) * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 t = ap[i];
      ang[4 * i] = t.x;
      ang[4 * i + 1] = t.y;
      ang[4 * i + 2] = t.z;
      ang[4 * i + 3] = t.w;
    }
  }
  uint4 kna = make_uint4(0, 0, 0, 0), knb = kna, vn = kna;
  if (owner) {
    kna = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * D + c * 8);
    knb = *reinterpret_cast<const uint4*>(a.k_new + static_cast<size_t>(j) * D + (c ^ 4) * 8);
    vn = *reinterpret_cast<const uint4*>(a.v_new + static_cast<size_t>(j) * D + c * 8);
  }

  float qv[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) rope_chunk(qa[g], qb[g], ang, lower, qv[g]);
  float kf[2][8], vf[2][8];
  bool valid[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int p = p0 + r + 32 * h;
    valid[h] = p < L;
    if (p == pos) {  // the new token: rotate k, append k/v to the caches
      rope_chunk(kna, knb, ang, lower, kf[h]);
      unpack8(vn, vf[h]);
      uint32_t kw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) kw[e] = pack_bf16x2(kf[h][2 * e], kf[h][2 * e + 1]);  // exact: already bf16 values
      const size_t off = (static_cast<size_t>(j) * a.max_len + pos) * D + c * 8;
      *reinterpret_cast<uint4*>(a.k_cache + off) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
      *reinterpret_cast<uint4*>(a.v_cache + off) = vn;
    } else {
      unpack8(kraw[h], kf[h]);
      unpack8(vraw[h], vf[h]);
    }
  }

  // scores in the log2 domain; the 8 lanes of a position sum their partial dots
  float sc[2][G];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d = fmaf(qv[g][e], kf[h][e], d);
      d = add_dpp<0xB1>(d);   // + lane ^ 1
      d = add_dpp<0x4E>(d);   // + lane ^ 2
      d = add_dpp<0x141>(d);  // + lane 7-i of the 8: full 8-lane sum
      sc[h][g] = valid[h] ? d * a.scale_log2 : -INFINITY;
    }

  // chunk maximum per head (finite: position p0 < L is always valid)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(fmaxf(sc[0][g], sc[1][g]));
    if (lane == 0) max_s[wave][g] = m;
  }
  __syncthreads();
  float mloc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float m = max_s[0][g];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, max_s[w][g]);
    mloc[g] = m;
  }

  // probabilities, their sum (one lane per position counts), and this
  // thread's share of the unnormalised output
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float e0 = valid[0] ? exp2f(sc[0][g] - mloc[g]) : 0.f;
    const float e1 = valid[1] ? exp2f(sc[1][g] - mloc[g]) : 0.f;
    const float l = wave_sum(c == 0 ? e0 + e1 : 0.f);
    if (lane == 0) sum_s[wave][g] = l;
#pragma unroll
    for (int e = 0; e < 8; ++e) o_s[g][r][c * 8 + e] = e0 * vf[0][e] + e1 * vf[1][e];
  }
  __syncthreads();
  float* part = a.part + (static_cast<size_t>(j) * a.nsplit + s) * PS;
  for (int t = tid; t < G * D; t += kDecThreads) {
    const int g = t / D, d = t % D;
    float acc = 0.f;
#pragma unroll 8
    for (int rr = 0; rr < kDecThreads / 8; ++rr) acc += o_s[g][rr][d];
    part[t] = acc;
  }
  if (tid < G) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) l += sum_s[w][tid];
    part[G * D + tid] = mloc[tid];
    part[G * D + G + tid] = l;
  }
}

// Merge of the chunk partials of one KV head, one 1024-thread workgroup per
// KV head. Thread -> output element t = (head, dim) of the G*64 outputs and
// slice q of the chunks (chunks q, q + NQ, ...). Each thread folds its chunks
// with a running maximum, loading 8 chunks per step with every load in
// flight; the NQ slices are then combined through LDS.
constexpr int kMergeThreads = 1024;

template <int G>
__global__ __launch_bounds__(kMergeThreads) void gqa_combine_kernel(DecodeArgs a) {
  constexpr int D = kD;
  constexpr int PS = part_stride<G>();
  constexpr int NT = G * D;                   // outputs per KV head
  constexpr int NQ = kMergeThreads / NT;      // chunk slices
  constexpr int B = 8;                        // chunks per step per thread
  __shared__ float m_s[kMergeThreads], l_s[kMergeThreads], o_s[kMergeThreads];
  const int tid = threadIdx.x, t = tid % NT, q = tid / NT, g = t / D;
  const int j = blockIdx.x;
  const int pos = a.pos_dev ? *a.pos_dev : a.pos;
  if (pos < 0 || pos >= a.max_len || pos >= a.angle_rows) return;
  const int nact = (pos + kDecChunk) / kDecChunk;
  const float* base = a.part + static_cast<size_t>(j) * a.nsplit * PS;
  float M = -INFINITY, Ls = 0.f, acc = 0.f;
  for (int k0 = q; k0 < nact; k0 += NQ * B) {
    float mb[B], lb[B], ob[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int k = k0 + b * NQ;
      mb[b] = -INFINITY;
      lb[b] = ob[b] = 0.f;
      if (k < nact) {
        const float* pk = base + static_cast<size_t>(k) * PS;
        mb[b] = pk[G * D + g];
        lb[b] = pk[G * D + G + g];
        ob[b] = pk[t];
      }
    }
    float bm = M;
#pragma unroll
    for (int b = 0; b < B; ++b) bm = fmaxf(bm, mb[b]);  // finite: chunk k0 < nact is active
    const float keep = exp2f(M - bm);                   // 0 on the first step
    acc *= keep;
    Ls *= keep;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float w = exp2f(mb[b] - bm);  // 0 for the chunks past nact
      acc = fmaf(w, ob[b], acc);
      Ls = fmaf(w, lb[b], Ls);
    }
    M = bm;
  }
  m_s[tid] = M;
  l_s[tid] = Ls;
  o_s[tid] = acc;
  __syncthreads();
  if (q == 0) {
    float Mx = M;  // slice 0 always holds chunk 0
#pragma unroll
    for (int qq = 1; qq < NQ; ++qq) Mx = fmaxf(Mx, m_s[qq * NT + t]);
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
      const float w = exp2f(m_s[qq * NT + t] - Mx);  // 0 for an empty slice
      lt = fmaf(w, l_s[qq * NT + t], lt);
      ot = fmaf(w, o_s[qq * NT + t], ot);
    }
    a.out[static_cast<size_t>(j) * NT + t] = f32_to_bf16(ot / lt);
  }
}

// ---------------------------------------------------------------------------
// Prefill / MHA: causal (optional) flash attention over strided Q, K, V.
// Block = 64 queries of one head, 256 threads: thread -> (query t/4, quarter
// t%4). K/V tiles of 64 keys are staged in LDS as fp32; the online softmax
// keeps a running max and sum per query (log2 domain).
// ---------------------------------------------------------------------------
struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  long long q_hs, q_rs;  // element strides: per head, per row
  long long k_hs, k_rs;
  long long v_hs, v_rs;
  long long o_hs, o_rs;
  int H, Hkv, Sq, Skv;
  int out_rows;  // rows of out to write; rows in [Sq, out_rows) are zero-filled
  int causal;
  int q_offset;  // absolute position of query row 0 (keys <= it are visible)
  float scale_log2;
};

constexpr int kPfQ = 64, kPfK = 64;

__global__ __launch_bounds__(256) void attention_prefill_kernel(PrefillArgs a) {
  __shared__ float k_s[kPfK][kD + 1];
  __shared__ float v_s[kPfK][kD];
  __shared__ float p_s[kPfQ][kPfK + 1];
  const int tid = threadIdx.x;
  const int h = blockIdx.y, hk = h / (a.H / a.Hkv);
  const int q0 = blockIdx.x * kPfQ;
  const int qi = tid >> 2, sub = tid & 3;
  const int qrow = q0 + qi;
  const bool qvalid = qrow < a.Sq;
  const int qpos = a.q_offset + qrow;
  if (q0 >= a.Sq) {  // padding rows only (uniform per block)
    if (qrow < a.out_rows) {
      uint16_t* op = a.out + h * a.o_hs + static_cast<long long>(qrow) * a.o_rs + sub * 16;
#pragma unroll
      for (int i = 0; i < 16; ++i) op[i] = 0;
    }
    return;
  }

  float qv[kD];
  {
    const uint16_t* qp = a.q + h * a.q_hs + static_cast<long long>(qvalid ? qrow : 0) * a.q_rs;
#pragma unroll
    for (int d = 0; d < kD; d += 8) {
      const uint4 t = *reinterpret_cast<const uint4*>(qp + d);
      const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qv[d + 2 * e] = lo_bf16(w[e]) * a.scale_log2;
        qv[d + 2 * e + 1] = hi_bf16(w[e]) * a.scale_log2;
      }
    }
  }
  float o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = 0.f;
  float m = -INFINITY, l = 0.f;

  // keys visible to the block: up to the last query's position (causal)
  int kend = a.Skv;
  if (a.causal) {
    const int last = a.q_offset + min(q0 + kPfQ, a.Sq) - 1;
    kend = min(kend, last + 1);
  }
  for (int k0 = 0; k0 < kend; k0 += kPfK) {
    __syncthreads();
    for (int e = tid; e < kPfK * (kD / 8); e += 256) {
      const int kr = e / (kD / 8), dc = (e % (kD / 8)) * 8;
      const int key = k0 + kr;
      uint4 kt = make_uint4(0, 0, 0, 0), vt = make_uint4(0, 0, 0, 0);
      if (key < a.Skv) {
        kt = *reinterpret_cast<const uint4*>(a.k + hk * a.k_hs + static_cast<long long>(key) * a.k_rs + dc);
        vt = *reinterpret_cast<const uint4*>(a.v + hk * a.v_hs + static_cast<long long>(key) * a.v_rs + dc);
      }
      const uint32_t kw[4] = {kt.x, kt.y, kt.z, kt.w}, vw[4] = {vt.x, vt.y, vt.z, vt.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        k_s[kr][dc + 2 * q] = lo_bf16(kw[q]);
        k_s[kr][dc + 2 * q + 1] = hi_bf16(kw[q]);
        v_s[kr][dc + 2 * q] = lo_bf16(vw[q]);
        v_s[kr][dc + 2 * q + 1] = hi_bf16(vw[q]);
      }
    }
    __syncthreads();
    // scores for keys sub*16 .. sub*16+15
    float sc[16];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kr = sub * 16 + i, key = k0 + kr;
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < kD; ++e) d = fmaf(qv[e], k_s[kr][e], d);
      const bool vis = key < a.Skv && (!a.causal || key <= qpos);
      sc[i] = vis ? d : -INFINITY;
      tmax = fmaxf(tmax, sc[i]);
    }
    // the 4 threads of a query are lanes 4q..4q+3
    tmax = fmaxf(tmax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                           static_cast<int>(0xff800000u), __builtin_bit_cast(int, tmax), 0xB1, 0xf, 0xf, false)));
    tmax = fmaxf(tmax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                           static_cast<int>(0xff800000u), __builtin_bit_cast(int, tmax), 0x4E, 0xf, 0xf, false)));
    const float mnew = fmaxf(m, tmax);
    const float alpha = (mnew == -INFINITY) ? 1.f : exp2f(m - mnew);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = (sc[i] == -INFINITY) ? 0.f : exp2f(sc[i] - mnew);
      psum += p;
      p_s[qi][sub * 16 + i] = p;
    }
    psum = add_dpp<0xB1>(psum);
    psum = add_dpp<0x4E>(psum);
    l = l * alpha + psum;
    m = mnew;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] *= alpha;
    __syncthreads();
    for (int kr = 0; kr < kPfK; ++kr) {
      const float p = p_s[qi][kr];
#pragma unroll
      for (int i = 0; i < 16; ++i) o[i] = fmaf(p, v_s[kr][sub * 16 + i], o[i]);
    }
  }
  if (qvalid) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* op = a.out + h * a.o_hs + static_cast<long long>(qrow) * a.o_rs + sub * 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) op[i] = f32_to_bf16(o[i] * inv);
  } else if (qrow < a.out_rows) {
    uint16_t* op = a.out + h * a.o_hs + static_cast<long long>(qrow) * a.o_rs + sub * 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) op[i] = 0;
  }
}

}  // namespace
}  // namespace iron

using namespace iron;

static int decode_nsplit(int max_len) { return (max_len + kDecChunk - 1) / kDecChunk; }

extern "C" long long iron_gqa_decode_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim != kD || max_len <= 0) return -1;
  const int G = n_heads / n_kv_heads;
  const long long part = static_cast<long long>(n_kv_heads) * decode_nsplit(max_len) * (G * kD + 2 * G) * 4;
  return 256 + part;  // 256 reserved bytes, then partials
}

extern "C" int iron_gqa_decode(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                               const float* angles, int angle_rows, void* out, void* workspace, int n_heads,
                               int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev, float scale,
                               void* stream) {
  IRON_REQUIRE(q && k_new && v_new && k_cache && v_cache && angles && out && workspace,
               "iron_gqa_decode: null pointer");
  IRON_REQUIRE(head_dim == kD, "iron_gqa_decode: head_dim=%d (only 64 is supported)", head_dim);
  IRON_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "iron_gqa_decode: n_heads=%d must be a multiple of n_kv_heads=%d", n_heads, n_kv_heads);
  const int G = n_heads / n_kv_heads;
  IRON_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "iron_gqa_decode: group size %d not in {1,2,4,8}", G);
  IRON_REQUIRE(n_kv_heads * 4 <= 256, "iron_gqa_decode: at most 64 KV heads");
  IRON_REQUIRE(max_len > 0 && angle_rows > 0, "iron_gqa_decode: max_len and angle_rows must be positive");
  IRON_REQUIRE(pos_dev || (pos >= 0 && pos < max_len && pos < angle_rows),
               "iron_gqa_decode: pos=%d outside the cache (max_len=%d) or angle table (%d rows)", pos, max_len,
               angle_rows);
  IRON_REQUIRE(aligned16(q) && aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) && aligned16(v_cache) &&
                   aligned16(angles),
               "iron_gqa_decode: q, k_new, v_new, the caches and the angle table must be 16-byte aligned");
  IRON_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "iron_gqa_decode: workspace must be 256-byte aligned");
  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.angles = angles;
  a.out = static_cast<uint16_t*>(out);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
  a.pos_dev = pos_dev;
  a.pos = pos;
  a.max_len = max_len;
  a.angle_rows = angle_rows;
  a.nsplit = decode_nsplit(max_len);
  a.scale_log2 = scale * 1.4426950408889634f;
  dim3 grid(a.nsplit, n_kv_heads), block(kDecThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 cgrid(n_kv_heads), cblock(kMergeThreads);
  switch (G) {
    case 1:
      IRON_LAUNCH((gqa_decode_kernel<1>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<1>), cgrid, cblock, 0, s, a);
      break;
    case 2:
      IRON_LAUNCH((gqa_decode_kernel<2>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<2>), cgrid, cblock, 0, s, a);
      break;
    case 4:
      IRON_LAUNCH((gqa_decode_kernel<4>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<4>), cgrid, cblock, 0, s, a);
      break;
    default:
      IRON_LAUNCH((gqa_decode_kernel<8>), grid, block, 0, s, a);
      IRON_LAUNCH((gqa_combine_kernel<8>), cgrid, cblock, 0, s, a);
      break;
  }
  return check_launch("gqa_decode");
}

extern "C" int iron_attention_prefill(const void* q, const void* k, const void* v, void* out, int n_heads,
                                      int n_kv_heads, int seq_q, int seq_kv, int head_dim, long long q_head_stride,
                                      long long q_row_stride, long long kv_head_stride, long long kv_row_stride,
                                      long long o_head_stride, long long o_row_stride, int out_rows, int causal,
                                      int q_offset, float scale, void* stream) {
  IRON_REQUIRE(q && k && v && out, "iron_attention_prefill: null pointer");
  IRON_REQUIRE(head_dim == kD, "iron_attention_prefill: head_dim=%d (only 64 is supported)", head_dim);
  IRON_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "iron_attention_prefill: n_heads=%d must be a multiple of n_kv_heads=%d", n_heads, n_kv_heads);
  IRON_REQUIRE(seq_q > 0 && seq_kv > 0, "iron_attention_prefill: empty sequence");
  IRON_REQUIRE(q_offset >= 0, "iron_attention_prefill: q_offset must be >= 0");
  if (out_rows < seq_q) out_rows = seq_q;
  IRON_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && q_row_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                   kv_row_stride % 8 == 0 && kv_head_stride % 8 == 0,
               "iron_attention_prefill: rows must be 16-byte aligned");
  PrefillArgs a{static_cast<const uint16_t*>(q),
                static_cast<const uint16_t*>(k),
                static_cast<const uint16_t*>(v),
                static_cast<uint16_t*>(out),
                q_head_stride,
                q_row_stride,
                kv_head_stride,
                kv_row_stride,
                kv_head_stride,
                kv_row_stride,
                o_head_stride,
                o_row_stride,
                n_heads,
                n_kv_heads,
                seq_q,
                seq_kv,
                out_rows,
                causal,
                q_offset,
                scale * 1.4426950408889634f};
  dim3 grid((out_rows + kPfQ - 1) / kPfQ, n_heads), block(256);
  IRON_LAUNCH(attention_prefill_kernel, grid, block, 0, static_cast<hipStream_t>(stream), a);
  return check_launch("attention_prefill");
}
