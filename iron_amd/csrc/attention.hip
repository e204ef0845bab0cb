// GQA attention for decode (split-K flash-decode) and causal prefill.
//
// The decode device code (gqa_decode_chunk, its merge and the combine kernel)
// lives in decode_attn.hpp, shared with the one-launch decode step; this file
// holds the causal prefill kernel and the host entry points of both.
#include "iron_common.hpp"
#include "decode_attn.hpp"
#include "../../include/iron_hip.h"

#include <atomic>
#include <mutex>
#include <type_traits>

namespace iron {
namespace {

// ---------------------------------------------------------------------------
// Prefill / MHA: causal (optional) flash attention over strided Q, K, V on
// MFMA (v_mfma_f32_32x32x16_bf16).
//
// Workgroup = 4 waves = 128 queries of one head; each wave owns 32 queries and
// walks the visible keys in blocks of 64. K and V blocks are staged row-major
// in a 4-stage LDS ring filled by LDS-direct loads (buffer_load_dwordx4 ... lds,
// load_lds16: no VGPR staging, no LDS stores), up to three blocks ahead of the
// one being computed, one barrier per block. Per block a wave computes S^T = K Q^T (two 32x32 tiles): every lane
// then holds one query column (lane % 32) and 16 keys, so the softmax row
// statistics need only the lane's own registers and one exchange with lane ^ 32.
// The probabilities go to bf16 and feed O^T += V^T P^T directly from registers
// as the B operand; the k index of that product is a permutation of the
// block's keys that matches the S^T accumulator layout. The V^T operand comes
// straight from the row-major V block through ds_read_b64_tr_b16: in each
// 16-lane group, lane i receives element i % 4 of the 8-byte rows addressed by
// lanes 4j + i / 4 (j = 0..3), so lanes addressing 4 keys x 16 dims receive 16
// dims x 4 keys. K rows keep the 16-byte chunk c at slot c ^ ((key / 2) % 8)
// (16 rows of a ds_read_b128 on distinct banks); V rows at slot
// c ^ (((key / 2) % 2) * 4): a transposed read serves 32 lanes per LDS pass,
// 4 rows x 4 chunks, and this maps rows r and r + 2 to disjoint slot halves
// (with rows r and r + 1 on opposite bank halves, all 64 banks once).
// Online softmax in the log2 domain, fp32 statistics; output rows in
// [Sq, out_rows) are zero-filled (the MHA operator's padding).
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

typedef __bf16 fa_bf16x8 __attribute__((ext_vector_type(8)));
typedef float fa_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int fa_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int fa_u32x2 __attribute__((ext_vector_type(2)));

typedef short fa_i16x4 __attribute__((ext_vector_type(4)));

constexpr int kFaQ = 128;             // queries per workgroup (4 waves x 32)
constexpr int kFaK = 64;              // keys per block
constexpr int kFaStages = 4;          // K/V blocks resident (see the pipeline in the kernel)
constexpr int kFaBlock = kFaK * 128;  // bytes of a 64-row K (or V) block
constexpr int kOutStride = 72;        // output staging row (144 B)
constexpr int kFaLds = (kFaStages * 2 * kFaBlock) > (4 * 32 * kOutStride * 2) ? (kFaStages * 2 * kFaBlock)
                                                                               : (4 * 32 * kOutStride * 2);

// Lanes l and l ^ 32 exchange values in one VALU op (v_permlane32_swap_b32
// swaps the upper half of its first operand with the lower half of its
// second): with both operands x, the two results hold x[l] and x[l ^ 32] in
// every lane. Inline assembly, because the compiler's builtin for it kept only
// the first of the two results here. The s_nop covers the VALU-write to
// permlane-read hazard (the compiler emits the same before the builtin).
__device__ __forceinline__ void fa_pair(float x, float& r0, float& r1) {
  unsigned a = __builtin_bit_cast(unsigned, x), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float fa_pair_max(float x) {
  float r0, r1;
  fa_pair(x, r0, r1);
  return fmaxf(r0, r1);
}
__device__ __forceinline__ float fa_pair_sum(float x) {
  float r0, r1;
  fa_pair(x, r0, r1);
  return r0 + r1;
}

__device__ __forceinline__ int fa_k_slot(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }
__device__ __forceinline__ int fa_v_slot(int row, int chunk) { return chunk ^ (((row >> 1) & 1) << 2); }

// Wait until at most N of this wave's global loads are outstanding, then
// barrier (__syncthreads would wait for all of them). The memory clobber keeps
// the next stage's LDS reads below the barrier.
template <int N>
__device__ __forceinline__ void fa_wait_loads_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

__global__ __launch_bounds__(256) void attention_prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kFaLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, hh = lane >> 5;
  // Workgroup order: x = head, y = query tile. Causal tiles run heaviest
  // first (the last tile sees the most keys), and when H % 8 == 0 the heads
  // are permuted so that each XCD (workgroup b runs on XCD b % 8) holds
  // H / 8 consecutive heads, which share KV heads and so K/V blocks in its L2.
  const int bx = blockIdx.x;
  const int h = (a.H % 8 == 0) ? (bx % 8) * (a.H / 8) + bx / 8 : bx;
  const int hk = h / (a.H / a.Hkv);
  const int tile = a.causal ? static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y) : blockIdx.y;
  const int q0 = tile * kFaQ;
  if (q0 >= a.Sq) {  // padding rows only (uniform per workgroup)
    for (int e = tid; e < kFaQ * (kD / 8); e += 256) {
      const int r = q0 + (e >> 3), ch = e & 7;
      if (r < a.out_rows)
        *reinterpret_cast<fa_u32x4*>(a.out + h * a.o_hs + static_cast<long long>(r) * a.o_rs + ch * 8) =
            fa_u32x4{0, 0, 0, 0};
    }
    return;
  }
  const int qw = q0 + wave * 32;  // this wave's first query row

  // Q fragments (B operand of S^T): query qw + c, dims 16 kk + 8 hh .. + 8
  fa_bf16x8 qf[4];
  {
    const int qrow = min(qw + c, a.Sq - 1);
    const uint16_t* qp = a.q + h * a.q_hs + static_cast<long long>(qrow) * a.q_rs;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      qf[kk] = __builtin_bit_cast(fa_bf16x8, *reinterpret_cast<const fa_u32x4*>(qp + 16 * kk + 8 * hh));
  }
  // Use the Q fragments here, before any K/V load is issued: the compiler then
  // waits for these four loads now. Otherwise it counts them as outstanding at
  // their first use inside the key loop and waits there with vmcnt, which also
  // drains the K/V blocks the loop keeps in flight (the compiler does not count
  // those assembly loads).
  asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]));
  fa_f32x16 o[2];
#pragma unroll
  for (int j = 0; j < 16; ++j) o[0][j] = o[1][j] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int qpos = a.q_offset + qw + c;  // absolute position of this lane's query
  int kend = a.Skv;
  if (a.causal) kend = min(kend, a.q_offset + min(q0 + kFaQ, a.Sq));
  const int nb = (kend + kFaK - 1) / kFaK;
  const int wave_last = a.q_offset + min(qw + 31, a.Sq - 1);
  const int wave_first = a.q_offset + qw;  // keys <= it are visible to every query of the wave

  // Loader: a stage is [K block][V block], each 8 x 1 KiB of 8 rows; wave w
  // loads 1 KiB blocks 4w..4w+3 (0-7 K, 8-15 V). Lane l lands on row
  // 8 (b % 8) + l / 8, slot l % 8 and fetches the chunk that belongs there.
  // Keys past Skv load key Skv-1: finite values whose weights are zero.
  // Blocks are issued in order 0, 1, 2, ...: each lane keeps the byte offset of
  // its next row (from the head's K or V base, through a buffer resource: see
  // load_lds16) and bumps it by 64 rows per issue; only a block that runs past
  // Skv recomputes clamped offsets.
  const i32x4v rsrc_k = buffer_rsrc(a.k + hk * a.k_hs), rsrc_v = buffer_rsrc(a.v + hk * a.v_hs);
  unsigned coff[4], rsb[4], next_off[4];
  int lrow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = wave * 4 + j;
    const bool is_k = b < 8;
    const int r = (b & 7) * 8 + (lane >> 3), slot = lane & 7;
    const int chunk = is_k ? fa_k_slot(r, slot) : fa_v_slot(r, slot);  // both are involutions
    coff[j] = chunk * 16;
    rsb[j] = static_cast<unsigned>((is_k ? a.k_rs : a.v_rs) * 2);
    lrow[j] = r;
    next_off[j] = coff[j] + r * rsb[j];
  }
  auto issue = [&](int bi) {
    unsigned char* st = lds + (bi % kFaStages) * 2 * kFaBlock;
    const bool inside = bi * kFaK + kFaK <= a.Skv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned off = inside ? next_off[j] : coff[j] + min(bi * kFaK + lrow[j], a.Skv - 1) * rsb[j];
      load_lds16(wave * 4 + j < 8 ? rsrc_k : rsrc_v, off, st + (wave * 4 + j) * 1024);
      next_off[j] += kFaK * rsb[j];
    }
  };
  // this lane's transposed-read address inside a V block: 16-lane group g
  // covers dims 16 (g % 2) .. + 15 (+ 32 db) and keys 4 hh .. + 3 (+ 16 st, + 8)
  const int tr_row = 4 * hh + ((lane & 15) >> 2), tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // S^T = K Q^T for block bi: sc[b][j] is key 64 bi + 32 b + 8 (j / 4) + 4 hh + j % 4, query qw + c.
  // k_frags reads the block's K fragments (A operand: key 32 b + c, dims 16 kk + 8 hh .. + 8);
  // s_mfma runs the two independent accumulation chains (b = 0, 1) interleaved.
  auto k_frags = [&](int bi, fa_bf16x8 (&kf)[2][4]) {
    const unsigned char* ks = lds + (bi % kFaStages) * 2 * kFaBlock;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int kr = 32 * b + c;
        kf[b][kk] = __builtin_bit_cast(
            fa_bf16x8, *reinterpret_cast<const fa_u32x4*>(ks + kr * 128 + fa_k_slot(kr, 2 * kk + hh) * 16));
      }
  };
  auto s_mfma = [&](const fa_bf16x8 (&kf)[2][4], fa_f32x16 (&sc)[2]) {
    fa_f32x16 acc0 = {}, acc1 = {};  // the first MFMAs take an inline zero accumulator
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0][kk], qf[kk], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[1][kk], qf[kk], acc1, 0, 0, 0);
    }
    sc[0] = acc0;
    sc[1] = acc1;
  };
  auto scores = [&](int bi, fa_f32x16 (&sc)[2]) {
    fa_bf16x8 kf[2][4];
    k_frags(bi, kf);
    s_mfma(kf, sc);
  };
  auto visible = [&](int bi) { return !a.causal || bi * kFaK <= wave_last; };

  // Software pipeline over key blocks: iteration bi waits for block bi+1 and
  // reads its K fragments and block bi's V^T fragments, takes block bi's row
  // maximum, then runs block bi+1's S^T MFMAs, block bi's exponentials and its
  // P V MFMAs in one branch-free stretch, so that the matrix cores work while
  // the softmax occupies the VALU. Stages: bi (V being read), bi+1 (K being
  // read), bi+2 in flight, bi+3 being issued into the stage block bi-1 used.
  // On the last iteration the K fragments come from a stage no load writes any
  // more and the scores they give are not used.
#pragma unroll
  for (int p = 0; p < kFaStages - 1; ++p)
    if (p < nb) issue(p);
  static_assert(kFaStages == 4, "the wait counts below assume 4 stages");
  if (nb >= 3)
    fa_wait_loads_barrier<8>();
  else if (nb == 2)
    fa_wait_loads_barrier<4>();
  else
    fa_wait_loads_barrier<0>();
  fa_f32x16 sa[2], sb[2];
  scores(0, sa);  // block 0 is visible to every wave

  auto step = [&](int bi, fa_f32x16 (&cur)[2], fa_f32x16 (&nxt)[2]) {
    if (bi + 1 < nb) {
      if (bi + 2 < nb)
        fa_wait_loads_barrier<4>();
      else
        fa_wait_loads_barrier<0>();
      // block bi-1's stage is free: every wave passed this barrier after its last read of it
      if (bi + kFaStages - 1 < nb) issue(bi + kFaStages - 1);
    }
    if (!visible(bi)) return;  // every key of the block (and of the next) is after this wave's queries
    fa_bf16x8 kf[2][4];
    k_frags(bi + 1, kf);  // issued now; the compiler waits for them (exact LDS counts) before their MFMAs
    const int k0 = bi * kFaK;
    const unsigned char* vs = lds + (bi % kFaStages) * 2 * kFaBlock + kFaBlock;
      // V^T fragments for O^T += V^T P^T: k-step st, element i of lane (d, hh) is
      // key 16 st + 8 (i / 4) + 4 hh + i % 4 (two transposed reads of 4 keys each).
      // The address of (st, hl) is the (0, 0) one plus 2048 st + 1024 hl: the
      // swizzle (fa_v_slot) depends on bit 1 of the row only, which st and hl do
      // not change, so those steps become the reads' immediate offsets. As
      // builtins the reads get exact LDS waits (the K/V loads are assembly the
      // compiler does not count), so it can issue them early and wait only
      // before the P V MFMAs.
      fa_u32x2 vt[2][4][2];
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const int dim = 32 * db + tr_dim;
        const unsigned char* vb = vs + tr_row * 128 + fa_v_slot(tr_row, dim >> 3) * 16 + (dim & 7) * 2;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int hl = 0; hl < 2; ++hl)
            vt[db][st][hl] = __builtin_bit_cast(
                fa_u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                              (__attribute__((address_space(3))) fa_i16x4*)(vb + 2048 * st + 1024 * hl)));
      }
      // Online softmax in the log2 domain with c = scale * log2(e) > 0: the row
      // maximum is taken on the raw scores, p = 2^(s c - m) is one FMA and one
      // v_exp_f32. Only blocks that cross Skv or the causal diagonal of this
      // wave's queries are masked. The softmax VALU work, not the MFMAs,
      // bounds this loop.
      const float cs = a.scale_log2;
      float mx = -INFINITY;
      if (k0 + kFaK > a.Skv || (a.causal && k0 + kFaK - 1 > wave_first)) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = k0 + 32 * b + 8 * (j >> 2) + 4 * hh + (j & 3);
            const bool vis = key < a.Skv && (!a.causal || key <= qpos);
            cur[b][j] = vis ? cur[b][j] : -INFINITY;
            mx = fmaxf(mx, cur[b][j]);
          }
      } else {
        mx = fmaxf(fmaxf(cur[0][0], cur[0][1]), cur[0][2]);  // a chain of v_max3_f32
#pragma unroll
        for (int j = 3; j < 15; j += 2) mx = fmaxf(fmaxf(mx, cur[0][j]), cur[0][j + 1]);
        mx = fmaxf(fmaxf(mx, cur[0][15]), cur[1][0]);
#pragma unroll
        for (int j = 1; j < 15; j += 2) mx = fmaxf(fmaxf(mx, cur[1][j]), cur[1][j + 1]);
        mx = fmaxf(mx, cur[1][15]);
      }
      mx = fa_pair_max(mx);
      // Lazy rescaling: the running maximum m moves only when this block's
      // maximum exceeds it by more than 8 (log2 units), so p = 2^(s c - m) <= 2^8
      // stays well inside bf16/fp32 range and O is rarely rescaled. The result
      // sum(p v) / sum(p) does not depend on which m is used.
      const float mblk = mx * cs;
      const bool grow = mblk > m + 8.f;  // first visible block: m = -inf
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float alpha = grow ? __builtin_amdgcn_exp2f(m - mblk) : 1.f;  // 0 when m = -inf
        m = grow ? mblk : m;
        l *= alpha;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          o[0][j] *= alpha;
          o[1][j] *= alpha;
        }
      }
      const float moff = (m == -INFINITY) ? 0.f : m;  // keeps 2^(-inf - moff) = 0, never NaN
      s_mfma(kf, nxt);  // block bi+1's scores, independent of everything below
      // P^T fragments: pf[2 b + sp] element i = register 8 sp + i of s[b]
      fa_bf16x8 pf[4];
      float psum = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(cur[b][8 * sp + i], cs, -moff));
          const fa_u32x4 w = {cvt_pk_bf16(p[0], p[1]), cvt_pk_bf16(p[2], p[3]), cvt_pk_bf16(p[4], p[5]),
                              cvt_pk_bf16(p[6], p[7])};
          // the row sum of the bf16 weights the PV product uses, two per v_dot2
#pragma unroll
          for (int i = 0; i < 4; ++i) psum = dot2_bf16(w[i], 0x3f803f80u, psum);
          pf[2 * b + sp] = __builtin_bit_cast(fa_bf16x8, w);
        }
      l += psum;
      // O^T += V^T P^T over the block's 64 keys, 4 k-steps of 16
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const fa_u32x4 vw = {vt[db][st][0].x, vt[db][st][0].y, vt[db][st][1].x, vt[db][st][1].y};
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(fa_bf16x8, vw), pf[st], o[db], 0, 0, 0);
        }
  };
  for (int bi = 0; bi < nb; bi += 2) {
    step(bi, sa, sb);
    if (bi + 1 < nb) step(bi + 1, sb, sa);
  }

  l = fa_pair_sum(l);  // the two halves summed different keys of the same query
  const float inv = l > 0.f ? 1.f / l : 0.f;
  __syncthreads();  // every wave is done with the K/V tiles
  uint16_t* stg = reinterpret_cast<uint16_t*>(lds) + wave * 32 * kOutStride;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int d = 32 * db + 8 * (j >> 2) + 4 * hh + (j & 3);
      stg[c * kOutStride + d] = f32_to_bf16(o[db][j] * inv);
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i, r = e >> 3, ch = e & 7, q = qw + r;
    uint16_t* dst = a.out + h * a.o_hs + static_cast<long long>(q) * a.o_rs + ch * 8;
    if (q < a.Sq)
      *reinterpret_cast<fa_u32x4*>(dst) = *reinterpret_cast<const fa_u32x4*>(stg + r * kOutStride + ch * 8);
    else if (q < a.out_rows)
      *reinterpret_cast<fa_u32x4*>(dst) = fa_u32x4{0, 0, 0, 0};
  }
}

}  // namespace
}  // namespace iron

using namespace iron;

static int decode_nsplit(int max_len) { return (max_len + kDecChunk - 1) / kDecChunk; }

static int decode_part_stride(int G) {
  switch (G) {
    case 1: return part_stride<1>();
    case 2: return part_stride<2>();
    case 4: return part_stride<4>();
    default: return part_stride<8>();
  }
}

// Workspace layout: the arrival counters (one 128-byte line per KV head,
// rounded up to 256 bytes), then per KV head its nsplit chunk partials,
// each head's region rounded up to 256 bytes.
static long long decode_ctr_bytes(int n_kv_heads) { return (static_cast<long long>(n_kv_heads) * kCtrStride * 4 + 255) / 256 * 256; }
static long long decode_head_stride(int G, int max_len) {
  return (static_cast<long long>(decode_nsplit(max_len)) * decode_part_stride(G) + 63) / 64 * 64;
}

static bool decode_long_chunks(int n_kv_heads, int max_len, int pos, bool resident);

extern "C" int iron_gqa_decode_chunk_positions_ex(int n_heads, int n_kv_heads, int head_dim, int max_len, int pos,
                                                  int flags, void* stream) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim != kD || max_len <= 0) return -1;
  if (flags & ~(IRON_GQA_KV_RESIDENT | IRON_GQA_COUNTERS_ZERO)) return -1;
  const int G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return -1;
  const bool one = n_kv_heads % kXcds == 0 && xcd_round_robin(static_cast<hipStream_t>(stream)) == 1;
  return one && decode_long_chunks(n_kv_heads, max_len, pos, (flags & IRON_GQA_KV_RESIDENT) != 0)
             ? 16 * kDecWaves1
             : kDecChunk;
}

extern "C" int iron_gqa_decode_chunk_positions(int n_heads, int n_kv_heads, int head_dim, int max_len, int pos,
                                               void* stream) {
  return iron_gqa_decode_chunk_positions_ex(n_heads, n_kv_heads, head_dim, max_len, pos, 0, stream);
}

extern "C" long long iron_gqa_decode_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim != kD || max_len <= 0) return -1;
  const int G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return -1;
  return decode_ctr_bytes(n_kv_heads) + static_cast<long long>(n_kv_heads) * decode_head_stride(G, max_len) * 4;
}

// Checks and launches of one GQA decode step with its counters and partials
// in `workspace` (iron_gqa_decode_workspace_bytes() of the shape, 256-byte
// aligned). The arrival counters are zeroed by a small kernel first unless
// the caller keeps them at zero (IRON_GQA_COUNTERS_ZERO).
// One launch (n_kv_heads a multiple of 8 and the device dispatching workgroup
// ids congruent mod 8 to one XCD: each KV head's chunks on one XCD, merged by
// the last to finish) or the partials kernel plus the merge kernel.
// CUs of the current device (cached per device; 256 if it cannot be read).
static int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

// Whether the one-launch path takes 128-position chunks (kDecWaves1 waves) for
// a call at position `pos` (the position, or with a device position the
// caller's hint of it; -1: no hint, the cache's last slot). Below the switch,
// more and smaller chunks keep more CUs loading; above it, half the partials
// to merge and half the waves to dispatch win. With resident caches
// (IRON_GQA_KV_RESIDENT: K/V served from the Infinity Cache) the switch is
// where the active 128-position chunks of all KV heads reach half the CUs
// (decode in the model measured each way at KV 512 to 3968); with caches
// streamed from HBM it is where those chunks alone reach the CU count (8 KV
// heads: KV 2048 5.07 us with 64-position chunks against 5.31 with 128, KV
// 4096 6.20 against 5.89). Any choice gives a correct result.
static bool decode_long_chunks(int n_kv_heads, int max_len, int pos, bool resident) {
  const int p = pos < 0 || pos >= max_len ? max_len - 1 : pos;
  const long long active = static_cast<long long>(p / (16 * kDecWaves1) + 1) * n_kv_heads;
  return (resident ? 2 * active : active) >= device_cus();
}

template <int G, bool RES, bool TR>
static void gqa_decode_dispatch(const DecodeArgs& a, int n_kv_heads, bool one_launch, bool long_chunks, hipStream_t s) {
  const dim3 block(kDecThreads);
  if (one_launch) {
    // the workspace holds the 64-position partials either way
    DecodeArgs b = a;
    b.nsplit = (a.max_len + 16 * kDecWaves1 - 1) / (16 * kDecWaves1);
    if (long_chunks)
      IRON_GQA_DECODE_LAUNCH((gqa_decode_kernel<G, true, RES, kDecWaves1, TR>), dim3(b.nsplit * n_kv_heads),
                             dim3(kDecWaves1 * kWave), s, b);
    else
      IRON_GQA_DECODE_LAUNCH((gqa_decode_kernel<G, true, RES, 4, TR>), dim3(a.nsplit * n_kv_heads), block, s, a);
  } else {
    IRON_GQA_DECODE_LAUNCH((gqa_decode_kernel<G, false, RES, 4, TR>), dim3(a.nsplit, n_kv_heads), block, s, a);
    IRON_LAUNCH((gqa_combine_kernel<G>), dim3(n_kv_heads * G), dim3(kMergeThreads), 0, s, a);
  }
}

// The traced instance only while a phase trace is armed.
template <int G, bool RES>
static void gqa_decode_dispatch_tr(const DecodeArgs& a, int n_kv_heads, bool one_launch, bool long_chunks,
                                   hipStream_t s) {
  if (a.trace)
    gqa_decode_dispatch<G, RES, true>(a, n_kv_heads, one_launch, long_chunks, s);
  else
    gqa_decode_dispatch<G, RES, false>(a, n_kv_heads, one_launch, long_chunks, s);
}

static int gqa_decode_launch(const char* who, const void* q, const void* k_new, const void* v_new, void* k_cache,
                             void* v_cache, const float* angles, int angle_rows, void* out, void* workspace,
                             int n_heads, int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev,
                             float scale, void* stream, int flags) {
  IRON_REQUIRE((flags & ~(IRON_GQA_KV_RESIDENT | IRON_GQA_COUNTERS_ZERO)) == 0, "%s: unknown flags 0x%x", who,
               static_cast<unsigned>(flags));
  IRON_REQUIRE(q && k_new && v_new && k_cache && v_cache && angles && out && workspace, "%s: null pointer", who);
  IRON_REQUIRE(head_dim == kD, "%s: head_dim=%d (only 64 is supported)", who, head_dim);
  IRON_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "%s: n_heads=%d must be a multiple of n_kv_heads=%d", who, n_heads, n_kv_heads);
  const int G = n_heads / n_kv_heads;
  IRON_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "%s: group size %d not in {1,2,4,8}", who, G);
  IRON_REQUIRE(max_len > 0 && angle_rows > 0, "%s: max_len and angle_rows must be positive", who);
  IRON_REQUIRE(pos_dev || (pos >= 0 && pos < max_len && pos < angle_rows),
               "%s: pos=%d outside the cache (max_len=%d) or angle table (%d rows)", who, pos, max_len, angle_rows);
  IRON_REQUIRE(aligned16(q) && aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) && aligned16(v_cache) &&
                   aligned16(angles),
               "%s: q, k_new, v_new, the caches and the angle table must be 16-byte aligned", who);
  IRON_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "%s: workspace must be 256-byte aligned", who);
  IRON_REQUIRE(decode_head_stride(G, max_len) * 4 < (1LL << 31),
               "%s: max_len=%d: a KV head's chunk partials exceed the 2 GiB the merge addresses", who, max_len);
  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k_new = static_cast<const uint16_t*>(k_new);
  a.v_new = static_cast<const uint16_t*>(v_new);
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.angles = angles;
  a.out = static_cast<uint16_t*>(out);
  a.ctr = static_cast<unsigned*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + decode_ctr_bytes(n_kv_heads));
  a.head_stride = decode_head_stride(G, max_len);
  a.pos_dev = pos_dev;
  a.pos = pos;
  a.max_len = max_len;
  a.angle_rows = angle_rows;
  a.nsplit = decode_nsplit(max_len);
  a.scale_log2 = scale * 1.4426950408889634f;
  // at most one record per 64-position chunk of every KV head (the grid of either launch shape)
  if (int rc = take_trace(who, static_cast<long long>(a.nsplit) * n_kv_heads, &a.trace)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool one = n_kv_heads % kXcds == 0 && xcd_round_robin(s) == 1;
  const bool long_chunks = one && decode_long_chunks(n_kv_heads, max_len, pos, (flags & IRON_GQA_KV_RESIDENT) != 0);
  if (one && !(flags & IRON_GQA_COUNTERS_ZERO))
    IRON_LAUNCH(gqa_clear_counters_kernel, dim3(1), dim3(kWave), 0, s, a.ctr, n_kv_heads);
  if (flags & IRON_GQA_KV_RESIDENT) {
    switch (G) {
      case 1: gqa_decode_dispatch_tr<1, true>(a, n_kv_heads, one, long_chunks, s); break;
      case 2: gqa_decode_dispatch_tr<2, true>(a, n_kv_heads, one, long_chunks, s); break;
      case 4: gqa_decode_dispatch_tr<4, true>(a, n_kv_heads, one, long_chunks, s); break;
      default: gqa_decode_dispatch_tr<8, true>(a, n_kv_heads, one, long_chunks, s); break;
    }
  } else {
    switch (G) {
      case 1: gqa_decode_dispatch_tr<1, false>(a, n_kv_heads, one, long_chunks, s); break;
      case 2: gqa_decode_dispatch_tr<2, false>(a, n_kv_heads, one, long_chunks, s); break;
      case 4: gqa_decode_dispatch_tr<4, false>(a, n_kv_heads, one, long_chunks, s); break;
      default: gqa_decode_dispatch_tr<8, false>(a, n_kv_heads, one, long_chunks, s); break;
    }
  }
  return check_launch(who);
}

extern "C" int iron_gqa_decode(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                               const float* angles, int angle_rows, void* out, void* workspace, int n_heads,
                               int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev, float scale,
                               void* stream) {
  return gqa_decode_launch("iron_gqa_decode", q, k_new, v_new, k_cache, v_cache, angles, angle_rows, out, workspace,
                           n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream, 0);
}

extern "C" int iron_gqa_decode_ex(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                  const float* angles, int angle_rows, void* out, void* workspace, int n_heads,
                                  int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev, float scale,
                                  int flags, void* stream) {
  return gqa_decode_launch("iron_gqa_decode_ex", q, k_new, v_new, k_cache, v_cache, angles, angle_rows, out,
                           workspace, n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream, flags);
}

// The workspace of iron_gqa_decode_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends. Host code never passes `scratch`
// itself to a kernel (on the host that name is a stand-in, not a device
// address): its device address is looked up once per device with
// hipGetSymbolAddress, with that device current, and only that address is used.
static constexpr long long kDecodeScratchBytes = 4LL << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device (looked up on the first
// call per device), or nullptr with the error set.
static void* decode_scratch_ptr(const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("%s: device %d beyond the %d devices the library tracks", who, dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", who, dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

// Also resolves the calling device's scratch address (a hipGetSymbolAddress,
// which is not to be called under graph capture): call it once outside
// capture, and a captured iron_gqa_decode_noalloc only reads the cached address.
extern "C" long long iron_gqa_decode_noalloc_max_bytes(void) {
  decode_scratch_ptr("iron_gqa_decode_noalloc_max_bytes");
  return kDecodeScratchBytes;
}

extern "C" int iron_gqa_decode_noalloc(const void* q, const void* k_new, const void* v_new, void* k_cache,
                                       void* v_cache, const float* angles, int angle_rows, void* out, int n_heads,
                                       int n_kv_heads, int head_dim, int max_len, int pos, const int* pos_dev,
                                       float scale, void* stream) {
  const long long need = iron_gqa_decode_workspace_bytes(n_heads, n_kv_heads, head_dim, max_len);
  IRON_REQUIRE(need > 0, "iron_gqa_decode_noalloc: invalid shape (n_heads=%d, n_kv_heads=%d, head_dim=%d, max_len=%d)",
               n_heads, n_kv_heads, head_dim, max_len);
  IRON_REQUIRE(need <= kDecodeScratchBytes,
               "iron_gqa_decode_noalloc: this shape needs %lld bytes of scratch, more than the %lld the library "
               "holds per device (use iron_gqa_decode with a workspace)", need, kDecodeScratchBytes);
  void* ws = decode_scratch_ptr("iron_gqa_decode_noalloc");
  if (!ws) return IRON_EINVAL;
  return gqa_decode_launch("iron_gqa_decode_noalloc", q, k_new, v_new, k_cache, v_cache, angles, angle_rows, out, ws,
                           n_heads, n_kv_heads, head_dim, max_len, pos, pos_dev, scale, stream, 0);
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
  IRON_REQUIRE(scale > 0.f && scale < INFINITY, "iron_attention_prefill: scale=%g must be positive and finite",
               static_cast<double>(scale));
  if (out_rows < seq_q) out_rows = seq_q;
  IRON_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && q_row_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                   kv_row_stride % 8 == 0 && kv_head_stride % 8 == 0,
               "iron_attention_prefill: rows must be 16-byte aligned");
  // K/V rows are addressed by 32-bit byte offsets from each head's base
  IRON_REQUIRE(kv_row_stride >= 0 && static_cast<long long>(seq_kv) * kv_row_stride * 2 < (1LL << 31) - 256,
               "iron_attention_prefill: seq_kv=%d x kv_row_stride=%lld spans more than 2 GiB", seq_kv, kv_row_stride);
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
  IRON_REQUIRE(aligned16(out) && o_row_stride % 8 == 0 && o_head_stride % 8 == 0,
               "iron_attention_prefill: out rows must be 16-byte aligned");
  IRON_REQUIRE((out_rows + kFaQ - 1) / kFaQ < 65536, "iron_attention_prefill: out_rows=%d too large", out_rows);
  dim3 grid(n_heads, (out_rows + kFaQ - 1) / kFaQ), block(256);
  IRON_LAUNCH(attention_prefill_kernel, grid, block, 0, static_cast<hipStream_t>(stream), a);
  return check_launch("attention_prefill");
}
