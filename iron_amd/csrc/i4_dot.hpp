// Building blocks of the int4-group-32 inner products of the GEMV kernels.
//
// Dequant-free inner product: a nibble n placed in the mantissa of the bf16
// 0x4300 (=128) gives the exact value 128+n, so one v_bitop3_b32 builds two
// such weights at once and v_dot2c consumes them. For signed codes the nibble
// sign bit is flipped in the same op (offset binary, 128+(q+8) = 136+q). The
// constant part is removed per group with the group's x sum:
// sum((c+q) x) - c*sum(x). The group scale multiplies the group total once.
#pragma once

#include "iron_common.hpp"

namespace iron {

// Sum of squares of the 8 bf16 of a 16-byte chunk added to acc: one v_dot2
// per pair (a pair times itself), so no unpacking.
__device__ __forceinline__ float sumsq_chunk(uint4 v, float acc) {
  acc = dot2_bf16(v.x, v.x, acc);
  acc = dot2_bf16(v.y, v.y, acc);
  acc = dot2_bf16(v.z, v.z, acc);
  return dot2_bf16(v.w, v.w, acc);
}

constexpr uint32_t kBf16OnePair = 0x3f803f80u;  // (1.0, 1.0) as two bf16

// x chunk of one group (32 bf16) rearranged into the nibble-pair order:
// word q of the codes holds elements 8q..8q+7; the pair extracted at shift 4j
// is (element 8q+j, element 8q+j+4).
struct XGroup {
  uint32_t p[16];
  float sum;
};

// The group's x sum takes one v_dot2 with (1, 1) per pair.
__device__ __forceinline__ void build_xgroup(const uint4 (&xc)[4], XGroup& g) {
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t w0 = xc[q].x, w1 = xc[q].y, w2 = xc[q].z, w3 = xc[q].w;  // (x0,x1) (x2,x3) (x4,x5) (x6,x7)
    // v_perm_b32 byte selects over {hi: first operand, lo: second}: 0-3 the
    // second operand's bytes, 4-7 the first's
    g.p[q * 4 + 0] = __builtin_amdgcn_perm(w2, w0, 0x05040100u);  // (x0, x4)
    g.p[q * 4 + 1] = __builtin_amdgcn_perm(w2, w0, 0x07060302u);  // (x1, x5)
    g.p[q * 4 + 2] = __builtin_amdgcn_perm(w3, w1, 0x05040100u);  // (x2, x6)
    g.p[q * 4 + 3] = __builtin_amdgcn_perm(w3, w1, 0x07060302u);  // (x3, x7)
    s = dot2_bf16(w0, kBf16OnePair, s);
    s = dot2_bf16(w1, kBf16OnePair, s);
    s = dot2_bf16(w2, kBf16OnePair, s);
    s = dot2_bf16(w3, kBf16OnePair, s);
  }
  g.sum = s;
}

// Truth table of f(a, b, c) = (a & b) ^ c for v_bitop3_b32 (inputs 0xF0, 0xCC, 0xAA).
constexpr unsigned kAndXor = (0xF0u & 0xCCu) ^ 0xAAu;

// `magic` = 0x43084308 for signed codes (mask, then XOR sets the 0x4300
// exponent bits and flips the nibble sign bit: 128 + (q + 8)), 0x43004300 for
// unsigned codes (128 + n). One v_bitop3_b32 + one v_dot2c per weight pair.
__device__ __forceinline__ float i4_group_dot(uint4 c, const XGroup& g, uint32_t magic) {
  const uint32_t words[4] = {c.x, c.y, c.z, c.w};
  float acc = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t u = words[q];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t wpair = __builtin_amdgcn_bitop3_b32(u >> (4 * j), 0x000f000fu, magic, kAndXor);
      acc = dot2_bf16(wpair, g.p[q * 4 + j], acc);
    }
  }
  return acc;
}

// Group total sum(w' x) - offset * sum(x), w' = offset + q: one explicit FMA,
// so the rounding is the same in every kernel (a product shared by several
// rows would otherwise be computed once and subtracted, or fused per row,
// depending on the surrounding code).
__device__ __forceinline__ float i4_group_total(uint4 c, const XGroup& g, uint32_t magic, float offset) {
  return fmaf(-offset, g.sum, i4_group_dot(c, g, magic));
}

}  // namespace iron
