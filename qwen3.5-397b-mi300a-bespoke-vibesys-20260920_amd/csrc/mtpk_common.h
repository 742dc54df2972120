// Shared host/device helpers for libmtpk (gfx950).
//
// Everything here is plain integer/float arithmetic usable from device code and, with
// MTPK_HOST_TEST defined, from a host C++ build: the CPU tests compile this header with g++
// and emulate the MoE kernels' lane decomposition with it, so an indexing mistake fails on the
// CPU before any GPU run.
#pragma once

#include <stdint.h>

#ifdef MTPK_HOST_TEST
#define MTPK_HD inline
#else
#include <hip/hip_runtime.h>
#define MTPK_HD __host__ __device__ inline
#endif

namespace mtpk {

// ---------------------------------------------------------------- bf16 / fp32 bits

MTPK_HD uint32_t f32_bits(float f) {
  union { float f; uint32_t u; } v;
  v.f = f;
  return v.u;
}

MTPK_HD float bits_f32(uint32_t u) {
  union { float f; uint32_t u; } v;
  v.u = u;
  return v.f;
}

// fp32 -> bf16, round to nearest even. NaN stays a quiet NaN.
MTPK_HD uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

MTPK_HD float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// Split v into hi + lo with hi = v truncated to bf16 and lo = bf16_rne(v - hi). v - hi is exact
// in fp32 (v's low 16 mantissa bits, below 2^-7 |v|) and lo rounds it to 8 significant bits,
// so |hi + lo - v| <= 2^-15 |v|, against 2^-8 for a single bf16.
MTPK_HD void split_bf16(float v, uint16_t* hi, uint16_t* lo) {
  uint32_t u = f32_bits(v);
  uint32_t h = u & 0xffff0000u;
  *hi = (uint16_t)(h >> 16);
  *lo = f32_to_bf16(v - bits_f32(h));
}

// Exact three-way split: hi = v truncated to bf16, mid = the next 8 significant bits truncated,
// lo = bf16_rne of the remainder (at most 8 significant bits, so exact for normal values).
MTPK_HD void split3_bf16(float v, uint16_t* hi, uint16_t* mid, uint16_t* lo) {
  const uint32_t h = f32_bits(v) & 0xffff0000u;
  const float r = v - bits_f32(h);
  const uint32_t m = f32_bits(r) & 0xffff0000u;
  *hi = (uint16_t)(h >> 16);
  *mid = (uint16_t)(m >> 16);
  *lo = f32_to_bf16(r - bits_f32(m));
}

// e8m0 scale byte -> fp32 2^(s-127) with the pinned kernel conventions: 0 -> +0.0,
// 255 -> +inf (the byte lands in the fp32 exponent field).
MTPK_HD float e8m0_to_f32(uint32_t s) { return bits_f32((s & 0xffu) << 23); }

// e2m1 code (4 bits: sign, e1, e0, m) -> exact fp32 value, by building the fp32 fields.
// e != 0: 2^(e-1) * (1 + m/2) = exponent e + 126, top mantissa bit m. e == 0: m * 0.5.
MTPK_HD float fp4_to_f32(uint32_t code) {
  const uint32_t sign = (code & 8u) << 28;
  const uint32_t e = (code >> 1) & 3u, m = code & 1u;
  const uint32_t mag = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3f000000u : 0u);
  return bits_f32(sign | mag);
}

// Orderable key for a float: larger float -> larger key; -0.0 is folded onto +0.0 so the two
// zeros tie, as a float comparison says they do.
MTPK_HD uint32_t f32_order_key(float f) {
  uint32_t u = f32_bits(f);
  if (u == 0x80000000u) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// (value, index) -> 64-bit key whose max is the first-occurrence argmax: larger value wins,
// and among equal values the smaller index (its complement is larger).
MTPK_HD uint64_t argmax_key(float v, uint32_t index) {
  return ((uint64_t)f32_order_key(v) << 32) | (uint64_t)(0xffffffffu - index);
}

MTPK_HD uint32_t argmax_key_index(uint64_t key) { return 0xffffffffu - (uint32_t)(key & 0xffffffffu); }

// ---------------------------------------------------------------- MoE lane mapping
//
// One wave (64 lanes) computes a 16 x 16 output tile D[m][n] with v_mfma_f32_16x16x32_bf16:
// m = token slot of the work unit (A operand, activations), n = weight row within a 16-row tile
// (B operand, decoded MXFP4). Lane l is (g = l / 16, c = l % 16):
//   - as a B lane it owns weight row c and, in trip `tr`, the 32-element scale block
//     blk = 4 * tr + g of that row: one 16-byte load of packed nibbles (coalesced: the four g
//     lanes of a row read 64 contiguous bytes) and one scale byte;
//   - the block's 32 values feed four MFMAs h = 0..3, eight values each (packed dword h);
//   - as an A lane it owns token slot c and supplies the same eight K positions
//     blk * 32 + 8h + j, j = 0..7, from the activation row;
//   - D: lane (g, c) holds rows m = 4g + i (i = 0..3) of column n = c.
// Every K position of a trip is covered exactly once: (g, h, j) -> 32 (4 tr + g) + 8h + j.

struct MoeLane {
  int g, c;
};

MTPK_HD MoeLane moe_lane(int lane) { return MoeLane{lane >> 4, lane & 15}; }

// Scale block a B lane reads in trip tr.
MTPK_HD int moe_block(int tr, int g) { return 4 * tr + g; }

// K index of value j (0..7) of MFMA slot h (0..3) for lane group g in trip tr.
MTPK_HD int moe_k_index(int tr, int g, int h, int j) { return 32 * moe_block(tr, g) + 8 * h + j; }

// Token slot m held by output register i of lane group g.
MTPK_HD int moe_out_slot(int g, int i) { return 4 * g + i; }

}  // namespace mtpk
