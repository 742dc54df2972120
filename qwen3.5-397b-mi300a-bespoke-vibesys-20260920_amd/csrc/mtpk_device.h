// Device-side building blocks shared by the libmtpk translation units (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mtpk.h"
#include "mtpk_common.h"

namespace mtpk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ inline u32x4_t ld16(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }

__device__ inline u32x4_t zero16() { return u32x4_t{0u, 0u, 0u, 0u}; }

// 16-byte LDS read / write (ds_read_b128 / ds_write_b128; 16-byte aligned addresses).
__device__ inline u32x4_t lds16(const uint8_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }
__device__ inline void lds16_store(uint8_t* p, u32x4_t v) { *reinterpret_cast<u32x4_t*>(p) = v; }

// Raw buffer loads. A buffer resource covers [base, base + bytes); a load whose byte offset
// lies outside returns zeros and touches no memory, so a lane that has nothing to load gets
// the offset kOutOfRange instead of a branch around its load (branches around loads make the
// compiler wait for every outstanding load at the join, which would drain the trip ring).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;  // raw (unformatted) 32-bit buffer, gfx9 family

__device__ inline rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}

__device__ inline u32x4_t buf16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// The same with a wave-uniform byte offset `soff` (an SGPR operand) added to the per-lane
// `off`. Only `off` carries kOutOfRange; `soff` itself always stays inside the buffer.
__device__ inline u32x4_t buf16(rsrc_t r, uint32_t off, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, 0));
}

// Direct-to-LDS form of buf16: lane L's 16 bytes land at lds + 16 L (lds wave-uniform), and no
// register holds them. The load counts in vmcnt like the others, in issue order; the reader of
// the LDS bytes waits for it with vmcnt_wait.
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ inline void buf16_lds(rsrc_t r, uint32_t off, uint8_t* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, (int)off, 0, 0, 0);
}

// s_waitcnt vmcnt(N) alone (gfx9 encoding, expcnt and lgkmcnt fields at their no-wait values):
// every vector memory load but the N most recently issued has completed.
template <int N>
__device__ inline void vmcnt_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

__device__ inline uint32_t buf1(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}

__device__ inline int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Scalar (constant-cache) load of p[i] for a wave-uniform p and i, from memory that an earlier
// launch wrote and this one only reads.
typedef const __attribute__((address_space(4))) int32_t* kc_i32_t;
__device__ inline int32_t sload(const int32_t* p, int i) { return ((kc_i32_t)p)[i]; }

// The e8m0 scales of D consecutive trips of one weight row: bytes [4 tr0, 4 tr0 + 4D) of the
// row, one 8- or 16-byte load instead of D byte loads. Trip tr0 + s of lane group g reads byte
// 4s + g, i.e. byte g of dword s.
template <int D>
struct ScaleChunk;

template <>
struct ScaleChunk<2> {
  uint32_t d[2];
  __device__ inline void load(rsrc_t r, uint32_t off) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t v = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
    d[0] = v[0];
    d[1] = v[1];
  }
  __device__ inline uint32_t byte(int s, int g) const { return (d[s] >> (8 * g)) & 0xffu; }
};

template <>
struct ScaleChunk<4> {
  uint32_t d[4];
  __device__ inline void load(rsrc_t r, uint32_t off) {
    const u32x4_t v = buf16(r, off);
    d[0] = v[0];
    d[1] = v[1];
    d[2] = v[2];
    d[3] = v[3];
  }
  __device__ inline uint32_t byte(int s, int g) const { return (d[s] >> (8 * g)) & 0xffu; }
};

// Scheduling fence between the steps of a trip ring: the compiler may not move any instruction
// across it, so each step's refill loads stay behind that step's MFMAs and the loads consumed
// next are always the oldest outstanding ones (the wait before them leaves D-1 trips in flight).
__device__ inline void ring_fence() { __builtin_amdgcn_sched_barrier(0); }

// Decode parameters of one 32-element block with e8m0 scale byte s: the fp32 scale operand of
// the hardware convert, and the mask applied to the packed codes first.
// The convert takes only the exponent field of its fp32 scale, so s = 0 (fp32 +0.0) acts as
// 2^-127, the OCP reading of that byte, where the pinned kernel decode gives +-0.0. For such a
// block only the codes' sign bits are kept: +-0 * 2^-127 is exactly +-0.0, the sign from the
// code as in the pinned decode. Bytes 1..254 are exact as they are (bf16 has fp32's exponent
// range, so the subnormal products of byte 1 and the overflow to +-inf at 253..254 come out as
// in fp32; checked bit for bit on the GPU). Byte 255, the OCP NaN scale, gives NaN for every
// code, where the pinned decode gives +-inf for nonzero codes: experts holding such a block
// are refused at load (`mtpk_scale_scan`).
struct BlockScale {
  float f;
  uint32_t keep;
};

__device__ inline BlockScale block_scale(uint32_t s) {
  s &= 0xffu;
  return BlockScale{e8m0_to_f32(s), s ? 0xffffffffu : 0x88888888u};
}

// Eight e2m1 codes of one packed dword (code j = nibble j, low nibble first) times the block
// scale, as eight bf16 in element order: the hardware fp4 -> bf16 convert with the e8m0 scale
// applied (one instruction per byte).
__device__ inline bf16x8_t decode8(uint32_t w, const BlockScale& b) {
  w &= b.keep;
  const float scale = b.f;
  const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  const bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  const bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  const u32x4_t r{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                  __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)};
  return __builtin_bit_cast(bf16x8_t, r);
}

__device__ inline bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ inline f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Typed scalar loads/stores selected by a runtime dtype code.
__device__ inline int64_t load_index(const void* p, int dtype, int64_t i) {
  return dtype == MTPK_I64 ? reinterpret_cast<const int64_t*>(p)[i]
                           : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

__device__ inline float load_float(const void* p, int dtype, int64_t i) {
  return dtype == MTPK_F32 ? reinterpret_cast<const float*>(p)[i]
                           : bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

__device__ inline void store_float(void* p, int dtype, int64_t i, float v) {
  if (dtype == MTPK_F32)
    reinterpret_cast<float*>(p)[i] = v;
  else
    reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

__device__ inline void store_index(void* p, int dtype, int64_t i, int64_t v) {
  if (dtype == MTPK_I64)
    reinterpret_cast<int64_t*>(p)[i] = v;
  else
    reinterpret_cast<int32_t*>(p)[i] = (int32_t)v;
}

// Wave-wide reductions over 64 lanes (butterfly: every lane ends with the result).
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, o, kWave);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, kWave);
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  }
  return v;
}

// Inclusive prefix sum across the wave.
__device__ inline int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

// Eight consecutive f32 or bf16 values of p at element i, as floats (bf16: one 16-byte load), and
// the inverse (bf16 rounded to nearest even); the row norms and the fused MoE combine + norm.
__device__ inline void load8(const void* p, int dt, int64_t i, float* v) {
  if (dt == MTPK_F32) {
    const float* f = reinterpret_cast<const float*>(p) + i;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = f[j];
  } else {
    const u32x4_t d = ld16(reinterpret_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bits_f32(d[j] << 16);
      v[2 * j + 1] = bits_f32(d[j] & 0xffff0000u);
    }
  }
}

__device__ inline void store8(void* p, int dt, int64_t i, const float* v) {
  if (dt == MTPK_F32) {
    float* f = reinterpret_cast<float*>(p) + i;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = v[j];
  } else {
    u32x4_t d;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      d[j] = (uint32_t)f32_to_bf16(v[2 * j]) | ((uint32_t)f32_to_bf16(v[2 * j + 1]) << 16);
    *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(p) + i) = d;
  }
}

}  // namespace mtpk
