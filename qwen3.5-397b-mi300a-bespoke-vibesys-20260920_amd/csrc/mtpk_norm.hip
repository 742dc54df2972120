// Row normalisations of the verify / draft forward for gfx950, one launch each instead of the
// chain of elementwise and reduction kernels the torch spelling takes:
//   kind 0  Qwen RMSNorm          y = x * rsqrt(mean(x^2) + eps) * (1 + w)      (model.py:587-604)
//   kind 1  gated RMSNorm         y = x * rsqrt(mean(x^2) + eps) * w * silu(g)  (model.py:613-619)
//   kind 2  L2 norm               y = x * rsqrt(sum(x^2) + eps) * scale         (DeltaNet q / k)
// with, optionally, a residual add in front (x <- x + res in x's dtype, the sum also written
// out, as `x = x + mixer` then `rmsnorm(x)`) and rotate-half RoPE behind (on the first rot_dim channels
// of the bf16-rounded result, model.py:631-635). Row r is head r % heads_per_token of token
// r / heads_per_token, read at token * token_stride + head * head_stride, so head slices of a
// projection output are read in place; with a gather table, token r reads input token
// gather[r * gather_stride] (an embedding row by token id). Output token r is written at
// r * out_token_stride + head * dim (two norms can fill the halves of one concatenated row).
// fp32 arithmetic throughout.
//
// Layout of the work (rows of a multiple of 2048 elements without RoPE: k_rownorm_row, one row
// per workgroup): a row of `dim` elements is split over G = min(64, dim / 8) lanes, each
// lane holding chunks of 8 consecutive elements (chunk c = lane-in-group + G * i); a wave
// holds 64 / G rows, a workgroup 4 waves. The sum of squares is a butterfly over the G lanes.

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kNormMaxChunks = 16;  // dim <= 64 * 8 * 16 = 8192

struct NormArgs {
  const void* x;
  int x_dt;
  int64_t x_ts, x_hs;
  const void* res;
  int res_dt;
  void* sum_out;
  const void* w;
  int w_dt;
  int kind;
  float eps, scale;
  const void* gate;
  int g_dt;
  int64_t g_ts, g_hs;
  const float* cos_t;
  const float* sin_t;
  const int64_t* pos;
  int rot;
  void* out;
  int o_dt;
  int64_t rows;
  int hpt, dim;
  const int64_t* gather;  // input token of output token r: gather[r * gather_stride] (or r)
  int64_t gather_stride, gather_rows;
  int64_t o_ts;  // output token stride (elements)
};

// the input token read for output token `tok` (a gathered id outside the table reads its
// nearest row: the callers check ids on the host, this keeps every read in bounds)
__device__ inline int64_t norm_src_token(const NormArgs& a, int64_t tok) {
  if (!a.gather) return tok;
  const int64_t g = a.gather[tok * a.gather_stride];
  return g < 0 ? 0 : (g >= a.gather_rows ? a.gather_rows - 1 : g);
}

__device__ inline float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <int G>
__global__ __launch_bounds__(256) void k_rownorm(NormArgs a) {
  constexpr int RPW = kWave / G;  // rows per wave
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int gl = lane % G;
  const int64_t row = ((int64_t)blockIdx.x * 4 + wave) * RPW + lane / G;
  const bool ok = row < a.rows;  // rows past the end compute on row 0 and store nothing
  const int64_t r = ok ? row : 0;
  const int64_t tok = r / a.hpt, head = r - tok * a.hpt;
  const int nch = a.dim / 8 / G;  // chunks per lane (a.dim is a multiple of 8 G)
  const int64_t xo = norm_src_token(a, tok) * a.x_ts + head * a.x_hs;
  const int64_t oo = tok * a.o_ts + head * a.dim;
  float v[kNormMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    if (i < nch) {
      const int e = (gl + G * i) * 8;
      load8(a.x, a.x_dt, xo + e, v[i]);
      if (a.res) {
        float rv[8];
        load8(a.res, a.res_dt, oo + e, rv);
        // the sum in x's dtype, as `x = x + res` computes it
#pragma unroll
        for (int j = 0; j < 8; ++j)
          v[i][j] = a.x_dt == MTPK_BF16 ? round_bf16(v[i][j] + rv[j]) : v[i][j] + rv[j];
        if (ok) store8(a.sum_out, a.x_dt, oo + e, v[i]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[i][j] * v[i][j];
    }
  }
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
  const float inv = a.kind == 2 ? rsqrtf(ss + a.eps) : rsqrtf(ss / (float)a.dim + a.eps);
  const int64_t go = tok * a.g_ts + head * a.g_hs;
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i) {
    if (i < nch) {
      const int e = (gl + G * i) * 8;
      float y[8];
      if (a.kind == 2) {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = v[i][j] * inv * a.scale;
      } else {
        float wv[8];
        load8(a.w, a.w_dt, e, wv);
        if (a.kind == 0) {
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = (v[i][j] * inv) * (1.f + wv[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = v[i][j] * inv * wv[j];
          if (a.gate) {
            float gv[8];
            load8(a.gate, a.g_dt, go + e, gv);
#pragma unroll
            for (int j = 0; j < 8; ++j) y[j] = y[j] * (gv[j] / (1.f + __expf(-gv[j])));
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = y[j];
    }
  }
  if (a.cos_t) {
    // rotate-half on channels [0, rot) of the normed values in the output dtype (one chunk per
    // lane): channel e's partner is e + rot/2 (e < rot/2, negated) or e - rot/2. For rot a
    // multiple of 16 it sits on lane gl +- rot/16; for rot = 2, 4, 8 it is channel e ^ rot/2
    // of the same chunk.
    const int half = a.rot / 2;
    const int64_t p = a.pos[tok];
    const int e0 = gl * 8;
    float rv[8], pv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) rv[j] = a.o_dt == MTPK_BF16 ? round_bf16(v[0][j]) : v[0][j];
    if (half >= 8) {
      const int sh = half / 8;
      const bool lower = e0 < half;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float up = __shfl(rv[j], lane + sh, kWave);  // partner for the lower half
        const float dn = __shfl(rv[j], lane - sh, kWave);  // partner for the upper half
        pv[j] = lower ? -up : dn;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float q = half == 1 ? rv[j ^ 1] : half == 2 ? rv[j ^ 2] : rv[j ^ 4];
        pv[j] = (j & half) ? q : -q;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (e0 + j < a.rot) {
        const float c = a.cos_t[p * a.rot + e0 + j], sn = a.sin_t[p * a.rot + e0 + j];
        v[0][j] = rv[j] * c + pv[j] * sn;
      }
    }
  }
  if (!ok) return;
#pragma unroll
  for (int i = 0; i < kNormMaxChunks; ++i)
    if (i < nch) store8(a.out, a.o_dt, oo + (gl + G * i) * 8, v[i]);
}

// Wide rows (dim >= 1024, no RoPE): one row per workgroup, NCH chunks of 8 per thread, so a
// few hundred rows still fill the chip; the weight (and gate) loads are issued before the
// reduction, which goes through the four waves' partial sums in LDS.
template <int NCH>
__global__ __launch_bounds__(256) void k_rownorm_row(NormArgs a) {
  __shared__ float part[4];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int64_t r = blockIdx.x;
  const int64_t tok = r / a.hpt, head = r - tok * a.hpt;
  const int64_t xo = norm_src_token(a, tok) * a.x_ts + head * a.x_hs, oo = tok * a.o_ts + head * a.dim;
  const int64_t go = tok * a.g_ts + head * a.g_hs;
  float v[NCH][8], wv[NCH][8], gv[NCH][8];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int e = (tid + 256 * i) * 8;
    load8(a.x, a.x_dt, xo + e, v[i]);
    if (a.kind != 2) load8(a.w, a.w_dt, e, wv[i]);
    if (a.gate) load8(a.gate, a.g_dt, go + e, gv[i]);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int e = (tid + 256 * i) * 8;
    if (a.res) {
      float rv[8];
      load8(a.res, a.res_dt, oo + e, rv);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[i][j] = a.x_dt == MTPK_BF16 ? round_bf16(v[i][j] + rv[j]) : v[i][j] + rv[j];
      store8(a.sum_out, a.x_dt, oo + e, v[i]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += v[i][j] * v[i][j];
  }
  ss = wave_sum(ss);
  if (lane == 0) part[wave] = ss;
  __syncthreads();
  ss = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = a.kind == 2 ? rsqrtf(ss + a.eps) : rsqrtf(ss / (float)a.dim + a.eps);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (a.kind == 2)
        y[j] = v[i][j] * inv * a.scale;
      else if (a.kind == 0)
        y[j] = (v[i][j] * inv) * (1.f + wv[i][j]);
      else
        y[j] = a.gate ? (v[i][j] * inv * wv[i][j]) * (gv[i][j] / (1.f + __expf(-gv[i][j])))
                      : v[i][j] * inv * wv[i][j];
    }
    store8(a.out, a.o_dt, oo + (tid + 256 * i) * 8, y);
  }
}

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int mtpk_rownorm(const void* x, int x_dtype, int64_t x_token_stride, int64_t x_head_stride,
                 const void* res, int res_dtype, void* sum_out, const void* w, int w_dtype,
                 int kind, float eps, float scale, const void* gate, int gate_dtype,
                 int64_t gate_token_stride, int64_t gate_head_stride, const float* rope_cos,
                 const float* rope_sin, const int64_t* rope_pos, int rot_dim, void* out,
                 int out_dtype, int64_t rows, int heads_per_token, int dim, const int64_t* gather,
                 int64_t gather_stride, int64_t gather_rows, int64_t out_token_stride,
                 void* stream) {
  auto fdt = [](int d) { return d == MTPK_F32 || d == MTPK_BF16; };
  if (!x || !out || !fdt(x_dtype) || !fdt(out_dtype)) return MTPK_EINVAL;
  if (kind < 0 || kind > 2 || rows < 0 || heads_per_token < 1 || dim < 8 || dim % 8) return MTPK_EINVAL;
  if (kind != 2 && (!w || !fdt(w_dtype))) return MTPK_EINVAL;
  if (gate && (kind != 1 || !fdt(gate_dtype))) return MTPK_EINVAL;
  if (res && (!sum_out || !fdt(res_dtype) || heads_per_token != 1 || x_token_stride != dim))
    return MTPK_EINVAL;
  // 0: outputs packed, token stride heads_per_token * dim; the residual form is packed throughout
  if (out_token_stride == 0) out_token_stride = (int64_t)heads_per_token * dim;
  if (out_token_stride < (int64_t)heads_per_token * dim || out_token_stride % 8 ||
      (res && (gather || out_token_stride != dim)) || (gather && gather_rows < 1))
    return MTPK_EINVAL;
  const int g = dim / 8 >= 64 ? 64 : dim / 8;
  if (g & (g - 1)) return MTPK_EINVAL;  // G a power of two
  if (dim % (8 * g) || dim / (8 * g) > kNormMaxChunks) return MTPK_EINVAL;
  if (rope_cos) {
    // one chunk per lane; rot a multiple of 16, or 2, 4 or 8 (inside the first chunk)
    const bool small = rot_dim == 2 || rot_dim == 4 || rot_dim == 8;
    if (!rope_sin || !rope_pos || dim > 512 || rot_dim > dim || !(small || rot_dim % 16 == 0))
      return MTPK_EINVAL;
  }
  // 16-byte bf16 accesses: every row start and stride on an 8-element boundary
  if (x_dtype == MTPK_BF16 && (x_token_stride % 8 || x_head_stride % 8 || !aligned16(x)))
    return MTPK_EINVAL;
  if (out_dtype == MTPK_BF16 && !aligned16(out)) return MTPK_EINVAL;
  if (gate && gate_dtype == MTPK_BF16 &&
      (gate_token_stride % 8 || gate_head_stride % 8 || !aligned16(gate)))
    return MTPK_EINVAL;
  if (res && ((res_dtype == MTPK_BF16 && !aligned16(res)) || !aligned16(sum_out))) return MTPK_EINVAL;
  if (w && w_dtype == MTPK_BF16 && !aligned16(w)) return MTPK_EINVAL;
  if (rows == 0) return 0;
  NormArgs a{x,        x_dtype,  x_token_stride, x_head_stride, res,   res_dtype,  sum_out,
             w,        w_dtype,  kind,           eps,           scale, gate,       gate_dtype,
             gate_token_stride, gate_head_stride, rope_cos,     rope_sin, rope_pos, rot_dim,
             out,      out_dtype, rows,          heads_per_token, dim,
             gather,   gather_stride, gather_rows, out_token_stride};
  const hipStream_t st = (hipStream_t)stream;
  if (!rope_cos && dim % 2048 == 0 && dim <= 8192) {  // one row per workgroup
    if (rows > INT32_MAX) return MTPK_EINVAL;
    const dim3 grid((unsigned)rows);
    switch (dim / 2048) {
      case 1: hipLaunchKernelGGL(k_rownorm_row<1>, grid, dim3(256), 0, st, a); break;
      case 2: hipLaunchKernelGGL(k_rownorm_row<2>, grid, dim3(256), 0, st, a); break;
      case 3: hipLaunchKernelGGL(k_rownorm_row<3>, grid, dim3(256), 0, st, a); break;
      default: hipLaunchKernelGGL(k_rownorm_row<4>, grid, dim3(256), 0, st, a); break;
    }
    return status_of(hipGetLastError());
  }
  const int rpw = 64 / g;
  const int64_t wgs = (rows + 4 * rpw - 1) / (4 * rpw);
  if (wgs > INT32_MAX) return MTPK_EINVAL;
  switch (g) {
    case 64: hipLaunchKernelGGL(k_rownorm<64>, dim3((unsigned)wgs), dim3(256), 0, st, a); break;
    case 32: hipLaunchKernelGGL(k_rownorm<32>, dim3((unsigned)wgs), dim3(256), 0, st, a); break;
    case 16: hipLaunchKernelGGL(k_rownorm<16>, dim3((unsigned)wgs), dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL(k_rownorm<8>, dim3((unsigned)wgs), dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(k_rownorm<4>, dim3((unsigned)wgs), dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(k_rownorm<2>, dim3((unsigned)wgs), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(k_rownorm<1>, dim3((unsigned)wgs), dim3(256), 0, st, a); break;
  }
  return status_of(hipGetLastError());
}

}  // extern "C"
