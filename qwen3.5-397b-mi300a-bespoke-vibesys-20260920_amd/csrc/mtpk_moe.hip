// Routed MXFP4 MoE for gfx950: work-list prep, gate_up + SiLU, down, fixed-order combine.
//
// Data flow for one call (all on the caller's stream, no host sync, static launch shapes):
//   prep      routing -> expert-grouped `sorted` + work units (expert, first, count <= 16)
//   gate_up   per (unit, 16 intermediate rows): MXFP4 decoded in registers, bf16 MFMA with the
//             unit's activation rows, K split over the 4 waves of the workgroup and reduced in
//             LDS; SiLU(gate) * up written as bf16 hi/lo planes (16 significant bits)
//   down      per (unit, 64 hidden rows): same decode, MFMA over both inter planes; fp32 y
//   combine   per token: sum of weight * y over its top_k assignments in j order
// The weight stream is the only HBM-sized traffic; nothing dequantised is ever stored.
// Lane mapping and K coverage of one MFMA tile: see mtpk_common.h ("MoE lane mapping").

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kUnitTokens = MTPK_MOE_UNIT_TOKENS;
constexpr int kMoeWaves = 4;
constexpr int kMoeThreads = kMoeWaves * kWave;
constexpr int kPrepThreads = 1024;

// ---------------------------------------------------------------- prep

__global__ __launch_bounds__(kPrepThreads) void k_moe_prep(
    const void* __restrict__ a_expert, int edt, const void* __restrict__ a_weight, int wdt,
    int assignments, int lo, int n_experts, int32_t* __restrict__ sorted,
    int32_t* __restrict__ units, int max_units, int32_t* __restrict__ n_units) {
  __shared__ int cnt[MTPK_MAX_EXPERTS];
  __shared__ int wtot_c[kPrepThreads / kWave], wtot_u[kPrepThreads / kWave];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;

  for (int e = tid; e < n_experts; e += kPrepThreads) cnt[e] = 0;
  __syncthreads();
  for (int a = tid; a < assignments; a += kPrepThreads) {
    const int64_t ex = load_index(a_expert, edt, a) - lo;
    if (ex >= 0 && ex < n_experts && load_float(a_weight, wdt, a) != 0.f) atomicAdd(&cnt[ex], 1);
  }
  __syncthreads();

  // Each thread owns `per` consecutive experts; a block-wide exclusive scan of the per-thread
  // (assignment count, unit count) pairs gives every expert its first position and first unit.
  const int per = (n_experts + kPrepThreads - 1) / kPrepThreads;
  const int e0 = tid * per;
  int sc = 0, su = 0;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < n_experts) {
      const int c = cnt[e];
      sc += c;
      su += (c + kUnitTokens - 1) / kUnitTokens;
    }
  }
  const int ic = wave_incl_scan(sc, lane), iu = wave_incl_scan(su, lane);
  if (lane == kWave - 1) {
    wtot_c[wv] = ic;
    wtot_u[wv] = iu;
  }
  __syncthreads();
  int pc = ic - sc, pu = iu - su, total_units = 0;
  for (int w = 0; w < kPrepThreads / kWave; ++w) {
    if (w < wv) {
      pc += wtot_c[w];
      pu += wtot_u[w];
    }
    total_units += wtot_u[w];
  }
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e >= n_experts) break;
    const int c = cnt[e];
    const int nu = (c + kUnitTokens - 1) / kUnitTokens;
    for (int j = 0; j < nu; ++j) {
      const int u = pu + j;
      if (u < max_units) {
        units[3 * u + 0] = e;
        units[3 * u + 1] = pc + j * kUnitTokens;
        units[3 * u + 2] = min(kUnitTokens, c - j * kUnitTokens);
      }
    }
    cnt[e] = pc;  // from here on: the claim cursor of expert e
    pc += c;
    pu += nu;
  }
  if (tid == 0) *n_units = min(total_units, max_units);
  __syncthreads();
  for (int a = tid; a < assignments; a += kPrepThreads) {
    const int64_t ex = load_index(a_expert, edt, a) - lo;
    if (ex >= 0 && ex < n_experts && load_float(a_weight, wdt, a) != 0.f)
      sorted[atomicAdd(&cnt[ex], 1)] = a;
  }
}

// ---------------------------------------------------------------- gate_up + SiLU
//
// Work item = (unit u, tile of 16 intermediate rows nt); items are unit-major. The four waves
// of a workgroup take trips w, w+4, ... of the K loop (a trip is 4 scale blocks = 128 K per
// wave: one 16-byte weight load per lane per projection) and reduce their partial tiles in LDS.
// XP = bf16 planes of x (1: bf16 activations; 3: an fp32 activation split exactly).
// OP = bf16 planes written for inter (2 or 3). C = trips whose loads are issued together.

template <int XP, int OP, int C>
__global__ __launch_bounds__(kMoeThreads) void k_moe_gate_up(
    const uint16_t* __restrict__ x, int64_t x_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int I, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ units, const int32_t* __restrict__ n_units_p, int max_units,
    int top_k, uint16_t* __restrict__ inter, int64_t inter_plane) {
  __shared__ f32x4_t red[kMoeWaves - 1][2][kWave];
  const int n_units = min(*n_units_p, max_units);
  const int ntile = I >> 4;
  const int n_items = n_units * ntile;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int64_t row_bytes = K >> 1;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int u = item / ntile, nt = item - u * ntile;
    const int e = units[3 * u], first = units[3 * u + 1], cnt = units[3 * u + 2];
    const bool alive = ln.c < cnt;
    const int tok = sorted[first + (alive ? ln.c : 0)] / top_k;
    const int64_t grow = (int64_t)e * (2 * I) + nt * 16 + ln.c;
    const uint8_t* pg = wq + grow * row_bytes;
    const uint8_t* pu = pg + (int64_t)I * row_bytes;
    const uint8_t* sg = ws + grow * nb;
    const uint8_t* su = sg + (int64_t)I * nb;
    const uint16_t* px = x + (int64_t)tok * K;

    f32x4_t accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    for (int t0 = wave; t0 < ntrip; t0 += kMoeWaves * C) {
      u32x4_t wg[C], wu[C], xv[C][XP][4];
      uint32_t sgv[C], suv[C];
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        const int tr = t0 + kMoeWaves * cc, blk = moe_block(tr, ln.g);
        const bool ok = tr < ntrip && blk < nb;
        wg[cc] = ok ? ld16(pg + blk * 16) : zero16();
        wu[cc] = ok ? ld16(pu + blk * 16) : zero16();
        sgv[cc] = ok ? sg[blk] : 0u;
        suv[cc] = ok ? su[blk] : 0u;
#pragma unroll
        for (int p = 0; p < XP; ++p)
#pragma unroll
          for (int h = 0; h < 4; ++h)
            xv[cc][p][h] = (ok && alive) ? ld16(px + p * x_plane + blk * 32 + 8 * h) : zero16();
      }
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        const float fg = e8m0_to_f32(sgv[cc]), fu = e8m0_to_f32(suv[cc]);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const bf16x8_t bg = decode8(wg[cc][h], fg), bu = decode8(wu[cc][h], fu);
#pragma unroll
          for (int p = 0; p < XP; ++p) {
            const bf16x8_t av = as_bf16x8(xv[cc][p][h]);
            accg = mfma16x16x32(av, bg, accg);
            accu = mfma16x16x32(av, bu, accu);
          }
        }
      }
    }
    if (wave > 0) {
      red[wave - 1][0][lane] = accg;
      red[wave - 1][1][lane] = accu;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < kMoeWaves - 1; ++w) {
        accg += red[w][0][lane];
        accu += red[w][1][lane];
      }
      const int n = nt * 16 + ln.c;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = moe_out_slot(ln.g, i);
        if (m < cnt) {
          const int64_t a = sorted[first + m];
          const float gt = accg[i];
          const float v = gt / (1.f + __expf(-gt)) * accu[i];
          uint16_t* dst = inter + a * I + n;
          if (OP == 2) {
            uint16_t hi, lo;
            split_bf16(v, &hi, &lo);
            dst[0] = hi;
            dst[inter_plane] = lo;
          } else {
            uint16_t hi, mid, lo;
            split3_bf16(v, &hi, &mid, &lo);
            dst[0] = hi;
            dst[inter_plane] = mid;
            dst[2 * inter_plane] = lo;
          }
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- down
//
// Work item = (unit u, 64 hidden rows): wave w owns 16 rows and the whole K (= intermediate)
// loop; IP = bf16 planes of inter; C = trips per load batch.

template <int IP, int C>
__global__ __launch_bounds__(kMoeThreads) void k_moe_down(
    const uint16_t* __restrict__ inter, int64_t inter_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int H, const int32_t* __restrict__ sorted,
    const int32_t* __restrict__ units, const int32_t* __restrict__ n_units_p, int max_units,
    float* __restrict__ y) {
  const int n_units = min(*n_units_p, max_units);
  const int rtiles = H >> 4;
  const int ntile = (rtiles + kMoeWaves - 1) / kMoeWaves;
  const int n_items = n_units * ntile;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int64_t row_bytes = K >> 1;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int u = item / ntile, nt = item - u * ntile;
    const int rt = nt * kMoeWaves + wave;
    if (rt >= rtiles) continue;
    const int e = units[3 * u], first = units[3 * u + 1], cnt = units[3 * u + 2];
    const bool alive = ln.c < cnt;
    const int64_t a_lane = sorted[first + (alive ? ln.c : 0)];
    const int64_t row = (int64_t)e * H + rt * 16 + ln.c;
    const uint8_t* pw = wq + row * row_bytes;
    const uint8_t* ps = ws + row * nb;
    const uint16_t* pa = inter + a_lane * K;

    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int t0 = 0; t0 < ntrip; t0 += C) {
      u32x4_t wv[C], av[C][IP][4];
      uint32_t sv[C];
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        const int tr = t0 + cc, blk = moe_block(tr, ln.g);
        const bool ok = tr < ntrip && blk < nb;
        wv[cc] = ok ? ld16(pw + blk * 16) : zero16();
        sv[cc] = ok ? ps[blk] : 0u;
#pragma unroll
        for (int p = 0; p < IP; ++p)
#pragma unroll
          for (int h = 0; h < 4; ++h)
            av[cc][p][h] = (ok && alive) ? ld16(pa + p * inter_plane + blk * 32 + 8 * h) : zero16();
      }
#pragma unroll
      for (int cc = 0; cc < C; ++cc) {
        const float fs = e8m0_to_f32(sv[cc]);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const bf16x8_t b = decode8(wv[cc][h], fs);
#pragma unroll
          for (int p = 0; p < IP; ++p) acc = mfma16x16x32(as_bf16x8(av[cc][p][h]), b, acc);
        }
      }
    }
    const int n = rt * 16 + ln.c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = moe_out_slot(ln.g, i);
      if (m < cnt) y[(int64_t)sorted[first + m] * H + n] = acc[i];
    }
  }
}

// ---------------------------------------------------------------- combine

__global__ __launch_bounds__(256) void k_moe_combine(
    const float* __restrict__ y, const void* __restrict__ a_expert, int edt,
    const void* __restrict__ a_weight, int wdt, int top_k, int H, int lo, int hi,
    void* __restrict__ out, int odt) {
  const int t = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= H) return;
  float acc = 0.f;
  for (int j = 0; j < top_k; ++j) {
    const int64_t a = (int64_t)t * top_k + j;
    const int64_t e = load_index(a_expert, edt, a);
    const float w = load_float(a_weight, wdt, a);
    if (e >= lo && e < hi && w != 0.f) acc += w * y[a * H + n];
  }
  store_float(out, odt, (int64_t)t * H + n, acc);
}

// ---------------------------------------------------------------- plane split

__global__ __launch_bounds__(256) void k_split_planes(const float* __restrict__ src, int64_t n,
                                                      int nplanes, uint16_t* __restrict__ planes) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = src[i];
    uint16_t hi, mid, lo;
    if (nplanes == 2) {
      split_bf16(v, &hi, &lo);
      planes[i] = hi;
      planes[n + i] = lo;
    } else {
      split3_bf16(v, &hi, &mid, &lo);
      planes[i] = hi;
      planes[n + i] = mid;
      planes[2 * n + i] = lo;
    }
  }
}

// ---------------------------------------------------------------- dequant probe / API

__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ packed,
                                                 const uint8_t* __restrict__ scale, int64_t rows,
                                                 int K, int mode, float* __restrict__ out) {
  const int64_t half = K >> 1, nb = K >> 5;
  const int64_t total = rows * half;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / half, col = i - r * half;
    const uint32_t b = packed[i];
    const uint32_t s = scale[r * nb + (2 * col) / 32];
    float v0, v1;
    if (mode == 0) {
      const float f = e8m0_to_f32(s);
      v0 = fp4_to_f32(b & 15u) * f;
      v1 = fp4_to_f32(b >> 4) * f;
    } else {
      const bf16x2_t p = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(b, e8m0_to_f32(s), 0);
      const uint32_t bits = __builtin_bit_cast(uint32_t, p);
      v0 = bf16_to_f32((uint16_t)(bits & 0xffffu));
      v1 = bf16_to_f32((uint16_t)(bits >> 16));
    }
    out[r * K + 2 * col] = v0;
    out[r * K + 2 * col + 1] = v1;
  }
}

__global__ __launch_bounds__(64) void k_probe_mfma(const uint16_t* __restrict__ a,
                                                   const uint16_t* __restrict__ b,
                                                   float* __restrict__ d) {
  const int l = threadIdx.x;
  const bf16x8_t av = as_bf16x8(ld16(a + 8 * l));
  const bf16x8_t bv = as_bf16x8(ld16(b + 8 * l));
  const f32x4_t r = mfma16x16x32(av, bv, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
  for (int i = 0; i < 4; ++i) d[4 * l + i] = r[i];
}

// ---------------------------------------------------------------- host launchers

namespace {

struct MoeLaunch {
  int grid_gate_up, grid_down;
};

template <typename KernelT>
int persistent_grid(KernelT kernel, int64_t items, int& cache) {
  if (items <= 0) return 0;
  if (cache == 0) cache = occupancy_per_cu(kernel, kMoeThreads);
  const int64_t cap = (int64_t)device_cu_count() * cache;
  return (int)(items < cap ? items : cap);
}

bool dtype_index_ok(int d) { return d == MTPK_I32 || d == MTPK_I64; }
bool dtype_float_ok(int d) { return d == MTPK_F32 || d == MTPK_BF16; }

constexpr int kGateUpChunk = 2;
constexpr int kDownChunk = 2;

template <int XP, int OP>
int launch_gate_up(const uint16_t* x, int64_t x_plane, int K, const uint8_t* wq,
                   const uint8_t* ws, int I, const int32_t* sorted, const int32_t* units,
                   const int32_t* n_units, int max_units, int top_k, uint16_t* inter,
                   int64_t inter_plane, hipStream_t st) {
  static int occ = 0;
  auto kern = k_moe_gate_up<XP, OP, kGateUpChunk>;
  const int grid = persistent_grid(kern, (int64_t)max_units * (I >> 4), occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, x, x_plane, K, wq, ws, I,
                     sorted, units, n_units, max_units, top_k, inter, inter_plane);
  return status_of(hipGetLastError());
}

template <int IP>
int launch_down(const uint16_t* inter, int64_t inter_plane, int K, const uint8_t* wq,
                const uint8_t* ws, int H, const int32_t* sorted, const int32_t* units,
                const int32_t* n_units, int max_units, float* y, hipStream_t st) {
  static int occ = 0;
  auto kern = k_moe_down<IP, kDownChunk>;
  const int64_t ntile = ((H >> 4) + kMoeWaves - 1) / kMoeWaves;
  const int grid = persistent_grid(kern, (int64_t)max_units * ntile, occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, inter, inter_plane, K, wq, ws,
                     H, sorted, units, n_units, max_units, y);
  return status_of(hipGetLastError());
}

}  // namespace

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int64_t mtpk_moe_max_units(int64_t assignments, int64_t local_experts) {
  if (assignments <= 0 || local_experts <= 0) return 0;
  const int64_t distinct = assignments < local_experts ? assignments : local_experts;
  return distinct + assignments / kUnitTokens;
}

int64_t mtpk_moe_workspace_bytes(int64_t tokens, int64_t top_k, int64_t local_experts,
                                 int64_t inter, int64_t hidden, int x_dtype) {
  const int64_t a = tokens * top_k;
  const int64_t mu = mtpk_moe_max_units(a, local_experts);
  const int64_t planes = x_dtype == MTPK_F32 ? 3 : 2;
  int64_t b = align256(a * 4) + align256(3 * mu * 4) + 256;
  if (x_dtype == MTPK_F32) b += align256(3 * tokens * hidden * 2);
  b += align256(planes * a * inter * 2) + align256(a * hidden * 4);
  return b;
}

int mtpk_moe_prep(const void* a_expert, int expert_dtype, const void* a_weight, int weight_dtype,
                  int64_t assignments, int expert_lo, int expert_hi, int32_t* sorted,
                  int32_t* units, int64_t max_units, int32_t* n_units, void* stream) {
  const int64_t ne = (int64_t)expert_hi - expert_lo;
  if (!a_expert || !a_weight || !sorted || !units || !n_units) return MTPK_EINVAL;
  if (!dtype_index_ok(expert_dtype) || !dtype_float_ok(weight_dtype)) return MTPK_EINVAL;
  if (ne <= 0 || ne > MTPK_MAX_EXPERTS || assignments < 0 || assignments > INT32_MAX)
    return MTPK_EINVAL;
  if (max_units < 0 || max_units > INT32_MAX / 3) return MTPK_EINVAL;
  hipLaunchKernelGGL(k_moe_prep, dim3(1), dim3(kPrepThreads), 0, (hipStream_t)stream, a_expert,
                     expert_dtype, a_weight, weight_dtype, (int)assignments, expert_lo, (int)ne,
                     sorted, units, (int)max_units, n_units);
  return status_of(hipGetLastError());
}

int mtpk_moe_gate_up(const uint16_t* x_planes, int x_nplanes, int64_t tokens, int64_t hidden,
                     const uint8_t* gate_up, const uint8_t* gate_up_scale, int64_t local_experts,
                     int64_t inter_dim, const int32_t* sorted, const int32_t* units,
                     const int32_t* n_units, int64_t max_units, int top_k, uint16_t* inter,
                     int inter_planes, int64_t assignments, void* stream) {
  if (!x_planes || !gate_up || !gate_up_scale || !sorted || !units || !n_units || !inter)
    return MTPK_EINVAL;
  if (hidden <= 0 || hidden % 32 || inter_dim <= 0 || inter_dim % 32 || top_k <= 0)
    return MTPK_EINVAL;
  if (hidden > (1 << 20) || inter_dim > (1 << 20) || local_experts <= 0) return MTPK_EINVAL;
  if (!aligned16(x_planes) || !aligned16(gate_up) || !aligned16(inter)) return MTPK_EINVAL;
  if (max_units <= 0 || max_units > INT32_MAX / inter_dim) return MTPK_EINVAL;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t xp = tokens * hidden, ip = assignments * inter_dim;
  if (x_nplanes == 1 && inter_planes == 2)
    return launch_gate_up<1, 2>(x_planes, xp, (int)hidden, gate_up, gate_up_scale,
                                (int)inter_dim, sorted, units, n_units, (int)max_units, top_k,
                                inter, ip, st);
  if (x_nplanes == 3 && inter_planes == 3)
    return launch_gate_up<3, 3>(x_planes, xp, (int)hidden, gate_up, gate_up_scale,
                                (int)inter_dim, sorted, units, n_units, (int)max_units, top_k,
                                inter, ip, st);
  return MTPK_EINVAL;
}

int mtpk_moe_down(const uint16_t* inter, int inter_planes, int64_t assignments, int64_t inter_dim,
                  const uint8_t* down, const uint8_t* down_scale, int64_t local_experts,
                  int64_t hidden, const int32_t* sorted, const int32_t* units,
                  const int32_t* n_units, int64_t max_units, float* y, void* stream) {
  if (!inter || !down || !down_scale || !sorted || !units || !n_units || !y) return MTPK_EINVAL;
  if (hidden <= 0 || hidden % 32 || inter_dim <= 0 || inter_dim % 32 || local_experts <= 0)
    return MTPK_EINVAL;
  if (!aligned16(inter) || !aligned16(down)) return MTPK_EINVAL;
  if (max_units <= 0 || max_units > INT32_MAX / hidden) return MTPK_EINVAL;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t ip = assignments * inter_dim;
  if (inter_planes == 2)
    return launch_down<2>(inter, ip, (int)inter_dim, down, down_scale, (int)hidden, sorted, units,
                          n_units, (int)max_units, y, st);
  if (inter_planes == 3)
    return launch_down<3>(inter, ip, (int)inter_dim, down, down_scale, (int)hidden, sorted, units,
                          n_units, (int)max_units, y, st);
  return MTPK_EINVAL;
}

int mtpk_moe_combine(const float* y, const void* a_expert, int expert_dtype, const void* a_weight,
                     int weight_dtype, int64_t tokens, int top_k, int64_t hidden, int expert_lo,
                     int expert_hi, void* out, int out_dtype, void* stream) {
  if (!y || !a_expert || !a_weight || !out) return MTPK_EINVAL;
  if (!dtype_index_ok(expert_dtype) || !dtype_float_ok(weight_dtype) || !dtype_float_ok(out_dtype))
    return MTPK_EINVAL;
  if (tokens < 0 || tokens > 65535 || hidden <= 0 || top_k <= 0) return MTPK_EINVAL;
  if (tokens == 0) return 0;
  const dim3 grid((unsigned)((hidden + 255) / 256), (unsigned)tokens);
  hipLaunchKernelGGL(k_moe_combine, grid, dim3(256), 0, (hipStream_t)stream, y, a_expert,
                     expert_dtype, a_weight, weight_dtype, top_k, (int)hidden, expert_lo,
                     expert_hi, out, out_dtype);
  return status_of(hipGetLastError());
}

int mtpk_split_planes(const float* src, int64_t n, int nplanes, uint16_t* planes, void* stream) {
  if (!src || !planes || n < 0 || (nplanes != 2 && nplanes != 3)) return MTPK_EINVAL;
  if (n == 0) return 0;
  const int64_t blocks = (n + 255) / 256;
  const int grid = (int)(blocks < 4096 ? blocks : 4096);
  hipLaunchKernelGGL(k_split_planes, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, n,
                     nplanes, planes);
  return status_of(hipGetLastError());
}

int mtpk_fused_moe(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                   const uint8_t* gate_up, const uint8_t* gate_up_scale, const uint8_t* down,
                   const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                   const void* a_expert, int expert_dtype, const void* a_weight, int weight_dtype,
                   int top_k, int expert_lo, int expert_hi, void* workspace,
                   int64_t workspace_bytes, void* out, void* stream) {
  if (!x || !out || !workspace || !dtype_float_ok(x_dtype)) return MTPK_EINVAL;
  if (tokens < 0 || top_k <= 0 || top_k > MTPK_MAX_TOP_K) return MTPK_EINVAL;
  if ((int64_t)expert_hi - expert_lo != local_experts) return MTPK_EINVAL;
  if (workspace_bytes <
      mtpk_moe_workspace_bytes(tokens, top_k, local_experts, inter_dim, hidden, x_dtype))
    return MTPK_EINVAL;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return MTPK_EINVAL;
  if (tokens == 0) return 0;
  const int64_t a = tokens * top_k;
  const int64_t mu = mtpk_moe_max_units(a, local_experts);
  char* p = static_cast<char*>(workspace);
  int32_t* sorted = reinterpret_cast<int32_t*>(p);
  p += align256(a * 4);
  int32_t* units = reinterpret_cast<int32_t*>(p);
  p += align256(3 * mu * 4);
  int32_t* n_units = reinterpret_cast<int32_t*>(p);
  p += 256;
  const uint16_t* xplanes = static_cast<const uint16_t*>(x);
  int xp = 1, ip = 2;
  int rc;
  if (x_dtype == MTPK_F32) {
    uint16_t* planes = reinterpret_cast<uint16_t*>(p);
    p += align256(3 * tokens * hidden * 2);
    rc = mtpk_split_planes(static_cast<const float*>(x), tokens * hidden, 3, planes, stream);
    if (rc) return rc;
    xplanes = planes;
    xp = 3;
    ip = 3;
  }
  uint16_t* inter = reinterpret_cast<uint16_t*>(p);
  p += align256((int64_t)ip * a * inter_dim * 2);
  float* y = reinterpret_cast<float*>(p);
  rc = mtpk_moe_prep(a_expert, expert_dtype, a_weight, weight_dtype, a, expert_lo, expert_hi,
                     sorted, units, mu, n_units, stream);
  if (rc) return rc;
  rc = mtpk_moe_gate_up(xplanes, xp, tokens, hidden, gate_up, gate_up_scale, local_experts,
                        inter_dim, sorted, units, n_units, mu, top_k, inter, ip, a, stream);
  if (rc) return rc;
  rc = mtpk_moe_down(inter, ip, a, inter_dim, down, down_scale, local_experts, hidden, sorted,
                     units, n_units, mu, y, stream);
  if (rc) return rc;
  return mtpk_moe_combine(y, a_expert, expert_dtype, a_weight, weight_dtype, tokens, top_k,
                          hidden, expert_lo, expert_hi, out, x_dtype, stream);
}

int mtpk_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale, int64_t rows, int64_t k,
                       int mode, float* out, void* stream) {
  if (!packed || !scale || !out || rows < 0 || k <= 0 || k % 32 || (mode != 0 && mode != 1))
    return MTPK_EINVAL;
  if (k > (1 << 24)) return MTPK_EINVAL;
  const int64_t total = rows * (k / 2);
  if (total == 0) return 0;
  const int64_t blocks = (total + 255) / 256;
  const int grid = (int)(blocks < 16384 ? blocks : 16384);
  hipLaunchKernelGGL(k_dequant, dim3(grid), dim3(256), 0, (hipStream_t)stream, packed, scale,
                     rows, (int)k, mode, out);
  return status_of(hipGetLastError());
}

int mtpk_probe_mfma_16x16x32(const uint16_t* a_lanes, const uint16_t* b_lanes, float* d_lanes,
                             void* stream) {
  if (!a_lanes || !b_lanes || !d_lanes) return MTPK_EINVAL;
  if (!aligned16(a_lanes) || !aligned16(b_lanes)) return MTPK_EINVAL;
  hipLaunchKernelGGL(k_probe_mfma, dim3(1), dim3(64), 0, (hipStream_t)stream, a_lanes, b_lanes,
                     d_lanes);
  return status_of(hipGetLastError());
}

}  // extern "C"
