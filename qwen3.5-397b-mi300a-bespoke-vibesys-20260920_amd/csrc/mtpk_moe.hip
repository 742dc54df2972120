// Routed MXFP4 MoE for gfx950: work-list prep, gate_up + SiLU, down, fixed-order combine.
//
// Two pipelines, chosen by batch size (launch shapes depend only on tokens and top_k; no host
// sync), all on the caller's stream:
//   unit path (tokens > 4): prep -> gate_up -> down -> combine
//     prep      routing -> expert-grouped `sorted` + work units (expert, first, count <= 16)
//     gate_up   per (unit, 16 intermediate rows): MXFP4 decoded in registers by the hardware
//               fp4 converter, bf16 MFMA with the unit's activation rows; SiLU(gate) * up stored
//               as bf16 hi/lo planes (16 significant bits)
//     down      per (unit, 64 hidden rows): same decode, MFMA over both planes; fp32 y
//     combine   per token: sum of weight * y over its top_k assignments in j order
//   direct path (tokens <= 4): gate_up with one unit per assignment (no prep), then a
//     per-token down that also combines (no y, no combine launch)
// Each wave keeps a ring of trips (weight + activation loads) in flight ahead of the MFMAs.
// The weight stream is the only HBM-sized traffic; nothing dequantised is ever stored.
// Lane mapping and K coverage of one MFMA tile: see mtpk_common.h ("MoE lane mapping").

#include <mutex>

#include "mtpk_device.h"
#include "mtpk_gemm_tile.h"
#include "mtpk_host.h"
#include "mtpk_layer.h"

namespace mtpk {

constexpr int kUnitTokens = MTPK_MOE_UNIT_TOKENS;
constexpr int kMoeWaves = 4;
constexpr int kMoeThreads = kMoeWaves * kWave;
constexpr int kPrepThreads = 1024;

// ---------------------------------------------------------------- prep

// The prep's LDS: per-expert counts (then claim cursors) and the per-wave scan totals.
template <int NT>
struct PrepSmem {
  static constexpr int kTot = MTPK_MAX_EXPERTS * 4;
  static constexpr int kBytes = kTot + 2 * (NT / kWave) * 4;
};

// The counting sort on one workgroup of NT threads. The live test of a thread's first
// kPrepKeep assignments is kept in registers from the counting pass for the placing pass, which
// then reloads the routing only past them.
constexpr int kPrepKeep = 4;

template <int NT>
__device__ inline void prep_body(const void* __restrict__ a_expert, int edt,
                                 const void* __restrict__ a_weight, int wdt, int assignments,
                                 int lo, int n_experts, int32_t* __restrict__ sorted,
                                 int32_t* __restrict__ units, int max_units,
                                 int32_t* __restrict__ n_units, uint8_t* smem) {
  constexpr int kPrepThreads = NT;
  int* cnt = reinterpret_cast<int*>(smem);
  int* wtot_c = reinterpret_cast<int*>(smem + PrepSmem<NT>::kTot);
  int* wtot_u = wtot_c + NT / kWave;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;

  int keep[kPrepKeep];  // local expert of assignment tid + i * NT, or -1 when it is dead
#pragma unroll
  for (int i = 0; i < kPrepKeep; ++i) {
    const int a = tid + i * kPrepThreads;
    keep[i] = -1;
    if (a < assignments) {
      const int64_t ex = load_index(a_expert, edt, a) - lo;
      if (ex >= 0 && ex < n_experts && load_float(a_weight, wdt, a) != 0.f) keep[i] = (int)ex;
    }
  }
  for (int e = tid; e < n_experts; e += kPrepThreads) cnt[e] = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPrepKeep; ++i)
    if (keep[i] >= 0) atomicAdd(&cnt[keep[i]], 1);
  for (int a = tid + kPrepKeep * kPrepThreads; a < assignments; a += kPrepThreads) {
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
#pragma unroll
  for (int i = 0; i < kPrepKeep; ++i)
    if (keep[i] >= 0) sorted[atomicAdd(&cnt[keep[i]], 1)] = tid + i * kPrepThreads;
  for (int a = tid + kPrepKeep * kPrepThreads; a < assignments; a += kPrepThreads) {
    const int64_t ex = load_index(a_expert, edt, a) - lo;
    if (ex >= 0 && ex < n_experts && load_float(a_weight, wdt, a) != 0.f)
      sorted[atomicAdd(&cnt[ex], 1)] = a;
  }
}

__global__ __launch_bounds__(kPrepThreads) void k_moe_prep(
    const void* __restrict__ a_expert, int edt, const void* __restrict__ a_weight, int wdt,
    int assignments, int lo, int n_experts, int32_t* __restrict__ sorted,
    int32_t* __restrict__ units, int max_units, int32_t* __restrict__ n_units) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[PrepSmem<kPrepThreads>::kBytes];
  prep_body<kPrepThreads>(a_expert, edt, a_weight, wdt, assignments, lo, n_experts, sorted, units,
                          max_units, n_units, smem);
}

// ---------------------------------------------------------------- work units
//
// Unit mode: units come from the prep kernel's list (expert, first position in `sorted`,
// count <= 16). Direct mode (small batches): every assignment is its own unit, read straight from
// the routing with the live test applied in place, so no prep launch is needed.

struct UnitSrc {
  const int32_t* units;
  const int32_t* sorted;
  const int32_t* n_units;
  int max_units;
  const void* a_expert;
  const void* a_weight;
  int edt, wdt, lo, n_experts, assignments, direct;
};

__device__ inline int unit_count(const UnitSrc& s) {
  return s.direct ? s.assignments : min(*s.n_units, s.max_units);
}

__device__ inline void unit_get(const UnitSrc& s, int u, int& e, int& first, int& cnt) {
  if (s.direct) {
    const int64_t ex = load_index(s.a_expert, s.edt, u) - s.lo;
    const bool live = ex >= 0 && ex < s.n_experts && load_float(s.a_weight, s.wdt, u) != 0.f;
    e = live ? (int)ex : 0;
    first = u;
    cnt = live ? 1 : 0;
  } else {
    e = s.units[3 * u];
    first = s.units[3 * u + 1];
    cnt = s.units[3 * u + 2];
  }
}

__device__ inline int unit_member(const UnitSrc& s, int pos) { return s.direct ? pos : s.sorted[pos]; }

// SiLU(gate) * up, stored as OP bf16 planes (hi, lo) or (hi, mid, lo) whose sum is the value.
template <int OP>
__device__ inline void store_planes(uint16_t* dst, int64_t plane, float v) {
  if (OP == 2) {
    uint16_t hi, lo;
    split_bf16(v, &hi, &lo);
    dst[0] = hi;
    dst[plane] = lo;
  } else {
    uint16_t hi, mid, lo;
    split3_bf16(v, &hi, &mid, &lo);
    dst[0] = hi;
    dst[plane] = mid;
    dst[2 * plane] = lo;
  }
}

// ---------------------------------------------------------------- gate_up + SiLU
//
// Item = (unit, 16 intermediate rows n): the gate rows n and the matching up rows I + n share
// every activation load, so SiLU(gate) * up is formed in registers. Each wave streams its trips
// (a trip = one 32-element scale block per lane group, i.e. 128 K of 16 rows: one 16-byte load
// per lane per projection) through a ring of D trips in flight: the loads of trip i + D are
// issued right after trip i is consumed, so every wave keeps D trips outstanding.
// SPLIT = 4: the workgroup's 4 waves share one item, each taking a contiguous quarter of the K
// trips, and reduce their partial tiles in LDS (small batches: 4x the waves in flight).
// SPLIT = 1: every wave owns whole items (wide batches). XP = bf16 planes of x; OP = planes of
// the stored intermediate. SV: the scales of D trips arrive in one 4D-byte load per row
// (rows whose scale bytes are a multiple of 16), else one byte load per trip.

template <int XP>
struct GuTrip {
  u32x4_t wg, wu;
  uint32_t sg, su;
  u32x4_t xv[XP][4];
};

template <int XP, int OP, int SPLIT, int D, bool SV>
__global__ __launch_bounds__(kMoeThreads) void k_moe_gate_up(
    const uint16_t* __restrict__ x, int64_t x_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int I, UnitSrc src, int top_k, uint16_t* __restrict__ inter,
    int64_t inter_plane) {
  __shared__ f32x4_t red[SPLIT > 1 ? SPLIT - 1 : 1][2][kWave];
  const int ntile = I >> 4;
  const int n_items = unit_count(src) * ntile;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int T = (ntrip + SPLIT - 1) / SPLIT;
  const int tbase = SPLIT > 1 ? wave * T : 0;
  const int64_t row_bytes = K >> 1;
  const int item0 = SPLIT > 1 ? (int)blockIdx.x : (int)blockIdx.x * kMoeWaves + wave;
  const int istep = SPLIT > 1 ? (int)gridDim.x : (int)gridDim.x * kMoeWaves;
  const rsrc_t rx = make_rsrc(x, (uint32_t)(XP * x_plane * 2));
  const uint32_t exp_bytes = (uint32_t)(2 * I) * (uint32_t)row_bytes;

  for (int item = item0; item < n_items; item += istep) {
    const int u = item / ntile, nt = item - u * ntile;
    int e, first, cnt;
    unit_get(src, u, e, first, cnt);
    if (cnt == 0) continue;  // uniform over the item's waves
    const bool alive = ln.c < cnt;
    const int tok = unit_member(src, first + (alive ? ln.c : 0)) / top_k;
    const int eu = uniform(e);
    const rsrc_t rw = make_rsrc(wq + (int64_t)eu * exp_bytes, exp_bytes);
    const rsrc_t rs = make_rsrc(ws + (int64_t)eu * (2 * I) * nb, (uint32_t)(2 * I * nb));
    const uint32_t row = (uint32_t)(nt * 16 + ln.c);
    const uint32_t og = row * (uint32_t)row_bytes, ou = og + (uint32_t)I * (uint32_t)row_bytes;
    const uint32_t osg = row * (uint32_t)nb, osu = osg + (uint32_t)(I * nb);
    const uint32_t ox = alive ? (uint32_t)tok * (uint32_t)K * 2u : kOutOfRange;

    // Offsets of valid loads stay below 2^31 (buffers are checked to be smaller), so OR-ing
    // bit 31 into an offset sends that load out of range without a select or a branch.
    auto issue = [&](GuTrip<XP>& r, int i) {
      const int tr = tbase + i;
      const int blk = moe_block(tr, ln.g);
      const uint32_t bad = (uint32_t)!(i < T && tr < ntrip && blk < nb) << 31;
      const uint32_t kb = (uint32_t)blk * 16u;
      r.wg = buf16(rw, (og + kb) | bad);
      r.wu = buf16(rw, (ou + kb) | bad);
      if (!SV) {
        r.sg = buf1(rs, (osg + (uint32_t)blk) | bad);
        r.su = buf1(rs, (osu + (uint32_t)blk) | bad);
      }
#pragma unroll
      for (int p = 0; p < XP; ++p)
#pragma unroll
        for (int h = 0; h < 4; ++h)
          r.xv[p][h] = buf16(rx, (ox + (uint32_t)(p * x_plane + blk * 32 + 8 * h) * 2u) | bad);
    };
    ScaleChunk<D> cg, cu, ng, nu;
    auto issue_chunk = [&](ScaleChunk<D>& a, ScaleChunk<D>& b, int i) {
      const int tr = tbase + i;
      const uint32_t bad = (uint32_t)!(i < T && tr < ntrip) << 31;
      a.load(rs, (osg + 4u * (uint32_t)tr) | bad);
      b.load(rs, (osu + 4u * (uint32_t)tr) | bad);
    };
    f32x4_t accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    auto consume = [&](const GuTrip<XP>& r, int s) {
      const BlockScale fg = block_scale(SV ? cg.byte(s, ln.g) : r.sg);
      const BlockScale fu = block_scale(SV ? cu.byte(s, ln.g) : r.su);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const bf16x8_t bg = decode8(r.wg[h], fg), bu = decode8(r.wu[h], fu);
#pragma unroll
        for (int p = 0; p < XP; ++p) {
          const bf16x8_t av = as_bf16x8(r.xv[p][h]);
          accg = mfma16x16x32(av, bg, accg);
          accu = mfma16x16x32(av, bu, accu);
        }
      }
    };
    GuTrip<XP> ring[D];
    if (SV) issue_chunk(cg, cu, 0);
#pragma unroll
    for (int s = 0; s < D; ++s) {
      issue(ring[s], s);
      ring_fence();
    }
    for (int t = 0; t < T; t += D) {
      if (SV) issue_chunk(ng, nu, t + D);
#pragma unroll
      for (int s = 0; s < D; ++s) {
        consume(ring[s], s);
        issue(ring[s], t + s + D);
        ring_fence();
      }
      if (SV) {
        cg = ng;
        cu = nu;
      }
    }

    const int n = nt * 16 + ln.c;
    if (SPLIT > 1) {
      if (wave > 0) {
        red[wave - 1][0][lane] = accg;
        red[wave - 1][1][lane] = accu;
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w = 0; w < SPLIT - 1; ++w) {
          accg += red[w][0][lane];
          accu += red[w][1][lane];
        }
      }
    }
    if (SPLIT == 1 || wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = moe_out_slot(ln.g, i);
        if (m < cnt) {
          const int64_t a = unit_member(src, first + m);
          const float gt = accg[i];
          store_planes<OP>(inter + a * I + n, inter_plane, gt / (1.f + __expf(-gt)) * accu[i]);
        }
      }
    }
    if (SPLIT > 1) __syncthreads();
  }
}

// ---------------------------------------------------------------- down (unit mode)
//
// Wave item = (unit, R tiles of 16 hidden rows) over the whole K (= intermediate) loop: the
// unit's activation operand (IP planes of the intermediate) is loaded once per trip and reused
// by the R row tiles, and the trips stream through a ring of D in flight. y f32 per assignment.

template <int IP, int R>
struct DnTrip {
  u32x4_t w[R];
  uint32_t s[R];
  u32x4_t av[IP][4];
};

template <int IP, int R, int D, bool SV>
__global__ __launch_bounds__(kMoeThreads) void k_moe_down(
    const uint16_t* __restrict__ inter, int64_t inter_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int H, UnitSrc src, float* __restrict__ y) {
  const int rtiles = H >> 4;
  const int ntile = (rtiles + R - 1) / R;
  const int n_items = unit_count(src) * ntile;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int64_t row_bytes = K >> 1;
  const rsrc_t ra = make_rsrc(inter, (uint32_t)(IP * inter_plane * 2));
  const uint32_t exp_bytes = (uint32_t)H * (uint32_t)row_bytes;

  for (int item = blockIdx.x * kMoeWaves + wave; item < n_items; item += gridDim.x * kMoeWaves) {
    const int u = item / ntile, nt = item - u * ntile;
    int e, first, cnt;
    unit_get(src, u, e, first, cnt);
    if (cnt == 0) continue;
    const bool alive = ln.c < cnt;
    const uint32_t oa =
        alive ? (uint32_t)unit_member(src, first + ln.c) * (uint32_t)K * 2u : kOutOfRange;
    const int eu = uniform(e);
    const rsrc_t rw = make_rsrc(wq + (int64_t)eu * exp_bytes, exp_bytes);
    const rsrc_t rs = make_rsrc(ws + (int64_t)eu * H * nb, (uint32_t)(H * nb));
    // Tiles past the last row tile (only when H/16 is not a multiple of R) recompute the last
    // tile and are not stored, which keeps the loads free of a per-tile condition.
    uint32_t ow[R], os[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rt = min(nt * R + r, rtiles - 1);
      const uint32_t row = (uint32_t)(rt * 16 + ln.c);
      ow[r] = row * (uint32_t)row_bytes;
      os[r] = row * (uint32_t)nb;
    }
    auto issue = [&](DnTrip<IP, R>& t, int tr) {
      const int blk = moe_block(tr, ln.g);
      const uint32_t bad = (uint32_t)!(tr < ntrip && blk < nb) << 31;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        t.w[r] = buf16(rw, (ow[r] + (uint32_t)blk * 16u) | bad);
        if (!SV) t.s[r] = buf1(rs, (os[r] + (uint32_t)blk) | bad);
      }
#pragma unroll
      for (int p = 0; p < IP; ++p)
#pragma unroll
        for (int h = 0; h < 4; ++h)
          t.av[p][h] = buf16(ra, (oa + (uint32_t)(p * inter_plane + blk * 32 + 8 * h) * 2u) | bad);
    };
    ScaleChunk<D> cs[R], ns[R];
    auto issue_chunk = [&](ScaleChunk<D>* c, int tr) {
      const uint32_t bad = (uint32_t)!(tr < ntrip) << 31;
#pragma unroll
      for (int r = 0; r < R; ++r) c[r].load(rs, (os[r] + 4u * (uint32_t)tr) | bad);
    };
    f32x4_t acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](const DnTrip<IP, R>& t, int s) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const BlockScale fs = block_scale(SV ? cs[r].byte(s, ln.g) : t.s[r]);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const bf16x8_t b = decode8(t.w[r][h], fs);
#pragma unroll
          for (int p = 0; p < IP; ++p) acc[r] = mfma16x16x32(as_bf16x8(t.av[p][h]), b, acc[r]);
        }
      }
    };
    DnTrip<IP, R> ring[D];
    if (SV) issue_chunk(cs, 0);
#pragma unroll
    for (int s = 0; s < D; ++s) {
      issue(ring[s], s);
      ring_fence();
    }
    for (int t = 0; t < ntrip; t += D) {
      if (SV) issue_chunk(ns, t + D);
#pragma unroll
      for (int s = 0; s < D; ++s) {
        consume(ring[s], s);
        issue(ring[s], t + s + D);
        ring_fence();
      }
      if (SV)
#pragma unroll
        for (int r = 0; r < R; ++r) cs[r] = ns[r];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (nt * R + r >= rtiles) continue;
      const int n = (nt * R + r) * 16 + ln.c;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = moe_out_slot(ln.g, i);
        if (m < cnt) y[(int64_t)unit_member(src, first + m) * H + n] = acc[r][i];
      }
    }
  }
}

// ---------------------------------------------------------------- down + combine (direct mode)
//
// Small batches: workgroup item = (token t, 16 hidden rows). Wave w takes the token's
// assignments j = w, w+4, ...; for each live one it streams that expert's 16 rows (one token
// column, so the A operand is lane c == 0) and adds weight_j * (down_e . inter_a); the four
// waves' partial rows are summed in LDS in wave order and written as the token's output. No y
// round trip and no separate combine launch; the result does not depend on scheduling.

template <int IP, int D, bool SV>
__global__ __launch_bounds__(kMoeThreads) void k_moe_down_token(
    const uint16_t* __restrict__ inter, int64_t inter_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int H, const void* __restrict__ a_expert, int edt,
    const void* __restrict__ a_weight, int wdt, int lo, int n_experts, int tokens, int top_k,
    void* __restrict__ out, int odt) {
  __shared__ float red[kMoeWaves][16];
  const int rtiles = H >> 4;
  const int n_items = tokens * rtiles;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int64_t row_bytes = K >> 1;
  const rsrc_t ra = make_rsrc(inter, (uint32_t)(IP * inter_plane * 2));
  const uint32_t exp_bytes = (uint32_t)H * (uint32_t)row_bytes;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int t = item / rtiles, rt = item - t * rtiles;
    float tot = 0.f;
    for (int j = wave; j < top_k; j += kMoeWaves) {
      const int64_t a = (int64_t)t * top_k + j;
      const int64_t ex = load_index(a_expert, edt, a) - lo;
      const float wj = load_float(a_weight, wdt, a);
      if (!(ex >= 0 && ex < n_experts && wj != 0.f)) continue;  // uniform per wave
      const int eu = uniform((int)ex);
      const rsrc_t rw = make_rsrc(wq + (int64_t)eu * exp_bytes, exp_bytes);
      const rsrc_t rs = make_rsrc(ws + (int64_t)eu * H * nb, (uint32_t)(H * nb));
      const uint32_t row = (uint32_t)(rt * 16 + ln.c);
      const uint32_t ow = row * (uint32_t)row_bytes, os = row * (uint32_t)nb;
      const uint32_t oa = ln.c == 0 ? (uint32_t)a * (uint32_t)K * 2u : kOutOfRange;
      auto issue = [&](DnTrip<IP, 1>& r, int tr) {
        const int blk = moe_block(tr, ln.g);
        const uint32_t bad = (uint32_t)!(tr < ntrip && blk < nb) << 31;
        r.w[0] = buf16(rw, (ow + (uint32_t)blk * 16u) | bad);
        if (!SV) r.s[0] = buf1(rs, (os + (uint32_t)blk) | bad);
#pragma unroll
        for (int p = 0; p < IP; ++p)
#pragma unroll
          for (int h = 0; h < 4; ++h)
            r.av[p][h] = buf16(ra, (oa + (uint32_t)(p * inter_plane + blk * 32 + 8 * h) * 2u) | bad);
      };
      ScaleChunk<D> cs, ns;
      auto issue_chunk = [&](ScaleChunk<D>& c, int tr) {
        c.load(rs, (os + 4u * (uint32_t)tr) | ((uint32_t)!(tr < ntrip) << 31));
      };
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      auto consume = [&](const DnTrip<IP, 1>& r, int s) {
        const BlockScale fs = block_scale(SV ? cs.byte(s, ln.g) : r.s[0]);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const bf16x8_t b = decode8(r.w[0][h], fs);
#pragma unroll
          for (int p = 0; p < IP; ++p) acc = mfma16x16x32(as_bf16x8(r.av[p][h]), b, acc);
        }
      };
      DnTrip<IP, 1> ring[D];
      if (SV) issue_chunk(cs, 0);
#pragma unroll
      for (int s = 0; s < D; ++s) {
        issue(ring[s], s);
        ring_fence();
      }
      for (int tr = 0; tr < ntrip; tr += D) {
        if (SV) issue_chunk(ns, tr + D);
#pragma unroll
        for (int s = 0; s < D; ++s) {
          consume(ring[s], s);
          issue(ring[s], tr + s + D);
          ring_fence();
        }
        if (SV) cs = ns;
      }
      tot += wj * acc[0];  // lanes 0..15 hold row m = 0 (the token) of column n = c
    }
    if (lane < 16) red[wave][lane] = tot;
    __syncthreads();
    if (wave == 0 && lane < 16) {
      float v = red[0][lane];
#pragma unroll
      for (int w = 1; w < kMoeWaves; ++w) v += red[w][lane];
      store_float(out, odt, (int64_t)t * H + rt * 16 + lane, v);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- shared expert term

// The shared expert's term of a MoE layer, out = routed + sigmoid(gate) * shared, with the
// torch chain's rounding points (`Model.moe`, model.py:2871-2872): the routed sum, the sigmoid
// and the product are each rounded to the output dtype before the final add, so the fused
// layer gives the same values as the three separate elementwise ops.
struct SharedTerm {
  const void* shared;  // [T, H] of dtype sdt, or null
  int sdt;
  const void* gate;  // pre-sigmoid logit of token t at gate[t * gate_stride]
  int gdt;
  int64_t gate_stride;
  // or, when set, the shared expert's down projection as the split-K GEMM leaves it: ks fp32
  // planes of [T, H] (`plane` = T * H apart), summed in split order and rounded to the output
  // dtype, which are the values the GEMM's own reduction would store
  const float* part;
  int ks;
  int64_t plane;
};

__device__ inline bool shared_active(const SharedTerm& st) { return st.shared || st.part; }

__device__ inline float round_to(int dt, float v) {
  return dt == MTPK_BF16 ? bf16_to_f32(f32_to_bf16(v)) : v;
}

__device__ inline float shared_gate(const SharedTerm& st, int t, int odt) {
  const float g = load_float(st.gate, st.gdt, (int64_t)t * st.gate_stride);
  return round_to(odt, 1.f / (1.f + expf(-g)));
}

__device__ inline float shared_value(const SharedTerm& st, int64_t i, int odt) {
  if (!st.part) return load_float(st.shared, st.sdt, i);
  // the planes loaded together, then summed in split order
  constexpr int kPlanes = 8;
  float v = 0.f;
  for (int k0 = 0; k0 < st.ks; k0 += kPlanes) {
    float p[kPlanes];
#pragma unroll
    for (int k = 0; k < kPlanes; ++k) p[k] = k0 + k < st.ks ? st.part[(k0 + k) * st.plane + i] : 0.f;
#pragma unroll
    for (int k = 0; k < kPlanes; ++k)
      if (k0 + k < st.ks) v += p[k];
  }
  return round_to(odt, v);
}

__device__ inline float add_shared(const SharedTerm& st, float gs, float routed, int64_t i, int odt) {
  const float prod = round_to(odt, gs * shared_value(st, i, odt));
  return round_to(odt, routed) + prod;
}

// ---------------------------------------------------------------- single-token units (direct mode)
//
// In direct mode every unit is one assignment, i.e. one token column of the MFMA tile. The
// activation row is then staged once in LDS (lanes c >= 1 read a zero row) instead of being
// loaded per trip, so a trip is only the weight loads and a wave keeps its whole K range in
// flight at once (one memory latency per item instead of one per ring turn).

constexpr int kSingleTrips = 8;    // trips a wave keeps in flight (its whole K range)
constexpr int kSingleQuarter = kSingleTrips * 128;  // K elements per wave in gate_up

// The e8m0 scales of 8 consecutive trips of one weight row: 32 bytes, two 16-byte loads.
struct ScaleRow8 {
  u32x4_t lo, hi;
  __device__ inline void load(rsrc_t r, uint32_t off, uint32_t bad) {
    lo = buf16(r, off | bad);
    hi = buf16(r, (off + 16u) | bad);
  }
  __device__ inline uint32_t byte(int s, int g) const {
    const uint32_t d = s < 4 ? lo[s & 3] : hi[s & 3];
    return (d >> (8 * g)) & 0xffu;
  }
};

// gate_up, one token per unit: item = (assignment, 16 intermediate rows); wave w takes trips
// [8w, 8w + 8) (K <= 4096), stages that quarter of the token's XP activation planes in its own
// LDS region, issues all 8 trips of gate and up weights, then reduces the four partial tiles
// in LDS in wave order.
// LDS of the single-token gate_up: each wave's activation quarter (XP planes), a zero row for
// the A lanes c >= 1, and the partial tiles of waves 1..3 for the reduction.
template <int XP>
struct SingleSmem {
  static constexpr int kPlaneBytes = kSingleQuarter * 2;  // 2 KB
  static constexpr int kZero = kMoeWaves * XP * kPlaneBytes;
  static constexpr int kRed = kZero + kPlaneBytes;
  static constexpr int kBytes = kRed + (kMoeWaves - 1) * 2 * kWave * 16;
};

template <int XP, int OP, bool SV>
__device__ inline void gate_up_single_body(
    const uint16_t* __restrict__ x, int64_t x_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int I, const UnitSrc& src, int top_k,
    uint16_t* __restrict__ inter, int64_t inter_plane, uint8_t* smem, int bid, int nblk) {
  constexpr int kPlaneBytes = SingleSmem<XP>::kPlaneBytes;
  typedef uint8_t Planes[XP][kPlaneBytes];
  typedef f32x4_t RedPair[2][kWave];
  Planes* xs = reinterpret_cast<Planes*>(smem);
  uint8_t* zero = smem + SingleSmem<XP>::kZero;  // the A rows of lanes c >= 1
  RedPair* red = reinterpret_cast<RedPair*>(smem + SingleSmem<XP>::kRed);
  const int ntile = I >> 4;
  const int n_items = unit_count(src) * ntile;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int tbase = wave * kSingleTrips;
  const int64_t row_bytes = K >> 1;
  const rsrc_t rx = make_rsrc(x, (uint32_t)(XP * x_plane * 2));
  const uint32_t exp_bytes = (uint32_t)(2 * I) * (uint32_t)row_bytes;
  if (tid < kPlaneBytes / 16) reinterpret_cast<u32x4_t*>(zero)[tid] = zero16();
  __syncthreads();

  for (int item = bid; item < n_items; item += nblk) {
    const int u = item / ntile, nt = item - u * ntile;
    int e, first, cnt;
    unit_get(src, u, e, first, cnt);
    if (cnt == 0) continue;  // uniform over the workgroup
    const int tok = unit_member(src, first) / top_k;
    const int eu = uniform(e);
    const rsrc_t rw = make_rsrc(wq + (int64_t)eu * exp_bytes, exp_bytes);
    const rsrc_t rs = make_rsrc(ws + (int64_t)eu * (2 * I) * nb, (uint32_t)(2 * I * nb));
    const uint32_t row = (uint32_t)(nt * 16 + ln.c);
    const uint32_t og = row * (uint32_t)row_bytes, ou = og + (uint32_t)I * (uint32_t)row_bytes;
    const uint32_t osg = row * (uint32_t)nb, osu = osg + (uint32_t)(I * nb);

    // this wave's activation quarter: 16 bytes per lane per load, two loads per plane
    u32x4_t sreg[XP][2];
#pragma unroll
    for (int p = 0; p < XP; ++p)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int kel = tbase * 128 + (k * kWave + lane) * 8;
        const uint32_t bad = (uint32_t)!(kel < K) << 31;
        sreg[p][k] = buf16(rx, ((uint32_t)(p * x_plane + (int64_t)tok * K + kel) * 2u) | bad);
      }
    ScaleRow8 cg, cu;  // SV: the quarter's 32 scale bytes per row (nb a multiple of 32)
    const uint32_t sbad = (uint32_t)!(SV && tbase < ntrip) << 31;
    cg.load(rs, osg + 4u * (uint32_t)tbase, sbad);
    cu.load(rs, osu + 4u * (uint32_t)tbase, sbad);
    u32x4_t wg[kSingleTrips], wu[kSingleTrips];
#pragma unroll
    for (int i = 0; i < kSingleTrips; ++i) {
      const int tr = tbase + i;
      const int blk = moe_block(tr, ln.g);
      const uint32_t bad = (uint32_t)!(tr < ntrip && blk < nb) << 31;
      wg[i] = buf16(rw, (og + (uint32_t)blk * 16u) | bad);
      wu[i] = buf16(rw, (ou + (uint32_t)blk * 16u) | bad);
    }
    ring_fence();
#pragma unroll
    for (int p = 0; p < XP; ++p)
#pragma unroll
      for (int k = 0; k < 2; ++k)
        *reinterpret_cast<u32x4_t*>(&xs[wave][p][(k * kWave + lane) * 16]) = sreg[p][k];
    ring_fence();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes are visible to itself
    // lane (g, c): A values of trip i, slot h at base + 256 i + 16 h (c == 0: the token row)
    const uint8_t* abase[XP];
#pragma unroll
    for (int p = 0; p < XP; ++p) abase[p] = (ln.c == 0 ? &xs[wave][p][0] : zero) + ln.g * 64;
    f32x4_t accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kSingleTrips; ++i) {
      const int tr = tbase + i, blk = moe_block(tr, ln.g);
      uint32_t sg_, su_;
      if (SV) {
        sg_ = cg.byte(i, ln.g);
        su_ = cu.byte(i, ln.g);
      } else {
        const uint32_t bad = (uint32_t)!(tr < ntrip && blk < nb) << 31;
        sg_ = buf1(rs, (osg + (uint32_t)blk) | bad);
        su_ = buf1(rs, (osu + (uint32_t)blk) | bad);
      }
      const BlockScale fg = block_scale(sg_), fu = block_scale(su_);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const bf16x8_t bg = decode8(wg[i][h], fg), bu = decode8(wu[i][h], fu);
#pragma unroll
        for (int p = 0; p < XP; ++p) {
          const bf16x8_t av = as_bf16x8(*reinterpret_cast<const u32x4_t*>(abase[p] + 256 * i + 16 * h));
          accg = mfma16x16x32(av, bg, accg);
          accu = mfma16x16x32(av, bu, accu);
        }
      }
      ring_fence();  // one trip's LDS reads and decodes at a time
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
      if (ln.g == 0) {  // row m = 0 (the token) of column n = c
        const float gt = accg[0];
        store_planes<OP>(inter + (int64_t)unit_member(src, first) * I + nt * 16 + ln.c, inter_plane,
                         gt / (1.f + __expf(-gt)) * accu[0]);
      }
    }
    __syncthreads();
  }
}

template <int XP, int OP, bool SV>
__global__ __launch_bounds__(kMoeThreads) void k_moe_gate_up_single(
    const uint16_t* __restrict__ x, int64_t x_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int I, UnitSrc src, int top_k, uint16_t* __restrict__ inter,
    int64_t inter_plane) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[SingleSmem<XP>::kBytes];
  gate_up_single_body<XP, OP, SV>(x, x_plane, K, wq, ws, I, src, top_k, inter, inter_plane, smem,
                                  blockIdx.x, gridDim.x);
}

// down + combine, one token per unit: workgroup item = (token t, 16 hidden rows), 16 waves;
// wave w streams assignment t * top_k + j for j = w, w + 16, ... over its whole K (<= 1024:
// all 8 trips in flight), its intermediate row staged in its own LDS region. The weighted
// partial rows are summed in LDS in wave order.
constexpr int kSingleDownWaves = 16;

template <int IP, bool SV>
__global__ __launch_bounds__(kSingleDownWaves * kWave) void k_moe_down_single(
    const uint16_t* __restrict__ inter, int64_t inter_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int H, const void* __restrict__ a_expert, int edt,
    const void* __restrict__ a_weight, int wdt, int lo, int n_experts, int tokens, int top_k,
    void* __restrict__ out, int odt, SharedTerm sh) {
  constexpr int kPlaneBytes = kSingleQuarter * 2;  // 2 KB: K <= 1024
  __shared__ __attribute__((aligned(16))) uint8_t as_[kSingleDownWaves][IP][kPlaneBytes];
  __shared__ __attribute__((aligned(16))) uint8_t zero[kPlaneBytes];  // the A rows of lanes c >= 1
  __shared__ float red[kSingleDownWaves][16];
  __shared__ float s_prod[16];  // the shared expert's gated rows, made by an idle wave
  const int rtiles = H >> 4;
  const int n_items = tokens * rtiles;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int64_t row_bytes = K >> 1;
  const rsrc_t ra = make_rsrc(inter, (uint32_t)(IP * inter_plane * 2));
  const uint32_t exp_bytes = (uint32_t)H * (uint32_t)row_bytes;
  if (tid < kPlaneBytes / 16) reinterpret_cast<u32x4_t*>(zero)[tid] = zero16();
  __syncthreads();

  // With top_k < kSingleDownWaves the last wave streams no assignment: it fetches the shared
  // expert's term while the others stream, so the epilogue does not wait a memory round trip
  // for it.
  const bool pre_shared = shared_active(sh) && top_k < kSingleDownWaves;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int t = item / rtiles, rt = item - t * rtiles;
    if (pre_shared && wave == kSingleDownWaves - 1 && lane < 16)
      s_prod[lane] = round_to(odt, shared_gate(sh, t, odt) *
                                       shared_value(sh, (int64_t)t * H + rt * 16 + lane, odt));
    float tot = 0.f;
    for (int j = wave; j < top_k; j += kSingleDownWaves) {
      const int64_t a = (int64_t)t * top_k + j;
      const int64_t ex = load_index(a_expert, edt, a) - lo;
      const float wj = load_float(a_weight, wdt, a);
      if (!(ex >= 0 && ex < n_experts && wj != 0.f)) continue;  // uniform per wave
      const int eu = uniform((int)ex);
      const rsrc_t rw = make_rsrc(wq + (int64_t)eu * exp_bytes, exp_bytes);
      const rsrc_t rs = make_rsrc(ws + (int64_t)eu * H * nb, (uint32_t)(H * nb));
      const uint32_t row = (uint32_t)(rt * 16 + ln.c);
      const uint32_t ow = row * (uint32_t)row_bytes, os = row * (uint32_t)nb;
      u32x4_t sreg[IP][2];
#pragma unroll
      for (int p = 0; p < IP; ++p)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int kel = (k * kWave + lane) * 8;
          const uint32_t bad = (uint32_t)!(kel < K) << 31;
          sreg[p][k] = buf16(ra, ((uint32_t)(p * inter_plane + a * K + kel) * 2u) | bad);
        }
      ScaleRow8 cs;  // SV: the row's 32 scale bytes (K = 1024)
      cs.load(rs, os, (uint32_t)!SV << 31);
      u32x4_t w[kSingleTrips];
#pragma unroll
      for (int i = 0; i < kSingleTrips; ++i) {
        const int blk = moe_block(i, ln.g);
        const uint32_t bad = (uint32_t)!(i < ntrip && blk < nb) << 31;
        w[i] = buf16(rw, (ow + (uint32_t)blk * 16u) | bad);
      }
      ring_fence();
#pragma unroll
      for (int p = 0; p < IP; ++p)
#pragma unroll
        for (int k = 0; k < 2; ++k)
          *reinterpret_cast<u32x4_t*>(&as_[wave][p][(k * kWave + lane) * 16]) = sreg[p][k];
      ring_fence();
      __builtin_amdgcn_s_waitcnt(0xC07F);
      const uint8_t* abase[IP];
#pragma unroll
      for (int p = 0; p < IP; ++p) abase[p] = (ln.c == 0 ? &as_[wave][p][0] : zero) + ln.g * 64;
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < kSingleTrips; ++i) {
        const int blk = moe_block(i, ln.g);
        uint32_t sb;
        if (SV) {
          sb = cs.byte(i, ln.g);
        } else {
          const uint32_t bad = (uint32_t)!(i < ntrip && blk < nb) << 31;
          sb = buf1(rs, (os + (uint32_t)blk) | bad);
        }
        const BlockScale fs = block_scale(sb);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const bf16x8_t b = decode8(w[i][h], fs);
#pragma unroll
          for (int p = 0; p < IP; ++p)
            acc = mfma16x16x32(as_bf16x8(*reinterpret_cast<const u32x4_t*>(abase[p] + 256 * i + 16 * h)), b, acc);
        }
        ring_fence();  // one trip's LDS reads and decodes at a time
      }
      tot += wj * acc[0];  // lanes 0..15 hold row m = 0 (the token) of column n = c
    }
    if (lane < 16) red[wave][lane] = tot;
    __syncthreads();
    if (wave == 0 && lane < 16) {
      float v = red[0][lane];
#pragma unroll
      for (int w2 = 1; w2 < kSingleDownWaves; ++w2) v += red[w2][lane];
      const int64_t oi = (int64_t)t * H + rt * 16 + lane;
      if (pre_shared)
        v = round_to(odt, v) + s_prod[lane];  // add_shared's arithmetic, its product made early
      else if (shared_active(sh))
        v = add_shared(sh, shared_gate(sh, t, odt), v, oi, odt);
      store_float(out, odt, oi, v);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- LDS-staged unit kernels
//
// Wide batches: the 4 waves of a workgroup work on one unit, each on its own weight rows, so
// the unit's activation rows are shared. They are staged cooperatively into LDS in K chunks
// (double-buffered, one barrier per chunk) and every wave reads its MFMA A operand from LDS
// (ds_read_b128); only weights and scales go through the per-wave trip ring. This takes the
// activation loads off the vector memory path, where every lane of a wave costs address work
// even when most of the unit's 16 token slots are empty.

// Scalar (constant-cache) reads of the work list (`sload`). An item's unit record and the member
// ids of its staging rows are uniform over a wave, so they are read with scalar loads, outside
// the vector-memory queue the trip ring keeps full: a vector load there would make the item's
// first wait drain the ring. The list was written by an earlier launch and is read-only here.

// Wait for this wave's LDS operations, then workgroup barrier. Vector memory loads (the trip
// ring) stay in flight across it.
__device__ inline void lds_barrier() {
  ring_fence();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only (gfx9 encoding)
  __builtin_amdgcn_s_barrier();
  ring_fence();
}


// Byte g of each of four dwords, packed low to high: one 16-byte scale segment (four trips of
// four lane groups) reduced to the four bytes one lane group uses. sel01 / selc come from
// lane_byte_selectors(g).
__device__ inline uint32_t pick_lane_bytes(u32x4_t d, uint32_t sel01, uint32_t selc) {
  const uint32_t t01 = __builtin_amdgcn_perm(d[1], d[0], sel01);
  const uint32_t t23 = __builtin_amdgcn_perm(d[3], d[2], sel01);
  return __builtin_amdgcn_perm(t23, t01, selc);
}

// v_perm selectors: bytes {g of the low dword, g of the high dword, zero, zero}, then the
// low two bytes of each half.
__device__ inline uint32_t lane_byte_sel01(int g) {
  return (uint32_t)g | ((uint32_t)(4 + g) << 8) | 0x0c0c0000u;
}
constexpr uint32_t kLaneByteSelC = 0x05040100u;

// K elements of the activation rows staged per chunk, and the LDS bytes of one token row
// (NPL planes, padded by 16 bytes so the 16 token rows fall on different banks).
template <int KC, int NPL>
struct StageGeom {
  static constexpr int kPlaneBytes = KC * 2;
  static constexpr int kRow = KC * 2 * NPL + 16;
  static constexpr int kBuf = 16 * kRow;
  static constexpr int kBytesPerThread = 16 * KC * 2 * NPL / kMoeThreads;  // 64
  static_assert(kBytesPerThread == 64, "one staging step is 4 x 16 bytes per thread");
};

// gate_up, LDS variant (bf16 x, hi/lo intermediate, chunked scales). Item = (unit, 4 tiles of
// 16 intermediate rows), wave w takes tile 4q + w. Chunks of 512 K = 4 trips = one ring turn.
template <int D, int NW>
__global__ __launch_bounds__(NW * kWave) void k_moe_gate_up_lds(
    const uint16_t* __restrict__ x, int64_t x_elems, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int I, UnitSrc src, int top_k, uint16_t* __restrict__ inter,
    int64_t inter_plane) {
  constexpr int KC = 512, TPC = KC / 128;
  static_assert(D == TPC, "one ring turn per staged chunk");
  using G = StageGeom<KC, 1>;
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][G::kBuf];
  // with 8 waves the 32 scale rows of each wave no longer fit in the idle chunk buffer
  constexpr int kScaleScratch = NW * 32 * 128 + NW * 16;
  __shared__ __attribute__((aligned(16))) uint8_t sscr[NW == 4 ? 16 : kScaleScratch];
  constexpr int RPW = 16 / NW;  // staged token rows per wave
  const int ntile = I >> 4, ngroup = (ntile + NW - 1) / NW;
  const int n_items = min(sload(src.n_units, 0), src.max_units) * ngroup;
  const int tid = threadIdx.x, wave = uniform(tid / kWave), lane = tid & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = nb >> 2, nchunk = K / KC;
  const int64_t row_bytes = K >> 1;
  const rsrc_t rx = make_rsrc(x, (uint32_t)(x_elems * 2));
  const uint32_t exp_bytes = (uint32_t)(2 * I) * (uint32_t)row_bytes;
  // staging: load k of a chunk moves 16 bytes of token row 4k + wave at byte 16 * lane, so
  // every wave instruction reads one row's whole 1 KB chunk (eight full 128-byte lines)

  // The intermediate rows are held in registers and stored kHold items at a time (all of a
  // workgroup's items at M = 192), not at the end of each item: stores spread through the
  // weight stream cost the HBM read/write turnarounds (gate_up 300 -> 294 us at M = 192 with 12
  // items held, 256 VGPRs; the 4-wave form holds 4, keeping two workgroups per CU at M = 32).
  // Offsets are 32-bit, so a launch whose intermediate plane exceeds that stores at once.
  constexpr int kHold = NW == 8 ? 12 : 4;
  const bool hold = inter_plane <= INT32_MAX;
  uint32_t held_v[kHold][4];  // (hi | lo << 16) bf16 planes of the value
  int32_t held_d[kHold][4];   // its offset in a plane, or -1
  int held = 0;
  auto flush = [&]() {
#pragma unroll
    for (int h = 0; h < kHold; ++h)
      if (h < held)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (held_d[h][i] >= 0) {
            inter[held_d[h][i]] = (uint16_t)(held_v[h][i] & 0xffffu);
            inter[inter_plane + held_d[h][i]] = (uint16_t)(held_v[h][i] >> 16);
          }
    held = 0;
  };
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int u = item / ngroup, q = item - u * ngroup;
    const int e = sload(src.units, 3 * u), first = sload(src.units, 3 * u + 1);
    const int cnt = sload(src.units, 3 * u + 2);
    if (cnt == 0) continue;  // uniform over the workgroup
    // output assignments of this lane's four token slots, read now, used after the K loop
    int32_t om[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) om[i] = src.sorted[first + min(moe_out_slot(ln.g, i), cnt - 1)];
    const int nt_raw = q * NW + wave;
    const bool wave_ok = nt_raw < ntile;
    const int nt = wave_ok ? nt_raw : ntile - 1;
    const int eu = e;
    const rsrc_t rw = make_rsrc(wq + (int64_t)eu * exp_bytes, exp_bytes);
    const rsrc_t rs = make_rsrc(ws + (int64_t)eu * (2 * I) * nb, (uint32_t)(2 * I * nb));
    const uint32_t row = (uint32_t)(nt * 16 + ln.c);
    const uint32_t og = row * (uint32_t)row_bytes, ou = og + (uint32_t)I * (uint32_t)row_bytes;
    const uint32_t osg = row * (uint32_t)nb, osu = osg + (uint32_t)(I * nb);
    uint32_t sx[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int r = NW * k + wave;
      const int tok = sload(src.sorted, first + min(r, cnt - 1)) / top_k;
      sx[k] = r < cnt ? (uint32_t)tok * (uint32_t)K * 2u + (uint32_t)lane * 16u : kOutOfRange;
    }
    u32x4_t sreg[RPW];
    auto stage_load = [&](int c) {
      const uint32_t bad = (uint32_t)!(c < nchunk) << 31;
#pragma unroll
      for (int k = 0; k < RPW; ++k) sreg[k] = buf16(rx, (sx[k] + (uint32_t)c * (KC * 2)) | bad);
    };
    auto stage_store = [&](int b) {
#pragma unroll
      for (int k = 0; k < RPW; ++k) lds16_store(&xs[b][(NW * k + wave) * G::kRow + lane * 16], sreg[k]);
    };

    auto issue = [&](u32x4_t& wg, u32x4_t& wu, int tr) {
      const int blk = moe_block(tr, ln.g);
      const uint32_t bad = (uint32_t)!(tr < ntrip) << 31;
      const uint32_t kb = (uint32_t)blk * 16u;
      wg = buf16(rw, (og + kb) | bad);
      wu = buf16(rw, (ou + kb) | bad);
    };
    // Scales: the wave's 32 scale rows (16 gate rows, then the matching 16 up rows; nb bytes
    // each) come in with full-line loads, pass through this wave's slice of the idle chunk
    // buffer 1, and each lane keeps the bytes of its lane group packed per turn: sdg[T] byte s
    // is the gate scale of trip 4T + s (K <= 4096: at most 8 turns).
    const int segs = nb >> 4, units = 32 * segs;
    u32x4_t sload4[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = k * kWave + lane;
      const int rr = idx / segs, sg = idx - rr * segs;
      const uint32_t grow = rr < 16 ? (uint32_t)(nt * 16 + rr) : (uint32_t)(I + nt * 16 + rr - 16);
      const uint32_t bad = (uint32_t)!(idx < units) << 31;
      sload4[k] = buf16(rs, (grow * (uint32_t)nb + (uint32_t)sg * 16u) | bad);
    }
    ring_fence();
    uint32_t sdg[8], sdu[8];
    f32x4_t accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    uint32_t cur_g = 0u, cur_u = 0u;  // this turn's packed scales (selected per chunk)
    auto consume = [&](const u32x4_t& wg, const u32x4_t& wu, int s, const uint8_t* buf) {
      const BlockScale fg = block_scale(cur_g >> (8 * s));
      const BlockScale fu = block_scale(cur_u >> (8 * s));
      const uint8_t* arow = buf + ln.c * G::kRow + ((4 * s + ln.g) * 32) * 2;
      u32x4_t a[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) a[h] = lds16(arow + 16 * h);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const bf16x8_t bg = decode8(wg[h], fg), bu = decode8(wu[h], fu);
        accg = mfma16x16x32(as_bf16x8(a[h]), bg, accg);
        accu = mfma16x16x32(as_bf16x8(a[h]), bu, accu);
      }
    };

    // prologue: chunk 0 loads first, then the scales and weights of the first D trips, so
    // that waiting for chunk 0 leaves the whole ring in flight; chunk 1 loads behind them
    stage_load(0);
    ring_fence();
    u32x4_t rg[D], ru[D];
#pragma unroll
    for (int s = 0; s < D; ++s) issue(rg[s], ru[s], s);
    ring_fence();
    {
      uint8_t* scr = (NW == 4 ? xs[1] : sscr) + wave * (32 * nb);
      uint8_t* spare = (NW == 4 ? xs[1] : sscr) + NW * 32 * nb + wave * 16;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // lanes past the wave's scale rows store their (zero) load to a spare 16 bytes past the
        // slices instead of branching around the store
        const int idx = k * kWave + lane;
        lds16_store(idx < units ? scr + idx * 16 : spare, sload4[k]);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // the wave reads back only its own slice
      const uint32_t sel01 = lane_byte_sel01(ln.g);
#pragma unroll
      for (int T = 0; T < 8; ++T) {
        if (T < nchunk) {
          sdg[T] = pick_lane_bytes(lds16(scr + ln.c * nb + 16 * T), sel01, kLaneByteSelC);
          sdu[T] = pick_lane_bytes(lds16(scr + (16 + ln.c) * nb + 16 * T), sel01, kLaneByteSelC);
        } else {
          sdg[T] = 0u;
          sdu[T] = 0u;
        }
      }
    }
    stage_store(0);
    stage_load(1);
    lds_barrier();  // also: every wave is done with its scale slice before chunk 1 lands
    // nchunk >= 1 (K is a positive multiple of KC): a bottom-tested loop keeps the ring
    // issue above in the prologue's block instead of letting it sink past the barrier
    int c = 0;
#pragma clang loop unroll(disable)
    do {
      const int t = c * D;
      const uint8_t* buf = xs[c & 1];
      // turn c's scales, by selects on the uniform c (indexing a register array by c would
      // move it to scratch, and rotating it makes every entry loop-carried)
      cur_g = sdg[0];
      cur_u = sdu[0];
#pragma unroll
      for (int T = 1; T < 8; ++T)
        if (c == T) {
          cur_g = sdg[T];
          cur_u = sdu[T];
        }
      // trips are consumed and refilled in pairs: the two refills of a row are adjacent
      // 64-byte segments issued back to back
#pragma unroll
      for (int s = 0; s < D; s += 2) {
        consume(rg[s], ru[s], s, buf);
        consume(rg[s + 1], ru[s + 1], s + 1, buf);
        ring_fence();
        issue(rg[s], ru[s], t + s + D);
        issue(rg[s + 1], ru[s + 1], t + s + 1 + D);
        ring_fence();
      }
      if (c + 1 < nchunk) stage_store((c + 1) & 1);
      stage_load(c + 2);
      lds_barrier();
    } while (++c < nchunk);

    const int n = nt * 16 + ln.c;
    if (!hold) {
      if (wave_ok) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (moe_out_slot(ln.g, i) < cnt) {
            const float gt = accg[i];
            store_planes<2>(inter + (int64_t)om[i] * I + n, inter_plane, gt / (1.f + __expf(-gt)) * accu[i]);
          }
        }
      }
      continue;
    }
    uint32_t pv[4];
    int32_t pd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float gt = accg[i];
      uint16_t hi, lo;
      split_bf16(gt / (1.f + __expf(-gt)) * accu[i], &hi, &lo);  // store_planes<2>'s split
      pv[i] = (uint32_t)hi | ((uint32_t)lo << 16);
      pd[i] = (wave_ok && moe_out_slot(ln.g, i) < cnt) ? om[i] * I + n : -1;
    }
    // into slot `held` by selects on the uniform count (an indexed register array would go to
    // scratch)
#pragma unroll
    for (int h = 0; h < kHold; ++h)
      if (h == held)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          held_v[h][i] = pv[i];
          held_d[h][i] = pd[i];
        }
    if (++held == kHold) flush();
  }
  flush();
}

// down, LDS variant (hi/lo intermediate planes, chunked scales). Item = (unit, 4 x R tiles of
// 16 hidden rows), wave w takes tiles (4q + w) R .. + R. Chunks of 256 K = 2 trips = one turn
// of the D = 2 ring; each chunk stages both planes. Items are software-pipelined: the workgroup
// issues its next grid-stride item's scale rows when an item starts and, while the item runs its
// last two chunks, the next one's first two activation chunks and first D ring trips, so an item
// starts with its loads in flight instead of waiting a full memory latency with the ring drained.
template <int R>
__global__ __launch_bounds__(kMoeThreads) void k_moe_down_lds(
    const uint16_t* __restrict__ inter, int64_t inter_plane, int K, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, int H, UnitSrc src, float* __restrict__ y) {
  constexpr int D = 2, KC = 256;
  constexpr int kScr = R * 16 * 32;  // a wave's scale rows (K <= 1024: at most 32 bytes each)
  using G = StageGeom<KC, 2>;
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][G::kBuf];
  __shared__ __attribute__((aligned(16))) uint8_t sscr[kMoeWaves * kScr];
  const int rtiles = H >> 4;
  const int ngroup = (rtiles + kMoeWaves * R - 1) / (kMoeWaves * R);
  const int n_items = min(sload(src.n_units, 0), src.max_units) * ngroup;
  const int tid = threadIdx.x, wave = uniform(tid / kWave), lane = tid & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int nb = K >> 5, ntrip = nb >> 2, nchunk = K / KC;  // nchunk is even (K % 512 == 0)
  const uint32_t row_bytes = (uint32_t)(K >> 1);
  const rsrc_t ra = make_rsrc(inter, (uint32_t)(2 * inter_plane * 2));
  const uint32_t exp_bytes = (uint32_t)H * row_bytes;
  const int segs = nb >> 4, nscale = R * 16 * segs;  // 16-byte scale pieces of a wave's rows
  // Offsets split into a per-lane part (voffset) and a wave-uniform per-item part (soffset).
  // Weights: lane (g, c) reads row c of each tile. Staging: load k of a chunk moves token row
  // 4k + wave, plane (lane >= 32), 16-byte column lane & 31, so every wave instruction reads
  // two whole 512-byte plane segments (full 128-byte lines).
  const uint32_t vrow = (uint32_t)ln.c * row_bytes;
  const int sp = lane >> 5, scol = lane & 31;
  const uint32_t vst = (uint32_t)sp * (uint32_t)inter_plane * 2u + (uint32_t)scol * 16u;
  uint8_t* const scr = sscr + wave * kScr;
  const uint32_t sel01 = lane_byte_sel01(ln.g);

  // A work item: expert, first sorted assignment, count, this wave's first tile, and the
  // staged token rows' byte offsets (-1: no such row). cnt == 0 marks "no item".
  struct Item {
    int e, first, cnt, tile0;
    int tok[4];
  };
  auto fetch = [&](int it) {
    Item m{0, 0, 0, 0, {-1, -1, -1, -1}};
    if (it < n_items) {
      const int u = it / ngroup, q = it - u * ngroup;
      m.e = sload(src.units, 3 * u);
      m.first = sload(src.units, 3 * u + 1);
      m.cnt = sload(src.units, 3 * u + 2);
      m.tile0 = (q * kMoeWaves + wave) * R;
      if (m.cnt > 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int r = 4 * k + wave;
          const int a = sload(src.sorted, m.first + min(r, m.cnt - 1));
          m.tok[k] = r < m.cnt ? a * K * 2 : -1;
        }
      }
    }
    return m;
  };
  auto tile_off = [&](int tile0, int r) { return (uint32_t)min(tile0 + r, rtiles - 1) * 16u * row_bytes; };
  // one ring slot: tile r (first tile tile0) of trip tr of the expert at `w`; out of range
  // (no memory access) when !live
  auto load_w = [&](const uint8_t* w, int tile0, int r, int tr, bool live) {
    const uint32_t off = (vrow + (uint32_t)moe_block(tr, ln.g) * 16u) | ((uint32_t)!live << 31);
    return buf16(make_rsrc(w, exp_bytes), off, tile_off(tile0, r));
  };
  u32x4_t sreg[4];
  auto stage_load = [&](const Item& m, int c) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = m.tok[k];
      sreg[k] = buf16(ra, vst | ((uint32_t)(t < 0) << 31), (uint32_t)max(t, 0) + (uint32_t)c * (KC * 2));
    }
  };
  auto stage_store = [&](int b) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      lds16_store(&xs[b][(4 * k + wave) * G::kRow + sp * G::kPlaneBytes + scol * 16], sreg[k]);
  };
  // The wave's R * 16 scale rows (nb bytes each) come in with full-line direct-to-LDS loads into
  // the wave's own LDS scratch (piece idx at 16 idx; lanes past the pieces load out of range
  // into the scratch's unread tail), and each lane keeps its lane group's bytes packed per four
  // trips: pd[r][Q] byte s is tile r's trip 4Q + s.
  auto scale_load = [&](const Item& m) {
    const rsrc_t rs = make_rsrc(ws + (int64_t)m.e * H * nb, (uint32_t)(H * nb));
    ring_fence();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = k * kWave + lane;
      const int rr = idx / segs, sg = idx - rr * segs;
      const uint32_t grow = (uint32_t)(min(m.tile0 + rr / 16, rtiles - 1) * 16 + (rr & 15));
      const bool live = m.cnt > 0 && idx < nscale;
      buf16_lds(rs, (grow * (uint32_t)nb + (uint32_t)sg * 16u) | ((uint32_t)!live << 31), scr + k * kWave * 16);
    }
    ring_fence();
  };
  uint32_t pd[R][2];
  auto scale_unpack = [&]() {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int Q = 0; Q < 2; ++Q)
        pd[r][Q] = Q < segs ? pick_lane_bytes(lds16(scr + (r * 16 + ln.c) * nb + 16 * Q), sel01, kLaneByteSelC)
                            : 0u;
  };

  // Prologue of the workgroup's first item; every later item finds the same loads issued by
  // its predecessor's K loop. An item with cnt == 0 (none in a prep work list) only ever
  // issues out-of-range loads and stores nothing.
  u32x4_t ring[D][R];
  Item cur = fetch(blockIdx.x);
  scale_load(cur);
  stage_load(cur, 0);  // chunk 0 before the ring: waiting for it leaves the ring in flight
  ring_fence();
#pragma unroll
  for (int s = 0; s < D; ++s)
#pragma unroll
    for (int r = 0; r < R; ++r)
      ring[s][r] = load_w(wq + (int64_t)cur.e * exp_bytes, cur.tile0, r, s, cur.cnt > 0);
  ring_fence();
  stage_store(0);
  vmcnt_wait<D * R>();  // the scale rows, issued before chunk 0 and the ring
  scale_unpack();
  stage_load(cur, 1);
  lds_barrier();

  // y rows are held in registers and stored kHoldY items at a time, as gate_up holds its
  // intermediate: fewer read/write turnarounds in the weight stream (M = 192 layer 471.5 ->
  // 467 us, M = 32 179 -> 177.8 us), at 232 VGPRs (two workgroups per CU instead of three).
  constexpr int kHoldY = 4;
  float hy[kHoldY][R][4];  // the held items' outputs
  int32_t ho[kHoldY][4];   // their output assignments per token slot, or -1
  int ht[kHoldY];          // their first tiles
  int nhy = 0;
  auto flush_y = [&]() {
#pragma unroll
    for (int h = 0; h < kHoldY; ++h)
      if (h < nhy)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (ht[h] + r >= rtiles) continue;
          const int n = (ht[h] + r) * 16 + ln.c;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (ho[h][i] >= 0) y[(int64_t)ho[h][i] * H + n] = hy[h][r][i];
        }
    nhy = 0;
  };
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const Item nxt = fetch(item + gridDim.x);
    // The scratch is free once this item's scales are unpacked (their LDS reads completed): the
    // next item's scale rows go in now, ahead of every load of this item's K loop.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    scale_load(nxt);
    const bool pf = nxt.cnt > 0, live = cur.cnt > 0;
    const uint8_t* const wc = wq + (int64_t)cur.e * exp_bytes;
    const uint8_t* const wn = wq + (int64_t)nxt.e * exp_bytes;
    int32_t om[4];  // output assignments of this lane's token slots, used after the K loop
#pragma unroll
    for (int i = 0; i < 4; ++i)
      om[i] = live ? src.sorted[cur.first + min(moe_out_slot(ln.g, i), cur.cnt - 1)] : 0;

    f32x4_t acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    uint32_t cs[R];
    int csh = 0;  // bit offset of this chunk's first trip within the packed dword
    // trip s of the chunk, tile by tile; each tile's ring slot is refilled with trip tr (of the
    // next item once tr runs past this one's) as soon as its MFMAs are issued
    auto consume = [&](int s, const uint8_t* buf, int tr) {
      const uint8_t* arow = buf + ln.c * G::kRow + ((4 * s + ln.g) * 32) * 2;
      u32x4_t a[2][4];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int h = 0; h < 4; ++h) a[p][h] = lds16(arow + p * G::kPlaneBytes + 16 * h);
      const bool nx = tr >= ntrip;  // uniform
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const BlockScale fs = block_scale(cs[r] >> (csh + 8 * s));
        bf16x8_t b[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) b[h] = decode8(ring[s][r][h], fs);
        ring[s][r] = load_w(nx ? wn : wc, nx ? nxt.tile0 : cur.tile0, r, nx ? tr - ntrip : tr, nx ? pf : live);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          acc[r] = mfma16x16x32(as_bf16x8(a[0][h]), b[h], acc[r]);
          acc[r] = mfma16x16x32(as_bf16x8(a[1][h]), b[h], acc[r]);
        }
        ring_fence();
      }
    };

    int c = 0;  // nchunk >= 2: bottom-tested loop
#pragma clang loop unroll(disable)
    do {
      const uint8_t* buf = xs[c & 1];
      // this chunk's two trips are bytes 2 (c & 1) .. +1 of dword c >> 1 (selects, not indexing)
#pragma unroll
      for (int r = 0; r < R; ++r) cs[r] = (c >> 1) ? pd[r][1] : pd[r][0];
      csh = 16 * (c & 1);
#pragma unroll
      for (int s = 0; s < D; ++s) consume(s, buf, c * D + s + D);
      // buffer (c + 1) & 1 was last read in chunk c - 1; past the last chunk it takes the next
      // item's chunk 0 (nchunk is even)
      stage_store((c + 1) & 1);
      stage_load(c + 2 < nchunk ? cur : nxt, c + 2 < nchunk ? c + 2 : c + 2 - nchunk);
      lds_barrier();
    } while (++c < nchunk);
    // the next item's scale rows, issued before the K loop (the last stage_store waited for
    // every load but the last chunk's D R refills and the next item's chunk 1)
    vmcnt_wait<D * R + 4>();
    scale_unpack();

    if (cur.cnt > 0) {  // into slot nhy by selects on the uniform count (not indexing)
#pragma unroll
      for (int h = 0; h < kHoldY; ++h)
        if (h == nhy) {
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) hy[h][r][i] = acc[r][i];
#pragma unroll
          for (int i = 0; i < 4; ++i) ho[h][i] = moe_out_slot(ln.g, i) < cur.cnt ? om[i] : -1;
          ht[h] = cur.tile0;
        }
      if (++nhy == kHoldY) flush_y();
    }
    cur = nxt;
  }
  flush_y();
}

// ---------------------------------------------------------------- combine (unit mode)
//
// out[t, n..n+3] = sum_j w_j * y[t*top_k + j, n..n+3] over live assignments, in j order. The
// routing of a group of G j is loaded first, then all of the group's live y rows at once, then
// they are summed in j order: two memory latencies per group. Few tokens: G = 16, one group up
// to top_k = 16 (M = 32: 6.4 against 6.7 us); many tokens, where the launch streams tens of MB of
// y, G = 4 (M = 192: 8.9 against 9.7 us with G = 16).
constexpr int kCombineGroup = 16;
constexpr int64_t kCombineWideTokens = 96;

template <int G>
__global__ __launch_bounds__(256) void k_moe_combine(
    const float* __restrict__ y, const void* __restrict__ a_expert, int edt,
    const void* __restrict__ a_weight, int wdt, int top_k, int H, int lo, int hi,
    void* __restrict__ out, int odt, SharedTerm st) {
  const int t = blockIdx.y;
  const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (n >= H) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < top_k; j0 += G) {
    float w[G];
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const int j = j0 + q;
      w[q] = 0.f;
      if (j < top_k) {
        const int64_t a = (int64_t)t * top_k + j;
        const int64_t e = load_index(a_expert, edt, a);
        const float wv = load_float(a_weight, wdt, a);
        if (e >= lo && e < hi) w[q] = wv;
      }
    }
    u32x4_t yv[G];
#pragma unroll
    for (int q = 0; q < G; ++q)
      yv[q] = w[q] != 0.f ? ld16(y + ((int64_t)t * top_k + j0 + q) * H + n) : zero16();
#pragma unroll
    for (int q = 0; q < G; ++q)
      if (w[q] != 0.f)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += w[q] * bits_f32(yv[q][c]);
  }
  if (shared_active(st)) {
    const float gs = shared_gate(st, t, odt);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = add_shared(st, gs, acc[c], (int64_t)t * H + n + c, odt);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) store_float(out, odt, (int64_t)t * H + n + c, acc[c]);
}

// The combine followed by the next norm's residual add, in one launch (the last launch of a MoE
// layer whose output feeds `add_rmsnorm(x, moe_out, w)`, model.py:587-604): one workgroup of
// 256 NCH threads per token, thread c taking the 8 columns 8c .. 8c + 7, which are chunk c / 256
// of thread c % 256 in k_rownorm_row<NCH>. Each thread issues all of its loads at once (the live
// assignments' y rows, the shared term's split-K planes, x and the norm weight), computes
// k_moe_combine's value (the same j-order sum, shared term and bf16 rounding), then
// s = bf16(x + value) and its squares; thread (i, r) continues the running sum of squares of
// thread (i - 1, r) through LDS, so the sums the last 256 threads reduce are the row kernel's,
// and y = s * rsqrt(mean(s^2) + eps) * (1 + w). sum_out and normed equal the combine launch
// followed by the residual-form row norm bit for bit; the layer output itself is not stored.
template <int NCH>
__global__ __launch_bounds__(256 * NCH) void k_moe_combine_norm(
    const float* __restrict__ y, const void* __restrict__ a_expert, int edt,
    const void* __restrict__ a_weight, int wdt, int top_k, int H, int lo, int hi, SharedTerm st,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw, float eps,
    uint16_t* __restrict__ sum_out, uint16_t* __restrict__ normed) {
  constexpr int G = kCombineGroup, kPl = 8;  // assignments per pass, shared planes held at once
  __shared__ float run[256];
  __shared__ float part[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1);
  const int chunk = tid >> 8, r = tid & 255;
  const int n = tid * 8;  // == (r + 256 chunk) * 8
  const int64_t base = (int64_t)t * H + n;
  float xv[8], wn[8];
  load8(x, MTPK_BF16, base, xv);
  load8(nw, MTPK_BF16, n, wn);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < top_k; j0 += G) {
    float w[G];
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const int j = j0 + q;
      w[q] = 0.f;
      if (j < top_k) {
        const int64_t a = (int64_t)t * top_k + j;
        const int64_t e = load_index(a_expert, edt, a);
        const float wv = load_float(a_weight, wdt, a);
        if (e >= lo && e < hi) w[q] = wv;
      }
    }
    u32x4_t yv[G][2];
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const float* row = y + ((int64_t)t * top_k + j0 + q) * H + n;
      yv[q][0] = w[q] != 0.f ? ld16(row) : zero16();
      yv[q][1] = w[q] != 0.f ? ld16(row + 4) : zero16();
    }
#pragma unroll
    for (int q = 0; q < G; ++q)
      if (w[q] != 0.f)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] += w[q] * bits_f32(yv[q][c >> 2][c & 3]);
  }
  float o[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) o[c] = round_to(MTPK_BF16, acc[c]);
  if (shared_active(st)) {
    const float gs = shared_gate(st, t, MTPK_BF16);
    float sv[8];
    if (st.part) {  // split-K planes summed in split order (shared_value's arithmetic)
#pragma unroll
      for (int c = 0; c < 8; ++c) sv[c] = 0.f;
      for (int k0 = 0; k0 < st.ks; k0 += kPl) {
        u32x4_t pv[kPl][2];
#pragma unroll
        for (int k = 0; k < kPl; ++k) {
          const float* pl = st.part + (k0 + k) * st.plane + base;
          pv[k][0] = k0 + k < st.ks ? ld16(pl) : zero16();
          pv[k][1] = k0 + k < st.ks ? ld16(pl + 4) : zero16();
        }
#pragma unroll
        for (int k = 0; k < kPl; ++k)
          if (k0 + k < st.ks)
#pragma unroll
            for (int c = 0; c < 8; ++c) sv[c] += bits_f32(pv[k][c >> 2][c & 3]);
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) sv[c] = round_to(MTPK_BF16, sv[c]);
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) sv[c] = load_float(st.shared, st.sdt, base + c);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) o[c] = o[c] + round_to(MTPK_BF16, gs * sv[c]);  // add_shared
  }
  float v[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) v[c] = round_to(MTPK_BF16, xv[c] + round_to(MTPK_BF16, o[c]));
  store8(sum_out, MTPK_BF16, base, v);
  // the row kernel's per-thread sum of squares runs over chunks 0 .. NCH - 1 in order
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (i > 0) {
      __syncthreads();
      if (chunk == i) ss = run[r];
    }
    if (chunk == i) {
#pragma unroll
      for (int c = 0; c < 8; ++c) ss += v[c] * v[c];
      if (i + 1 < NCH) run[r] = ss;
    }
  }
  if (chunk == NCH - 1) {
    ss = wave_sum(ss);
    if (lane == 0) part[r / kWave] = ss;
  }
  __syncthreads();
  ss = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = rsqrtf(ss / (float)H + eps);
  float yn[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) yn[c] = (v[c] * inv) * (1.f + wn[c]);
  store8(normed, MTPK_BF16, base, yn);
}

// The combine of rows that already carry their routing weight (the staging of a down
// projection that applies the weight in its epilogue): out[t, n..n+3] = sum_j y[t*top_k + j]
// over live assignments (expert in [lo, hi) and weight != 0; dead rows are never read), in j
// order, in fp32, then the shared term when there is one. y is f32 or bf16 (YB).
template <bool YB>
__global__ __launch_bounds__(256) void k_moe_combine_rows(
    const void* __restrict__ y, const void* __restrict__ a_expert, int edt,
    const void* __restrict__ a_weight, int wdt, int top_k, int H, int lo, int hi,
    void* __restrict__ out, int odt, SharedTerm st) {
  const int t = blockIdx.y;
  const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (n >= H) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < top_k; j0 += kCombineGroup) {
    bool live[kCombineGroup];
    int64_t a[kCombineGroup];
#pragma unroll
    for (int q = 0; q < kCombineGroup; ++q) {
      const int j = j0 + q;
      a[q] = (int64_t)t * top_k + j;
      live[q] = false;
      if (j < top_k) {
        const int64_t e = load_index(a_expert, edt, a[q]);
        live[q] = e >= lo && e < hi && load_float(a_weight, wdt, a[q]) != 0.f;
      }
    }
    float v[kCombineGroup][4];
#pragma unroll
    for (int q = 0; q < kCombineGroup; ++q) {
      if (YB) {
        uint2 b = make_uint2(0u, 0u);
        if (live[q]) b = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(y) + a[q] * H + n);
        v[q][0] = bits_f32(b.x << 16);
        v[q][1] = bits_f32(b.x & 0xffff0000u);
        v[q][2] = bits_f32(b.y << 16);
        v[q][3] = bits_f32(b.y & 0xffff0000u);
      } else {
        const u32x4_t b = live[q] ? ld16(static_cast<const float*>(y) + a[q] * H + n) : zero16();
#pragma unroll
        for (int c = 0; c < 4; ++c) v[q][c] = bits_f32(b[c]);
      }
    }
#pragma unroll
    for (int q = 0; q < kCombineGroup; ++q)
      if (live[q])
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += v[q][c];
  }
  if (shared_active(st)) {
    const float gs = shared_gate(st, t, odt);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = add_shared(st, gs, acc[c], (int64_t)t * H + n + c, odt);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) store_float(out, odt, (int64_t)t * H + n + c, acc[c]);
}

// The shared term over a routed output already in `out` (the direct path, whose down kernel
// writes the routed sum itself).
__global__ __launch_bounds__(256) void k_moe_shared_glue(void* __restrict__ out, int odt, int H,
                                                         SharedTerm st) {
  const int t = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= H) return;
  const int64_t i = (int64_t)t * H + n;
  store_float(out, odt, i, add_shared(st, shared_gate(st, t, odt), load_float(out, odt, i), i, odt));
}

// ---------------------------------------------------------------- MoE layer co-launches
//
// The shared expert's down projection runs as GEMM tiles inside launches the routed experts
// need anyway (`mtpk_moe_layer`): beside the single-token gate_up items on the direct path, and
// beside the prep's counting sort on the unit path. The GEMM tiles take the lowest workgroup ids,
// so they are dispatched first and stream next to the routed work; each leaves its fp32 split-K
// partials for the final combine (`SharedTerm::part`).

template <int TT, bool SV>
__global__ __launch_bounds__(kMoeThreads) void k_moe_gate_up_single_gemm(
    GemmArgs g, int g_blocks, int g_gx, const uint16_t* __restrict__ x, int64_t x_plane, int K,
    const uint8_t* __restrict__ wq, const uint8_t* __restrict__ ws, int I, UnitSrc src, int top_k,
    uint16_t* __restrict__ inter, int64_t inter_plane) {
  constexpr int kA = GemmSmem<TT, 4>::kBytes, kB = SingleSmem<1>::kBytes;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kA > kB ? kA : kB];
  const int b = blockIdx.x;
  if (b < g_blocks) {
    gemm_tile<TT, 1, 4, false>(g, smem, b % g_gx, b / g_gx);
    return;
  }
  gate_up_single_body<1, 2, SV>(x, x_plane, K, wq, ws, I, src, top_k, inter, inter_plane, smem,
                                b - g_blocks, (int)gridDim.x - g_blocks);
}

constexpr int kPrepCoThreads = kMoeThreads;

template <int TT>
__global__ __launch_bounds__(kMoeThreads) void k_moe_prep_gemm(
    GemmArgs g, int g_gx, const void* __restrict__ a_expert, int edt,
    const void* __restrict__ a_weight, int wdt, int assignments, int lo, int n_experts,
    int32_t* __restrict__ sorted, int32_t* __restrict__ units, int max_units,
    int32_t* __restrict__ n_units) {
  constexpr int kA = GemmSmem<TT, 4>::kBytes, kB = PrepSmem<kPrepCoThreads>::kBytes;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kA > kB ? kA : kB];
  if (blockIdx.x == 0) {
    prep_body<kPrepCoThreads>(a_expert, edt, a_weight, wdt, assignments, lo, n_experts, sorted,
                              units, max_units, n_units, smem);
    return;
  }
  const int b = blockIdx.x - 1;
  gemm_tile<TT, 1, 4, false>(g, smem, b % g_gx, b / g_gx);
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
  if (mode == 0) {
    const int64_t total = rows * half;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
      const int64_t r = i / half, col = i - r * half;
      const uint32_t b = packed[i];
      const float f = e8m0_to_f32(scale[r * nb + (2 * col) / 32]);
      out[r * K + 2 * col] = fp4_to_f32(b & 15u) * f;
      out[r * K + 2 * col + 1] = fp4_to_f32(b >> 4) * f;
    }
    return;
  }
  // mode 1: the MoE kernels' decode8 on each packed dword (K % 32 == 0, so a dword never
  // straddles a row or a scale block)
  const int64_t words = rows * (half >> 2), wpr = half >> 2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / wpr, wc = i - r * wpr;
    const uint8_t* pb = packed + r * half + 4 * wc;
    const uint32_t w = (uint32_t)pb[0] | ((uint32_t)pb[1] << 8) | ((uint32_t)pb[2] << 16) |
                       ((uint32_t)pb[3] << 24);
    const bf16x8_t v = decode8(w, block_scale(scale[r * nb + (8 * wc) / 32]));
    const u32x4_t bits = __builtin_bit_cast(u32x4_t, v);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[r * K + 8 * wc + 2 * j] = bf16_to_f32((uint16_t)(bits[j] & 0xffffu));
      out[r * K + 8 * wc + 2 * j + 1] = bf16_to_f32((uint16_t)(bits[j] >> 16));
    }
  }
}

// Blocks the in-register decode cannot reproduce: scale byte 255 (the OCP NaN scale, where the
// pinned decode gives +-inf for nonzero codes and the hardware convert NaN) over a block that
// holds a nonzero-magnitude code. Block b is packed bytes [16 b, 16 b + 16) and scale byte b.
// Each thread tests 16 scale bytes with one load when `vec` (16-byte aligned scales) and reads
// packed bytes only for the blocks that carry scale 255; *bad counts the threads that found one.
__global__ __launch_bounds__(256) void k_scale_scan(const uint8_t* __restrict__ packed,
                                                    const uint8_t* __restrict__ scale,
                                                    int64_t blocks, int vec,
                                                    int32_t* __restrict__ bad) {
  int found = 0;
  auto check = [&](int64_t b) {
    if (scale[b] != 0xffu) return;
    const uint8_t* p = packed + 16 * b;
    uint32_t any = 0;
    for (int i = 0; i < 16; ++i) any |= p[i];
    if (any & 0x77u) found = 1;
  };
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t groups = vec ? blocks / 16 : 0;
  for (int64_t gi = tid; gi < groups; gi += stride) {
    const u32x4_t s = ld16(scale + 16 * gi);
    uint32_t ff = 0;  // nonzero when some byte of s is 0xff (zero-byte test on ~s)
#pragma unroll
    for (int j = 0; j < 4; ++j) ff |= (~s[j] - 0x01010101u) & s[j] & 0x80808080u;
    if (ff)
      for (int i = 0; i < 16; ++i) check(16 * gi + i);
  }
  for (int64_t b = groups * 16 + tid; b < blocks; b += stride) check(b);
  if (found) atomicAdd(bad, 1);
}

__global__ void k_zero_i32(int32_t* p) { *p = 0; }

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

// Batches of at most this many tokens take the direct path: per-assignment gate_up (no prep)
// and the per-token down + combine (no y, no combine launch).
constexpr int kDirectMaxTokens = 4;

bool dtype_index_ok(int d) { return d == MTPK_I32 || d == MTPK_I64; }
bool dtype_float_ok(int d) { return d == MTPK_F32 || d == MTPK_BF16; }

template <typename KernelT>
int grid_for(KernelT kernel, int64_t wgs_needed, int& cache) {
  if (wgs_needed <= 0) return 0;
  if (cache == 0) cache = occupancy_per_cu(kernel, kMoeThreads);
  const int64_t cap = (int64_t)device_cu_count() * cache;
  return (int)(wgs_needed < cap ? wgs_needed : cap);
}

template <int XP, int OP, int SPLIT, int D, bool SV>
int launch_gate_up_t(const uint16_t* x, int64_t x_plane, int K, const uint8_t* wq,
                     const uint8_t* ws, int I, const UnitSrc& src, int64_t max_units, int top_k,
                     uint16_t* inter, int64_t inter_plane, hipStream_t st) {
  static int occ = 0;
  auto kern = k_moe_gate_up<XP, OP, SPLIT, D, SV>;
  const int64_t items = max_units * (I >> 4);
  const int64_t wgs = SPLIT > 1 ? items : (items + kMoeWaves - 1) / kMoeWaves;
  const int grid = grid_for(kern, wgs, occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, x, x_plane, K, wq, ws, I, src,
                     top_k, inter, inter_plane);
  return status_of(hipGetLastError());
}

// Scale rows whose byte count is a multiple of 16 take the chunked scale loads (SV); for SPLIT
// = 4 each wave's quarter of the trips must also be a multiple of the ring depth.
bool chunked_scales(int K, int split, int D) {
  const int nb = K >> 5, ntrip = (nb + 3) >> 2, T = (ntrip + split - 1) / split;
  return nb % 16 == 0 && T % D == 0;
}

// Unit-mode gate_up with the activation rows staged in LDS (bf16 x, K a multiple of 512).
// Batches of at least this many tokens run gate_up with 8-wave workgroups (one staged copy of
// the unit's activation rows for 128 intermediate rows, one workgroup per CU at 256 VGPRs with
// its held outputs): measured 4-5% faster at 192 rows (Zipf routing, 393 units), slower at 32
// rows (M = 32 layer 180.0-180.9 against 178.8-179.2 us), where the 8 items per unit leave the
// grid a short tail of a few items per workgroup; at 48 rows (the draft steps' MoE) the MTP
// round took 8.29 against 8.32-8.33 ms.
constexpr int64_t kGateUpWideTokens = 48;

int launch_gate_up_lds(const uint16_t* x, int64_t x_elems, int K, const uint8_t* wq,
                       const uint8_t* ws, int I, const UnitSrc& src, int64_t max_units, int top_k,
                       uint16_t* inter, int64_t inter_plane, int64_t tokens, hipStream_t st) {
  if (tokens >= kGateUpWideTokens) {
    static int occ8 = 0;
    auto kern = k_moe_gate_up_lds<4, 8>;
    const int64_t items = max_units * (((I >> 4) + 7) / 8);
    if (occ8 == 0) occ8 = occupancy_per_cu(kern, 8 * kWave);
    const int64_t cap = (int64_t)device_cu_count() * occ8;
    const int grid = (int)(items < cap ? items : cap);
    if (grid == 0) return 0;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(8 * kWave), 0, st, x, x_elems, K, wq, ws, I, src,
                       top_k, inter, inter_plane);
    return status_of(hipGetLastError());
  }
  static int occ = 0;
  auto kern = k_moe_gate_up_lds<4, 4>;
  const int64_t items = max_units * (((I >> 4) + kMoeWaves - 1) / kMoeWaves);
  const int grid = grid_for(kern, items, occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, x, x_elems, K, wq, ws, I, src,
                     top_k, inter, inter_plane);
  return status_of(hipGetLastError());
}

// SPLIT = 4 while the item count would leave fewer than four waves per SIMD busy.
int launch_gate_up(int xp, const uint16_t* x, int64_t x_plane, int K, const uint8_t* wq,
                   const uint8_t* ws, int I, const UnitSrc& src, int64_t max_units, int top_k,
                   uint16_t* inter, int64_t inter_plane, hipStream_t st) {
  const bool split = max_units * (I >> 4) < (int64_t)device_cu_count() * 16;
  if (xp == 1 && !split && K % 512 == 0 && K <= 4096)
    return launch_gate_up_lds(x, x_plane, K, wq, ws, I, src, max_units, top_k, inter, inter_plane,
                              x_plane / K, st);
#define MTPK_GU(XP_, OP_, SP_, D_)                                                           \
  (chunked_scales(K, SP_, D_)                                                                \
       ? launch_gate_up_t<XP_, OP_, SP_, D_, true>(x, x_plane, K, wq, ws, I, src, max_units, \
                                                   top_k, inter, inter_plane, st)            \
       : launch_gate_up_t<XP_, OP_, SP_, D_, false>(x, x_plane, K, wq, ws, I, src, max_units, \
                                                    top_k, inter, inter_plane, st))
  if (xp == 1) return split ? MTPK_GU(1, 2, 4, 4) : MTPK_GU(1, 2, 1, 4);
  return split ? MTPK_GU(3, 3, 4, 2) : MTPK_GU(3, 3, 1, 2);
#undef MTPK_GU
}

template <int IP, int R, int D, bool SV>
int launch_down_t(const uint16_t* inter, int64_t inter_plane, int K, const uint8_t* wq,
                  const uint8_t* ws, int H, const UnitSrc& src, int64_t max_units, float* y,
                  hipStream_t st) {
  static int occ = 0;
  auto kern = k_moe_down<IP, R, D, SV>;
  const int64_t items = max_units * (((H >> 4) + R - 1) / R);
  const int grid = grid_for(kern, (items + kMoeWaves - 1) / kMoeWaves, occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, inter, inter_plane, K, wq, ws,
                     H, src, y);
  return status_of(hipGetLastError());
}

int launch_down_lds(const uint16_t* inter, int64_t inter_plane, int K, const uint8_t* wq,
                    const uint8_t* ws, int H, const UnitSrc& src, int64_t max_units, float* y,
                    hipStream_t st) {
  static int occ = 0;
  constexpr int R = 4;
  auto kern = k_moe_down_lds<R>;
  const int64_t items = max_units * (((H >> 4) + kMoeWaves * R - 1) / (kMoeWaves * R));
  const int grid = grid_for(kern, items, occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, inter, inter_plane, K, wq, ws,
                     H, src, y);
  return status_of(hipGetLastError());
}

template <int IP, int D, bool SV>
int launch_down_token_t(const uint16_t* inter, int64_t inter_plane, int K, const uint8_t* wq,
                        const uint8_t* ws, int H, const void* a_expert, int edt,
                        const void* a_weight, int wdt, int lo, int n_experts, int tokens,
                        int top_k, void* out, int odt, hipStream_t st) {
  static int occ = 0;
  auto kern = k_moe_down_token<IP, D, SV>;
  const int grid = grid_for(kern, (int64_t)tokens * (H >> 4), occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, inter, inter_plane, K, wq, ws,
                     H, a_expert, edt, a_weight, wdt, lo, n_experts, tokens, top_k, out, odt);
  return status_of(hipGetLastError());
}

// Direct mode with one token per unit: the single-token kernels when the K ranges fit their
// fixed trip counts (gate_up K <= 4096, down K <= 1024).
bool single_gate_up_ok(int K) { return K <= 4 * kSingleQuarter; }
bool single_down_ok(int K) { return K <= kSingleQuarter; }

template <int XP, int OP, bool SV>
int launch_gate_up_single(const uint16_t* x, int64_t x_plane, int K, const uint8_t* wq,
                          const uint8_t* ws, int I, const UnitSrc& src, int64_t units, int top_k,
                          uint16_t* inter, int64_t inter_plane, hipStream_t st) {
  static int occ = 0;
  auto kern = k_moe_gate_up_single<XP, OP, SV>;
  const int grid = grid_for(kern, units * (I >> 4), occ);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kMoeThreads), 0, st, x, x_plane, K, wq, ws, I, src,
                     top_k, inter, inter_plane);
  return status_of(hipGetLastError());
}

template <int IP, bool SV>
int launch_down_single(const uint16_t* inter, int64_t inter_plane, int K, const uint8_t* wq,
                       const uint8_t* ws, int H, const void* a_expert, int edt, const void* a_weight,
                       int wdt, int lo, int n_experts, int tokens, int top_k, void* out, int odt,
                       hipStream_t st, const SharedTerm& sh = SharedTerm{}) {
  static int occ = 0;
  auto kern = k_moe_down_single<IP, SV>;
  constexpr int threads = kSingleDownWaves * kWave;
  if (occ == 0) occ = occupancy_per_cu(kern, threads);
  const int64_t need = (int64_t)tokens * (H >> 4), cap = (int64_t)device_cu_count() * occ;
  const int grid = (int)(need < cap ? need : cap);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(threads), 0, st, inter, inter_plane, K, wq, ws, H,
                     a_expert, edt, a_weight, wdt, lo, n_experts, tokens, top_k, out, odt, sh);
  return status_of(hipGetLastError());
}

UnitSrc unit_list(const int32_t* units, const int32_t* sorted, const int32_t* n_units,
                  int64_t max_units) {
  UnitSrc s{};
  s.units = units;
  s.sorted = sorted;
  s.n_units = n_units;
  s.max_units = (int)max_units;
  s.direct = 0;
  return s;
}

UnitSrc unit_direct(const void* a_expert, int edt, const void* a_weight, int wdt, int lo, int hi,
                    int64_t assignments) {
  UnitSrc s{};
  s.a_expert = a_expert;
  s.a_weight = a_weight;
  s.edt = edt;
  s.wdt = wdt;
  s.lo = lo;
  s.n_experts = hi - lo;
  s.assignments = (int)assignments;
  s.direct = 1;
  return s;
}

bool gemm_shapes_ok(int64_t hidden, int64_t inter_dim, int64_t local_experts) {
  return hidden > 0 && hidden % 32 == 0 && inter_dim > 0 && inter_dim % 32 == 0 &&
         hidden <= (1 << 20) && inter_dim <= (1 << 20) && local_experts > 0 &&
         local_experts <= MTPK_MAX_EXPERTS;
}

}  // namespace

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int mtpk_moe_direct_max_tokens(void) { return kDirectMaxTokens; }

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
  // fewer units than the bound would drop assignments that down and combine still expect
  if (max_units < mtpk_moe_max_units(assignments, ne) || max_units > INT32_MAX / 3) return MTPK_EINVAL;
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
  if (!gemm_shapes_ok(hidden, inter_dim, local_experts) || top_k <= 0) return MTPK_EINVAL;
  if (!aligned16(x_planes) || !aligned16(gate_up) || !aligned16(inter)) return MTPK_EINVAL;
  if (max_units <= 0 || max_units > INT32_MAX / inter_dim ||
      max_units < mtpk_moe_max_units(assignments, local_experts))
    return MTPK_EINVAL;
  if (!((x_nplanes == 1 && inter_planes == 2) || (x_nplanes == 3 && inter_planes == 3)))
    return MTPK_EINVAL;
  return launch_gate_up(x_nplanes, x_planes, tokens * hidden, (int)hidden, gate_up, gate_up_scale,
                        (int)inter_dim, unit_list(units, sorted, n_units, max_units), max_units,
                        top_k, inter, assignments * inter_dim, (hipStream_t)stream);
}

int mtpk_moe_gate_up_direct(const uint16_t* x_planes, int x_nplanes, int64_t tokens,
                            int64_t hidden, const uint8_t* gate_up, const uint8_t* gate_up_scale,
                            int64_t local_experts, int64_t inter_dim, const void* a_expert,
                            int expert_dtype, const void* a_weight, int weight_dtype, int top_k,
                            int expert_lo, int expert_hi, uint16_t* inter, int inter_planes,
                            void* stream) {
  if (!x_planes || !gate_up || !gate_up_scale || !a_expert || !a_weight || !inter)
    return MTPK_EINVAL;
  if (!gemm_shapes_ok(hidden, inter_dim, local_experts) || top_k <= 0) return MTPK_EINVAL;
  if (!dtype_index_ok(expert_dtype) || !dtype_float_ok(weight_dtype)) return MTPK_EINVAL;
  if ((int64_t)expert_hi - expert_lo != local_experts) return MTPK_EINVAL;
  if (!aligned16(x_planes) || !aligned16(gate_up) || !aligned16(inter)) return MTPK_EINVAL;
  if (tokens < 0 || tokens * top_k > INT32_MAX / inter_dim) return MTPK_EINVAL;
  if (!((x_nplanes == 1 && inter_planes == 2) || (x_nplanes == 3 && inter_planes == 3)))
    return MTPK_EINVAL;
  const int64_t a = tokens * top_k;
  if (a == 0) return 0;
  const UnitSrc src =
      unit_direct(a_expert, expert_dtype, a_weight, weight_dtype, expert_lo, expert_hi, a);
  const hipStream_t st = (hipStream_t)stream;
  if (single_gate_up_ok((int)hidden)) {
#define MTPK_GS(XP_, OP_, SV_)                                                                   \
  launch_gate_up_single<XP_, OP_, SV_>(x_planes, tokens * hidden, (int)hidden, gate_up,         \
                                       gate_up_scale, (int)inter_dim, src, a, top_k, inter,      \
                                       a * inter_dim, st)
    const bool sv = (hidden / 32) % 32 == 0;
    if (x_nplanes == 1) return sv ? MTPK_GS(1, 2, true) : MTPK_GS(1, 2, false);
    return sv ? MTPK_GS(3, 3, true) : MTPK_GS(3, 3, false);
#undef MTPK_GS
  }
  return launch_gate_up(x_nplanes, x_planes, tokens * hidden, (int)hidden, gate_up,
                        gate_up_scale, (int)inter_dim, src, a, top_k, inter, a * inter_dim, st);
}

int mtpk_moe_down(const uint16_t* inter, int inter_planes, int64_t assignments, int64_t inter_dim,
                  const uint8_t* down, const uint8_t* down_scale, int64_t local_experts,
                  int64_t hidden, const int32_t* sorted, const int32_t* units,
                  const int32_t* n_units, int64_t max_units, float* y, void* stream) {
  if (!inter || !down || !down_scale || !sorted || !units || !n_units || !y) return MTPK_EINVAL;
  if (!gemm_shapes_ok(hidden, inter_dim, local_experts)) return MTPK_EINVAL;
  if (!aligned16(inter) || !aligned16(down)) return MTPK_EINVAL;
  if (max_units <= 0 || max_units > INT32_MAX / hidden ||
      max_units < mtpk_moe_max_units(assignments, local_experts))
    return MTPK_EINVAL;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t ip = assignments * inter_dim;
  const UnitSrc src = unit_list(units, sorted, n_units, max_units);
  const bool sv = chunked_scales((int)inter_dim, 1, 2);
  // the LDS kernel marks absent staging rows with an offset >= 2^31 (past the whole inter buffer)
  if (inter_planes == 2 && inter_dim % 512 == 0 && inter_dim <= 1024 && ip * 4 < (int64_t(1) << 31))
    return launch_down_lds(inter, ip, (int)inter_dim, down, down_scale, (int)hidden, src,
                           max_units, y, st);
  if (inter_planes == 2)
    return sv ? launch_down_t<2, 4, 2, true>(inter, ip, (int)inter_dim, down, down_scale,
                                             (int)hidden, src, max_units, y, st)
              : launch_down_t<2, 4, 2, false>(inter, ip, (int)inter_dim, down, down_scale,
                                              (int)hidden, src, max_units, y, st);
  if (inter_planes == 3)
    return sv ? launch_down_t<3, 2, 2, true>(inter, ip, (int)inter_dim, down, down_scale,
                                             (int)hidden, src, max_units, y, st)
              : launch_down_t<3, 2, 2, false>(inter, ip, (int)inter_dim, down, down_scale,
                                              (int)hidden, src, max_units, y, st);
  return MTPK_EINVAL;
}

int mtpk_moe_down_combine(const uint16_t* inter, int inter_planes, int64_t inter_dim,
                          const uint8_t* down, const uint8_t* down_scale, int64_t local_experts,
                          int64_t hidden, const void* a_expert, int expert_dtype,
                          const void* a_weight, int weight_dtype, int64_t tokens, int top_k,
                          int expert_lo, int expert_hi, void* out, int out_dtype, void* stream) {
  if (!inter || !down || !down_scale || !a_expert || !a_weight || !out) return MTPK_EINVAL;
  if (!gemm_shapes_ok(hidden, inter_dim, local_experts) || top_k <= 0) return MTPK_EINVAL;
  if (!dtype_index_ok(expert_dtype) || !dtype_float_ok(weight_dtype) || !dtype_float_ok(out_dtype))
    return MTPK_EINVAL;
  if ((int64_t)expert_hi - expert_lo != local_experts) return MTPK_EINVAL;
  if (!aligned16(inter) || !aligned16(down)) return MTPK_EINVAL;
  if (tokens < 0 || tokens * (hidden >> 4) > INT32_MAX || tokens * top_k > INT32_MAX / inter_dim)
    return MTPK_EINVAL;
  if (tokens == 0) return 0;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t ip = tokens * top_k * inter_dim;
  if (single_down_ok((int)inter_dim) && (inter_planes == 2 || inter_planes == 3)) {
#define MTPK_DS(IP_, SV_)                                                                     \
  launch_down_single<IP_, SV_>(inter, ip, (int)inter_dim, down, down_scale, (int)hidden,      \
                               a_expert, expert_dtype, a_weight, weight_dtype, expert_lo,     \
                               (int)local_experts, (int)tokens, top_k, out, out_dtype, st)
    const bool sv = inter_dim == 1024;
    if (inter_planes == 2) return sv ? MTPK_DS(2, true) : MTPK_DS(2, false);
    return sv ? MTPK_DS(3, true) : MTPK_DS(3, false);
#undef MTPK_DS
  }
#define MTPK_DT(IP_, D_, SV_)                                                              \
  launch_down_token_t<IP_, D_, SV_>(inter, ip, (int)inter_dim, down, down_scale, (int)hidden, \
                                    a_expert, expert_dtype, a_weight, weight_dtype, expert_lo, \
                                    (int)local_experts, (int)tokens, top_k, out, out_dtype, st)
  if (inter_planes == 2)
    return chunked_scales((int)inter_dim, 1, 4) ? MTPK_DT(2, 4, true) : MTPK_DT(2, 4, false);
  if (inter_planes == 3)
    return chunked_scales((int)inter_dim, 1, 2) ? MTPK_DT(3, 2, true) : MTPK_DT(3, 2, false);
#undef MTPK_DT
  return MTPK_EINVAL;
}

int mtpk_moe_combine(const float* y, const void* a_expert, int expert_dtype, const void* a_weight,
                     int weight_dtype, int64_t tokens, int top_k, int64_t hidden, int expert_lo,
                     int expert_hi, void* out, int out_dtype, void* stream) {
  if (!y || !a_expert || !a_weight || !out) return MTPK_EINVAL;
  if (!dtype_index_ok(expert_dtype) || !dtype_float_ok(weight_dtype) || !dtype_float_ok(out_dtype))
    return MTPK_EINVAL;
  if (tokens < 0 || tokens > 65535 || hidden <= 0 || hidden % 4 || top_k <= 0) return MTPK_EINVAL;
  if (!aligned16(y)) return MTPK_EINVAL;
  if (tokens == 0) return 0;
  const dim3 grid((unsigned)((hidden / 4 + 255) / 256), (unsigned)tokens);
  hipLaunchKernelGGL(tokens < kCombineWideTokens ? k_moe_combine<kCombineGroup> : k_moe_combine<4>,
                     grid, dim3(256), 0, (hipStream_t)stream, y, a_expert,
                     expert_dtype, a_weight, weight_dtype, top_k, (int)hidden, expert_lo,
                     expert_hi, out, out_dtype, SharedTerm{});
  return status_of(hipGetLastError());
}

int mtpk_moe_combine_rows(const void* y, int y_dtype, const void* a_expert, int expert_dtype,
                          const void* a_weight, int weight_dtype, int64_t tokens, int top_k,
                          int64_t hidden, int expert_lo, int expert_hi, const void* shared,
                          int shared_dtype, const void* shared_gate, int gate_dtype,
                          int64_t gate_stride, void* out, int out_dtype, void* stream) {
  if (!y || !a_expert || !a_weight || !out) return MTPK_EINVAL;
  if (!dtype_float_ok(y_dtype) || !dtype_index_ok(expert_dtype) || !dtype_float_ok(weight_dtype) ||
      !dtype_float_ok(out_dtype))
    return MTPK_EINVAL;
  if (tokens < 0 || tokens > 65535 || hidden <= 0 || hidden % 4 || top_k <= 0) return MTPK_EINVAL;
  if (reinterpret_cast<uintptr_t>(y) & (y_dtype == MTPK_F32 ? 15u : 7u)) return MTPK_EINVAL;
  if (shared && (!shared_gate || !dtype_float_ok(shared_dtype) || !dtype_float_ok(gate_dtype) ||
                 gate_stride < 0))
    return MTPK_EINVAL;
  if (tokens == 0) return 0;
  const SharedTerm st{shared, shared_dtype, shared_gate, gate_dtype, gate_stride};
  const dim3 grid((unsigned)((hidden / 4 + 255) / 256), (unsigned)tokens);
  auto kern = y_dtype == MTPK_F32 ? k_moe_combine_rows<false> : k_moe_combine_rows<true>;
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, (hipStream_t)stream, y, a_expert, expert_dtype,
                     a_weight, weight_dtype, top_k, (int)hidden, expert_lo, expert_hi, out,
                     out_dtype, st);
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
  return mtpk_fused_moe_shared(x, x_dtype, tokens, hidden, gate_up, gate_up_scale, down,
                               down_scale, local_experts, inter_dim, a_expert, expert_dtype,
                               a_weight, weight_dtype, top_k, expert_lo, expert_hi, nullptr, 0,
                               nullptr, 0, 0, workspace, workspace_bytes, out, stream);
}

int mtpk_fused_moe_shared(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                          const uint8_t* gate_up, const uint8_t* gate_up_scale, const uint8_t* down,
                          const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                          const void* a_expert, int expert_dtype, const void* a_weight,
                          int weight_dtype, int top_k, int expert_lo, int expert_hi,
                          const void* shared, int shared_dtype, const void* shared_gate,
                          int gate_dtype, int64_t gate_stride, void* workspace,
                          int64_t workspace_bytes, void* out, void* stream) {
  if (!x || !out || !workspace || !dtype_float_ok(x_dtype)) return MTPK_EINVAL;
  if (shared && (!shared_gate || !dtype_float_ok(shared_dtype) || !dtype_float_ok(gate_dtype) ||
                 gate_stride < 0))
    return MTPK_EINVAL;
  if (tokens > 65535 || hidden <= 0 || hidden % 4) return MTPK_EINVAL;  // the combine's grid
  const SharedTerm st{shared, shared_dtype, shared_gate, gate_dtype, gate_stride};
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
  if (tokens <= kDirectMaxTokens) {
    rc = mtpk_moe_gate_up_direct(xplanes, xp, tokens, hidden, gate_up, gate_up_scale,
                                 local_experts, inter_dim, a_expert, expert_dtype, a_weight,
                                 weight_dtype, top_k, expert_lo, expert_hi, inter, ip, stream);
    if (rc) return rc;
    rc = mtpk_moe_down_combine(inter, ip, inter_dim, down, down_scale, local_experts, hidden,
                               a_expert, expert_dtype, a_weight, weight_dtype, tokens, top_k,
                               expert_lo, expert_hi, out, x_dtype, stream);
    if (rc || !shared) return rc;
    hipLaunchKernelGGL(k_moe_shared_glue, dim3((unsigned)((hidden + 255) / 256), (unsigned)tokens),
                       dim3(256), 0, (hipStream_t)stream, out, x_dtype, (int)hidden, st);
    return status_of(hipGetLastError());
  }
  rc = mtpk_moe_prep(a_expert, expert_dtype, a_weight, weight_dtype, a, expert_lo, expert_hi,
                     sorted, units, mu, n_units, stream);
  if (rc) return rc;
  rc = mtpk_moe_gate_up(xplanes, xp, tokens, hidden, gate_up, gate_up_scale, local_experts,
                        inter_dim, sorted, units, n_units, mu, top_k, inter, ip, a, stream);
  if (rc) return rc;
  rc = mtpk_moe_down(inter, ip, a, inter_dim, down, down_scale, local_experts, hidden, sorted,
                     units, n_units, mu, y, stream);
  if (rc) return rc;
  const dim3 grid((unsigned)((hidden / 4 + 255) / 256), (unsigned)tokens);
  hipLaunchKernelGGL(tokens < kCombineWideTokens ? k_moe_combine<kCombineGroup> : k_moe_combine<4>,
                     grid, dim3(256), 0, (hipStream_t)stream, y, a_expert,
                     expert_dtype, a_weight, weight_dtype, top_k, (int)hidden, expert_lo,
                     expert_hi, out, x_dtype, st);
  return status_of(hipGetLastError());
}

}  // extern "C"

namespace {

// Token tiles of 16 weight rows per wave, 4 waves: the tile count of one fused-layer GEMM.
int64_t layer_tiles(int64_t cols) { return (cols + 63) / 64; }

struct LayerPlan {
  int64_t routed, topw, topi, sgate, wr, wsg, act, wd, total;
  int ksr, kss, ksd;
};

LayerPlan layer_plan(int64_t tokens, int64_t hidden, int64_t router_rows, int64_t shared_inter,
                     int64_t top_k, int64_t local_experts, int64_t inter_dim) {
  LayerPlan p{};
  p.ksr = gemm_splits(tokens, router_rows, hidden, kEpiStore);
  p.kss = gemm_splits(tokens, 2 * shared_inter, hidden, kEpiSilu);
  p.ksd = gemm_splits(tokens, hidden, shared_inter, kEpiStore);
  int64_t o = align256(mtpk_moe_workspace_bytes(tokens, top_k, local_experts, inter_dim, hidden,
                                                MTPK_BF16));
  p.topw = o;
  o += align256(tokens * top_k * 4);
  p.topi = o;
  o += align256(tokens * top_k * 4);
  p.sgate = o;
  o += align256(tokens * 2);
  p.wr = o;
  o += align256((int64_t)p.ksr * tokens * router_rows * 4);
  p.wsg = o;
  o += align256((int64_t)p.kss * tokens * 2 * shared_inter * 4);
  p.act = o;
  o += align256(tokens * shared_inter * 2);
  p.wd = o;
  o += align256((int64_t)p.ksd * tokens * hidden * 4);
  p.total = o;
  return p;
}

GemmArgs layer_gemm(const uint16_t* x, const uint16_t* w, int64_t m, int64_t n, int64_t k, int ks,
                    int epi, float* part) {
  const int64_t cols = epi == kEpiSilu ? n / 2 : n;
  return GemmArgs{x, w, (int)m, (int)n, (int)k, ks, epi, MTPK_BF16, (int)cols, nullptr, part,
                  nullptr, (int)layer_tiles(cols), gemm_groups(m)};
}

template <int TT, bool SV>
int launch_gate_up_single_gemm(const GemmArgs& g, const uint16_t* x, int64_t x_plane, int K,
                               const uint8_t* wq, const uint8_t* ws, int I, const UnitSrc& src,
                               int64_t units, int top_k, uint16_t* inter, int64_t inter_plane,
                               hipStream_t st) {
  static int occ = 0;
  auto kern = k_moe_gate_up_single_gemm<TT, SV>;
  const int g_gx = (int)gemm_grid_x(g.tiles, g.RG), g_blocks = g_gx * g.KS;
  const int routed = grid_for(kern, units * (I >> 4), occ);
  hipLaunchKernelGGL(kern, dim3(g_blocks + routed), dim3(kMoeThreads), 0, st, g, g_blocks, g_gx,
                     x, x_plane, K, wq, ws, I, src, top_k, inter, inter_plane);
  return status_of(hipGetLastError());
}

template <int TT>
int launch_prep_gemm(const GemmArgs& g, const void* a_expert, int edt, const void* a_weight,
                     int wdt, int64_t assignments, int lo, int n_experts, int32_t* sorted,
                     int32_t* units, int64_t max_units, int32_t* n_units, hipStream_t st) {
  const int g_gx = (int)gemm_grid_x(g.tiles, g.RG);
  hipLaunchKernelGGL(k_moe_prep_gemm<TT>, dim3(1 + g_gx * g.KS), dim3(kMoeThreads), 0, st, g,
                     g_gx, a_expert, edt, a_weight, wdt, (int)assignments, lo, n_experts, sorted,
                     units, (int)max_units, n_units);
  return status_of(hipGetLastError());
}

}  // namespace

extern "C" {

int64_t mtpk_moe_layer_workspace_bytes(int64_t tokens, int64_t hidden, int64_t router_rows,
                                       int64_t shared_inter, int top_k, int64_t local_experts,
                                       int64_t inter_dim) {
  if (tokens <= 0 || tokens > 256 || hidden <= 0 || router_rows <= 1 || shared_inter <= 0 ||
      top_k <= 0 || local_experts <= 0 || inter_dim <= 0)
    return 0;
  return layer_plan(tokens, hidden, router_rows, shared_inter, top_k, local_experts, inter_dim)
      .total;
}

int mtpk_moe_layer_supported(const void* h, int64_t tokens, int64_t hidden, const void* router_gate,
                             int64_t router_rows, const void* shared_gate_up,
                             const void* shared_down, int64_t shared_inter, const void* gate_up,
                             const void* gate_up_scale, const void* down, const void* down_scale,
                             int64_t local_experts, int64_t inter_dim, int top_k, int expert_lo,
                             int expert_hi) {
  if (!h || !router_gate || !shared_gate_up || !shared_down || !gate_up || !gate_up_scale ||
      !down || !down_scale)
    return 0;
  if (tokens < 0 || tokens > 256 || tokens > 65535) return 0;
  const int64_t experts = router_rows - 1;  // the router's last row is the shared expert's gate
  if (experts <= 0 || experts > MTPK_MAX_ROUTER_EXPERTS || top_k <= 0 || top_k > MTPK_MAX_TOP_K ||
      top_k > experts)
    return 0;
  if ((int64_t)expert_hi - expert_lo != local_experts || expert_lo < 0 || expert_hi > experts)
    return 0;
  if (!gemm_shapes_ok(hidden, inter_dim, local_experts) || hidden % kGemmKC ||
      shared_inter <= 0 || shared_inter % kGemmKC || shared_inter % 16 || hidden % 4)
    return 0;
  if (!aligned16(h) || !aligned16(router_gate) || !aligned16(shared_gate_up) ||
      !aligned16(shared_down) || !aligned16(gate_up) || !aligned16(down))
    return 0;
  if (router_rows * hidden * 2 > 0x7fffffffLL || 2 * shared_inter * hidden * 2 > 0x7fffffffLL)
    return 0;
  // the co-launches run 4-wave GEMM tiles
  if (tokens > 0 && (gemm_waves(tokens, router_rows, kEpiStore) != 4 ||
                     gemm_waves(tokens, 2 * shared_inter, kEpiSilu) != 4 ||
                     gemm_waves(tokens, hidden, kEpiStore) != 4))
    return 0;
  return 1;
}

}  // extern "C"

namespace {

// The next norm's residual form, fused into a layer's last launch (mtpk_moe_layer_add_norm).
struct AddNorm {
  const uint16_t* x;  // residual rows [tokens, hidden]
  const uint16_t* w;  // norm weight [hidden]
  float eps;
  uint16_t* sum_out;  // x + the layer's output
  uint16_t* normed;   // rmsnorm(sum_out) * (1 + w)
};

int moe_layer_run(const uint16_t* h, int64_t tokens, int64_t hidden, const uint16_t* router_gate,
                  int64_t router_rows, const uint16_t* shared_gate_up,
                  const uint16_t* shared_down, int64_t shared_inter, const uint8_t* gate_up,
                  const uint8_t* gate_up_scale, const uint8_t* down, const uint8_t* down_scale,
                  int64_t local_experts, int64_t inter_dim, int top_k, int expert_lo,
                  int expert_hi, float* top_w, int32_t* top_i, void* workspace,
                  int64_t workspace_bytes, void* out, const AddNorm* an, void* stream) {
  if (!workspace || (!out && !an) || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return MTPK_EINVAL;
  if (!mtpk_moe_layer_supported(h, tokens, hidden, router_gate, router_rows, shared_gate_up,
                                shared_down, shared_inter, gate_up, gate_up_scale, down, down_scale,
                                local_experts, inter_dim, top_k, expert_lo, expert_hi))
    return MTPK_EINVAL;
  const int64_t experts = router_rows - 1;
  if (tokens == 0) return 0;
  const LayerPlan pl =
      layer_plan(tokens, hidden, router_rows, shared_inter, top_k, local_experts, inter_dim);
  if (workspace_bytes < pl.total) return MTPK_EINVAL;
  char* w = static_cast<char*>(workspace);
  float* tw = top_w ? top_w : reinterpret_cast<float*>(w + pl.topw);
  int32_t* ti = top_i ? top_i : reinterpret_cast<int32_t*>(w + pl.topi);
  uint16_t* sgate = reinterpret_cast<uint16_t*>(w + pl.sgate);
  float* wr = reinterpret_cast<float*>(w + pl.wr);
  float* wsg = reinterpret_cast<float*>(w + pl.wsg);
  uint16_t* act = reinterpret_cast<uint16_t*>(w + pl.act);
  float* wd = reinterpret_cast<float*>(w + pl.wd);
  const hipStream_t st = (hipStream_t)stream;

  // 1. router logits and the shared expert's gate/up, one launch (split-K partials)
  int rc = launch_gemm_pair(layer_gemm(h, router_gate, tokens, router_rows, hidden, pl.ksr, kEpiStore, wr),
                            layer_gemm(h, shared_gate_up, tokens, 2 * shared_inter, hidden, pl.kss, kEpiSilu, wsg),
                            st);
  if (rc) return rc;
  // 2. softmax top-k from the router partials, the shared gate logit, act = silu(gate) * up
  RouteActArgs ra{wr, pl.ksr, (int)tokens, (int)router_rows, (int)experts, top_k, tw, ti,
                  MTPK_I32, sgate, wsg, pl.kss, (int)shared_inter, act, 0};
  rc = launch_route_act(ra, st);
  if (rc) return rc;
  // 3.. the routed experts, with the shared down projection's tiles in the first routed launch
  // and its gated term in the last
  const GemmArgs gd = layer_gemm(act, shared_down, tokens, hidden, shared_inter, pl.ksd, kEpiStore, wd);
  SharedTerm sh{};
  sh.gate = sgate;
  sh.gdt = MTPK_BF16;
  sh.gate_stride = 1;
  sh.part = wd;
  sh.ks = pl.ksd;
  sh.plane = tokens * hidden;
  const int64_t a = tokens * top_k;
  const int64_t mu = mtpk_moe_max_units(a, local_experts);
  char* p = w;
  int32_t* sorted = reinterpret_cast<int32_t*>(p);
  p += align256(a * 4);
  int32_t* units = reinterpret_cast<int32_t*>(p);
  p += align256(3 * mu * 4);
  int32_t* n_units = reinterpret_cast<int32_t*>(p);
  p += 256;
  uint16_t* inter = reinterpret_cast<uint16_t*>(p);
  p += align256(2 * a * inter_dim * 2);
  float* y = reinterpret_cast<float*>(p);
  const int tt = gemm_tt(tokens);
  static_assert(kDirectMaxTokens <= 16, "the direct path's GEMM tiles hold one token tile");
  if (tokens <= kDirectMaxTokens && single_gate_up_ok((int)hidden) && single_down_ok((int)inter_dim)) {
    if (an) return MTPK_EINVAL;  // the direct path's down launch writes the output itself
    const UnitSrc src = unit_direct(ti, MTPK_I32, tw, MTPK_F32, expert_lo, expert_hi, a);
    const bool sv = (hidden / 32) % 32 == 0;
#define MTPK_GSG(TT_)                                                                          \
  (sv ? launch_gate_up_single_gemm<TT_, true>(gd, h, tokens * hidden, (int)hidden, gate_up,     \
                                              gate_up_scale, (int)inter_dim, src, a, top_k,     \
                                              inter, a * inter_dim, st)                         \
      : launch_gate_up_single_gemm<TT_, false>(gd, h, tokens * hidden, (int)hidden, gate_up,    \
                                               gate_up_scale, (int)inter_dim, src, a, top_k,    \
                                               inter, a * inter_dim, st))
    rc = MTPK_GSG(1);  // at most 4 token rows: one token tile
#undef MTPK_GSG
    if (rc) return rc;
    const int64_t ip = a * inter_dim;
    return inter_dim == 1024
               ? launch_down_single<2, true>(inter, ip, (int)inter_dim, down, down_scale,
                                             (int)hidden, ti, MTPK_I32, tw, MTPK_F32, expert_lo,
                                             (int)local_experts, (int)tokens, top_k, out,
                                             MTPK_BF16, st, sh)
               : launch_down_single<2, false>(inter, ip, (int)inter_dim, down, down_scale,
                                              (int)hidden, ti, MTPK_I32, tw, MTPK_F32, expert_lo,
                                              (int)local_experts, (int)tokens, top_k, out,
                                              MTPK_BF16, st, sh);
  }
#define MTPK_PG(TT_)                                                                          \
  launch_prep_gemm<TT_>(gd, ti, MTPK_I32, tw, MTPK_F32, a, expert_lo, (int)local_experts, sorted, \
                        units, mu, n_units, st)
  switch (tt) {
    case 1: rc = MTPK_PG(1); break;
    case 2: rc = MTPK_PG(2); break;
    case 3: rc = MTPK_PG(3); break;
    default: rc = MTPK_PG(4); break;
  }
#undef MTPK_PG
  if (rc) return rc;
  rc = mtpk_moe_gate_up(h, 1, tokens, hidden, gate_up, gate_up_scale, local_experts, inter_dim,
                        sorted, units, n_units, mu, top_k, inter, 2, a, stream);
  if (rc) return rc;
  rc = mtpk_moe_down(inter, 2, a, inter_dim, down, down_scale, local_experts, hidden, sorted,
                     units, n_units, mu, y, stream);
  if (rc) return rc;
  if (an) {
    const dim3 g1((unsigned)tokens);
#define MTPK_CN(N_)                                                                             \
  hipLaunchKernelGGL(k_moe_combine_norm<N_>, g1, dim3(256 * N_), 0, st, y, ti, MTPK_I32, tw, MTPK_F32, \
                     top_k, (int)hidden, expert_lo, expert_hi, sh, an->x, an->w, an->eps,          \
                     an->sum_out, an->normed)
    if (hidden == 2048)
      MTPK_CN(1);
    else
      MTPK_CN(2);
#undef MTPK_CN
    return status_of(hipGetLastError());
  }
  const dim3 grid((unsigned)((hidden / 4 + 255) / 256), (unsigned)tokens);
  hipLaunchKernelGGL(tokens < kCombineWideTokens ? k_moe_combine<kCombineGroup> : k_moe_combine<4>,
                     grid, dim3(256), 0, st, y, ti, MTPK_I32, tw, MTPK_F32, top_k,
                     (int)hidden, expert_lo, expert_hi, out, MTPK_BF16, sh);
  return status_of(hipGetLastError());
}

}  // namespace

extern "C" {

int mtpk_moe_layer(const uint16_t* h, int64_t tokens, int64_t hidden, const uint16_t* router_gate,
                   int64_t router_rows, const uint16_t* shared_gate_up,
                   const uint16_t* shared_down, int64_t shared_inter, const uint8_t* gate_up,
                   const uint8_t* gate_up_scale, const uint8_t* down, const uint8_t* down_scale,
                   int64_t local_experts, int64_t inter_dim, int top_k, int expert_lo,
                   int expert_hi, float* top_w, int32_t* top_i, void* workspace,
                   int64_t workspace_bytes, void* out, void* stream) {
  if (!out) return MTPK_EINVAL;
  return moe_layer_run(h, tokens, hidden, router_gate, router_rows, shared_gate_up, shared_down,
                       shared_inter, gate_up, gate_up_scale, down, down_scale, local_experts,
                       inter_dim, top_k, expert_lo, expert_hi, top_w, top_i, workspace,
                       workspace_bytes, out, nullptr, stream);
}

int mtpk_moe_layer_add_norm(const uint16_t* h, int64_t tokens, int64_t hidden,
                            const uint16_t* router_gate, int64_t router_rows,
                            const uint16_t* shared_gate_up, const uint16_t* shared_down,
                            int64_t shared_inter, const uint8_t* gate_up,
                            const uint8_t* gate_up_scale, const uint8_t* down,
                            const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                            int top_k, int expert_lo, int expert_hi, float* top_w, int32_t* top_i,
                            void* workspace, int64_t workspace_bytes, const uint16_t* residual,
                            const uint16_t* norm_w, float eps, uint16_t* sum_out,
                            uint16_t* normed_out, void* stream) {
  if (!residual || !norm_w || !sum_out || !normed_out) return MTPK_EINVAL;
  if (tokens <= kDirectMaxTokens || (hidden != 2048 && hidden != 4096)) return MTPK_EINVAL;
  if (!aligned16(residual) || !aligned16(norm_w) || !aligned16(sum_out) || !aligned16(normed_out))
    return MTPK_EINVAL;
  const AddNorm an{residual, norm_w, eps, sum_out, normed_out};
  return moe_layer_run(h, tokens, hidden, router_gate, router_rows, shared_gate_up, shared_down,
                       shared_inter, gate_up, gate_up_scale, down, down_scale, local_experts,
                       inter_dim, top_k, expert_lo, expert_hi, top_w, top_i, workspace,
                       workspace_bytes, nullptr, &an, stream);
}

}  // extern "C"

// The static scratch of mtpk_fused_moe_static. In host code `g_moe_scratch` names a host-side
// stand-in, not device memory: its device address comes from hipGetSymbolAddress, taken once per
// device (with that device current) on the entry point's first call there, and only that address
// is ever passed to a kernel.
static __device__ __align__(256) uint8_t g_moe_scratch[MTPK_MOE_STATIC_SCRATCH];

namespace {

constexpr int kScratchDevices = 64;
std::once_flag g_scratch_once[kScratchDevices];
void* g_scratch_ptr[kScratchDevices];
hipError_t g_scratch_err[kScratchDevices];

// Device address of this device's g_moe_scratch, or null with *err set.
void* moe_scratch_of_current_device(int* err) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = status_of(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kScratchDevices) {
    *err = MTPK_ENODEV;
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(g_moe_scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
  });
  if (!g_scratch_ptr[dev]) {
    *err = g_scratch_err[dev] != hipSuccess ? status_of(g_scratch_err[dev]) : MTPK_ENODEV;
    return nullptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int mtpk_fused_moe_static(const void* x, int x_dtype, int64_t tokens, int64_t hidden,
                          const uint8_t* gate_up, const uint8_t* gate_up_scale, const uint8_t* down,
                          const uint8_t* down_scale, int64_t local_experts, int64_t inter_dim,
                          const void* a_expert, int expert_dtype, const void* a_weight,
                          int weight_dtype, int top_k, int expert_lo, int expert_hi,
                          const void* shared, int shared_dtype, const void* shared_gate,
                          int gate_dtype, int64_t gate_stride, void* out, void* stream) {
  if (tokens < 0 || top_k <= 0 || top_k > MTPK_MAX_TOP_K || local_experts <= 0 || inter_dim <= 0 ||
      hidden <= 0 || !dtype_float_ok(x_dtype))
    return MTPK_EINVAL;
  const int64_t need =
      mtpk_moe_workspace_bytes(tokens, top_k, local_experts, inter_dim, hidden, x_dtype);
  if (need > MTPK_MOE_STATIC_SCRATCH) return MTPK_ETOOBIG;
  int err = 0;
  void* scratch = moe_scratch_of_current_device(&err);
  if (!scratch) return err;
  return mtpk_fused_moe_shared(x, x_dtype, tokens, hidden, gate_up, gate_up_scale, down, down_scale,
                               local_experts, inter_dim, a_expert, expert_dtype, a_weight,
                               weight_dtype, top_k, expert_lo, expert_hi, shared, shared_dtype,
                               shared_gate, gate_dtype, gate_stride, scratch,
                               MTPK_MOE_STATIC_SCRATCH, out, stream);
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

int mtpk_scale_scan(const uint8_t* packed, const uint8_t* scale, int64_t blocks,
                    int32_t* bad_count, void* stream) {
  if (!packed || !scale || !bad_count || blocks < 0) return MTPK_EINVAL;
  const hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_zero_i32, dim3(1), dim3(1), 0, st, bad_count);
  if (blocks > 0) {
    const int vec = aligned16(scale) ? 1 : 0;
    const int64_t work = vec ? blocks / 16 + 16 : blocks;
    const int64_t wgs = (work + 255) / 256;
    const int grid = (int)(wgs < 8192 ? wgs : 8192);
    hipLaunchKernelGGL(k_scale_scan, dim3(grid), dim3(256), 0, st, packed, scale, blocks, vec,
                       bad_count);
  }
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
