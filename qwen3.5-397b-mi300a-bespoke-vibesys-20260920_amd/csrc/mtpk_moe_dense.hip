// Routed bf16 experts for gfx950: the MTP draft layer of the real checkpoint, whose experts are
// dense bf16 while the target layers' are MXFP4 (`mtp_dense_moe.grouped_moe`,
// mtp_dense_moe.py:642-745, and its prep / gate_up / down / combine kernels).
//
// The work list and the combine are the MXFP4 MoE's: mtpk_moe_prep sorts the live assignments
// (owned expert, nonzero weight) by expert into units of <= 16, and mtpk_moe_combine sums
// out[t] = sum_j w_j y[t k + j] in j order. Between them two weight-streaming kernels, one
// workgroup per (tile of 64 weight rows, unit); each reads its rows of the unit's expert once
// for all of the unit's tokens:
//   gate_up: A = the unit's token rows of x, B = gate rows r and up rows I + r of the expert;
//            inter[a, r] = silu(gate) * up, stored as two bf16 planes hi + lo (hi = truncation,
//            lo = the rounded remainder, 16 significant bits together).
//   down:    A = the unit's inter rows, both planes (one MFMA each), B = down rows r;
//            y[a, r] in f32.
// v_mfma_f32_16x16x32_bf16 with the MoE kernels' lane layout: lane (g, c) supplies K positions
// 8 g .. 8 g + 7 of each 32-K step for weight row c (B) and token slot c (A), and holds
// D[slot 4 g + i][row c]. The A rows are staged in LDS per 256-K chunk (double-buffered, one
// barrier per chunk); the weights stream through a ring of 8 steps of 16-byte buffer loads per
// lane and stream, with the expert's base in the buffer resource so that the in-expert offsets
// stay 32-bit. A workgroup whose unit is at or past n_units returns at once, so the grid depends
// only on the sizes (graph capturable).

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kDnKC = 256;                // K per staged chunk
constexpr int kDnSteps = kDnKC / 32;      // MFMA steps per chunk
constexpr int kDnRing = kDnSteps;         // ring depth: one chunk of steps (see mtpk_gemm.hip)
constexpr int kDnRow = kDnKC * 2 + 16;    // LDS bytes of one staged row (padded)
constexpr int kDnWaves = 4;
constexpr int kDnThreads = kDnWaves * kWave;
constexpr int kDnTile = 16 * kDnWaves;    // weight rows per workgroup

struct DenseMoeArgs {
  const uint16_t* a;  // gate_up: x bf16 [T, K]; down: inter planes bf16 [2, A, K]
  const uint16_t* w;  // expert weights bf16 [E, N, K]
  const int32_t* sorted;
  const int32_t* units;
  const int32_t* n_units;
  int64_t A;          // assignments
  int top_k;
  int T;              // tokens
  int N, K;           // weight rows per expert (gate_up 2I, down H), reduction dim
  int cols;           // output columns (I for gate_up, H for down)
  uint16_t* inter;    // gate_up output planes [2, A, I]
  float* y;           // down output [A, H]
};

template <bool GATE_UP>
__global__ __launch_bounds__(kDnThreads) void k_moe_dense(DenseMoeArgs a) {
  constexpr int P = GATE_UP ? 1 : 2;  // A-operand planes
  constexpr int S = GATE_UP ? 2 : 1;  // weight streams (gate and up rows)
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][P][16 * kDnRow];
  const int unit = blockIdx.y;
  if (unit >= sload(a.n_units, 0)) return;
  const int e = sload(a.units, 3 * unit), first = sload(a.units, 3 * unit + 1);
  const int cnt = sload(a.units, 3 * unit + 2);
  const int tid = threadIdx.x, wave = uniform(tid / kWave), lane = tid & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int r0 = blockIdx.x * kDnTile + 16 * wave + ln.c;  // this lane's weight row / column
  const bool rok = r0 < a.cols;
  const int nchunk = a.K / kDnKC;

  const rsrc_t rw = make_rsrc(a.w + (int64_t)e * a.N * a.K, (uint32_t)((int64_t)a.N * a.K * 2));
  const uint32_t wbase[2] = {
      (uint32_t)((int64_t)r0 * a.K * 2),
      (uint32_t)((int64_t)(r0 + (S > 1 ? a.N / 2 : 0)) * a.K * 2)};
  auto issue = [&](u32x4_t* v, int st) {
    const bool in = rok && st < nchunk * kDnSteps;
#pragma unroll
    for (int s = 0; s < S; ++s)
      v[s] = buf16(rw, in ? wbase[s] + (uint32_t)((32 * st + 8 * ln.g) * 2) : kOutOfRange);
  };

  // Staging: piece j of a plane moves 16 bytes of slot row (256 j + tid) / 32, column
  // (tid % 32) * 16. The slot's source row is fixed for the workgroup.
  const int64_t a_bytes = GATE_UP ? (int64_t)a.T * a.K * 2 : 2 * a.A * a.K * 2;
  const rsrc_t ra = make_rsrc(a.a, (uint32_t)a_bytes);
  uint32_t src[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = (j * kDnThreads + tid) >> 5;
    if (m < cnt) {
      const int aid = a.sorted[first + m];
      const int64_t row = GATE_UP ? aid / a.top_k : aid;
      src[j] = (uint32_t)((row * a.K + (tid & 31) * 8) * 2);
    } else {
      src[j] = kOutOfRange;
    }
  }
  const uint32_t plane_bytes = (uint32_t)(a.A * a.K * 2);
  u32x4_t sreg[P][2];
  auto stage_load = [&](int c) {
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bool ok = c < nchunk && src[j] != kOutOfRange;
        sreg[p][j] = buf16(ra, ok ? src[j] + p * plane_bytes + (uint32_t)(c * kDnKC * 2) : kOutOfRange);
      }
  };
  auto stage_store = [&](int b) {
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int q = j * kDnThreads + tid;
        lds16_store(&xs[b][p][(q >> 5) * kDnRow + (q & 31) * 16], sreg[p][j]);
      }
  };

  f32x4_t acc[S];
#pragma unroll
  for (int s = 0; s < S; ++s) acc[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  stage_load(0);
  ring_fence();
  u32x4_t ring[kDnRing][S];
#pragma unroll
  for (int st = 0; st < kDnRing; ++st) issue(ring[st], st);
  ring_fence();
  stage_store(0);
  stage_load(1);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the LDS stores, not the buffer loads
  __syncthreads();
  int c = 0;
#pragma clang loop unroll(disable)
  do {
    // the next step's staged A rows read before this step's MFMAs, so their LDS latency does
    // not sit between the MFMAs and the ring refill (813 -> 811 us at 48 rows, Zipf)
    u32x4_t av[P];
#pragma unroll
    for (int p = 0; p < P; ++p) av[p] = lds16(&xs[c & 1][p][ln.c * kDnRow + (8 * ln.g) * 2]);
#pragma unroll
    for (int st = 0; st < kDnSteps; ++st) {
      u32x4_t an[P];
      if (st + 1 < kDnSteps) {
#pragma unroll
        for (int p = 0; p < P; ++p)
          an[p] = lds16(&xs[c & 1][p][ln.c * kDnRow + (32 * (st + 1) + 8 * ln.g) * 2]);
      }
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int p = 0; p < P; ++p)
          acc[s] = mfma16x16x32(as_bf16x8(av[p]), as_bf16x8(ring[st][s]), acc[s]);
      ring_fence();
      issue(ring[st], c * kDnSteps + st + kDnRing);
      ring_fence();
      if (st + 1 < kDnSteps) {
#pragma unroll
        for (int p = 0; p < P; ++p) av[p] = an[p];
      }
    }
    if (c + 1 < nchunk) stage_store((c + 1) & 1);
    stage_load(c + 2);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __syncthreads();
  } while (++c < nchunk);

  if (!rok) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * ln.g + i;
    if (m >= cnt) continue;
    const int64_t aid = a.sorted[first + m];
    if (GATE_UP) {
      const float g = acc[0][i];
      const float v = g / (1.f + __expf(-g)) * acc[S - 1][i];
      uint16_t hi, lo;
      split_bf16(v, &hi, &lo);
      a.inter[aid * a.cols + r0] = hi;
      a.inter[(a.A + aid) * a.cols + r0] = lo;
    } else {
      a.y[aid * a.cols + r0] = acc[0][i];
    }
  }
}

struct DenseLayout {
  int64_t A, max_units;
  int64_t sorted, units, n_units, inter, y, total;  // byte offsets into the workspace
};

DenseLayout dense_layout(int64_t tokens, int64_t top_k, int64_t experts, int64_t inter,
                         int64_t hidden) {
  DenseLayout l{};
  l.A = tokens * top_k;
  l.max_units = mtpk_moe_max_units(l.A, experts);
  int64_t at = 0;
  l.sorted = at;
  at += align256(l.A * 4);
  l.units = at;
  at += align256(3 * l.max_units * 4);
  l.n_units = at;
  at += 256;
  l.inter = at;
  at += align256(2 * l.A * inter * 2);
  l.y = at;
  at += align256(l.A * hidden * 4);
  l.total = at;
  return l;
}

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int64_t mtpk_moe_dense_workspace_bytes(int64_t tokens, int64_t top_k, int64_t local_experts,
                                       int64_t inter, int64_t hidden) {
  if (tokens <= 0 || top_k <= 0 || local_experts <= 0 || inter <= 0 || hidden <= 0) return 256;
  return dense_layout(tokens, top_k, local_experts, inter, hidden).total;
}

int mtpk_moe_dense(const uint16_t* x, int64_t tokens, int64_t hidden, const uint16_t* gate_up,
                   const uint16_t* down, int64_t local_experts, int64_t inter_dim,
                   const void* a_expert, int expert_dtype, const void* a_weight, int weight_dtype,
                   int top_k, int expert_lo, int expert_hi, void* workspace,
                   int64_t workspace_bytes, uint16_t* out, void* stream) {
  if (!x || !gate_up || !down || !a_expert || !a_weight || !workspace || !out) return MTPK_EINVAL;
  if (tokens < 0 || top_k < 1 || local_experts < 1 || expert_hi - expert_lo != local_experts)
    return MTPK_EINVAL;
  if (hidden <= 0 || inter_dim <= 0 || hidden % kDnKC || inter_dim % kDnKC) return MTPK_EINVAL;
  if (!aligned16(x) || !aligned16(gate_up) || !aligned16(down) || !aligned16(out) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255))
    return MTPK_EINVAL;
  const int64_t A = tokens * top_k;
  // 32-bit buffer offsets: one expert's weights, x, the intermediate planes
  if (2 * inter_dim * hidden * 2 > 0x7fffffffLL || tokens * hidden * 2 > 0x7fffffffLL ||
      2 * A * inter_dim * 2 > 0x7fffffffLL || A > INT32_MAX / 4)
    return MTPK_EINVAL;
  if (tokens == 0) return 0;
  const DenseLayout l = dense_layout(tokens, top_k, local_experts, inter_dim, hidden);
  if (workspace_bytes < l.total || l.max_units > 65535) return MTPK_EINVAL;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + l.sorted);
  int32_t* units = reinterpret_cast<int32_t*>(ws + l.units);
  int32_t* n_units = reinterpret_cast<int32_t*>(ws + l.n_units);
  uint16_t* inter = reinterpret_cast<uint16_t*>(ws + l.inter);
  float* y = reinterpret_cast<float*>(ws + l.y);
  int rc = mtpk_moe_prep(a_expert, expert_dtype, a_weight, weight_dtype, A, expert_lo, expert_hi,
                         sorted, units, l.max_units, n_units, stream);
  if (rc) return rc;
  const hipStream_t st = (hipStream_t)stream;
  DenseMoeArgs g{x, gate_up, sorted, units, n_units, A, top_k, (int)tokens, (int)(2 * inter_dim),
                 (int)hidden, (int)inter_dim, inter, nullptr};
  hipLaunchKernelGGL(k_moe_dense<true>,
                     dim3((unsigned)((inter_dim + kDnTile - 1) / kDnTile), (unsigned)l.max_units),
                     dim3(kDnThreads), 0, st, g);
  if ((rc = status_of(hipGetLastError()))) return rc;
  DenseMoeArgs d{inter, down, sorted, units, n_units, A, top_k, (int)tokens, (int)hidden,
                 (int)inter_dim, (int)hidden, nullptr, y};
  hipLaunchKernelGGL(k_moe_dense<false>,
                     dim3((unsigned)((hidden + kDnTile - 1) / kDnTile), (unsigned)l.max_units),
                     dim3(kDnThreads), 0, st, d);
  if ((rc = status_of(hipGetLastError()))) return rc;
  return mtpk_moe_combine(y, a_expert, expert_dtype, a_weight, weight_dtype, tokens, top_k, hidden,
                          expert_lo, expert_hi, out, MTPK_BF16, stream);
}

}  // extern "C"
