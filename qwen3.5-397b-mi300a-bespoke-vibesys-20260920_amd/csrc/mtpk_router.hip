// Fused router for gfx950: softmax over the expert logits, top-k, renormalise. One wave per
// token row; the row's logits live in registers (PER per lane, expert e at lane e % 64, slot
// e / 64).
//
// Selection ranks by logit: softmax is strictly increasing in it, so this is the probability
// order of the exact softmax, with equal logits broken by the lower index (first occurrence).
// Each lane keeps the best of its free slots (the lowest slot among equal logits, i.e. its lowest
// index); a round takes the wave maximum of those keys with DPP (row shifts, then the row
// broadcasts: no LDS round trips), finds the lanes holding it with one ballot and, on a tie
// between lanes, the lowest index with a second DPP reduction; only the winning lane rescans its
// slots. Weights: the reference's arithmetic (router_fused.py:85-107), p = exp(l - max) / S with
// S the sum over every expert's exp(l - max), then each selected p divided by the sum of the
// selected p accumulated in selection order.

#include "mtpk_device.h"
#include "mtpk_gemm_tile.h"
#include "mtpk_host.h"
#include "mtpk_layer.h"

namespace mtpk {

// Wave-wide reductions to lane 63 by DPP (gfx9 row_shr 1, 2, 4, 8 inside each 16-lane row, then
// row_bcast 15 into rows 1 and 3 and row_bcast 31 into rows 2 and 3), read back as a uniform
// value. `id` is the operation's identity, taken by lanes whose DPP source lies outside the row.
template <typename Op>
__device__ inline uint32_t dpp_reduce(uint32_t v, uint32_t id, Op op) {
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, 0x111, 0xf, 0xf, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, 0x112, 0xf, 0xf, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, 0x114, 0xf, 0xf, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, 0x118, 0xf, 0xf, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, 0x142, 0xa, 0xf, false));
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, 0x143, 0xc, 0xf, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ inline uint32_t dpp_max_u32(uint32_t v) {
  return dpp_reduce(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ inline uint32_t dpp_min_u32(uint32_t v) {
  return dpp_reduce(v, 0xffffffffu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ inline float dpp_max_f32(float v) {
  return bits_f32(dpp_reduce(f32_bits(v), f32_bits(-INFINITY),
                             [](uint32_t a, uint32_t b) { return f32_bits(fmaxf(bits_f32(a), bits_f32(b))); }));
}

__device__ inline float dpp_sum_f32(float v) {
  return bits_f32(dpp_reduce(f32_bits(v), 0u,
                             [](uint32_t a, uint32_t b) { return f32_bits(bits_f32(a) + bits_f32(b)); }));
}

// The row's logits in registers: lane l holds logits l + 64 j (j < PER). Every lane issues its
// loads at once, and loads past E return zeros (unused) without a branch around them.
template <int PER, bool BF16>
__device__ inline void load_logits_row(const void* __restrict__ routing, int64_t stride, int row,
                                       int E, int lane, float (&lg)[PER]) {
  constexpr int elt = BF16 ? 2 : 4;
  const rsrc_t r = make_rsrc(static_cast<const uint8_t*>(routing) + (int64_t)row * stride * elt,
                             (uint32_t)(E * elt));
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t off = (uint32_t)((lane + kWave * j) * elt);
    lg[j] = BF16 ? bf16_to_f32((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0))
                 : bits_f32(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
  }
}

// The same row as the split-K GEMM leaves it: KS fp32 partial planes [KS, rows, cols], summed in
// split order and rounded to bf16, i.e. the bf16 logits the GEMM's reduction would store. Also
// returns column E (the shared expert's gate logit, when the row has one) summed the same way
// and not rounded; its loads travel with the row's.
template <int PER>
__device__ inline float load_logits_partials(const float* __restrict__ part, int KS, int rows,
                                             int cols, int row, int E, int lane, float (&lg)[PER]) {
  float acc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) acc[j] = 0.f;
  // four planes' loads in flight at once, then summed in split order
  constexpr int kPlanes = 4;
  const bool extra = E < cols;
  float ge = 0.f;
  for (int k0 = 0; k0 < KS; k0 += kPlanes) {
    float v[kPlanes][PER], ve[kPlanes];
#pragma unroll
    for (int i = 0; i < kPlanes; ++i) {
      const bool in = k0 + i < KS;
      const rsrc_t r = make_rsrc(part + ((int64_t)(in ? k0 + i : 0) * rows + row) * cols,
                                 (uint32_t)((E + (extra ? 1 : 0)) * 4));
#pragma unroll
      for (int j = 0; j < PER; ++j)
        v[i][j] = bits_f32(__builtin_amdgcn_raw_buffer_load_b32(
            r, (int)(in && lane + kWave * j < E ? (uint32_t)((lane + kWave * j) * 4) : kOutOfRange), 0, 0));
      ve[i] = bits_f32(__builtin_amdgcn_raw_buffer_load_b32(
          r, (int)(in && extra ? (uint32_t)(E * 4) : kOutOfRange), 0, 0));
    }
#pragma unroll
    for (int i = 0; i < kPlanes; ++i)
      if (k0 + i < KS) {
#pragma unroll
        for (int j = 0; j < PER; ++j) acc[j] += v[i][j];
        ge += ve[i];
      }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) lg[j] = bf16_to_f32(f32_to_bf16(acc[j]));
  return ge;
}

// softmax -> top-k -> renormalise of one row whose logits lane l holds at slots j (expert
// l + 64 j), written to row `row` of top_w / top_i. Runs on a whole wave (the DPP reductions).
template <int PER>
__device__ inline void route_row(float (&lg)[PER], int row, int E, int top_k, int lane,
                                 float* __restrict__ top_w, void* __restrict__ top_i, int idt) {
  float e_[PER];
  uint32_t key[PER];  // order key of a free slot (>= 1), 0 once taken or past E
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const bool in = lane + kWave * j < E;
    lg[j] = in ? lg[j] : -INFINITY;
    m = fmaxf(m, lg[j]);
  }
  m = dpp_max_f32(m);
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const bool in = lane + kWave * j < E;
    e_[j] = in ? __expf(lg[j] - m) : 0.f;
    part += e_[j];
    // a key of 0 marks "no candidate"; only NaNs with every payload bit set map below 1
    key[j] = in ? max(f32_order_key(lg[j]), 1u) : 0u;
  }
  // the softmax probabilities p = e / S; a selected p is then divided by the selected p's sum
  const float denom = dpp_sum_f32(part);
#pragma unroll
  for (int j = 0; j < PER; ++j) e_[j] = e_[j] / denom;

  // this lane's best free slot: strictly larger keys only, so the lowest slot wins a tie
  uint32_t bk = 0;
  int bj = 0;
  float bp = 0.f;
  auto rescan = [&]() {
    bk = 0;
    bj = 0;
    bp = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (key[j] > bk) {
        bk = key[j];
        bj = j;
        bp = e_[j];
      }
  };
  rescan();
  float my_w = 0.f, total = 0.f;
  int my_i = 0;
  for (int r = 0; r < top_k; ++r) {
    const uint32_t mk = dpp_max_u32(bk);
    const uint64_t holders = __ballot(bk == mk);
    int owner, sel;
    if (__popcll(holders) == 1) {
      owner = __ffsll((unsigned long long)holders) - 1;
      sel = owner + kWave * __builtin_amdgcn_readlane(bj, owner);
    } else {  // equal logits on several lanes: the lowest expert index
      sel = (int)dpp_min_u32(bk == mk ? (uint32_t)(lane + kWave * bj) : 0xffffffffu);
      owner = sel & (kWave - 1);
    }
    const float ps = bits_f32((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(bp), owner));
    if (lane == owner) {
      const int slot = sel / kWave;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (j == slot) key[j] = 0u;
      rescan();
    }
    total += ps;
    if (lane == r) {
      my_w = ps;
      my_i = sel;
    }
  }
  if (lane < top_k) {
    top_w[(int64_t)row * top_k + lane] = my_w / total;
    store_index(top_i, idt, (int64_t)row * top_k + lane, my_i);
  }
}

template <int PER, bool BF16>
__global__ __launch_bounds__(256) void k_route_topk(const void* __restrict__ routing,
                                                    int64_t stride, int tokens, int E, int top_k,
                                                    float* __restrict__ top_w,
                                                    void* __restrict__ top_i, int idt) {
  const int row = uniform(blockIdx.x * 4 + (threadIdx.x / kWave));  // per wave: resources in SGPRs
  const int lane = threadIdx.x & (kWave - 1);
  if (row >= tokens) return;  // uniform over the wave: every DPP below runs with all lanes
  float lg[PER];
  load_logits_row<PER, BF16>(routing, stride, row, E, lane, lg);
  route_row<PER>(lg, row, E, top_k, lane, top_w, top_i, idt);
}

// The MoE layer's second launch (after the router and shared gate_up GEMM tiles have left their
// split-K partials): workgroups [0, route_blocks) route four token rows each from the router's
// partials and store the shared gate's logit (column E) rounded to bf16; the others finish the
// shared expert's gate_up, act[m, j] = bf16(silu(gate) * up) from its partials, 256 values each.
// Both halves reproduce the bits of the GEMM's own reduction launch.
template <int PER>
__global__ __launch_bounds__(256) void k_route_act(RouteActArgs a) {
  if ((int)blockIdx.x < a.route_blocks) {
    const int row = uniform(blockIdx.x * 4 + (threadIdx.x / kWave));  // per wave: resources in SGPRs
    const int lane = threadIdx.x & (kWave - 1);
    if (row >= a.rows) return;  // uniform over the wave
    float lg[PER];
    const float g = load_logits_partials<PER>(a.rpart, a.rks, a.rows, a.rcols, row, a.E, lane, lg);
    if (a.sgate && lane == 0) a.sgate[row] = f32_to_bf16(g);
    route_row<PER>(lg, row, a.E, a.top_k, lane, a.top_w, a.top_i, a.idt);
    return;
  }
  const int64_t idx = (int64_t)(blockIdx.x - a.route_blocks) * 256 + threadIdx.x;
  if (idx >= (int64_t)a.rows * a.scols) return;
  const int64_t m = idx / a.scols, col = idx - m * a.scols;
  a.act[idx] = f32_to_bf16(gemm_reduce_value(a.spart, a.sks, a.rows, a.scols, kEpiSilu, m, col));
}

int launch_route_act(const RouteActArgs& a, hipStream_t st) {
  RouteActArgs b = a;
  b.route_blocks = (a.rows + 3) / 4;
  const int64_t act_blocks = ((int64_t)a.rows * a.scols + 255) / 256;
  const unsigned grid = (unsigned)(b.route_blocks + act_blocks);
  const int per = (a.E + kWave - 1) / kWave;
  if (per <= 4)
    hipLaunchKernelGGL(k_route_act<4>, dim3(grid), dim3(256), 0, st, b);
  else if (per <= 8)
    hipLaunchKernelGGL(k_route_act<8>, dim3(grid), dim3(256), 0, st, b);
  else
    hipLaunchKernelGGL(k_route_act<16>, dim3(grid), dim3(256), 0, st, b);
  return status_of(hipGetLastError());
}

template <int PER>
int launch_route(const void* routing, int rdt, int64_t tokens, int64_t stride, int E, int top_k,
                 float* top_w, void* top_i, int idt, hipStream_t st) {
  const unsigned grid = (unsigned)((tokens + 3) / 4);
  if (rdt == MTPK_BF16)
    hipLaunchKernelGGL((k_route_topk<PER, true>), dim3(grid), dim3(256), 0, st, routing, stride,
                       (int)tokens, E, top_k, top_w, top_i, idt);
  else
    hipLaunchKernelGGL((k_route_topk<PER, false>), dim3(grid), dim3(256), 0, st, routing, stride,
                       (int)tokens, E, top_k, top_w, top_i, idt);
  return status_of(hipGetLastError());
}

}  // namespace mtpk

using namespace mtpk;

extern "C" int mtpk_route_topk(const void* routing, int routing_dtype, int64_t tokens,
                               int64_t row_stride, int experts_out, int top_k, float* top_w,
                               void* top_i, int index_dtype, void* stream) {
  if (!routing || !top_w || !top_i) return MTPK_EINVAL;
  if (routing_dtype != MTPK_F32 && routing_dtype != MTPK_BF16) return MTPK_EINVAL;
  if (index_dtype != MTPK_I32 && index_dtype != MTPK_I64) return MTPK_EINVAL;
  if (experts_out <= 0 || experts_out > MTPK_MAX_ROUTER_EXPERTS) return MTPK_EINVAL;
  if (top_k <= 0 || top_k > MTPK_MAX_TOP_K || top_k > experts_out) return MTPK_EINVAL;
  if (tokens < 0 || tokens > ((int64_t)1 << 30) || row_stride < experts_out) return MTPK_EINVAL;
  if (tokens == 0) return 0;
  const hipStream_t st = (hipStream_t)stream;
  const int per = (experts_out + kWave - 1) / kWave;
  if (per <= 1)
    return launch_route<1>(routing, routing_dtype, tokens, row_stride, experts_out, top_k, top_w,
                           top_i, index_dtype, st);
  if (per <= 2)
    return launch_route<2>(routing, routing_dtype, tokens, row_stride, experts_out, top_k, top_w,
                           top_i, index_dtype, st);
  if (per <= 4)
    return launch_route<4>(routing, routing_dtype, tokens, row_stride, experts_out, top_k, top_w,
                           top_i, index_dtype, st);
  if (per <= 8)
    return launch_route<8>(routing, routing_dtype, tokens, row_stride, experts_out, top_k, top_w,
                           top_i, index_dtype, st);
  return launch_route<16>(routing, routing_dtype, tokens, row_stride, experts_out, top_k, top_w,
                          top_i, index_dtype, st);
}
