// Fused router for gfx950: softmax over the expert logits, top-k, renormalise. One wave per
// token row; the row's logits live in registers (PER per lane), the k selection rounds are
// 64-bit wave max reductions over (logit, index) keys.
//
// Selection ranks by logit: softmax is strictly increasing in it, so this is the probability
// order of the exact softmax, with equal logits broken by the lower index (first occurrence).
// Weights follow the reference arithmetic (router_fused.py:85-107): p = exp(l - max) / sum,
// then each selected p divided by the sum of the selected ones, accumulated in selection order.

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

template <int PER>
__global__ __launch_bounds__(256) void k_route_topk(const void* __restrict__ routing, int rdt,
                                                    int64_t stride, int tokens, int E, int top_k,
                                                    float* __restrict__ top_w,
                                                    void* __restrict__ top_i, int idt) {
  const int row = blockIdx.x * 4 + (threadIdx.x / kWave);
  const int lane = threadIdx.x & (kWave - 1);
  if (row >= tokens) return;
  float lg[PER], p[PER];
  bool free_[PER];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + kWave * j;
    lg[j] = e < E ? load_float(routing, rdt, (int64_t)row * stride + e) : -INFINITY;
    free_[j] = e < E;
    m = fmaxf(m, lg[j]);
  }
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    p[j] = free_[j] ? __expf(lg[j] - m) : 0.f;
    s += p[j];
  }
  s = wave_sum(s);
#pragma unroll
  for (int j = 0; j < PER; ++j) p[j] = p[j] / s;

  float my_w = 0.f, total = 0.f;
  int my_i = 0;
  for (int r = 0; r < top_k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const uint64_t key = free_[j] ? argmax_key(lg[j], (uint32_t)(lane + kWave * j)) : 0ull;
      best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    const int sel = (int)argmax_key_index(best);
    const int owner = sel & (kWave - 1), slot = sel / kWave;
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (j == slot) {
        ps = p[j];
        if (lane == owner) free_[j] = false;
      }
    }
    ps = __shfl(ps, owner, kWave);
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

template <int PER>
int launch_route(const void* routing, int rdt, int64_t tokens, int64_t stride, int E, int top_k,
                 float* top_w, void* top_i, int idt, hipStream_t st) {
  const unsigned grid = (unsigned)((tokens + 3) / 4);
  hipLaunchKernelGGL(k_route_topk<PER>, dim3(grid), dim3(256), 0, st, routing, rdt, stride,
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
