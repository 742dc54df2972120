// Speculative rejection sampling and temperature sampling over the vocabulary, for gfx950.
//
// Method (Leviathan, Kalman & Matias 2023, Alg. 1; Chen et al. 2023): with p_i =
// softmax(target_i / T) and q_i = softmax(draft_i / T), draft token x_i is accepted iff
// u_i * q_i(x_i) <= p_i(x_i); at the first rejection i a token is drawn from
// norm(max(0, p_i - q_i)) (from p_i if that residual is all zero), and if all k drafts are
// accepted the bonus token is drawn from p_k. A draw from weights w with uniform r is the
// smallest index v with cumsum(w)[v] > r * sum(w), or the last positive index if rounding
// leaves none.
//
// Three launches for rejection (four for plain sampling), streaming the logits with 16-byte loads:
//   stats : (chunk, row) workgroups -> per-chunk (max, sum exp(z - max)) of z = logit / T
//   decide + mass: (chunk, lane) workgroups; each first makes its lane's decision (a wave per
//           verify row -> row softmax constants, margins, the accept length and the draw), then
//           sums its chunk's draw weights. Plain sampling: a wave per row for the row constants,
//           then (chunk, row) workgroups for the mass
//   pick  : one workgroup per item -> the chunk where the cumulative mass crosses r * total
//           (one wave: scan and ballot over the chunk masses), then a block scan inside it;
//           writes the token (and the emitted row)
// Every sum runs in a fixed order, so results are deterministic for fixed shapes.

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kRsThreads = 256;
constexpr int kRsPerThread = 16;
constexpr int kRsChunk = kRsThreads * kRsPerThread;  // 4096 logits per workgroup

// One draw: weights from target row `trow` (and draft row `drow` for a residual, else -1).
struct RsItem {
  int trow, drow, a, pad;
  float mt, st, mq, sq;
};

struct RsRows {
  const void* target;
  const void* draft;
  int dt;
  int64_t vocab;
  int vec;  // 16-byte vector loads allowed
};

// The 16 logits of thread `tid` in chunk `c` of a row, scaled by 1/T; invalid slots -> -inf.
__device__ inline void rs_load(const void* base, int dt, int vec, int64_t row, int64_t vocab, int c,
                               int tid, float inv_t, float (&z)[kRsPerThread]) {
  const int64_t i0 = (int64_t)c * kRsChunk + (int64_t)tid * kRsPerThread;
  if (vec && i0 + kRsPerThread <= vocab) {
    if (dt == MTPK_BF16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(base) + row * vocab + i0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4_t v = ld16(p + 8 * h);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          z[8 * h + 2 * q] = bf16_to_f32((uint16_t)(v[q] & 0xffffu)) * inv_t;
          z[8 * h + 2 * q + 1] = bf16_to_f32((uint16_t)(v[q] >> 16)) * inv_t;
        }
      }
    } else {
      const float* p = reinterpret_cast<const float*>(base) + row * vocab + i0;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const u32x4_t v = ld16(p + 4 * h);
#pragma unroll
        for (int q = 0; q < 4; ++q) z[4 * h + q] = bits_f32(v[q]) * inv_t;
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) {
    const int64_t i = i0 + e;
    z[e] = i < vocab ? load_float(base, dt, row * vocab + i) * inv_t : -INFINITY;
  }
}

// Block-wide reductions over 256 threads (4 waves), result broadcast to every thread.
__device__ inline float block_max(float v, float* red) {
  v = wave_max(v);
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ inline float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int tid = threadIdx.x;
  __syncthreads();
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// rows [0, n_target) are target rows, [n_target, n_target + n_draft) draft rows.
__global__ __launch_bounds__(kRsThreads) void k_rs_stats(RsRows rr, int64_t n_target, float inv_t,
                                                        float2* __restrict__ part) {
  __shared__ float red[kRsThreads / kWave];
  const int c = blockIdx.x, nchunk = gridDim.x;
  const int64_t r = blockIdx.y;
  const bool is_t = r < n_target;
  const void* base = is_t ? rr.target : rr.draft;
  const int64_t row = is_t ? r : r - n_target;
  float z[kRsPerThread];
  rs_load(base, rr.dt, rr.vec, row, rr.vocab, c, threadIdx.x, inv_t, z);
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) m = fmaxf(m, z[e]);
  m = block_max(m, red);
  // A chunk of -inf logits (a masked stretch of the vocabulary) has no mass: (-inf, 0), not the
  // NaN of exp(-inf - -inf). m is uniform over the workgroup, so is the branch.
  float s = 0.f;
  if (m > -INFINITY) {
#pragma unroll
    for (int e = 0; e < kRsPerThread; ++e) s += __expf(z[e] - m);
  }
  s = block_sum(s, red);
  if (threadIdx.x == 0) part[r * nchunk + c] = make_float2(m, s);
}

// A chunk partial's share of a row sum with row max m; a massless (-inf) chunk adds nothing.
__device__ inline float rs_share(float2 v, float m) { return v.x > -INFINITY ? v.y * __expf(v.x - m) : 0.f; }

// A lane's first chunk partial of row r (chunk = lane), or the empty (-inf, 0).
__device__ inline float2 rs_first_partial(const float2* part, int64_t r, int nchunk) {
  const int lane = threadIdx.x & (kWave - 1);
  return lane < nchunk ? part[r * nchunk + lane] : make_float2(-INFINITY, 0.f);
}

// Combine a row's chunk partials (one wave): max M and sum S of exp(z - M). v0 is the lane's
// first partial (rs_first_partial), loaded ahead by the caller so that its latency overlaps
// other loads.
__device__ inline float2 rs_row_stats(float2 v0, const float2* part, int64_t r, int nchunk) {
  const int lane = threadIdx.x & (kWave - 1);
  float m = v0.x;
  for (int c = lane + kWave; c < nchunk; c += kWave) m = fmaxf(m, part[r * nchunk + c].x);
  m = wave_max(m);
  float s = rs_share(v0, m);
  for (int c = lane + kWave; c < nchunk; c += kWave) s += rs_share(part[r * nchunk + c], m);
  return make_float2(m, wave_sum(s));
}

// Rejection decision for lane b by one workgroup of kDecideWaves waves: its waves take the t
// verify rows in parallel (row softmax constants and the margin p(x) - u q(x)), then the first
// negative margin is the accept length, and *s_item (LDS) the draw it leads to. Outputs are
// written only where the pointers are non-null.
constexpr int kDecideWaves = 4;
constexpr int kMaxT = 64;

__device__ void rs_decide_lane(const RsRows& rr, const float2* __restrict__ part, int nchunk, int B,
                               int k, float inv_t, const int64_t* __restrict__ draft_tokens,
                               const float* __restrict__ u_accept, int b, float* s_mg, float4* s_st,
                               RsItem* s_item, RsItem* __restrict__ items,
                               int64_t* __restrict__ accept_len, float* __restrict__ margin) {
  const int t = k + 1;
  const int wv = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int64_t n_target = (int64_t)B * t;
  for (int i = wv; i < t; i += kDecideWaves) {
    // The rows' chunk partials, then the token and its two logits: the partials do not depend
    // on the token, so their loads are in flight while the token's chain runs.
    const float2 pt = rs_first_partial(part, (int64_t)b * t + i, nchunk);
    const float2 pq = i < k ? rs_first_partial(part, n_target + (int64_t)b * k + i, nchunk)
                            : make_float2(-INFINITY, 0.f);
    const int64_t x = i < k ? draft_tokens[(int64_t)b * k + i] : -1;
    const float ua = i < k ? u_accept[(int64_t)b * k + i] : 0.f;
    const bool in_vocab = x >= 0 && x < rr.vocab;
    float lt = 0.f, lq = 0.f;
    if (in_vocab) {
      lt = load_float(rr.target, rr.dt, ((int64_t)b * t + i) * rr.vocab + x) * inv_t;
      lq = load_float(rr.draft, rr.dt, ((int64_t)b * k + i) * rr.vocab + x) * inv_t;
    }
    const float2 st = rs_row_stats(pt, part, (int64_t)b * t + i, nchunk);
    float2 sq = make_float2(0.f, 1.f);
    float mg = 0.f;
    if (i < k) {
      sq = rs_row_stats(pq, part, n_target + (int64_t)b * k + i, nchunk);
      if (in_vocab) {
        const float p = __expf(lt - st.x) / st.y, q = __expf(lq - sq.x) / sq.y;
        mg = p - ua * q;
      } else {
        mg = -1.f;  // a token outside the vocabulary is never accepted
      }
    }
    if (lane == 0) {
      s_mg[i] = mg;
      s_st[i] = make_float4(st.x, st.y, sq.x, sq.y);
      if (margin && i < k) margin[(int64_t)b * k + i] = mg;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int a = k;
    for (int i = 0; i < k; ++i)
      if (!(s_mg[i] >= 0.f)) {  // a NaN margin (a fully masked row) rejects too
        a = i;
        break;
      }
    const float4 sa = s_st[a];
    RsItem it;
    it.trow = b * t + a;
    it.drow = a < k ? b * k + a : -1;
    it.a = a;
    it.pad = 0;
    it.mt = sa.x;
    it.st = sa.y;
    it.mq = sa.z;
    it.sq = sa.w;
    *s_item = it;
    if (items) items[b] = it;
    if (accept_len) accept_len[b] = a;
  }
  __syncthreads();
}

// Plain sampling: item r draws from target row r.
__global__ __launch_bounds__(kWave) void k_rs_rows(const float2* __restrict__ part, int nchunk,
                                                  RsItem* __restrict__ items) {
  const int r = blockIdx.x;
  const float2 st = rs_row_stats(rs_first_partial(part, r, nchunk), part, r, nchunk);
  if (threadIdx.x == 0) {
    RsItem it;
    it.trow = r;
    it.drow = -1;
    it.a = 0;
    it.pad = 0;
    it.mt = st.x;
    it.st = st.y;
    it.mq = 0.f;
    it.sq = 1.f;
    items[r] = it;
  }
}

// Draw weights of this thread's 16 slots from the logits z (target) and zq (draft): target p,
// and the residual max(0, p - q) when the item has a draft row.
__device__ inline void rs_weights_of(const RsItem& it, const float (&z)[kRsPerThread],
                                     const float (&zq)[kRsPerThread], float (&wr)[kRsPerThread],
                                     float (&wp)[kRsPerThread]) {
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) wp[e] = __expf(z[e] - it.mt) / it.st;
  if (it.drow >= 0) {
#pragma unroll
    for (int e = 0; e < kRsPerThread; ++e) wr[e] = fmaxf(wp[e] - __expf(zq[e] - it.mq) / it.sq, 0.f);
  } else {
#pragma unroll
    for (int e = 0; e < kRsPerThread; ++e) wr[e] = 0.f;
  }
}

__device__ inline void rs_weights(const RsRows& rr, const RsItem& it, int c, float inv_t,
                                  float (&wr)[kRsPerThread], float (&wp)[kRsPerThread]) {
  float z[kRsPerThread], zq[kRsPerThread];
  rs_load(rr.target, rr.dt, rr.vec, it.trow, rr.vocab, c, threadIdx.x, inv_t, z);
  if (it.drow >= 0) rs_load(rr.draft, rr.dt, rr.vec, it.drow, rr.vocab, c, threadIdx.x, inv_t, zq);
  rs_weights_of(it, z, zq, wr, wp);
}

// Per-chunk sums of an item's draw weights, one workgroup per (chunk, item).
__global__ __launch_bounds__(kRsThreads) void k_rs_mass(RsRows rr, const RsItem* __restrict__ items,
                                                       int nchunk, float inv_t,
                                                       float2* __restrict__ mass) {
  __shared__ float2 red[kRsThreads / kWave];
  const int c = blockIdx.x;
  const int item = blockIdx.y;
  const RsItem it = items[item];
  float wr[kRsPerThread], wp[kRsPerThread];
  rs_weights(rr, it, c, inv_t, wr, wp);
  float sr = 0.f, sp = 0.f;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) {
    sr += wr[e];
    sp += wp[e];
  }
  sr = wave_sum(sr);
  sp = wave_sum(sp);
  const int tid = threadIdx.x;
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = make_float2(sr, sp);
  __syncthreads();
  if (tid == 0) {
    const float2 a = red[0], b = red[1], d = red[2], e = red[3];
    mass[(int64_t)item * nchunk + c] =
        make_float2((a.x + b.x) + (d.x + e.x), (a.y + b.y) + (d.y + e.y));
  }
}

// Rejection: the lane's decision and its draw's per-chunk mass in one launch, one workgroup per
// (chunk, lane). Every chunk's workgroup makes the lane's decision itself (a few KB of chunk
// partials and 2k logits, the same deterministic result in each), so no launch separates the
// decision from the mass; the chunk-0 workgroup writes the decision's outputs.
__global__ __launch_bounds__(kRsThreads) void k_rs_decide_mass(
    RsRows rr, const float2* __restrict__ part, int nchunk, int B, int k, float inv_t,
    const int64_t* __restrict__ draft_tokens, const float* __restrict__ u_accept,
    RsItem* __restrict__ items, int64_t* __restrict__ accept_len, float* __restrict__ margin,
    float2* __restrict__ mass) {
  static_assert(kRsThreads == kWave * kDecideWaves, "one decision per workgroup");
  __shared__ float s_mg[kMaxT];
  __shared__ float4 s_st[kMaxT];
  __shared__ RsItem s_item;
  __shared__ float2 red[kRsThreads / kWave];
  const int c = blockIdx.x, b = blockIdx.y;
  const bool first = c == 0;
  rs_decide_lane(rr, part, nchunk, B, k, inv_t, draft_tokens, u_accept, b, s_mg, s_st, &s_item,
                 first ? items : nullptr, first ? accept_len : nullptr, first ? margin : nullptr);
  const RsItem it = s_item;
  float wr[kRsPerThread], wp[kRsPerThread];
  rs_weights(rr, it, c, inv_t, wr, wp);
  float sr = 0.f, sp = 0.f;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) {
    sr += wr[e];
    sp += wp[e];
  }
  sr = wave_sum(sr);
  sp = wave_sum(sp);
  const int tid = threadIdx.x;
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = make_float2(sr, sp);
  __syncthreads();
  if (tid == 0) {
    const float2 a = red[0], b2 = red[1], d = red[2], e = red[3];
    mass[(int64_t)b * nchunk + c] =
        make_float2((a.x + b2.x) + (d.x + e.x), (a.y + b2.y) + (d.y + e.y));
  }
}

__device__ inline float wave_incl_scan_f(float v, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const float u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

__global__ __launch_bounds__(kRsThreads) void k_rs_pick(
    RsRows rr, const RsItem* __restrict__ items, const float2* __restrict__ mass, int nchunk,
    float inv_t, const float* __restrict__ u_sample, int64_t* __restrict__ token,
    const int64_t* __restrict__ draft_tokens, int k, int64_t* __restrict__ emitted) {
  __shared__ float wtot[kRsThreads / kWave];
  __shared__ int s_chunk, s_use_r, s_fallback, s_best;
  __shared__ float s_before, s_target;
  const int item = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  const RsItem it = items[item];
  const int64_t dtok = emitted && tid < k ? draft_tokens[(int64_t)item * k + tid] : 0;
  if (wv == 0) {
    // One wave finds the chunk where the cumulative mass crosses r * total: totals by a wave
    // sum, then 64 chunks at a time by an inclusive scan and a ballot.
    const float u = u_sample[item];
    const float2* row_mass = mass + (int64_t)item * nchunk;
    const float2 m0 = lane < nchunk ? row_mass[lane] : make_float2(0.f, 0.f);
    float tr = m0.x, tp = m0.y;
    for (int c = lane + kWave; c < nchunk; c += kWave) {
      const float2 m = row_mass[c];
      tr += m.x;
      tp += m.y;
    }
    tr = wave_sum(tr);
    tp = wave_sum(tp);
    const int use_r = it.drow >= 0 && tr > 0.f;
    const float target = u * (use_r ? tr : tp);
    float cum = 0.f;
    int chunk = -1, last_pos = 0;
    for (int g0 = 0; g0 < nchunk; g0 += kWave) {
      const int c = g0 + lane;
      float2 m = m0;
      if (g0 > 0) m = c < nchunk ? row_mass[c] : make_float2(0.f, 0.f);
      const float w = use_r ? m.x : m.y;
      const float inc = wave_incl_scan_f(w, lane);
      const uint64_t hit = __ballot(c < nchunk && cum + inc > target);
      if (hit) {
        const int f = __ffsll((long long)hit) - 1;
        chunk = g0 + f;
        cum += __shfl(inc - w, f, kWave);
        break;
      }
      const uint64_t positive = __ballot(w > 0.f);
      if (positive) last_pos = g0 + 63 - __clzll((long long)positive);
      cum += __shfl(inc, kWave - 1, kWave);
    }
    if (lane == 0) {
      s_fallback = chunk < 0;
      s_chunk = chunk < 0 ? last_pos : chunk;
      s_use_r = use_r;
      s_before = cum;
      s_target = target;
      s_best = INT32_MAX;
    }
  }
  __syncthreads();
  const int c = s_chunk;
  float wr[kRsPerThread], wp[kRsPerThread];
  rs_weights(rr, it, c, inv_t, wr, wp);
  float w[kRsPerThread];
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) w[e] = s_use_r ? wr[e] : wp[e];
  float mine = 0.f;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) mine += w[e];
  const float inc = wave_incl_scan_f(mine, lane);
  if (lane == kWave - 1) wtot[wv] = inc;
  __syncthreads();
  float off = s_before;
  for (int q = 0; q < wv; ++q) off += wtot[q];
  float run = off + inc - mine;
  const int64_t i0 = (int64_t)c * kRsChunk + (int64_t)tid * kRsPerThread;
  int hit = INT32_MAX, lastp = -1;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) {
    run += w[e];
    if (w[e] > 0.f) lastp = (int)(i0 + e);
    if (hit == INT32_MAX && !s_fallback && run > s_target && w[e] > 0.f) hit = (int)(i0 + e);
  }
  atomicMin(&s_best, hit);
  __syncthreads();
  // Rounding can leave no crossing inside the chunk: take the chunk's last positive slot.
  const int need_last = s_best == INT32_MAX;
  __syncthreads();
  if (need_last) {
    if (tid == 0) s_best = -1;
    __syncthreads();
    atomicMax(&s_best, lastp);
    __syncthreads();
  }
  // the emitted row by its first k + 1 threads at once (draft token i was loaded at the start)
  if (tid <= k) {
    const int64_t v = s_best < 0 ? 0 : s_best;
    if (tid == 0) token[item] = v;
    if (emitted) emitted[(int64_t)item * (k + 1) + tid] = tid < it.a ? dtok : v;
  }
}

int64_t rs_chunks(int64_t vocab) { return (vocab + kRsChunk - 1) / kRsChunk; }

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int64_t mtpk_rejection_workspace_bytes(int64_t batch, int k, int64_t vocab) {
  if (batch <= 0 || k < 0 || vocab <= 0) return 0;
  const int64_t nchunk = rs_chunks(vocab);
  const int64_t rows = batch * (2 * (int64_t)k + 1);
  return align256(rows * nchunk * (int64_t)sizeof(float2)) +
         align256(batch * (int64_t)sizeof(RsItem)) +
         align256(batch * nchunk * (int64_t)sizeof(float2));
}

int mtpk_rejection_sample(const void* target, const void* draft, int dtype, int64_t batch, int k,
                          int64_t vocab, const int64_t* draft_tokens, const float* u_accept,
                          const float* u_sample, float temperature, void* workspace,
                          int64_t workspace_bytes, int64_t* accept_len, int64_t* token,
                          int64_t* emitted, float* margin, void* stream) {
  if (!target || !u_sample || !workspace || !accept_len || !token) return MTPK_EINVAL;
  if (dtype != MTPK_F32 && dtype != MTPK_BF16) return MTPK_EINVAL;
  if (batch <= 0 || batch > 65535 || k < 0 || k > 63 || vocab <= 0 || vocab > INT32_MAX / 2)
    return MTPK_EINVAL;
  if (k > 0 && (!draft || !draft_tokens || !u_accept)) return MTPK_EINVAL;
  if (!(temperature > 0.f) || !(temperature < INFINITY)) return MTPK_EINVAL;
  if (workspace_bytes < mtpk_rejection_workspace_bytes(batch, k, vocab)) return MTPK_EINVAL;
  if (!aligned16(workspace)) return MTPK_EINVAL;
  const int64_t nchunk = rs_chunks(vocab);
  if (nchunk > 65535) return MTPK_EINVAL;
  const int t = k + 1;
  const int64_t rows = batch * (t + (int64_t)k);
  if (rows > 65535) return MTPK_EINVAL;
  const int per_vec = dtype == MTPK_BF16 ? 8 : 4;
  RsRows rr{target, draft, dtype, vocab,
            (int)(aligned16(target) && (k == 0 || aligned16(draft)) && vocab % per_vec == 0)};
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  float2* part = reinterpret_cast<float2*>(ws);
  ws += align256(batch * (2 * (int64_t)k + 1) * nchunk * (int64_t)sizeof(float2));
  RsItem* items = reinterpret_cast<RsItem*>(ws);
  ws += align256(batch * (int64_t)sizeof(RsItem));
  float2* mass = reinterpret_cast<float2*>(ws);
  const float inv_t = 1.f / temperature;
  const hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_rs_stats, dim3((unsigned)nchunk, (unsigned)rows), dim3(kRsThreads), 0, st,
                     rr, batch * t, inv_t, part);
  int rc = status_of(hipGetLastError());
  if (rc) return rc;
  hipLaunchKernelGGL(k_rs_decide_mass, dim3((unsigned)nchunk, (unsigned)batch), dim3(kRsThreads), 0,
                     st, rr, part, (int)nchunk, (int)batch, k, inv_t, draft_tokens, u_accept, items,
                     accept_len, margin, mass);
  if ((rc = status_of(hipGetLastError()))) return rc;
  hipLaunchKernelGGL(k_rs_pick, dim3((unsigned)batch), dim3(kRsThreads), 0, st, rr, items, mass,
                     (int)nchunk, inv_t, u_sample, token, draft_tokens, k, emitted);
  return status_of(hipGetLastError());
}

int64_t mtpk_sample_workspace_bytes(int64_t rows, int64_t vocab) {
  return mtpk_rejection_workspace_bytes(rows, 0, vocab);
}

int mtpk_sample_rows(const void* logits, int dtype, int64_t rows, int64_t vocab, float temperature,
                     const float* u, void* workspace, int64_t workspace_bytes, int64_t* token,
                     void* stream) {
  if (!logits || !u || !workspace || !token) return MTPK_EINVAL;
  if (dtype != MTPK_F32 && dtype != MTPK_BF16) return MTPK_EINVAL;
  if (rows <= 0 || rows > 65535 || vocab <= 0 || vocab > INT32_MAX / 2) return MTPK_EINVAL;
  if (!(temperature > 0.f) || !(temperature < INFINITY)) return MTPK_EINVAL;
  if (workspace_bytes < mtpk_sample_workspace_bytes(rows, vocab) || !aligned16(workspace))
    return MTPK_EINVAL;
  const int64_t nchunk = rs_chunks(vocab);
  if (nchunk > 65535) return MTPK_EINVAL;
  const int per_vec = dtype == MTPK_BF16 ? 8 : 4;
  RsRows rr{logits, nullptr, dtype, vocab, (int)(aligned16(logits) && vocab % per_vec == 0)};
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  float2* part = reinterpret_cast<float2*>(ws);
  ws += align256(rows * nchunk * (int64_t)sizeof(float2));
  RsItem* items = reinterpret_cast<RsItem*>(ws);
  ws += align256(rows * (int64_t)sizeof(RsItem));
  float2* mass = reinterpret_cast<float2*>(ws);
  const float inv_t = 1.f / temperature;
  const hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_rs_stats, dim3((unsigned)nchunk, (unsigned)rows), dim3(kRsThreads), 0, st,
                     rr, rows, inv_t, part);
  int rc = status_of(hipGetLastError());
  if (rc) return rc;
  hipLaunchKernelGGL(k_rs_rows, dim3((unsigned)rows), dim3(kWave), 0, st, part, (int)nchunk, items);
  if ((rc = status_of(hipGetLastError()))) return rc;
  hipLaunchKernelGGL(k_rs_mass, dim3((unsigned)nchunk, (unsigned)rows),
                     dim3(kRsThreads), 0, st, rr, items, (int)nchunk, inv_t, mass);
  if ((rc = status_of(hipGetLastError()))) return rc;
  hipLaunchKernelGGL(k_rs_pick, dim3((unsigned)rows), dim3(kRsThreads), 0, st, rr, items, mass,
                     (int)nchunk, inv_t, u, token, nullptr, 0, nullptr);
  return status_of(hipGetLastError());
}

}  // extern "C"
