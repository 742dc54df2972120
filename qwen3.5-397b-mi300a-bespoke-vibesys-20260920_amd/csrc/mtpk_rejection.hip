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
// Four launches, streaming the logits with 16-byte loads:
//   stats : (chunk, row) workgroups -> per-chunk (max, sum exp(z - max)) of z = logit / T
//   decide: one workgroup per lane (a wave per verify row -> row softmax constants, margins, the
//           accept length and the draw it leads to); plain sampling: a wave per row for the row
//           constants
//   mass  : (chunk, item) workgroups -> the chunk's sums of the draw weights
//   pick  : one workgroup per item -> the chunk where the cumulative mass crosses r * total
//           (one wave: scan and ballot over the chunk masses), then a block scan inside it;
//           writes the token (and the emitted row)
// The exponentials are base-2 with the temperature folded into one FMA (exp(l / T - m) =
// exp2(l log2(e) / T - m log2(e))), and no division touches a logit: at the quotient form the
// mass launch was bound by the VALU (20 us against 9.2 us now for config 4).
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

// rows [0, n_target) are target rows, [n_target, n_target + n_draft) draft rows.
constexpr float kLog2e = 1.4426950408889634f;

// Chunk partials in one block reduction: each thread's (max, sum of exp relative to that max)
// over its 16 raw logits, rescaled to the wave max and summed per wave, then the four waves
// combined by thread 0 in a fixed order. With a = log2(e) / T, exp(l / T - m / T) = exp2(l a -
// m a): one FMA and one exp2 per logit. The partial is (M / T, S) for the chunk's raw max M;
// M / T equals the max of the scaled logits (scaling by 1 / T > 0 keeps the order, rounding
// included).
__global__ __launch_bounds__(kRsThreads) void k_rs_stats(RsRows rr, int64_t n_target, float inv_t,
                                                        float2* __restrict__ part) {
  __shared__ float2 red[kRsThreads / kWave];
  const int c = blockIdx.x, nchunk = gridDim.x;
  const int64_t r = blockIdx.y;
  const bool is_t = r < n_target;
  const void* base = is_t ? rr.target : rr.draft;
  const int64_t row = is_t ? r : r - n_target;
  float l[kRsPerThread];
  rs_load(base, rr.dt, rr.vec, row, rr.vocab, c, threadIdx.x, 1.f, l);
  const float a = inv_t * kLog2e;
  float ml = -INFINITY;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) ml = fmaxf(ml, l[e]);
  // A stretch of -inf logits (a masked part of the vocabulary) has no mass: (-inf, 0), not the
  // NaN of exp(-inf - -inf).
  float s = 0.f;
  if (ml > -INFINITY) {
    const float b = ml * a;
#pragma unroll
    for (int e = 0; e < kRsPerThread; ++e) s += __builtin_amdgcn_exp2f(fmaf(l[e], a, -b));
  }
  const float mw = wave_max(ml);
  s = ml > -INFINITY ? s * __builtin_amdgcn_exp2f((ml - mw) * a) : 0.f;
  s = wave_sum(s);
  const int tid = threadIdx.x;
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = make_float2(mw, s);
  __syncthreads();
  if (tid == 0) {
    float m = red[0].x;
#pragma unroll
    for (int w = 1; w < kRsThreads / kWave; ++w) m = fmaxf(m, red[w].x);
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < kRsThreads / kWave; ++w)
      sum += red[w].x > -INFINITY ? red[w].y * __builtin_amdgcn_exp2f((red[w].x - m) * a) : 0.f;
    part[r * nchunk + c] = make_float2(m * inv_t, sum);
  }
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

// The round's acceptance outputs in sampling mode (the outputs of greedy acceptance over the
// emitted rows, `mtpk_greedy_accept`), made by the sampler's own launches. The sampler's accept
// length a fixes all of them but the bonus token: emitted[s] is draft s for s < a and the drawn
// token from a on, so the stop ids can only shorten the accept below a through the drafts, and
// the budget clamps it the same way. lim = min(a, first stop among drafts 0 .. a - 1, budget - 1,
// >= 0); lengths = lim + 1 on an active lane (1 otherwise), the bonus token emitted[lim]. Every
// pointer but the inputs may be null, as for the greedy acceptance; `lengths` non-null turns
// the outputs on.
struct RsAccept {
  const uint8_t* active;
  const int64_t* pos;
  const int64_t* budget;
  const int64_t* stops;
  int n_stops, conv_k1;
  int64_t* accept_len;
  int64_t* lengths;
  int64_t* packed_src;
  int32_t* packed_cu;
  int64_t* conv_idx;
  uint8_t* keep;
  int64_t* bonus;
  int64_t* next_pos;
  int64_t* budget_left;
  uint8_t* live;
  int64_t* hidden_src;
};

// A lane's acceptance inputs that do not depend on the draw, loaded into registers where a
// launch starts (stop ids and drafts up to kRsPre of them), so that the tables written after
// the decision wait for no memory round trip.
constexpr int kRsPre = 8;
struct RsLanePre {
  int64_t bud, pos;
  bool act;
  int64_t sv[kRsPre], dv[kRsPre];
};

__device__ inline RsLanePre rs_lane_pre(const RsAccept& acc, int b, int k,
                                        const int64_t* __restrict__ draft_tokens) {
  RsLanePre p;
  p.bud = acc.budget[b];
  p.pos = acc.pos ? acc.pos[b] : 0;
  p.act = acc.active[b] != 0;
  const int64_t* srow = acc.stops + (int64_t)b * acc.n_stops;
#pragma unroll
  for (int u = 0; u < kRsPre; ++u) {
    p.sv[u] = u < acc.n_stops ? srow[u] : 0;
    p.dv[u] = u < k ? draft_tokens[(int64_t)b * k + u] : 0;
  }
  return p;
}

__device__ inline bool rs_is_stop(const RsAccept& acc, const RsLanePre& p, int b, int64_t tok) {
  bool hit = false;
#pragma unroll
  for (int u = 0; u < kRsPre; ++u) hit |= u < acc.n_stops && p.sv[u] == tok;
  for (int q = kRsPre; q < acc.n_stops; ++q) hit |= acc.stops[(int64_t)b * acc.n_stops + q] == tok;
  return hit;
}

// draft s of lane b, from the registers when s < kRsPre (selects, not indexing)
__device__ inline int64_t rs_draft(const RsLanePre& p, int b, int k, int s,
                                   const int64_t* __restrict__ draft_tokens) {
  int64_t v = 0;
#pragma unroll
  for (int u = 0; u < kRsPre; ++u) v = u == s ? p.dv[u] : v;
  return s < kRsPre ? v : draft_tokens[(int64_t)b * k + s];
}

// Lane b's tables from the sampler's accept length a (one thread): returns lim.
__device__ int rs_lane_tables(const RsAccept& acc, const RsLanePre& p, int b, int k, int a,
                              const int64_t* __restrict__ draft_tokens) {
  const int t = k + 1;
  int lim = a;
  for (int s = 0; s < a; ++s)
    if (rs_is_stop(acc, p, b, rs_draft(p, b, k, s, draft_tokens))) {
      lim = s;
      break;
    }
  if (p.bud - 1 < lim) lim = (int)(p.bud - 1);
  if (lim < 0) lim = 0;
  const int len = p.act ? lim + 1 : 1;
  if (acc.accept_len) acc.accept_len[b] = lim;
  acc.lengths[b] = len;
  if (acc.next_pos) acc.next_pos[b] = p.pos + lim + 1;
  if (acc.budget_left) acc.budget_left[b] = p.bud - (lim + 1);
  if (acc.hidden_src) acc.hidden_src[b] = (int64_t)b * t + lim;
  if (acc.keep)
    for (int s = 0; s < t; ++s) acc.keep[(int64_t)b * t + s] = (p.act && s <= lim) ? 1 : 0;
  if (acc.conv_idx)
    for (int w = 0; w < acc.conv_k1; ++w) {
      const int v = len + w;
      acc.conv_idx[(int64_t)b * acc.conv_k1 + w] = v < acc.conv_k1 + t - 1 ? v : acc.conv_k1 + t - 1;
    }
  return lim;
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
                               int64_t* __restrict__ accept_len, float* __restrict__ margin,
                               const RsAccept& acc) {
  const int t = k + 1;
  const int wv = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int64_t n_target = (int64_t)B * t;
  RsLanePre pre{};
  if (acc.lengths && threadIdx.x == 0) pre = rs_lane_pre(acc, b, k, draft_tokens);
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
    it.pad = acc.lengths ? rs_lane_tables(acc, pre, b, k, a, draft_tokens) : 0;  // lim
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

// Rejection: the lane's decision, one workgroup per lane (its own launch: made inside every mass
// workgroup instead, its dependent loads delay each workgroup's stream, 14.6 us for the mass
// launch against 9.2 + 4.8 us for the two).
__global__ __launch_bounds__(kRsThreads) void k_rs_decide(
    RsRows rr, const float2* __restrict__ part, int nchunk, int B, int k, float inv_t,
    const int64_t* __restrict__ draft_tokens, const float* __restrict__ u_accept,
    RsItem* __restrict__ items, int64_t* __restrict__ accept_len, float* __restrict__ margin,
    RsAccept acc) {
  static_assert(kRsThreads == kWave * kDecideWaves, "one decision per workgroup");
  __shared__ float s_mg[kMaxT];
  __shared__ float4 s_st[kMaxT];
  __shared__ RsItem s_item;
  const int b = blockIdx.x;
  rs_decide_lane(rr, part, nchunk, B, k, inv_t, draft_tokens, u_accept, b, s_mg, s_st, &s_item,
                 items, accept_len, margin, acc);
}

// The draw weights in base-2 form: p = exp(l / T - mt) / st = exp2(l * a - bt) with a = log2(e) /
// T and bt = log2(e) mt + log2(st) (bq likewise for the draft row), one FMA and one exp2 per slot
// where the quotient form costs two exps and two IEEE divisions per slot pair: the mass pass
// streams 2 x vocab logits per item, and at the division form it was bound by the VALU rather
// than by HBM.
struct RsExp {
  float a, bt, bq;
  bool has_q;
};

__device__ inline RsExp rs_exp(const RsItem& it, float inv_t) {
  RsExp x;
  x.a = inv_t * kLog2e;
  x.bt = it.mt * kLog2e + __log2f(it.st);
  x.bq = it.mq * kLog2e + __log2f(it.sq);
  x.has_q = it.drow >= 0;
  return x;
}

// Draw weights of this thread's 16 slots from the raw logits l (target) and lq (draft): target
// p, and the residual max(0, p - q) when the item has a draft row. A -inf logit weighs 0.
__device__ inline void rs_weights_of(const RsExp& x, const float (&l)[kRsPerThread],
                                     const float (&lq)[kRsPerThread], float (&wr)[kRsPerThread],
                                     float (&wp)[kRsPerThread]) {
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) wp[e] = __builtin_amdgcn_exp2f(fmaf(l[e], x.a, -x.bt));
  if (x.has_q) {
#pragma unroll
    for (int e = 0; e < kRsPerThread; ++e)
      wr[e] = fmaxf(wp[e] - __builtin_amdgcn_exp2f(fmaf(lq[e], x.a, -x.bq)), 0.f);
  } else {
#pragma unroll
    for (int e = 0; e < kRsPerThread; ++e) wr[e] = 0.f;
  }
}

__device__ inline void rs_weights(const RsRows& rr, const RsItem& it, int c, float inv_t,
                                  float (&wr)[kRsPerThread], float (&wp)[kRsPerThread]) {
  float l[kRsPerThread], lq[kRsPerThread];
  rs_load(rr.target, rr.dt, rr.vec, it.trow, rr.vocab, c, threadIdx.x, 1.f, l);
  if (it.drow >= 0) rs_load(rr.draft, rr.dt, rr.vec, it.drow, rr.vocab, c, threadIdx.x, 1.f, lq);
  rs_weights_of(rs_exp(it, inv_t), l, lq, wr, wp);
}

__device__ inline float wave_incl_scan_f(float v, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const float u = __shfl_up(v, o, kWave);
    if (lane >= o) v += u;
  }
  return v;
}

struct RsPickLds {
  float wtot[kRsThreads / kWave];
  int chunk, use_r, fallback, best;
  float before, target;
};

// The draw of `item` by the whole workgroup from its per-chunk masses `row_mass` (residual,
// target): one wave finds the chunk where the cumulative mass crosses u * total (a wave sum for
// the totals, then 64 chunks at a time by an inclusive scan and a ballot), then a block scan
// inside that chunk. Writes token[item] and, when `emitted` is set, the emitted row.
__device__ void rs_pick(const RsRows& rr, const RsItem& it, const float2* row_mass, int nchunk,
                        float inv_t, float u, int64_t item, int64_t* __restrict__ token,
                        const int64_t* __restrict__ draft_tokens, int k,
                        int64_t* __restrict__ emitted, RsPickLds& sh, const RsAccept& acc) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  const int64_t dtok = emitted && tid < k ? draft_tokens[item * k + tid] : 0;
  RsLanePre pre{};
  int64_t lim_draft = 0;  // emitted[lim] when lim < a: draft lim
  if (acc.lengths && tid == 0) {
    pre = rs_lane_pre(acc, (int)item, k, draft_tokens);
    if (it.pad < it.a) lim_draft = rs_draft(pre, (int)item, k, it.pad, draft_tokens);
  }
  if (wv == 0) {
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
      sh.fallback = chunk < 0;
      sh.chunk = chunk < 0 ? last_pos : chunk;
      sh.use_r = use_r;
      sh.before = cum;
      sh.target = target;
      sh.best = INT32_MAX;
    }
  }
  __syncthreads();
  const int c = sh.chunk;
  float wr[kRsPerThread], wp[kRsPerThread];
  rs_weights(rr, it, c, inv_t, wr, wp);
  float w[kRsPerThread];
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) w[e] = sh.use_r ? wr[e] : wp[e];
  float mine = 0.f;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) mine += w[e];
  const float inc = wave_incl_scan_f(mine, lane);
  if (lane == kWave - 1) sh.wtot[wv] = inc;
  __syncthreads();
  float off = sh.before;
  for (int q = 0; q < wv; ++q) off += sh.wtot[q];
  float run = off + inc - mine;
  const int64_t i0 = (int64_t)c * kRsChunk + (int64_t)tid * kRsPerThread;
  int hit = INT32_MAX, lastp = -1;
#pragma unroll
  for (int e = 0; e < kRsPerThread; ++e) {
    run += w[e];
    if (w[e] > 0.f) lastp = (int)(i0 + e);
    if (hit == INT32_MAX && !sh.fallback && run > sh.target && w[e] > 0.f) hit = (int)(i0 + e);
  }
  atomicMin(&sh.best, hit);
  __syncthreads();
  // Rounding can leave no crossing inside the chunk: take the chunk's last positive slot.
  const int need_last = sh.best == INT32_MAX;
  __syncthreads();
  if (need_last) {
    if (tid == 0) sh.best = -1;
    __syncthreads();
    atomicMax(&sh.best, lastp);
    __syncthreads();
  }
  // the emitted row by its first k + 1 threads at once (draft token i was loaded at the start)
  if (tid <= k) {
    const int64_t v = sh.best < 0 ? 0 : sh.best;
    if (tid == 0) token[item] = v;
    if (emitted) emitted[item * (k + 1) + tid] = tid < it.a ? dtok : v;
  }
  // sampling-mode acceptance: the lane's bonus token emitted[lim] (lim in the item's pad) and
  // whether the lane stays live, as the greedy acceptance over the emitted row gives them
  if (acc.lengths && tid == 0) {
    const int lim = it.pad;
    const int64_t v = sh.best < 0 ? 0 : sh.best;
    const int64_t bn = lim < it.a ? lim_draft : v;
    if (acc.bonus) acc.bonus[item] = bn;
    if (acc.live) acc.live[item] = (!rs_is_stop(acc, pre, (int)item, bn) && pre.bud - (lim + 1) > 0) ? 1 : 0;
  }
}

// The pack offsets of sampling-mode acceptance, from the lanes' lengths (written by the decide
// launch): packed_cu = exclusive prefix of lengths over the B lanes, and packed_src[dst] = lane
// * t + local for the lane whose packed rows hold dst (as `mtpk_greedy_accept`). One workgroup,
// four lanes per thread (B <= 1024).
constexpr int kRsPackLanes = 4 * kRsThreads;

__device__ void rs_pack(const RsAccept& acc, int B, int t) {
  __shared__ int cu[kRsPackLanes + 1];
  __shared__ int wtot[kRsThreads / kWave];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  int v[4], sum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = 4 * tid + q;
    v[q] = j < B ? (int)acc.lengths[j] : 0;
    sum += v[q];
  }
  const int inc = wave_incl_scan(sum, lane);
  if (lane == kWave - 1) wtot[wv] = inc;
  __syncthreads();
  int run = inc - sum;
  for (int w = 0; w < wv; ++w) run += wtot[w];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = 4 * tid + q;
    run += v[q];
    if (j < B) cu[j + 1] = run;
  }
  if (tid == 0) cu[0] = 0;
  __syncthreads();
  if (acc.packed_cu)
    for (int j = tid; j <= B; j += kRsThreads) acc.packed_cu[j] = cu[j];
  if (acc.packed_src)
    for (int dst = tid; dst < B * t; dst += kRsThreads) {
      int lo = 1, hi = B + 1;  // lane = #{i in 1..B : cu[i] <= dst}, clamped to B - 1
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (cu[mid] <= dst)
          lo = mid + 1;
        else
          hi = mid;
      }
      int ln = lo - 1;
      if (ln > B - 1) ln = B - 1;
      int local = dst - cu[ln];
      local = local < 0 ? 0 : (local > t - 1 ? t - 1 : local);
      acc.packed_src[dst] = (int64_t)ln * t + local;
    }
}

// The draw in a launch of its own (one workgroup per item), after the mass launch.
// With sampling-mode acceptance one more workgroup (the last) makes the pack offsets.
__global__ __launch_bounds__(kRsThreads) void k_rs_pick(
    RsRows rr, const RsItem* __restrict__ items, const float2* __restrict__ mass, int nchunk,
    float inv_t, const float* __restrict__ u_sample, int64_t* __restrict__ token,
    const int64_t* __restrict__ draft_tokens, int k, int64_t* __restrict__ emitted, int n_items,
    RsAccept acc) {
  __shared__ RsPickLds sh;
  const int item = blockIdx.x;
  if (item >= n_items) {  // uniform: the pack workgroup
    rs_pack(acc, n_items, k + 1);
    return;
  }
  rs_pick(rr, items[item], mass + (int64_t)item * nchunk, nchunk, inv_t, u_sample[item], item,
          token, draft_tokens, k, emitted, sh, acc);
}

// Chunks per mass workgroup. Measured at config 4 (48 items of two 248320-logit rows): 1 chunk
// (2928 workgroups) 9.2 us, 2 and 4 chunks 1-3 us slower in the whole acceptance: more
// workgroups in flight hide the item load each one starts with better than longer streams do.
// (A variant whose last workgroup per item also made the draw, found by an agent-scope arrival
// counter, lost 3-20 us to the counter's same-address atomics.)
constexpr int kRsMassChunks = 1;

// Per-chunk sums of an item's draw weights (residual, target), one workgroup per (G chunks,
// item), every load of its chunks in flight before the first is used.
template <int G>
__global__ __launch_bounds__(kRsThreads) void k_rs_mass(RsRows rr, const RsItem* __restrict__ items,
                                                       int nchunk, float inv_t,
                                                       float2* __restrict__ mass) {
  __shared__ float2 red[G][kRsThreads / kWave];
  const int c0 = blockIdx.x * G;
  const int item = blockIdx.y;
  const int tid = threadIdx.x;
  const RsItem it = items[item];
  auto reduce = [&](int g, const float (&wr)[kRsPerThread], const float (&wp)[kRsPerThread]) {
    float sr = 0.f, sp = 0.f;
#pragma unroll
    for (int e = 0; e < kRsPerThread; ++e) {
      sr += wr[e];
      sp += wp[e];
    }
    sr = wave_sum(sr);
    sp = wave_sum(sp);
    if ((tid & (kWave - 1)) == 0) red[g][tid / kWave] = make_float2(sr, sp);
  };
  if (rr.vec && rr.dt == MTPK_BF16) {
    // Every load of the G chunks (two rows) goes out before the first is used: 16-byte buffer
    // loads, slots past the row reading zeros, which the index test below turns into -inf as
    // rs_load does. The logits stay raw: the temperature is in RsExp.
    const uint32_t bytes = (uint32_t)(rr.vocab * 2);
    const bool has_q = it.drow >= 0;
    const RsExp ex = rs_exp(it, inv_t);
    const rsrc_t rt = make_rsrc(reinterpret_cast<const uint16_t*>(rr.target) + it.trow * rr.vocab, bytes);
    const rsrc_t rq = make_rsrc(reinterpret_cast<const uint16_t*>(rr.draft) +
                                    (has_q ? it.drow : 0) * rr.vocab, has_q ? bytes : 0u);
    u32x4_t vt[G][2], vq[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t i = (int64_t)(c0 + g) * kRsChunk + (int64_t)tid * kRsPerThread + 8 * h;
        const uint32_t off = i < rr.vocab ? (uint32_t)(i * 2) : kOutOfRange;
        vt[g][h] = buf16(rt, off);
        vq[g][h] = buf16(rq, has_q ? off : kOutOfRange);
      }
#pragma unroll
    for (int g = 0; g < G; ++g) {  // a chunk past the row is all -inf: zero mass, not stored
      float z[kRsPerThread], zq[kRsPerThread];
      const int64_t i0 = (int64_t)(c0 + g) * kRsChunk + (int64_t)tid * kRsPerThread;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e = 8 * h + 2 * q;
          const bool in0 = i0 + e < rr.vocab, in1 = i0 + e + 1 < rr.vocab;
          z[e] = in0 ? bf16_to_f32((uint16_t)(vt[g][h][q] & 0xffffu)) : -INFINITY;
          z[e + 1] = in1 ? bf16_to_f32((uint16_t)(vt[g][h][q] >> 16)) : -INFINITY;
          zq[e] = in0 ? bf16_to_f32((uint16_t)(vq[g][h][q] & 0xffffu)) : -INFINITY;
          zq[e + 1] = in1 ? bf16_to_f32((uint16_t)(vq[g][h][q] >> 16)) : -INFINITY;
        }
      float wr[kRsPerThread], wp[kRsPerThread];
      rs_weights_of(ex, z, zq, wr, wp);
      reduce(g, wr, wp);
    }
  } else {
    for (int g = 0; g < G && c0 + g < nchunk; ++g) {
      float wr[kRsPerThread], wp[kRsPerThread];
      rs_weights(rr, it, c0 + g, inv_t, wr, wp);
      reduce(g, wr, wp);
    }
  }
  __syncthreads();
  if (tid < G && c0 + tid < nchunk) {
    const float2 a = red[tid][0], b = red[tid][1], d = red[tid][2], e = red[tid][3];
    mass[(int64_t)item * nchunk + c0 + tid] =
        make_float2((a.x + b.x) + (d.x + e.x), (a.y + b.y) + (d.y + e.y));
  }
}

int64_t rs_chunks(int64_t vocab) { return (vocab + kRsChunk - 1) / kRsChunk; }
int64_t rs_groups(int64_t nchunk) { return (nchunk + kRsMassChunks - 1) / kRsMassChunks; }

// Workspace layout shared by both entry points: chunk partials | items | chunk masses.
struct RsWorkspace {
  float2* part;
  RsItem* items;
  float2* mass;
};

RsWorkspace rs_workspace(void* workspace, int64_t items, int64_t rows, int64_t nchunk) {
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  RsWorkspace w;
  w.part = reinterpret_cast<float2*>(ws);
  ws += align256(rows * nchunk * (int64_t)sizeof(float2));
  w.items = reinterpret_cast<RsItem*>(ws);
  ws += align256(items * (int64_t)sizeof(RsItem));
  w.mass = reinterpret_cast<float2*>(ws);
  return w;
}

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

}  // extern "C"

namespace {

// The four launches of rejection sampling; with acc.lengths set also the acceptance outputs
// (decide writes the lane tables, pick the bonus token and liveness, one more pick workgroup
// the pack offsets).
int rejection_launch(const void* target, const void* draft, int dtype, int64_t batch, int k,
                     int64_t vocab, const int64_t* draft_tokens, const float* u_accept,
                     const float* u_sample, float temperature, void* workspace,
                     int64_t workspace_bytes, int64_t* accept_len, int64_t* token,
                     int64_t* emitted, float* margin, const RsAccept& acc, void* stream) {
  if (!target || !u_sample || !workspace || !token) return MTPK_EINVAL;
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
  const RsWorkspace w = rs_workspace(workspace, batch, batch * (2 * (int64_t)k + 1), nchunk);
  const float inv_t = 1.f / temperature;
  const hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_rs_stats, dim3((unsigned)nchunk, (unsigned)rows), dim3(kRsThreads), 0, st,
                     rr, batch * t, inv_t, w.part);
  int rc = status_of(hipGetLastError());
  if (rc) return rc;
  hipLaunchKernelGGL(k_rs_decide, dim3((unsigned)batch), dim3(kRsThreads), 0, st, rr, w.part,
                     (int)nchunk, (int)batch, k, inv_t, draft_tokens, u_accept, w.items, accept_len,
                     margin, acc);
  if ((rc = status_of(hipGetLastError()))) return rc;
  hipLaunchKernelGGL(k_rs_mass<kRsMassChunks>, dim3((unsigned)rs_groups(nchunk), (unsigned)batch),
                     dim3(kRsThreads), 0, st, rr, w.items, (int)nchunk, inv_t, w.mass);
  if ((rc = status_of(hipGetLastError()))) return rc;
  const bool pack = acc.lengths && (acc.packed_cu || acc.packed_src);
  hipLaunchKernelGGL(k_rs_pick, dim3((unsigned)(batch + (pack ? 1 : 0))), dim3(kRsThreads), 0, st, rr,
                     w.items, w.mass, (int)nchunk, inv_t, u_sample, token, draft_tokens, k, emitted,
                     (int)batch, acc);
  return status_of(hipGetLastError());
}

}  // namespace

extern "C" {

int mtpk_rejection_sample(const void* target, const void* draft, int dtype, int64_t batch, int k,
                          int64_t vocab, const int64_t* draft_tokens, const float* u_accept,
                          const float* u_sample, float temperature, void* workspace,
                          int64_t workspace_bytes, int64_t* accept_len, int64_t* token,
                          int64_t* emitted, float* margin, void* stream) {
  if (!accept_len) return MTPK_EINVAL;
  const RsAccept none{};
  return rejection_launch(target, draft, dtype, batch, k, vocab, draft_tokens, u_accept, u_sample,
                          temperature, workspace, workspace_bytes, accept_len, token, emitted,
                          margin, none, stream);
}

int mtpk_rejection_accept(const void* target, const void* draft, int dtype, int64_t batch, int k,
                          int64_t vocab, const int64_t* draft_tokens, const float* u_accept,
                          const float* u_sample, float temperature, void* workspace,
                          int64_t workspace_bytes, const uint8_t* active, const int64_t* pos,
                          const int64_t* budget, const int64_t* stops, int n_stops, int conv_k1,
                          int64_t* accept_len, int64_t* lengths, int64_t* packed_src,
                          int32_t* packed_cu, int64_t* conv_idx, uint8_t* keep, int64_t* bonus,
                          int64_t* next_pos, int64_t* budget_left, uint8_t* live,
                          int64_t* hidden_src, int64_t* token, int64_t* emitted, void* stream) {
  if (!active || !budget || !accept_len || !lengths) return MTPK_EINVAL;
  if (batch > kRsPackLanes || n_stops < 0 || (n_stops > 0 && !stops) || conv_k1 < 0) return MTPK_EINVAL;
  if (next_pos && !pos) return MTPK_EINVAL;
  const RsAccept acc{active,     pos,     budget,  stops, n_stops,  conv_k1,     accept_len,
                     lengths,    packed_src, packed_cu, conv_idx, keep, bonus, next_pos,
                     budget_left, live,   hidden_src};
  return rejection_launch(target, draft, dtype, batch, k, vocab, draft_tokens, u_accept, u_sample,
                          temperature, workspace, workspace_bytes, nullptr, token, emitted, nullptr,
                          acc, stream);
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
  const RsWorkspace w = rs_workspace(workspace, rows, rows, nchunk);
  const float inv_t = 1.f / temperature;
  const hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_rs_stats, dim3((unsigned)nchunk, (unsigned)rows), dim3(kRsThreads), 0, st,
                     rr, rows, inv_t, w.part);
  int rc = status_of(hipGetLastError());
  if (rc) return rc;
  hipLaunchKernelGGL(k_rs_rows, dim3((unsigned)rows), dim3(kWave), 0, st, w.part, (int)nchunk,
                     w.items);
  if ((rc = status_of(hipGetLastError()))) return rc;
  hipLaunchKernelGGL(k_rs_mass<kRsMassChunks>, dim3((unsigned)rs_groups(nchunk), (unsigned)rows),
                     dim3(kRsThreads), 0, st, rr, w.items, (int)nchunk, inv_t, w.mass);
  if ((rc = status_of(hipGetLastError()))) return rc;
  const RsAccept none{};
  hipLaunchKernelGGL(k_rs_pick, dim3((unsigned)rows), dim3(kRsThreads), 0, st, rr, w.items, w.mass,
                     (int)nchunk, inv_t, u, token, nullptr, 0, nullptr, (int)rows, none);
  return status_of(hipGetLastError());
}

}  // extern "C"
