// Verify-step tail for gfx950: row argmax over the vocabulary and greedy acceptance with its
// rollback indices.
//
// argmax: the vocabulary is cut into chunks so rows x chunks workgroups stream the logits at
// HBM rate; each workgroup reduces (value, index) keys whose maximum is the first-occurrence
// argmax (mtpk_common.h argmax_key), so the split and the reduction order cannot change the
// answer. A second tiny kernel takes the max over a row's chunk keys.
// greedy accept: one workgroup, one thread per verify row (B <= 1024), plus a block scan for
// the prefix-pack offsets.

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kArgmaxThreads = 256;
// 16-byte loads in flight per thread, and the workgroup count the chunking aims at. Measured
// over [192 | 48, 248320] bf16: 4 loads beat 2/8/16, and about 1536 workgroups (six per CU,
// all resident at once at this kernel's occupancy, the same number on every CU at 192 and 48
// rows) beat 512/768/1024/2048/4096 (greedy accept at 192 rows: 24.4 us against 25.9 us at
// 1024, whose 4.5 per CU leave half the CUs a workgroup longer, and 6144/12288/24576 with
// shorter chunks: greedy accept 30/42/64 us); a 1024-thread workgroup per row, which would drop
// the second launch, streams at only about 40 GB/s per CU and lost at every row count. Numbering
// the workgroups row-fastest (each row's chunks on one XCD) measured the same.
constexpr int kArgmaxLoads = 4;
constexpr int64_t kArgmaxWorkgroups = 1536;

__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_partial(
    const void* __restrict__ logits, int dt, int64_t stride, int64_t vocab, int64_t chunk,
    int vec, uint64_t* __restrict__ partials) {
  const int64_t row = blockIdx.y;
  const int64_t begin = (int64_t)blockIdx.x * chunk;
  const int64_t end = begin + chunk < vocab ? begin + chunk : vocab;
  const int tid = threadIdx.x;
  uint64_t best = 0;
  if (vec && dt == MTPK_BF16) {
    // kArgmaxLoads 16-byte loads in flight per thread. A chunk of 8 values updates the thread's best
    // only if its float max beats it strictly (an equal value has a later index, so the earlier
    // one stays: the key order), and then at the chunk's first index holding that max; +0 and
    // -0 compare equal as the keys fold them. A chunk holding a NaN takes the key path.
    const uint16_t* base = reinterpret_cast<const uint16_t*>(logits) + row * stride;
    float bv = -INFINITY;
    int64_t bi = -1;
    auto chunk8 = [&](const u32x4_t& v, int64_t i0) {
      float f[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f[2 * q] = bits_f32(v[q] << 16);
        f[2 * q + 1] = bits_f32(v[q] & 0xffff0000u);
      }
      bool nan = false;
      float m8 = f[0];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        nan |= f[j] != f[j];
        m8 = fmaxf(m8, f[j]);
      }
      if (nan) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint64_t k = argmax_key(f[j], (uint32_t)(i0 + j));
          best = k > best ? k : best;
        }
      } else if (m8 > bv || bi < 0) {
        int first = 7;
#pragma unroll
        for (int j = 7; j >= 0; --j)
          if (f[j] == m8) first = j;
        bv = m8;
        bi = i0 + first;
      }
    };
    // The chunk as one buffer, streamed kArgmaxLoads 16-byte slots per thread at a time and
    // software-pipelined: the next group's loads are issued before the current group is
    // scanned, so 2 kArgmaxLoads loads stay in flight. Slots past the chunk read zeros and are
    // skipped by the index test.
    constexpr int64_t step = (int64_t)kArgmaxThreads * 8;  // elements per slot over the workgroup
    const int64_t n = end - begin;
    const rsrc_t rr = make_rsrc(base + begin, (uint32_t)(n * 2));
    const int64_t iters = (n + kArgmaxLoads * step - 1) / (kArgmaxLoads * step);
    u32x4_t va[kArgmaxLoads], vb[kArgmaxLoads];
    auto issue = [&](u32x4_t* v, int64_t it) {
#pragma unroll
      for (int u = 0; u < kArgmaxLoads; ++u) {
        const int64_t e = (it * kArgmaxLoads + u) * step + (int64_t)tid * 8;
        v[u] = buf16(rr, e < n ? (uint32_t)(e * 2) : kOutOfRange);
      }
    };
    auto scan = [&](const u32x4_t* v, int64_t it) {
#pragma unroll
      for (int u = 0; u < kArgmaxLoads; ++u) {
        const int64_t i0 = begin + (it * kArgmaxLoads + u) * step + (int64_t)tid * 8;
        if (i0 + 8 <= end) {
          chunk8(v[u], i0);
        } else {
          for (int64_t q = i0; q < end; ++q) {
            const uint64_t k = argmax_key(bf16_to_f32(base[q]), (uint32_t)q);
            best = k > best ? k : best;
          }
        }
      }
    };
    issue(va, 0);
    for (int64_t it = 0; it < iters; it += 2) {
      issue(vb, it + 1);
      scan(va, it);
      if (it + 1 >= iters) break;
      issue(va, it + 2);
      scan(vb, it + 1);
    }
    if (bi >= 0) {
      const uint64_t k = argmax_key(bv, (uint32_t)bi);
      best = k > best ? k : best;
    }
  } else if (vec && dt == MTPK_F32) {
    const float* base = reinterpret_cast<const float*>(logits) + row * stride;
    for (int64_t i = begin + (int64_t)tid * 4; i < end; i += (int64_t)kArgmaxThreads * 4) {
      if (i + 4 <= end) {
        const u32x4_t v = ld16(base + i);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint64_t k = argmax_key(bits_f32(v[q]), (uint32_t)(i + q));
          best = k > best ? k : best;
        }
      } else {
        for (int64_t q = i; q < end; ++q) {
          const uint64_t k = argmax_key(base[q], (uint32_t)q);
          best = k > best ? k : best;
        }
      }
    }
  } else {
    for (int64_t i = begin + tid; i < end; i += kArgmaxThreads) {
      const uint64_t k = argmax_key(load_float(logits, dt, row * stride + i), (uint32_t)i);
      best = k > best ? k : best;
    }
  }
  best = wave_max_u64(best);
  __shared__ uint64_t part[kArgmaxThreads / kWave];
  if ((tid & (kWave - 1)) == 0) part[tid / kWave] = best;
  __syncthreads();
  if (tid == 0) {
    uint64_t b = part[0];
    for (int w = 1; w < kArgmaxThreads / kWave; ++w) b = part[w] > b ? part[w] : b;
    partials[row * gridDim.x + blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(256) void k_argmax_final(const uint64_t* __restrict__ partials,
                                                      int64_t rows, int chunks,
                                                      int64_t* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  uint64_t b = 0;
  for (int c = 0; c < chunks; ++c) {
    const uint64_t k = partials[row * chunks + c];
    b = k > b ? k : b;
  }
  out[row] = (int64_t)argmax_key_index(b);
}

constexpr int kAcceptThreads = 1024;
constexpr int kPre = 8;
constexpr int kKeyRows = 4096;  // B * t bound of the keys path: one u64 of LDS per verify row
constexpr int kKeyLoads = 32;   // key loads in flight per row in the keys fold

// keys (optional): the argmax chunk keys [B * t, chunks] of k_argmax_partial. The workgroup
// then first folds them into one key per verify row (a thread per row), writes the indices to
// sa_out and reads the verify columns from LDS: the argmax needs no second launch.
// forced_n (optional): a row with forced_n[j] > 0 accepts exactly min(forced_n[j], k) drafts,
// which are not generated output, so the stop ids and the budget do not clamp them and the
// budget is charged the one target token (graph_verify_wide.py:196-200, mtp_overlap.py:53-71);
// every other output follows from that accept length.
__global__ __launch_bounds__(kAcceptThreads) void k_greedy_accept(
    const uint64_t* __restrict__ keys, int chunks, int64_t* sa_out,
    const int64_t* sa, int64_t ss, const int64_t* __restrict__ draft, int64_t ds,
    const uint8_t* __restrict__ active, const int64_t* __restrict__ pos,
    const int64_t* __restrict__ budget, const int64_t* __restrict__ stops, int n_stops,
    const int64_t* __restrict__ forced_n, int B, int t, int conv_k1, int64_t* __restrict__ accept_len, int64_t* __restrict__ lengths,
    int64_t* __restrict__ packed_src, int32_t* __restrict__ packed_cu,
    int64_t* __restrict__ conv_idx, uint8_t* __restrict__ keep, int64_t* __restrict__ bonus,
    int64_t* __restrict__ next_pos, int64_t* __restrict__ budget_left,
    uint8_t* __restrict__ live, int64_t* __restrict__ hidden_src) {
  __shared__ int cu[kAcceptThreads + 1];
  __shared__ int wtot[kAcceptThreads / kWave];
  const int j = threadIdx.x, lane = j & (kWave - 1), wv = j / kWave;
  const int k = t - 1;
  __shared__ unsigned long long s_key[kKeyRows];
  int len = 0;
  // The lane's loads that do not depend on the step argmax (drafts, stop ids, budget, state) go
  // out before the key fold, so their latency overlaps it: kPre of each into registers.
  const int64_t* drow = draft + (int64_t)(j < B ? j : 0) * ds;
  const int64_t* srow = stops + (int64_t)(j < B ? j : 0) * n_stops;
  int64_t dv[kPre], sv[kPre];
  int64_t bud = 0, p0 = 0, fn = 0;
  bool act = false;
  if (j < B) {
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      dv[u] = u < k ? drow[u] : 0;
      sv[u] = u < n_stops ? srow[u] : 0;
    }
    bud = budget[j];
    act = active[j] != 0;
    fn = forced_n ? forced_n[j] : 0;
    p0 = next_pos ? pos[j] : 0;
  }
  if (keys) {
    // One thread per verify row folds the row's chunk keys in registers: up to kKeyLoads loads
    // in flight at once (one memory round trip), then any further keys kKeyLoads at a time. The
    // maximum key is the first-occurrence argmax whatever the order. (LDS atomics over all keys,
    // spread across the workgroup, measured 0.5-1 us slower at 8 and 32 chunks per row.)
    const int rows = B * t;
    for (int r = j; r < rows; r += kAcceptThreads) {
      const uint64_t* kr = keys + (int64_t)r * chunks;
      uint64_t bk = 0;
      for (int c0 = 0; c0 < chunks; c0 += kKeyLoads) {
        uint64_t x[kKeyLoads];
#pragma unroll
        for (int u = 0; u < kKeyLoads; ++u) x[u] = c0 + u < chunks ? kr[c0 + u] : 0;
#pragma unroll
        for (int u = 0; u < kKeyLoads; ++u) bk = x[u] > bk ? x[u] : bk;
      }
      const int64_t tok = (int64_t)argmax_key_index(bk);
      s_key[r] = (unsigned long long)tok;
      sa_out[(int64_t)(r / t) * ss + r % t] = tok;
    }
    __syncthreads();
  }
  if (j < B) {
    const int64_t* row = keys ? reinterpret_cast<const int64_t*>(s_key) + (int64_t)j * t
                              : sa + (int64_t)j * ss;
    // The first kPre verify columns into registers together: compared one after another they
    // would cost a memory round trip each.
    int64_t rv[kPre];
#pragma unroll
    for (int u = 0; u < kPre; ++u) rv[u] = u < t ? row[u] : 0;
    auto column = [&](int s) {
      int64_t v = 0;
#pragma unroll
      for (int u = 0; u < kPre; ++u) v = u == s ? rv[u] : v;
      return s < kPre ? v : row[s];
    };
    auto is_stop = [&](int64_t tok) {
      bool hit = false;
#pragma unroll
      for (int u = 0; u < kPre; ++u) hit |= u < n_stops && sv[u] == tok;
      for (int q = kPre; q < n_stops; ++q) hit |= srow[q] == tok;
      return hit;
    };
    int acc = 0;
    bool same = true;
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      same = same && u < k && dv[u] == rv[u];
      acc = same ? u + 1 : acc;
    }
    if (same)
      while (acc < k && drow[acc] == row[acc]) ++acc;
    int first_stop = t;
#pragma unroll
    for (int s = kPre - 1; s >= 0; --s)
      if (s < t && is_stop(rv[s])) first_stop = s;
    for (int s = kPre; s < t && first_stop == t; ++s)
      if (is_stop(row[s])) first_stop = s;
    int64_t lim = acc < first_stop ? acc : first_stop;
    if (bud - 1 < lim) lim = bud - 1;
    if (lim < 0) lim = 0;
    if (fn > 0) lim = fn < k ? fn : k;  // forced drafts: accepted as they are
    const int a = (int)lim;
    len = act ? a + 1 : 1;
    accept_len[j] = a;
    if (lengths) lengths[j] = len;
    const int64_t bn = column(a);
    if (bonus) bonus[j] = bn;
    if (next_pos) next_pos[j] = p0 + a + 1;
    const int64_t left = bud - (fn > 0 ? 1 : a + 1);
    if (budget_left) budget_left[j] = left;
    if (live) live[j] = (!is_stop(bn) && left > 0) ? 1 : 0;
    if (hidden_src) hidden_src[j] = (int64_t)j * t + a;
    if (keep)
      for (int s = 0; s < t; ++s) keep[(int64_t)j * t + s] = (act && s <= a) ? 1 : 0;
    if (conv_idx)
      for (int w = 0; w < conv_k1; ++w) {
        const int v = len + w;
        conv_idx[(int64_t)j * conv_k1 + w] = v < conv_k1 + t - 1 ? v : conv_k1 + t - 1;
      }
  }
  const int inc = wave_incl_scan(len, lane);
  if (lane == kWave - 1) wtot[wv] = inc;
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wv; ++w) off += wtot[w];
  if (j < B) cu[j + 1] = off + inc;
  if (j == 0) cu[0] = 0;
  __syncthreads();
  if (packed_cu) {
    if (j < B) packed_cu[j] = cu[j];
    if (j == 0) packed_cu[B] = cu[B];  // B may equal the thread count
  }
  if (packed_src) {
    const int total = B * t;
    for (int dst = j; dst < total; dst += kAcceptThreads) {
      // lane = #{i in 1..B : cu[i] <= dst}, clamped to B - 1 (graph_mtp.py:445)
      int lo = 1, hi = B + 1;
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
      packed_src[dst] = (int64_t)ln * t + local;
    }
  }
}

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int64_t mtpk_argmax_partials(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  // About kArgmaxWorkgroups workgroups over all rows, chunks of >= 2048 values.
  int64_t chunks = (kArgmaxWorkgroups + rows - 1) / rows;
  const int64_t by_len = (vocab + 2047) / 2048;
  if (chunks > by_len) chunks = by_len;
  if (chunks < 1) chunks = 1;
  if (chunks > 4096) chunks = 4096;
  return rows * chunks;
}

int mtpk_argmax_rows(const void* logits, int dtype, int64_t rows, int64_t vocab,
                     int64_t row_stride, uint64_t* partials, int64_t* out_index, void* stream) {
  if (!logits || !partials || !out_index) return MTPK_EINVAL;
  if (dtype != MTPK_F32 && dtype != MTPK_BF16) return MTPK_EINVAL;
  if (rows < 0 || rows > 65535 || vocab <= 0 || vocab > INT32_MAX || row_stride < vocab)
    return MTPK_EINVAL;
  if (rows == 0) return 0;
  const int per_vec = dtype == MTPK_BF16 ? 8 : 4;
  const int vec = aligned16(logits) && (row_stride % per_vec) == 0;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t chunks = mtpk_argmax_partials(rows, vocab) / rows;
  int64_t chunk = (vocab + chunks - 1) / chunks;
  chunk = (chunk + per_vec - 1) / per_vec * per_vec;
  hipLaunchKernelGGL(k_argmax_partial, dim3((unsigned)chunks, (unsigned)rows),
                     dim3(kArgmaxThreads), 0, st, logits, dtype, row_stride, vocab, chunk, vec,
                     partials);
  int rc = status_of(hipGetLastError());
  if (rc) return rc;
  hipLaunchKernelGGL(k_argmax_final, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st,
                     partials, rows, (int)chunks, out_index);
  return status_of(hipGetLastError());
}

namespace {

int greedy_accept_launch(const uint64_t* keys, int chunks, int64_t* sa_out,
                         const int64_t* step_argmax, int64_t sa_stride, const int64_t* draft,
                         int64_t draft_stride, const uint8_t* active, const int64_t* pos,
                         const int64_t* budget, const int64_t* stops, int n_stops,
                         const int64_t* forced_n, int batch, int t, int conv_k1, int64_t* accept_len, int64_t* lengths, int64_t* packed_src,
                         int32_t* packed_cu, int64_t* conv_idx, uint8_t* keep, int64_t* bonus,
                         int64_t* next_pos, int64_t* budget_left, uint8_t* live,
                         int64_t* hidden_src, void* stream) {
  if (!step_argmax || !active || !budget || !accept_len) return MTPK_EINVAL;
  if (batch <= 0 || batch > kAcceptThreads || t < 1 || t > 64) return MTPK_EINVAL;
  if (t > 1 && !draft) return MTPK_EINVAL;
  if (n_stops < 0 || (n_stops > 0 && !stops) || conv_k1 < 0) return MTPK_EINVAL;
  if (next_pos && !pos) return MTPK_EINVAL;
  if (sa_stride < t || (t > 1 && draft_stride < t - 1)) return MTPK_EINVAL;
  hipLaunchKernelGGL(k_greedy_accept, dim3(1), dim3(kAcceptThreads), 0, (hipStream_t)stream,
                     keys, chunks, sa_out, step_argmax, sa_stride, draft, draft_stride, active, pos,
                     budget, stops, n_stops, forced_n, batch, t, conv_k1, accept_len, lengths, packed_src,
                     packed_cu, conv_idx, keep, bonus, next_pos, budget_left, live, hidden_src);
  return status_of(hipGetLastError());
}

}  // namespace

int mtpk_greedy_accept(const int64_t* step_argmax, int64_t sa_stride, const int64_t* draft,
                       int64_t draft_stride, const uint8_t* active, const int64_t* pos,
                       const int64_t* budget, const int64_t* stops, int n_stops,
                       const int64_t* forced_n, int batch, int t, int conv_k1, int64_t* accept_len, int64_t* lengths, int64_t* packed_src,
                       int32_t* packed_cu, int64_t* conv_idx, uint8_t* keep, int64_t* bonus,
                       int64_t* next_pos, int64_t* budget_left, uint8_t* live,
                       int64_t* hidden_src, void* stream) {
  return greedy_accept_launch(nullptr, 0, nullptr, step_argmax, sa_stride, draft, draft_stride,
                              active, pos, budget, stops, n_stops, forced_n, batch, t, conv_k1, accept_len,
                              lengths, packed_src, packed_cu, conv_idx, keep, bonus, next_pos,
                              budget_left, live, hidden_src, stream);
}

int mtpk_greedy_accept_keys(const uint64_t* keys, int64_t chunks, int64_t* step_argmax,
                            int64_t sa_stride, const int64_t* draft, int64_t draft_stride,
                            const uint8_t* active, const int64_t* pos, const int64_t* budget,
                            const int64_t* stops, int n_stops, const int64_t* forced_n, int batch,
                            int t, int conv_k1, int64_t* accept_len, int64_t* lengths, int64_t* packed_src,
                            int32_t* packed_cu, int64_t* conv_idx, uint8_t* keep, int64_t* bonus,
                            int64_t* next_pos, int64_t* budget_left, uint8_t* live,
                            int64_t* hidden_src, void* stream) {
  if (!keys || chunks < 1 || chunks > 65535) return MTPK_EINVAL;
  if ((int64_t)batch * t > kKeyRows) return MTPK_EINVAL;
  return greedy_accept_launch(keys, (int)chunks, step_argmax, step_argmax, sa_stride, draft,
                              draft_stride, active, pos, budget, stops, n_stops, forced_n, batch, t, conv_k1,
                              accept_len, lengths, packed_src, packed_cu, conv_idx, keep, bonus,
                              next_pos, budget_left, live, hidden_src, stream);
}

int mtpk_argmax_keys(const void* logits, int dtype, int64_t rows, int64_t vocab,
                     int64_t row_stride, uint64_t* keys, void* stream) {
  if (!logits || !keys) return MTPK_EINVAL;
  if (dtype != MTPK_F32 && dtype != MTPK_BF16) return MTPK_EINVAL;
  if (rows < 0 || rows > 65535 || vocab <= 0 || vocab > INT32_MAX || row_stride < vocab)
    return MTPK_EINVAL;
  if (rows == 0) return 0;
  const int per_vec = dtype == MTPK_BF16 ? 8 : 4;
  const int vec = aligned16(logits) && (row_stride % per_vec) == 0;
  const int64_t chunks = mtpk_argmax_partials(rows, vocab) / rows;
  int64_t chunk = (vocab + chunks - 1) / chunks;
  chunk = (chunk + per_vec - 1) / per_vec * per_vec;
  hipLaunchKernelGGL(k_argmax_partial, dim3((unsigned)chunks, (unsigned)rows),
                     dim3(kArgmaxThreads), 0, (hipStream_t)stream, logits, dtype, row_stride, vocab,
                     chunk, vec, keys);
  return status_of(hipGetLastError());
}

}  // extern "C"
