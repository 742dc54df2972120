// Causal GQA attention of the verify rows over the paged bf16 KV cache (`verify_attention_paged`,
// model.py:1120-1205, which runs `paged_attn.decode_attention_paged` per verify row; the MTP
// layer's draft step `mtp._attn_rows`, mtp.py:233-279, is the same call with t = 1).
//
// Shapes: q bf16 [B, heads, t, hd]; K pool bf16 [pool_rows, kv_heads, hd] and V pool bf16
// [pool_rows / 16, kv_heads, hd, 16] (V transposed inside each 16-row block, so that a V tile
// is staged with contiguous reads and no transposition), 16-row blocks; lane b's key position p
// lives in pool row table[b][p / 16] * 16 + p % 16, i.e. block table[b][p / 16], slot p % 16.
// Query row s of lane b sits at position base_pos[b] + s and sees keys 0 .. base_pos[b] + s.
//
// One workgroup takes one (lane, kv head, group of up to 64 query rows, key split). The query
// rows of a kv head (group = heads / kv_heads q heads x t steps) share every key, so K and V are
// read from HBM once per (lane, kv head, split) and staged in LDS in tiles of 32 keys: K as
// [key][d], V as [d][key] (its cache layout) so that both MFMA B operands are 16-byte LDS reads. Each
// wave owns 16 query rows:
//   S = Q K^T   v_mfma_f32_16x16x32_bf16, A = Q (registers, loaded once), B = K tile
//   online softmax over the row's keys (base-2, running max m and sum l per row)
//   O += P V    A = P (bf16, re-laid out through a per-wave LDS patch), B = V tile
// With n_split > 1 every workgroup writes its unnormalised O with (m, l) per row and a second
// kernel merges the splits; with one split the workgroup writes the bf16 output directly.

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kAttnRows = 16 * kAttnWaves;  // query rows per workgroup
constexpr int kAttnKeys = 32;               // keys per staged tile
constexpr int kAttnBlock = 16;              // KV cache block size

template <int HD>
struct AttnGeom {
  static constexpr int kDs = HD / 32;                     // d steps of the QK^T MFMA
  static constexpr int kDt = HD / 16;                     // d tiles of the PV MFMA
  static constexpr int kKRow = HD * 2 + 16;               // K tile row (one key), padded
  static constexpr int kVRow = kAttnKeys * 2 + 16;        // V^T tile row (one d), padded
  static constexpr int kPRow = kAttnKeys * 2 + 16;        // P patch row (one query row)
  static constexpr int kKBytes = kAttnKeys * kKRow;
  static constexpr int kVBytes = HD * kVRow;
  static constexpr int kPBytes = 16 * kPRow;
  static constexpr int kPieces = kAttnKeys * HD * 2 / 16;  // 16-byte pieces of one K (or V) tile
  static constexpr int kLoads = kPieces / kAttnThreads;    // per thread and tensor
  static_assert(kLoads >= 1 && kPieces % kAttnThreads == 0, "tile must split evenly");
};

// Key range [k0, k1) of split `sp` of a lane whose keys are [0, ctx): splits of whole tiles.
__device__ __host__ inline void attn_split_range(int ctx, int n_split, int sp, int& k0, int& k1) {
  const int tiles = (ctx + kAttnKeys - 1) / kAttnKeys;
  const int per = (tiles + n_split - 1) / n_split;
  k0 = min(sp * per * kAttnKeys, ctx);
  k1 = min((sp + 1) * per * kAttnKeys, ctx);
}

// Max / sum over the 16 lanes of a DPP row (lanes 16r .. 16r + 15), every lane getting the
// result: quad_perm swaps (xor 1, xor 2) combine each quad, row_half_mirror (lane i with 7 - i
// inside each 8) the two quads of a half, row_mirror (i with 15 - i) the two halves. Register
// moves, no LDS round trip.
template <int CTRL>
__device__ inline float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

__device__ inline float row16_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
  return v;
}

__device__ inline float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return v;
}

// Where the query rows come from and the output rows go: element d of (lane b, q head h, step s)
// is at b * sb + h * sh + s * st + d of each tensor (unit stride over d). With `gate`, the stored
// output is bf16(bf16(o) * bf16(sigmoid(gate))), the rounding of the torch chain
// `out * torch.sigmoid(gate)` on bf16 tensors (`model.py:2158-2290`).
struct AttnRows {
  int64_t sb, sh, st;
  __device__ inline int64_t at(int b, int h, int s) const { return b * sb + h * sh + s * st; }
};
struct AttnIO {
  const uint16_t* q;
  AttnRows qr;
  uint16_t* out;
  AttnRows orow;
  const uint16_t* gate;  // may be null
  AttnRows gr;
};

__device__ inline uint16_t attn_out_value(const AttnIO& io, float v, int b, int h, int s, int d) {
  if (!io.gate) return f32_to_bf16(v);
  const float g = bf16_to_f32(io.gate[io.gr.at(b, h, s) + d]);
  const float sg = bf16_to_f32(f32_to_bf16(1.f / (1.f + expf(-g))));
  return f32_to_bf16(bf16_to_f32(f32_to_bf16(v)) * sg);
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void k_paged_attention(
    AttnIO io, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, int64_t pool_rows, const int32_t* __restrict__ table,
    int table_stride, const int64_t* __restrict__ base_pos, int t, int heads, int kvh,
    float scale_log2, int n_split, int row_groups, float* __restrict__ part_o,
    float* __restrict__ part_ml) {
  using G = AttnGeom<HD>;
  __shared__ __attribute__((aligned(16))) uint8_t ks[G::kKBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vs[G::kVBytes];
  __shared__ __attribute__((aligned(16))) uint8_t ps[kAttnWaves][G::kPBytes];
  const int group = heads / kvh, R = group * t;
  int id = blockIdx.x;
  const int rg = id % row_groups;
  id /= row_groups;
  const int kh = id % kvh, b = id / kvh;
  const int sp = blockIdx.y;
  const int tid = threadIdx.x, wave = uniform(tid / kWave), lane = tid & (kWave - 1);
  const int g = lane >> 4, c = lane & 15;
  const int64_t bp = base_pos[b];
  const int ctx = (int)bp + t;
  int k0, k1;
  attn_split_range(ctx, n_split, sp, k0, k1);
  if (k0 >= k1) return;  // uniform: an empty split writes nothing (the merge skips it)

  // this wave's query rows r = 64 rg + 16 wave + (0..15); row r = (q head kh*group + r / t,
  // step r % t). Lanes of A (row c) load their row; rows past R read zeros.
  const int rbase = kAttnRows * rg + 16 * wave;
  const int ra = rbase + c;
  const bool wave_live = rbase < R;  // uniform
  bf16x8_t qa[G::kDs];
  {
    const bool live = ra < R;
    const int hq = kh * group + (live ? ra / t : 0), st = live ? ra % t : 0;
    const uint16_t* qrow = io.q + io.qr.at(b, hq, st);
#pragma unroll
    for (int ds = 0; ds < G::kDs; ++ds)
      qa[ds] = live ? as_bf16x8(ld16(qrow + 32 * ds + 8 * g)) : as_bf16x8(zero16());
  }
  // D-layout rows of this lane: 4g + i; their positions (rows past R are masked everywhere)
  int qpos[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rbase + 4 * g + i;
    qpos[i] = r < R ? (int)bp + r % t : -1;
  }
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }
  f32x4_t o[G::kDt];
#pragma unroll
  for (int dt = 0; dt < G::kDt; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // staging of a 32-key tile = two 16-row cache blocks, whose physical ids (p0, p1) are two
  // scalar table reads. K [rows, kvh, HD]: piece p = j * 256 + tid is key p / (HD / 8),
  // 16-byte column p % (HD / 8), so a wave instruction reads whole key rows. V is stored
  // transposed per block, [blocks, kvh, HD, 16]: a block's slab for this kv head is HD rows of
  // 16 keys (HD * 32 contiguous bytes), and piece p is block p / (2 HD), channel d = (p % 2HD) / 2,
  // keys 8 ((p % 2HD) % 2) .. + 7: 16 contiguous bytes that land unchanged in LDS row d of the
  // [d][key] tile the PV MFMA reads. Keys at or past k1 are zero in both tiles.
  constexpr int kCols = HD / 8;
  const uint32_t pool_bytes = (uint32_t)min(pool_rows * kvh * HD * 2, (int64_t)0x7fffffff);
  const rsrc_t rk = make_rsrc(k_pool, pool_bytes), rv = make_rsrc(v_pool, pool_bytes);
  const int32_t* const trow = table + (int64_t)b * table_stride;
  auto tile_blocks = [&](int key0, int& p0, int& p1) {
    const int blk = key0 / kAttnBlock;
    p0 = sload(trow, min(blk, table_stride - 1));  // never past the lane's table row
    p1 = sload(trow, min(blk + 1, table_stride - 1));
  };
  u32x4_t kreg[G::kLoads], vreg[G::kLoads];
  auto stage_load = [&](int key0, int p0, int p1) {
#pragma unroll
    for (int j = 0; j < G::kLoads; ++j) {
      const int p = j * kAttnThreads + tid;
      const int kk = p / kCols, col = p % kCols;
      const int64_t krow = (int64_t)(kk < kAttnBlock ? p0 : p1) * kAttnBlock + kk % kAttnBlock;
      kreg[j] = buf16(rk, key0 + kk < k1 ? (uint32_t)(((krow * kvh + kh) * HD + col * 8) * 2)
                                         : kOutOfRange);
      const int bsel = p / (2 * HD), q2 = p % (2 * HD), d = q2 >> 1, half = q2 & 1;
      const int64_t vblk = bsel ? p1 : p0;
      vreg[j] = buf16(rv, key0 + kAttnBlock * bsel + 8 * half < k1
                              ? (uint32_t)((((vblk * kvh + kh) * HD + d) * kAttnBlock + 8 * half) * 2)
                              : kOutOfRange);
    }
  };
  auto stage_store = [&](int key0) {
#pragma unroll
    for (int j = 0; j < G::kLoads; ++j) {
      const int p = j * kAttnThreads + tid;
      lds16_store(ks + (p / kCols) * G::kKRow + (p % kCols) * 16, kreg[j]);
      const int bsel = p / (2 * HD), q2 = p % (2 * HD), d = q2 >> 1, half = q2 & 1;
      const int kfirst = key0 + kAttnBlock * bsel + 8 * half;
      u32x4_t vv = vreg[j];
      if (kfirst + 8 > k1) {  // the piece that straddles k1: zero its keys past the end
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = kfirst + 2 * e < k1 ? 0x0000ffffu : 0u;
          const uint32_t hi = kfirst + 2 * e + 1 < k1 ? 0xffff0000u : 0u;
          vv[e] &= lo | hi;
        }
      }
      lds16_store(vs + d * G::kVRow + (kAttnBlock * bsel + 8 * half) * 2, vv);
    }
  };

  uint8_t* const pw = ps[wave];
  int p0, p1;
  tile_blocks(k0, p0, p1);
  stage_load(k0, p0, p1);
  for (int key0 = k0; key0 < k1; key0 += kAttnKeys) {
    const int kn = key0 + kAttnKeys;
    if (kn < k1) tile_blocks(kn, p0, p1);  // scalar reads, ready by the next stage_load
    __syncthreads();  // the previous tile's LDS reads are done
    stage_store(key0);
    __syncthreads();
    if (kn < k1) stage_load(kn, p0, p1);  // next tile in flight meanwhile
    // A wave whose 16 query rows all lie past R (t = 1: 16 rows per kv head, one wave's worth)
    // stages its share of each tile and skips the tile's math and LDS reads.
    if (!wave_live) continue;

    // S = Q K^T for keys key0 + (0..15) and key0 + 16 + (0..15)
    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < G::kDs; ++ds) {
      const bf16x8_t kb0 = as_bf16x8(lds16(ks + c * G::kKRow + (32 * ds + 8 * g) * 2));
      const bf16x8_t kb1 = as_bf16x8(lds16(ks + (16 + c) * G::kKRow + (32 * ds + 8 * g) * 2));
      s0 = mfma16x16x32(qa[ds], kb0, s0);
      s1 = mfma16x16x32(qa[ds], kb1, s1);
    }
    // online softmax, base 2: row 4g + i, keys c and 16 + c of this lane. m is the row max
    // (uniform over the row's 16 lanes); l is this lane's own share of the row sum, reduced
    // over the 16 lanes once, after the last tile.
    const int pa = key0 + c, pb = key0 + 16 + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool la = pa < k1 && pa <= qpos[i], lb = pb < k1 && pb <= qpos[i];
      const float xa = la ? s0[i] * scale_log2 : -INFINITY;
      const float xb = lb ? s1[i] * scale_log2 : -INFINITY;
      const float tm = row16_max(fmaxf(xa, xb));
      const float mn = fmaxf(m[i], tm);
      const float alpha = mn == -INFINITY ? 1.f : exp2f(m[i] - mn);
      const float ea = la ? exp2f(xa - mn) : 0.f;
      const float eb = lb ? exp2f(xb - mn) : 0.f;
      l[i] = l[i] * alpha + (ea + eb);
      m[i] = mn;
#pragma unroll
      for (int dt = 0; dt < G::kDt; ++dt) o[dt][i] *= alpha;
      // P row 4g + i, keys c and 16 + c, as bf16 into the wave's patch
      *reinterpret_cast<__bf16*>(pw + (4 * g + i) * G::kPRow + c * 2) = (__bf16)ea;
      *reinterpret_cast<__bf16*>(pw + (4 * g + i) * G::kPRow + (16 + c) * 2) = (__bf16)eb;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // the wave's own patch writes, before reading them back
    const bf16x8_t pa8 = as_bf16x8(lds16(pw + c * G::kPRow + 8 * g * 2));
    // O += P V: B = V[keys 8g .. 8g + 7][d = 16 dt + c] from the transposed tile
#pragma unroll
    for (int dt = 0; dt < G::kDt; ++dt) {
      const bf16x8_t vb = as_bf16x8(lds16(vs + (16 * dt + c) * G::kVRow + 8 * g * 2));
      o[dt] = mfma16x16x32(pa8, vb, o[dt]);
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) l[i] = row16_sum(l[i]);
  // rows 4g + i of this lane: o[dt][i] is d = 16 dt + c
  const int64_t slot = ((int64_t)(b * kvh + kh) * row_groups + rg) * n_split + sp;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rl = 16 * wave + 4 * g + i;  // row within the workgroup
    const int r = kAttnRows * rg + rl;
    if (r >= R) continue;
    if (n_split == 1) {
      const float inv = 1.f / l[i];
      const int hq = kh * group + r / t, st = r % t;
      uint16_t* orow = io.out + io.orow.at(b, hq, st);
#pragma unroll
      for (int dt = 0; dt < G::kDt; ++dt)
        orow[16 * dt + c] = attn_out_value(io, o[dt][i] * inv, b, hq, st, 16 * dt + c);
    } else {
      float* po = part_o + (slot * kAttnRows + rl) * HD;
#pragma unroll
      for (int dt = 0; dt < G::kDt; ++dt) po[16 * dt + c] = o[dt][i];
      if (c == 0) {
        part_ml[(slot * kAttnRows + rl) * 2] = m[i];
        part_ml[(slot * kAttnRows + rl) * 2 + 1] = l[i];
      }
    }
  }
}

// Merge of the key splits: out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s,
// over the splits that hold keys of the row's lane. One thread per (row, 4 d values).
template <int HD>
__global__ __launch_bounds__(256) void k_attention_merge(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const int64_t* __restrict__ base_pos, int B, int t, int heads, int kvh, int n_split,
    int row_groups, AttnIO io) {
  const int group = heads / kvh;
  const int64_t rows = (int64_t)B * heads * t;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * (HD / 4)) return;
  const int64_t row = idx / (HD / 4);
  const int d = (int)(idx % (HD / 4)) * 4;
  const int st = (int)(row % t);
  const int64_t bh = row / t;
  const int hq = (int)(bh % heads), b = (int)(bh / heads);
  const int kh = hq / group, r = (hq % group) * t + st;
  const int rg = r / kAttnRows, rl = r % kAttnRows;
  const int ctx = (int)base_pos[b] + t;
  const int64_t base = ((int64_t)(b * kvh + kh) * row_groups + rg) * n_split;
  float mx = -INFINITY;
  for (int sp = 0; sp < n_split; ++sp) {
    int k0, k1;
    attn_split_range(ctx, n_split, sp, k0, k1);
    if (k0 < k1) mx = fmaxf(mx, part_ml[((base + sp) * kAttnRows + rl) * 2]);
  }
  float lsum = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < n_split; ++sp) {
    int k0, k1;
    attn_split_range(ctx, n_split, sp, k0, k1);
    if (k0 >= k1) continue;
    const int64_t pr = (base + sp) * kAttnRows + rl;
    const float ms = part_ml[pr * 2];
    const float w = ms == -INFINITY ? 0.f : exp2f(ms - mx);
    lsum += part_ml[pr * 2 + 1] * w;
    const float* po = part_o + pr * HD + d;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += po[e] * w;
  }
  const float inv = 1.f / lsum;
  uint16_t* orow = io.out + io.orow.at(b, hq, st) + d;
#pragma unroll
  for (int e = 0; e < 4; ++e) orow[e] = attn_out_value(io, acc[e] * inv, b, hq, st, d + e);
}

// Workgroups of k_paged_attention<HD> resident on the whole device at once.
int attention_slots(int hd) {
  static int occ[3] = {0, 0, 0};
  const int i = hd == 64 ? 0 : hd == 128 ? 1 : 2;
  if (occ[i] == 0) {
    occ[i] = hd == 64    ? occupancy_per_cu(k_paged_attention<64>, kAttnThreads)
             : hd == 128 ? occupancy_per_cu(k_paged_attention<128>, kAttnThreads)
                         : occupancy_per_cu(k_paged_attention<256>, kAttnThreads);
    if (occ[i] < 1) occ[i] = 1;
  }
  return device_cu_count() * occ[i];
}

// The largest key-split count whose workgroups all run in one round of resident slots, at
// least 8 tiles per split and at most 64 splits. A second, partly filled round leaves CUs idle
// for its whole length, and every extra split adds partials to the merge: at 48 lanes, 2 kv
// heads of 256 and 8192 keys (96 workgroups per split, 512 slots), 5 splits take 179 us per
// call against 199 us for 8 and 10 and 220 us for 12 and 16.
int attention_splits(int hd, int64_t B, int64_t kvh, int row_groups, int64_t max_ctx) {
  const int64_t wgs = B * kvh * row_groups;
  const int64_t fit = attention_slots(hd) / (wgs > 0 ? wgs : 1);
  const int64_t tiles = (max_ctx + kAttnKeys - 1) / kAttnKeys;
  const int64_t cap = tiles / 8 > 1 ? tiles / 8 : 1;  // at least 8 tiles per split
  int64_t n = fit < cap ? fit : cap;
  if (n > 64) n = 64;
  return n < 1 ? 1 : (int)n;
}

template <int HD>
int launch_attention(const AttnIO& io, const uint16_t* k_pool, const uint16_t* v_pool,
                     int64_t pool_rows, const int32_t* table, int table_stride,
                     const int64_t* base_pos, int B, int t, int heads, int kvh, float scale,
                     int n_split, float* part_o, float* part_ml, hipStream_t st) {
  const int row_groups = (heads / kvh * t + kAttnRows - 1) / kAttnRows;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(k_paged_attention<HD>, dim3(B * kvh * row_groups, n_split), dim3(kAttnThreads),
                     0, st, io, k_pool, v_pool, pool_rows, table, table_stride, base_pos, t, heads,
                     kvh, scale_log2, n_split, row_groups, part_o, part_ml);
  int rc = status_of(hipGetLastError());
  if (rc || n_split == 1) return rc;
  const int64_t threads = (int64_t)B * heads * t * (HD / 4);
  hipLaunchKernelGGL(k_attention_merge<HD>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     part_o, part_ml, base_pos, B, t, heads, kvh, n_split, row_groups, io);
  return status_of(hipGetLastError());
}

// This round's K and V rows into the paged caches (the cache writes of `attn_verify`,
// model.py:3519-3577, and `graph_mtp.py:857-860`): row (b, s) at position base_pos[b] + s goes to
// pool row table[b][pos / 16] * 16 + pos % 16, K as a [kv_heads, HD] row, V into channel d,
// slot pos % 16 of its block's transposed [kv_heads, HD, 16] slab. keep (optional, [B, t] at
// element strides keep_b, keep_s) leaves rows with keep == 0 untouched. A thread moves 8 channels of one (row, kv head); a
// position outside the table or a block outside the pool is not written.
__global__ __launch_bounds__(256) void k_kv_write(const uint16_t* __restrict__ k, int64_t k_row,
                                                  const uint16_t* __restrict__ v, int64_t v_row,
                                                  uint16_t* __restrict__ k_pool,
                                                  uint16_t* __restrict__ v_pool, int64_t pool_rows,
                                                  const int32_t* __restrict__ table, int table_stride,
                                                  const int64_t* __restrict__ base_pos,
                                                  const uint8_t* __restrict__ keep, int64_t keep_b,
                                                  int64_t keep_s, int B, int t, int kvh, int hd) {
  const int pieces = hd / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)B * t * kvh * pieces) return;
  const int piece = (int)(i % pieces);
  const int64_t rh = i / pieces;  // (row, kv head)
  const int h = (int)(rh % kvh);
  const int64_t row = rh / kvh;
  const int b = (int)(row / t), s = (int)(row - (int64_t)b * t);
  if (keep && !keep[b * keep_b + s * keep_s]) return;
  const int64_t pos = base_pos[b] + s;
  if (pos < 0 || pos / kAttnBlock >= table_stride) return;
  const int64_t blk = table[(int64_t)b * table_stride + pos / kAttnBlock];
  const int slot = (int)(pos % kAttnBlock);
  if (blk < 0 || (blk + 1) * kAttnBlock > pool_rows) return;
  const int d = piece * 8;
  const u32x4_t kv = ld16(k + row * k_row + h * hd + d);
  const u32x4_t vv = ld16(v + row * v_row + h * hd + d);
  *reinterpret_cast<u32x4_t*>(k_pool + ((blk * kAttnBlock + slot) * kvh + h) * hd + d) = kv;
  uint16_t* vs = v_pool + ((blk * kvh + h) * hd + d) * kAttnBlock + slot;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    vs[(2 * e) * kAttnBlock] = (uint16_t)(vv[e] & 0xffffu);
    vs[(2 * e + 1) * kAttnBlock] = (uint16_t)(vv[e] >> 16);
  }
}

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int mtpk_attention_splits(int64_t batch, int64_t t, int64_t heads, int64_t kv_heads,
                          int64_t head_dim, int64_t max_ctx) {
  if (batch <= 0 || t <= 0 || kv_heads <= 0 || heads % kv_heads) return 0;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
  const int row_groups = (int)((heads / kv_heads * t + kAttnRows - 1) / kAttnRows);
  return attention_splits((int)head_dim, batch, kv_heads, row_groups, max_ctx);
}

int64_t mtpk_attention_workspace_bytes(int64_t batch, int64_t t, int64_t heads, int64_t kv_heads,
                                       int64_t head_dim, int n_split) {
  if (batch <= 0 || t <= 0 || kv_heads <= 0 || heads % kv_heads || n_split <= 1) return 0;
  const int64_t row_groups = (heads / kv_heads * t + kAttnRows - 1) / kAttnRows;
  const int64_t slots = batch * kv_heads * row_groups * n_split * kAttnRows;
  return slots * (head_dim + 2) * 4;
}

namespace {

int paged_attention_io(const AttnIO& io, int64_t batch, int64_t t, int64_t heads, int64_t kv_heads,
                       int64_t head_dim, const uint16_t* k_pool, const uint16_t* v_pool,
                       int64_t pool_rows, const int32_t* block_table, int64_t table_stride,
                       const int64_t* base_pos, float scale, int n_split, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  if (!io.q || !k_pool || !v_pool || !block_table || !base_pos || !io.out) return MTPK_EINVAL;
  if (batch < 0 || t <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads) return MTPK_EINVAL;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return MTPK_EINVAL;
  if (pool_rows <= 0 || pool_rows * kv_heads * head_dim * 2 > 0x7fffffffLL) return MTPK_EINVAL;
  if (table_stride <= 0 || n_split < 1 || n_split > 64 || !(scale > 0.f)) return MTPK_EINVAL;
  if (!aligned16(io.q) || !aligned16(k_pool) || !aligned16(v_pool)) return MTPK_EINVAL;
  // 16-byte q loads: every q row starts on a 16-byte boundary
  if (io.qr.sb % 8 || io.qr.sh % 8 || io.qr.st % 8) return MTPK_EINVAL;
  if (batch * heads * t > INT32_MAX / 64) return MTPK_EINVAL;
  if (n_split > 1 &&
      (!workspace || workspace_bytes < mtpk_attention_workspace_bytes(batch, t, heads, kv_heads,
                                                                      head_dim, n_split)))
    return MTPK_EINVAL;
  if (batch == 0) return 0;
  const int64_t rg = (heads / kv_heads * t + kAttnRows - 1) / kAttnRows;
  float* part_o = (float*)workspace;
  float* part_ml = part_o ? part_o + batch * kv_heads * rg * n_split * kAttnRows * head_dim : nullptr;
  const hipStream_t st = (hipStream_t)stream;
#define MTPK_ATTN(HD_)                                                                          \
  launch_attention<HD_>(io, k_pool, v_pool, pool_rows, block_table, (int)table_stride, base_pos, \
                        (int)batch, (int)t, (int)heads, (int)kv_heads, scale, n_split, part_o,   \
                        part_ml, st)
  switch (head_dim) {
    case 64: return MTPK_ATTN(64);
    case 128: return MTPK_ATTN(128);
    default: return MTPK_ATTN(256);
  }
#undef MTPK_ATTN
}

}  // namespace

int mtpk_paged_attention(const uint16_t* q, int64_t batch, int64_t t, int64_t heads,
                         int64_t kv_heads, int64_t head_dim, const uint16_t* k_pool,
                         const uint16_t* v_pool, int64_t pool_rows, const int32_t* block_table,
                         int64_t table_stride, const int64_t* base_pos, float scale, int n_split,
                         void* workspace, int64_t workspace_bytes, uint16_t* out, void* stream) {
  const AttnRows dense{heads * t * head_dim, t * head_dim, head_dim};  // [B, heads, t, HD]
  const AttnIO io{q, dense, out, dense, nullptr, dense};
  return paged_attention_io(io, batch, t, heads, kv_heads, head_dim, k_pool, v_pool, pool_rows,
                            block_table, table_stride, base_pos, scale, n_split, workspace,
                            workspace_bytes, stream);
}

int mtpk_paged_attention_gated(const uint16_t* q, const int64_t* q_strides, const uint16_t* gate,
                               const int64_t* gate_strides, int64_t batch, int64_t t,
                               int64_t heads, int64_t kv_heads, int64_t head_dim,
                               const uint16_t* k_pool, const uint16_t* v_pool, int64_t pool_rows,
                               const int32_t* block_table, int64_t table_stride,
                               const int64_t* base_pos, float scale, int n_split, void* workspace,
                               int64_t workspace_bytes, uint16_t* out, const int64_t* out_strides,
                               void* stream) {
  if (!q_strides || !out_strides || (gate && !gate_strides)) return MTPK_EINVAL;
  const AttnRows qr{q_strides[0], q_strides[1], q_strides[2]};
  const AttnRows orow{out_strides[0], out_strides[1], out_strides[2]};
  const AttnRows gr = gate ? AttnRows{gate_strides[0], gate_strides[1], gate_strides[2]} : orow;
  const AttnIO io{q, qr, out, orow, gate, gr};
  return paged_attention_io(io, batch, t, heads, kv_heads, head_dim, k_pool, v_pool, pool_rows,
                            block_table, table_stride, base_pos, scale, n_split, workspace,
                            workspace_bytes, stream);
}

int mtpk_kv_write(const uint16_t* k, int64_t k_row_stride, const uint16_t* v, int64_t v_row_stride,
                  uint16_t* k_pool, uint16_t* v_pool, int64_t pool_rows, const int32_t* block_table,
                  int64_t table_stride, const int64_t* base_pos, const uint8_t* keep, int64_t keep_b,
                  int64_t keep_s, int64_t batch, int64_t t, int64_t kv_heads, int64_t head_dim,
                  void* stream) {
  if (!k || !v || !k_pool || !v_pool || !block_table || !base_pos) return MTPK_EINVAL;
  if (batch < 0 || t <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 8) return MTPK_EINVAL;
  if (k_row_stride < kv_heads * head_dim || v_row_stride < kv_heads * head_dim ||
      k_row_stride % 8 || v_row_stride % 8)
    return MTPK_EINVAL;
  if (!aligned16(k) || !aligned16(v) || !aligned16(k_pool) || pool_rows <= 0 || pool_rows % kAttnBlock)
    return MTPK_EINVAL;
  if (table_stride <= 0 || table_stride > INT32_MAX || batch * t * kv_heads * head_dim > INT32_MAX)
    return MTPK_EINVAL;
  if (keep && (keep_b < 0 || keep_s < 0)) return MTPK_EINVAL;
  if (batch == 0) return 0;
  const int64_t n = batch * t * kv_heads * (head_dim / 8);
  hipLaunchKernelGGL(k_kv_write, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     k, k_row_stride, v, v_row_stride, k_pool, v_pool, pool_rows, block_table,
                     (int)table_stride, base_pos, keep, keep_b, keep_s, (int)batch, (int)t,
                     (int)kv_heads, (int)head_dim);
  return status_of(hipGetLastError());
}

}  // extern "C"
