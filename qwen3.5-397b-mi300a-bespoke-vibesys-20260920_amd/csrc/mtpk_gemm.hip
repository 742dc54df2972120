// bf16 weight-streaming GEMM for few token rows on gfx950: Y[M, N] = X[M, K] . W[N, K]^T with
// M <= 256, the shape of the MTP draft step's projections (M = B = 48), the verify step's
// (M = B (k + 1) = 192), the LM head (`greedy_token`, mtp.py:640-658; N = vocab) and the shared
// expert / router of a decode or draft MoE layer (model.py:2811-2873). These are weight-
// bandwidth bound: every weight byte is read from HBM once, and the token rows are the MFMA's
// other operand. Above 64 rows the rows are split into groups of 64, one workgroup per
// (weight tile, row group).
//
// Workgroup = NW = 4 or 8 waves, tile = 16 NW weight rows (wave w: rows 16 w .. + 15; with the
// paired SiLU epilogue also the matching 16 "up" rows N/2 + ...) x all M tokens (TT = ceil(M / 16) MFMA token
// tiles). v_mfma_f32_16x16x32_bf16 with the lane layout of the MoE kernels: lane (g, c) supplies
// K positions 8 g .. 8 g + 7 of each 32-K step, for weight row c (B) and token row c of a tile (A).
// The token rows are staged in LDS in chunks of 256 K (double-buffered, one barrier per chunk);
// the weights stream through a ring of D = 8 steps (16 bytes per lane per step) per wave. Chunk
// c + 2 is loaded at the end of chunk c after that point's ring refills and stored at the end of
// chunk c + 1, when every ring load issued before it has been consumed (vmcnt retires in order).
//
// Split-K: grid.y = KS workgroups share a tile's K range; with KS > 1 each writes fp32 partials
// [KS, M, cols] and k_gemm_reduce sums them in split order and applies the epilogue, so the
// result does not depend on scheduling.
// Epilogues: 0 store, 1 out[m, j] = silu(y[m, j]) * y[m, N/2 + j] (j < N/2), 2 argmax over n of
// bf16(y[m, n]) with the first-occurrence rule (one key per row and tile, then a max over tiles),
// i.e. the argmax of the bf16 logits this kernel would store.

#include "mtpk_gemm_tile.h"
#include "mtpk_layer.h"

namespace mtpk {

template <int TT, int S, int NW, bool SILU>
__global__ __launch_bounds__(NW * kWave, 16 / NW) void k_gemm_skinny(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[GemmSmem<TT, NW>::kBytes];
  gemm_tile<TT, S, NW, SILU>(a, smem, blockIdx.x, blockIdx.y);
}

// Two GEMMs of the same token rows in one launch (the MoE layer's router and shared gate_up):
// workgroups [0, a_blocks) are the tiles of `a` (store epilogue), the rest those of `b` (SiLU
// pairing). Each workgroup runs one tile exactly as the GEMM's own launch would, so both leave
// the same partials.
template <int TT>
__global__ __launch_bounds__(4 * kWave, 4) void k_gemm_pair(GemmArgs a, GemmArgs b, int a_blocks,
                                                            int a_gx, int b_gx) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[GemmSmem<TT, 4>::kBytes];
  const int idx = blockIdx.x;
  if (idx < a_blocks)
    gemm_tile<TT, 1, 4, false>(a, smem, idx % a_gx, idx / a_gx);
  else
    gemm_tile<TT, 2, 4, true>(b, smem, (idx - a_blocks) % b_gx, (idx - a_blocks) / b_gx);
}

int launch_gemm_pair(const GemmArgs& a, const GemmArgs& b, hipStream_t st) {
  const int a_gx = (int)gemm_grid_x(a.tiles, a.RG), b_gx = (int)gemm_grid_x(b.tiles, b.RG);
  const int a_blocks = a_gx * a.KS;
  const unsigned grid = (unsigned)(a_blocks + b_gx * b.KS);
  switch (gemm_tt(a.M)) {
    case 1: hipLaunchKernelGGL(k_gemm_pair<1>, dim3(grid), dim3(4 * kWave), 0, st, a, b, a_blocks, a_gx, b_gx); break;
    case 2: hipLaunchKernelGGL(k_gemm_pair<2>, dim3(grid), dim3(4 * kWave), 0, st, a, b, a_blocks, a_gx, b_gx); break;
    case 3: hipLaunchKernelGGL(k_gemm_pair<3>, dim3(grid), dim3(4 * kWave), 0, st, a, b, a_blocks, a_gx, b_gx); break;
    default: hipLaunchKernelGGL(k_gemm_pair<4>, dim3(grid), dim3(4 * kWave), 0, st, a, b, a_blocks, a_gx, b_gx); break;
  }
  return status_of(hipGetLastError());
}

// The wide form (`gemm_wide`, 17..192 token rows on wide N: the LM heads of the draft step, 48
// rows, and of the verify step, 192 rows).
// One workgroup of NW waves per 16 NW RT weight rows, one workgroup per CU. Wave w owns weight
// rows 16 RT w .. + 16 RT - 1 (RT row tiles) against all TT token tiles, so one staged A
// fragment feeds RT MFMAs and one weight fragment TT.
//  - Weights: a register ring of D steps of 32 K (RT 16-byte loads per lane per step), as the
//    other weight streams here.
//  - Token rows: direct-to-LDS buffer loads (no registers held), KC-K chunks of TT x 16 rows x
//    2 KC bytes, NB chunks in flight. The 16-byte piece p of row r sits at slot p ^ (r & 7) of
//    the row, so the A reads of 8 consecutive rows hit distinct banks; every load instruction
//    still covers whole 128-byte lines.
//  - One barrier per chunk: each wave waits (vmcnt) for its own loads of the chunk, the barrier
//    makes all waves' loads visible and also frees the buffer read in the previous chunk, which
//    the chunk NB - 1 ahead is loaded into. The ring's register loads are waited for by the
//    compiler; the chunk wait is exact and keeps the ring and the later chunks in flight.
//  - Tile t walks the K chunks from chunk 7 t mod (K / KC) on: with every tile starting at K = 0
//    all workgroups read the same column range of rows 8 KB apart at the same moment, which
//    measured 583 against 552 us on [192, 4096] x [248320, 4096] (the weight stream alone 524
//    against 449 us). A column's sum order is then its tile's; nothing else depends on it.
// Measured there (graph replay over two weight copies, MI355X): 552 us with the argmax epilogue
// against 496 us for the library GEMM alone and 521 us with its argmax pass; the token rows'
// staging (75% of the weight bytes: 192 rows against 256 per tile, the most the register file
// holds accumulators for) costs about 100 us of it. The verify head's later form (the 8-wave,
// 2-row-tile configuration below) runs it in 506.5 us against 519-520 us for the library GEMM
// and its argmax pass.
// Epilogues: store (fp32 or bf16) or the first-occurrence argmax keys of bf16(y) per tile.
template <int TT, int NW, int RT, int KC, int NB, int D>
struct Wide {
  static constexpr int kRows = 16 * RT * NW;  // weight rows per tile
  static constexpr int kChunk = TT * 16 * KC * 2;
  static constexpr int kLoads = kChunk / 1024 / NW;  // direct loads per wave per chunk
  static constexpr int kSteps = KC / 32;            // ring steps per chunk
  static constexpr int kTurn = D / kSteps;          // chunks per loop turn
  static constexpr int kKeys = NB * kChunk;
  static constexpr int kBytes = kKeys + NW * TT * 16 * 8;
};
// 8 waves x 2 row tiles (two waves per SIMD, 195 VGPRs) measured 566-575 us against 637 us for
// 4 waves x 4 row tiles (accumulators shuffled between AGPRs and VGPRs in the loop); NB = 3
// against 4, D = 8 against 4 and 128-K chunks were equal or slower.
// At <= 64 rows (4 token tiles) the same form with RT = 4, 512-row tiles (194 VGPRs, one
// workgroup per CU): 372-373 us at 48 rows against 393-395 us with RT = 2, where the token rows
// are staged for twice as many tiles; NB = 4, 128-K chunks and 3 token tiles of 256-K chunks
// were equal or slower.
constexpr int kWideNW = 8, kWideKC = 64, kWideNB = 3, kWideD = 4;
constexpr int kWideKStep = kWideKC * (kWideD / (kWideKC / 32));  // K per loop turn

template <int TT, int NW, int RT, int KC, int NB, int D>
__global__ __launch_bounds__(NW * kWave, 1) void k_gemm_wide(GemmArgs a) {
  using C = Wide<TT, NW, RT, KC, NB, D>;
  constexpr int kChunk = C::kChunk, kLoads = C::kLoads, kSteps = C::kSteps, kTurn = C::kTurn;
  static_assert(kLoads * 1024 * NW == kChunk, "chunk split over the waves");
  static_assert(D % kSteps == 0 && NB >= 2, "ring depth in whole chunks");
  // Loads this wave issued after its loads of chunk c, at the chunk's wait: (NB - 2) chunks
  // and D RT ring loads plus kSteps RT per chunk already looped, for the prologue's chunks, and
  // (NB - 2) chunks plus (NB - 1) kSteps RT ring loads in the steady state. The smallest is exact
  // where it applies and waits only for consumed ring steps elsewhere.
  constexpr int kChunkWait = (NB - 2) * kLoads + RT * (D < kSteps * (NB - 1) ? D : kSteps * (NB - 1));
  static_assert(kChunkWait < 64, "vmcnt is a 6-bit counter");
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::kBytes];
  uint64_t(*kred)[TT * 16] = reinterpret_cast<uint64_t(*)[TT * 16]>(smem + C::kKeys);
  const int tid = threadIdx.x, wave = uniform(tid / kWave), lane = tid & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  const int tile = blockIdx.x;
  const int K = a.K, nchunk = K / KC, nstep = K / 32;
  const int rot = (int)(((int64_t)tile * 7) % nchunk);  // this tile's first chunk
  int wrow[RT];
  bool wok[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int row = tile * C::kRows + 16 * RT * wave + 16 * r + ln.c;
    wok[r] = row < a.N;
    wrow[r] = wok[r] ? row : 0;
  }
  const rsrc_t rw = make_rsrc(a.w, 0x7fffffff);
  const rsrc_t rx = make_rsrc(a.x, (uint32_t)((int64_t)a.M * K * 2));
  // weight step st (the st-th of this tile's rotated order): K = 32 st' + 8 g .. + 7 of row wrow[r]
  auto issue = [&](u32x4_t* v, int st) {
    const bool in = st < nstep;
    const int sr = (st + rot * kSteps) % nstep;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const uint32_t off = (uint32_t)(((int64_t)wrow[r] * K + 32 * sr + 8 * ln.g) * 2);
      v[r] = buf16(rw, (wok[r] && in) ? off : kOutOfRange);
    }
  };
  // chunk c into buffer c % NB: load j of this wave fills LDS bytes [1024 q, 1024 q + 1024) of
  // the chunk, q = kLoads wave + j: row (1024 q + 16 L) / (2 KC), slot s of that row <- piece
  // s ^ (row & 7)
  constexpr int kPieces = KC / 8;  // 16-byte pieces per row
  auto stage = [&](int c) {
    uint8_t* buf = smem + (c % NB) * kChunk;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int q = kLoads * wave + j, slot16 = 64 * q + lane;
      const int row = slot16 / kPieces, slot = slot16 % kPieces;
      const int piece = slot ^ (row & 7);
      const bool ok = c < nchunk && row < a.M;
      const int cr = (c + rot) % nchunk;
      buf16_lds(rx, ok ? (uint32_t)(((int64_t)row * K + cr * KC + piece * 8) * 2) : kOutOfRange,
                buf + 1024 * q);
    }
  };

  f32x4_t acc[RT][TT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[r][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // prologue: chunks 0 .. NB - 2, then D ring steps
#pragma unroll
  for (int c = 0; c < NB - 1; ++c) stage(c);
  ring_fence();
  u32x4_t ring[D][RT];
#pragma unroll
  for (int st = 0; st < D; ++st) issue(ring[st], st);
  ring_fence();

  // kTurn chunks per loop turn, so every ring slot index is a constant (a register array
  // indexed at run time would live in scratch); K is a multiple of kTurn KC (checked on launch)
  int c0 = 0;
#pragma clang loop unroll(disable)
  do {
#pragma unroll
    for (int h = 0; h < kTurn; ++h) {
      const int c = c0 + h;
      vmcnt_wait<kChunkWait>();  // this wave's loads of chunk c have landed
      __builtin_amdgcn_s_barrier();  // ... and every wave's; buffer (c - 1) % NB is free
      __asm__ volatile("" ::: "memory");  // no LDS read moves above the barrier
      ring_fence();
      stage(c + NB - 1);
      ring_fence();
      const uint8_t* buf = smem + (c % NB) * kChunk;
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        u32x4_t* slot = ring[h * kSteps + u];
        u32x4_t av[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          const int row = 16 * t + ln.c;
          av[t] = lds16(buf + row * (KC * 2) + (((4 * u + ln.g) ^ (row & 7)) * 16));
        }
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
          for (int t = 0; t < TT; ++t)
            acc[r][t] = mfma16x16x32(as_bf16x8(av[t]), as_bf16x8(slot[r]), acc[r][t]);
        ring_fence();
        issue(slot, c * kSteps + u + D);
        ring_fence();
      }
    }
    c0 += kTurn;
  } while (c0 < nchunk);

  // lane (g, c): acc[r][t][i] is token m = 16 t + 4 g + i, weight row wrow[r]
  if (a.epi == kEpiArgmax) {
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint64_t key = 0;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const float v = bf16_to_f32(f32_to_bf16(acc[r][t][i]));
          const uint64_t kr = wok[r] ? argmax_key(v, (uint32_t)wrow[r]) : 0;
          key = kr > key ? kr : key;
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const uint32_t lo = __shfl_xor((uint32_t)key, o, kWave);
          const uint32_t hi = __shfl_xor((uint32_t)(key >> 32), o, kWave);
          const uint64_t k2 = ((uint64_t)hi << 32) | lo;
          key = k2 > key ? k2 : key;
        }
        if (ln.c == 0) kred[wave][16 * t + 4 * ln.g + i] = key;
      }
    __syncthreads();
    for (int m = tid; m < a.M; m += NW * kWave) {
      uint64_t b = kred[0][m];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) b = kred[w2][m] > b ? kred[w2][m] : b;
      a.keys[(int64_t)m * a.tiles + tile] = b;
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * t + 4 * ln.g + i;
      if (m >= a.M) continue;
#pragma unroll
      for (int r = 0; r < RT; ++r)
        if (wok[r]) store_float(a.out, a.odt, (int64_t)m * a.cols + wrow[r], acc[r][t][i]);
    }
}

template <int TT, int RT>
void launch_wide(const GemmArgs& a, int tiles, hipStream_t st) {
  hipLaunchKernelGGL((k_gemm_wide<TT, kWideNW, RT, kWideKC, kWideNB, kWideD>),
                     dim3((unsigned)tiles), dim3(kWideNW * kWave), 0, st, a);
}

// Split-K reduction: out[m, col] = epilogue(sum over ks of part[ks, m, .]) in split order.
__global__ __launch_bounds__(256) void k_gemm_reduce(const float* __restrict__ part, int KS, int M,
                                                     int cols, int epi, void* __restrict__ out,
                                                     int odt) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * cols) return;
  const int64_t m = idx / cols, col = idx - m * cols;
  store_float(out, odt, m * cols + col, gemm_reduce_value(part, KS, M, cols, epi, m, col));
}

// One workgroup per row: the max over the row's tile keys (thousands for an LM head), strided
// over the threads, then over the waves.
__global__ __launch_bounds__(256) void k_gemm_argmax_final(const uint64_t* __restrict__ keys,
                                                           int M, int tiles,
                                                           int64_t* __restrict__ out) {
  __shared__ uint64_t red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  uint64_t b = 0;
  for (int t = tid; t < tiles; t += 256) {
    const uint64_t k = keys[(int64_t)m * tiles + t];
    b = k > b ? k : b;
  }
  b = wave_max_u64(b);
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = b;
  __syncthreads();
  if (tid == 0) {
    uint64_t r = red[0];
    for (int w = 1; w < 4; ++w) r = red[w] > r ? red[w] : r;
    out[m] = (int64_t)argmax_key_index(r);
  }
}

namespace {

template <int TT, int S, int NW, bool SILU>
void launch_gemm(const GemmArgs& a, int tiles, hipStream_t st) {
  // several row groups: tiles padded to a multiple of 8 (the XCD count) so that a tile's
  // groups share an XCD; the padding workgroups exit at once
  const int64_t grid = gemm_grid_x(tiles, a.RG);
  hipLaunchKernelGGL((k_gemm_skinny<TT, S, NW, SILU>), dim3((unsigned)grid, (unsigned)a.KS),
                     dim3(NW * kWave), 0, st, a);
}

template <int S, bool SILU>
void launch_gemm_tt(const GemmArgs& a, int tt, int tiles, hipStream_t st) {
  const bool wide = gemm_waves(a.M, a.N, a.epi) == 8;
  switch (tt) {
    case 1: wide ? launch_gemm<1, S, 8, SILU>(a, tiles, st) : launch_gemm<1, S, 4, SILU>(a, tiles, st); break;
    case 2: wide ? launch_gemm<2, S, 8, SILU>(a, tiles, st) : launch_gemm<2, S, 4, SILU>(a, tiles, st); break;
    case 3: wide ? launch_gemm<3, S, 8, SILU>(a, tiles, st) : launch_gemm<3, S, 4, SILU>(a, tiles, st); break;
    default: wide ? launch_gemm<4, S, 8, SILU>(a, tiles, st) : launch_gemm<4, S, 4, SILU>(a, tiles, st); break;
  }
}

}  // namespace

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int64_t mtpk_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int epilogue) {
  if (m <= 0 || m > kGemmMaxRows || n <= 0 || k <= 0 || k % kGemmKC || epilogue < 0 || epilogue > 2)
    return 0;
  const int ks = gemm_splits(m, n, k, epilogue);
  const int64_t tiles = gemm_tiles(m, n, epilogue);
  if (epilogue == kEpiArgmax) return m * tiles * 8;
  if (ks == 1) return 0;
  return (int64_t)ks * m * (epilogue == kEpiSilu ? n : gemm_cols(n, epilogue)) * 4;
}

int mtpk_gemm_bf16(const uint16_t* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                   int epilogue, void* out, int out_dtype, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  if (!x || !w || !out) return MTPK_EINVAL;
  if (m < 0 || m > kGemmMaxRows || n <= 0 || k <= 0 || k % kGemmKC || epilogue < 0 || epilogue > 2)
    return MTPK_EINVAL;
  if (epilogue == kEpiSilu && (n % 2 || (n / 2) % 16)) return MTPK_EINVAL;
  if (epilogue != kEpiArgmax && out_dtype != MTPK_F32 && out_dtype != MTPK_BF16) return MTPK_EINVAL;
  if (!aligned16(x) || !aligned16(w)) return MTPK_EINVAL;
  if (n * k * 2 > 0x7fffffffLL || m * k * 2 > 0x7fffffffLL || n > INT32_MAX / 2) return MTPK_EINVAL;
  if (workspace_bytes < mtpk_gemm_workspace_bytes(m > 0 ? m : 1, n, k, epilogue)) return MTPK_EINVAL;
  if (m == 0) return 0;
  const int ks = gemm_splits(m, n, k, epilogue);
  if ((ks > 1 || epilogue == kEpiArgmax) && !workspace) return MTPK_EINVAL;
  const int cols = gemm_cols(n, epilogue);
  const int tiles = (int)gemm_tiles(m, n, epilogue);
  GemmArgs a{x, w, (int)m, (int)n, (int)k, ks, epilogue, out_dtype, cols, out,
             ks > 1 ? static_cast<float*>(workspace) : nullptr,
             epilogue == kEpiArgmax ? static_cast<uint64_t*>(workspace) : nullptr, tiles,
             gemm_groups(m)};
  if ((int64_t)(tiles + 7) / 8 * 8 * a.RG > INT32_MAX) return MTPK_EINVAL;
  const hipStream_t st = (hipStream_t)stream;
  const int tt = gemm_tt(m);
  if (gemm_wide(m, n, epilogue)) {
    a.RG = 1;
    const int wtt = (int)((m + 15) / 16);
    static_assert(kGemmKC % kWideKStep == 0, "K (a multiple of kGemmKC) fills whole loop turns");
    if (wtt <= 4)
      launch_wide<4, 4>(a, tiles, st);
    else if (wtt <= 8)
      launch_wide<8, 2>(a, tiles, st);
    else
      launch_wide<12, 2>(a, tiles, st);
  } else if (epilogue == kEpiSilu)
    launch_gemm_tt<2, true>(a, tt, tiles, st);
  else
    launch_gemm_tt<1, false>(a, tt, tiles, st);
  int rc = status_of(hipGetLastError());
  if (rc) return rc;
  if (epilogue == kEpiArgmax) {
    hipLaunchKernelGGL(k_gemm_argmax_final, dim3((unsigned)m), dim3(256), 0, st,
                       a.keys, (int)m, tiles, static_cast<int64_t*>(out));
    return status_of(hipGetLastError());
  }
  if (ks > 1) {
    const int64_t total = m * cols;
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                       a.part, ks, (int)m, cols, epilogue, out, out_dtype);
    return status_of(hipGetLastError());
  }
  return 0;
}

}  // extern "C"
