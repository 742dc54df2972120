// The skinny bf16 GEMM's tile body and launch-shape rules, shared by the GEMM's own launches
// (mtpk_gemm.hip) and by the MoE layer's launches that run GEMM tiles beside other work
// (mtpk_moe.hip, mtpk_router.hip). See mtpk_gemm.hip for the design.
#pragma once

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kGemmKC = 256;  // K per staged chunk
enum { kEpiStore = 0, kEpiSilu = 1, kEpiArgmax = 2 };

struct GemmArgs {
  const uint16_t* x;
  const uint16_t* w;
  int M, N, K, KS, epi, odt, cols;  // cols: output columns (N, or N / 2 for the SiLU epilogue)
  void* out;
  float* part;
  uint64_t* keys;  // argmax: [M, tiles]
  int tiles;       // weight tiles of 16 NW rows
  int RG;          // row groups of 16 TT token rows (M > 64: RG = ceil(M / 64), TT = 4)
};

// LDS of one tile: two staging buffers of TT token tiles, then the argmax epilogue's keys.
template <int TT, int NW, int KC = kGemmKC>
struct GemmSmem {
  static constexpr int kStage = TT * 16 * (KC * 2 + 16);
  static constexpr int kKeys = 2 * kStage;
  static constexpr int kBytes = kKeys + NW * TT * 16 * 8;
};

// S weight streams per wave. SILU: S = 2, the gate row r and its up row N/2 + r (the SiLU
// product epilogue). Otherwise the S streams are the wave's rows r, r + 16 NW, ...: a tile is
// 16 NW S weight rows, and every staged activation read feeds S MFMAs. Only S = 1 is launched
// outside the SiLU pairing: two streams at 48 rows on the LM head measured 471 us against 437
// (half the waves resident, for half the LDS reads per weight byte).
template <int TT, int S, int NW, bool SILU, int KC = kGemmKC>
__device__ inline void gemm_tile(const GemmArgs& a, uint8_t* smem, int bx, int by) {
  static_assert(!SILU || S == 2, "the SiLU epilogue pairs two streams");
  constexpr int NT = NW * kWave;
  constexpr int kSteps = KC / 32;          // MFMA steps per chunk
  // Ring depth: one chunk of steps. The chunk-end wait for the staged token rows also waits for
  // every ring load issued before them (vmcnt retires in order), so a deeper ring would be
  // drained at each chunk boundary.
  constexpr int kRing = kSteps;
  constexpr int kRow = KC * 2 + 16;        // LDS bytes of one token row (padded)
  constexpr int kPieces = KC / 8;          // 16-byte pieces of a token row per chunk
  typedef uint8_t StageBuf[TT * 16 * kRow];
  typedef uint64_t KeyRow[TT * 16];
  StageBuf* xs = reinterpret_cast<StageBuf*>(smem);
  KeyRow* kred = reinterpret_cast<KeyRow*>(smem + GemmSmem<TT, NW, KC>::kKeys);
  const int tid = threadIdx.x, wave = uniform(tid / kWave), lane = tid & (kWave - 1);
  const MoeLane ln = moe_lane(lane);
  // Workgroup -> (weight tile, row group). With several row groups, the groups of one tile
  // get ids 8 apart: workgroup i runs on XCD i % 8 (checked on MI355X for 4096 workgroups), so
  // they run on one XCD close in time and can share its L2. Each group still does the tile's
  // full load and MFMA work. Measured at 192 rows this pays where the weight tiles are few
  // (N = 4096: 47 us against the library GEMM's 61) but not on wide N (the LM head: 881 against
  // 494 us), where callers keep the library GEMM.
  int tile = bx, rg = 0;
  if (a.RG > 1) {
    const int xcd = bx & 7, slot = bx >> 3;
    tile = (slot / a.RG) * 8 + xcd;
    rg = slot % a.RG;
    if (tile >= a.tiles) return;  // grid padding, before any barrier
  }
  const int ks = by;
  const int m0 = rg * 16 * TT;                             // first token row of this group
  const int Mg = a.M - m0 < 16 * TT ? a.M - m0 : 16 * TT;  // its rows
  const int kc_per = a.K / KC / a.KS;  // chunks of this split
  const int k0 = ks * kc_per * KC;
  const int nchunk = kc_per;
  // weight rows of this wave: stream s at r0 + s N/2 (SILU) or r0 + 16 NW s
  const int r0 = tile * 16 * NW * (SILU ? 1 : S) + 16 * wave + ln.c;
  int wrow[S];
  bool wok[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int r = SILU ? r0 + s * (a.N / 2) : r0 + s * 16 * NW;
    wok[s] = SILU ? r0 < a.cols : r < a.N;
    wrow[s] = wok[s] ? r : 0;
  }
  const rsrc_t rw = make_rsrc(a.w, 0x7fffffff);
  const rsrc_t rx = make_rsrc(a.x, (uint32_t)((int64_t)a.M * a.K * 2));
  // ring step st of this split: K = k0 + 32 st + 8 g .. + 7 of each stream's row
  auto issue = [&](u32x4_t* v, int st) {
    const bool in = st < nchunk * kSteps;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const uint32_t off = (uint32_t)(((int64_t)wrow[s] * a.K + k0 + 32 * st + 8 * ln.g) * 2);
      v[s] = buf16(rw, (wok[s] && in) ? off : kOutOfRange);
    }
  };
  // staging: load j moves 16 bytes of token row (NT j + tid) / kPieces, column
  // ((NT j + tid) % kPieces) * 16
  constexpr int kSL = TT * 16 * kPieces / NT;  // 16-byte loads per thread per chunk
  static_assert(kSL * NT == TT * 16 * kPieces, "staging split");
  u32x4_t sreg[kSL];
  auto stage_load = [&](int c) {
#pragma unroll
    for (int j = 0; j < kSL; ++j) {
      const int p = j * NT + tid, row = p / kPieces, col = p % kPieces;
      const bool ok = c < nchunk && row < Mg;
      sreg[j] = buf16(rx, ok ? (uint32_t)(((int64_t)(m0 + row) * a.K + k0 + c * KC + col * 8) * 2)
                             : kOutOfRange);
    }
  };
  auto stage_store = [&](int b) {
#pragma unroll
    for (int j = 0; j < kSL; ++j) {
      const int p = j * NT + tid, row = p / kPieces, col = p % kPieces;
      lds16_store(&xs[b][row * kRow + col * 16], sreg[j]);
    }
  };

  f32x4_t acc[S][TT];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[s][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  stage_load(0);
  ring_fence();
  u32x4_t ring[kRing][S];
#pragma unroll
  for (int st = 0; st < kRing; ++st) issue(ring[st], st);
  ring_fence();
  stage_store(0);
  stage_load(1);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __syncthreads();
  int c = 0;
#pragma clang loop unroll(disable)
  do {
    // The A operand (staged token rows) of step st + 1 is read from LDS before step st's MFMAs:
    // read after them, its latency sat between each step's MFMAs and its ring refill (the
    // refill is issued once the slot's MFMAs are), holding back the weight stream (the 48-row
    // LM head with the argmax epilogue 446 -> 432 us).
    const uint8_t* buf = xs[c & 1];
    const uint8_t* abase = buf + ln.c * kRow + (8 * ln.g) * 2;
    u32x4_t av[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) av[t] = lds16(abase + t * 16 * kRow);
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      u32x4_t* slot = ring[st];
      u32x4_t an[TT];
      if (st + 1 < kSteps) {
#pragma unroll
        for (int t = 0; t < TT; ++t) an[t] = lds16(abase + 64 * (st + 1) + t * 16 * kRow);
      }
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int t = 0; t < TT; ++t)
          acc[s][t] = mfma16x16x32(as_bf16x8(av[t]), as_bf16x8(slot[s]), acc[s][t]);
      ring_fence();
      issue(slot, c * kSteps + st + kRing);
      ring_fence();
      if (st + 1 < kSteps) {
#pragma unroll
        for (int t = 0; t < TT; ++t) av[t] = an[t];
      }
    }
    if (c + 1 < nchunk) stage_store((c + 1) & 1);
    stage_load(c + 2);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __syncthreads();
  } while (++c < nchunk);

  // lane (g, c): acc[s][t][i] is token m = 16 t + 4 g + i, column r0 (stream s)
  if (a.part) {  // fp32 partials [KS, M, cols] (or [KS, M, 2 cols] for SiLU), summed later
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * t + 4 * ln.g + i;
        if (m >= Mg) continue;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int col = SILU ? r0 + s * a.cols : wrow[s];  // SiLU partials: gate, then up
          if (!wok[s]) continue;
          a.part[((int64_t)ks * a.M + m0 + m) * (int64_t)((SILU ? 2 : 1) * a.cols) + col] = acc[s][t][i];
        }
      }
    return;
  }
  if (a.epi == kEpiArgmax) {
    // first-occurrence argmax of the bf16 values: the max key over this wave's 16 columns,
    // then over the NW waves
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint64_t key = 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const float v = bf16_to_f32(f32_to_bf16(acc[s][t][i]));
          const uint64_t ks_ = wok[s] ? argmax_key(v, (uint32_t)wrow[s]) : 0;
          key = ks_ > key ? ks_ : key;
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
    for (int m = tid; m < Mg; m += NT) {
      uint64_t b = kred[0][m];
      for (int w2 = 1; w2 < NW; ++w2) b = kred[w2][m] > b ? kred[w2][m] : b;
      a.keys[(int64_t)(m0 + m) * a.tiles + tile] = b;
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * t + 4 * ln.g + i;
      if (m >= Mg) continue;
      if (SILU) {
        if (!wok[0]) continue;
        const float g = acc[0][t][i];
        store_float(a.out, a.odt, (int64_t)(m0 + m) * a.cols + r0, g / (1.f + __expf(-g)) * acc[1][t][i]);
      } else {
#pragma unroll
        for (int s = 0; s < S; ++s)
          if (wok[s]) store_float(a.out, a.odt, (int64_t)(m0 + m) * a.cols + wrow[s], acc[s][t][i]);
      }
    }
}

// One element of the split-K reduction: out[m, col] = epilogue(sum over ks of part[ks, m, .]) in
// split order (the SiLU epilogue reads the gate half, then the up half of each partial row).
// The planes are loaded kReducePlanes at a time and then summed in split order, so a value waits
// for one memory latency per group of planes rather than one per plane.
constexpr int kReducePlanes = 8;

__device__ inline float gemm_reduce_value(const float* __restrict__ part, int KS, int M, int cols,
                                          int epi, int64_t m, int64_t col) {
  const int pc = epi == kEpiSilu ? 2 * cols : cols;
  float g = 0.f, u = 0.f;
  for (int k0 = 0; k0 < KS; k0 += kReducePlanes) {
    float vg[kReducePlanes], vu[kReducePlanes];
#pragma unroll
    for (int i = 0; i < kReducePlanes; ++i) {
      const float* p = part + ((int64_t)(k0 + i) * M + m) * pc;
      vg[i] = k0 + i < KS ? p[col] : 0.f;
      vu[i] = k0 + i < KS && epi == kEpiSilu ? p[cols + col] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kReducePlanes; ++i)
      if (k0 + i < KS) {
        g += vg[i];
        if (epi == kEpiSilu) u += vu[i];
      }
  }
  return epi == kEpiSilu ? g / (1.f + __expf(-g)) * u : g;
}

inline int gemm_cols(int64_t n, int epi) { return (int)(epi == kEpiSilu ? n / 2 : n); }

constexpr int64_t kGemmMaxRows = 256;  // 4 row groups of 64

// Row groups of 64 token rows: one below 65 rows (then TT = ceil(M / 16)), else ceil(M / 64)
// with TT = 4.
inline int gemm_groups(int64_t m) { return m <= 64 ? 1 : (int)((m + 63) / 64); }
inline int gemm_tt(int64_t m) { return m <= 64 ? (int)((m + 15) / 16) : 4; }

// Waves per workgroup. At TT >= 3 token tiles the 2 x TT x 8 KiB staged token rows hold a CU to
// three 4-wave workgroups; 8 waves sharing one staged copy double the resident waves, which
// measured 4% faster on [48 | 64, 4096] x [248320, 4096] (the LM head) but slower wherever the
// 128-row tiles leave fewer than two workgroups per CU (N = 4096: 8.8 -> 12.4 us).
inline int gemm_waves(int64_t m, int64_t n, int epi) {
  const int64_t cols = gemm_cols(n, epi);
  return (m + 15) / 16 >= 3 && cols / 128 >= 2 * (int64_t)device_cu_count() ? 8 : 4;
}

// The wide form for 17..192 token rows on wide N (the LM heads, mtpk_gemm.hip k_gemm_wide):
// one row group of token tiles against 16 x 8 RT-row weight tiles, the token rows staged by
// direct-to-LDS loads. Every weight is read once for all rows; the 64-row groups would stream the
// tile's weights once per group. Up to 64 rows the rows are padded to four token tiles and a
// tile is 512 weight rows (RT = 4), above that 8 or 12 token tiles against 256 rows (RT = 2,
// the accumulators' share of the registers). Measured on [M, 4096] x [248320, 4096] with the
// argmax epilogue: 372-374 us from 17 to 64 rows against 391-410 us for the 8-wave skinny tiles
// (128 rows, the token rows staged per tile twice as often), equal at 16 rows.
constexpr int kWideMinRows = 17, kWideMaxRows = 192;
inline bool gemm_wide(int64_t m, int64_t n, int epi) {
  return m >= kWideMinRows && m <= kWideMaxRows && epi != kEpiSilu &&
         gemm_cols(n, epi) >= 256 * 2 * (int64_t)device_cu_count();
}
inline int wide_row_tiles(int64_t m) { return m <= 64 ? 4 : 2; }

inline int64_t gemm_tiles(int64_t m, int64_t n, int epi) {
  const int64_t rows = gemm_wide(m, n, epi) ? 16 * 8 * wide_row_tiles(m) : 16 * gemm_waves(m, n, epi);
  return (gemm_cols(n, epi) + rows - 1) / rows;
}

// Split count: a power of two dividing K / 256, enough workgroups for ~3 per CU, at least 4
// chunks per split (2 at up to 64 rows, one row group: the MoE layer's router + shared expert
// launch at 1 row took 38 against 41 us, at 48 rows 416 against 418 us; at 192 rows, three row
// groups per tile, 2 chunks lost 9 us); argmax takes no split.
inline int gemm_splits(int64_t m, int64_t n, int64_t k, int epi) {
  if (epi == kEpiArgmax || gemm_wide(m, n, epi)) return 1;
  const int64_t tiles = gemm_tiles(m, n, epi);
  const int64_t chunks = k / kGemmKC;
  const int64_t wgs = tiles * gemm_groups(m);
  const int64_t want = (3 * (int64_t)device_cu_count() * 4 / gemm_waves(m, n, epi) + wgs - 1) / wgs;
  int ks = 1;
  const int64_t min_chunks = m <= 64 ? 2 : 4;
  while (ks * 2 <= want && chunks % (ks * 2) == 0 && chunks / (ks * 2) >= min_chunks) ks *= 2;
  return ks;
}

// Grid x extent of one GEMM launch (grid y = KS): with several row groups the tiles are padded to
// a multiple of 8 (the XCD count) so that a tile's groups share an XCD.
inline int64_t gemm_grid_x(int64_t tiles, int rg) { return rg > 1 ? (tiles + 7) / 8 * 8 * rg : tiles; }

}  // namespace mtpk
