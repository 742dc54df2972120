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

// The wide form (`gemm_wide`): TT token tiles in one row group, 8 waves x 2 weight streams,
// 128-K chunks (2 x TT x 16 padded 256-byte rows of LDS: 104 KiB at TT = 12, one workgroup per CU).
template <int TT>
__global__ __launch_bounds__(8 * kWave, 2) void k_gemm_wide(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[GemmSmem<TT, 8, 128>::kBytes];
  gemm_tile<TT, 2, 8, false, 128>(a, smem, blockIdx.x, blockIdx.y);
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
    if (wtt <= 8)
      hipLaunchKernelGGL(k_gemm_wide<8>, dim3((unsigned)tiles), dim3(8 * kWave), 0, st, a);
    else
      hipLaunchKernelGGL(k_gemm_wide<12>, dim3((unsigned)tiles), dim3(8 * kWave), 0, st, a);
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
