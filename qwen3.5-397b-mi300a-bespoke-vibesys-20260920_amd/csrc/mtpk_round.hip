// Round fill for gfx950: the device half of a speculative round's fill in one launch.
//
// The host writes one int64 row per buffer row into a pinned staging table and copies it over in
// one transfer; this kernel unpacks it into the captured round's static buffers and derives the
// fields the fill computes on the device (the round's block tables, block counts, KV write rows
// and the draft seed), which the reference writes with a copy per field and a chain of small
// tensor ops (`MTPVerifyRunner.fill`, graph_mtp.py:795-874), plus three index tables the
// round's steps would otherwise build with small launches of their own: every row's t
// positions (row major, for the verify rows, and step major, one contiguous row per draft step)
// and the commit's slot per row (-1 on padding rows, which the commit kernels skip). One
// workgroup per buffer row; the only sizeable traffic is the seed row (hidden * 2 bytes in
// bf16), copied with 16-byte loads.
//
// Draft feed: after each draft step, one launch puts the token the next step feeds into the
// token matrix (the forced id while the row has forced drafts left, else the step's greedy
// token), in place of a compare, a select and a column copy.

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {

constexpr int kFillThreads = 256;
// columns of a staging row: token, position, budget, slot, forced count, active, then the forced
// ids (max(t - 1, 1) columns) and the stop ids (n_stops columns)
constexpr int kStageToken = 0, kStagePos = 1, kStageBudget = 2, kStageSlot = 3, kStageForced = 4,
              kStageActive = 5, kStageIds = 6;

struct RoundFillArgs {
  const int64_t* staging;
  int t, width, n_stops, cols;
  const int32_t* lane_tables;  // [lanes, max_blocks]
  int64_t lanes;
  int max_blocks;
  int64_t block_size;
  int32_t reserved;
  const uint8_t* hidden_cache;  // [lanes, row_bytes]
  int64_t row_bytes;
  bool vec;  // row_bytes % 16 == 0 and both row bases 16-byte aligned
  int64_t *token_matrix, *pos, *budget, *slot_rows, *forced_n;
  uint8_t* active;
  int64_t *forced_ids, *stops;
  int32_t *block_table, *block_valid;
  int64_t* write_rows;
  uint8_t* draft_hidden;
  int64_t *pos_grid, *pos_steps, *commit_slots;  // [rows, t], [t, rows], [rows]
  int64_t rows;
};

// Python's floor division and remainder (the fill's `//` and `%` on int64 tensors)
__device__ inline int64_t floor_div(int64_t a, int64_t b) {
  const int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

__global__ __launch_bounds__(kFillThreads) void k_round_fill(RoundFillArgs a) {
  const int64_t j = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t* st = a.staging + j * a.cols;
  const int64_t p = st[kStagePos];
  const int64_t slot = st[kStageSlot];
  const bool act = st[kStageActive] != 0;
  // a slot outside the lanes reads nothing (the host checks slots before staging them): its
  // table row is the reserved block and its seed row zeros
  const bool slot_ok = slot >= 0 && slot < a.lanes;
  const bool own = act && slot_ok;
  const int32_t* lt = a.lane_tables + (slot_ok ? slot : 0) * (int64_t)a.max_blocks;
  if (tid == 0) {
    a.pos[j] = p;
    a.budget[j] = st[kStageBudget];
    a.slot_rows[j] = slot;
    a.forced_n[j] = st[kStageForced];
    a.active[j] = act ? 1 : 0;
    a.block_valid[j] = (int32_t)floor_div(p + a.t + a.block_size - 1, a.block_size);
    a.commit_slots[j] = act ? slot : -1;
  }
  for (int c = tid; c < a.t; c += kFillThreads) {
    a.token_matrix[j * a.t + c] = c == 0 ? st[kStageToken] : 0;
    // KV row of position p + c through this row's table (the reserved block on padding rows);
    // a position outside the table gets -1 (the host grows every lane's table to p + t first)
    const int64_t g = p + c;
    const int64_t col = floor_div(g, a.block_size);
    int64_t row = -1;
    if (col >= 0 && col < a.max_blocks) {
      const int64_t blk = own ? lt[col] : a.reserved;
      row = blk * a.block_size + (g - col * a.block_size);
    }
    a.write_rows[j * a.t + c] = row;
    a.pos_grid[j * a.t + c] = g;
    a.pos_steps[c * a.rows + j] = g;
  }
  for (int c = tid; c < a.width; c += kFillThreads) a.forced_ids[j * a.width + c] = st[kStageIds + c];
  for (int c = tid; c < a.n_stops; c += kFillThreads)
    a.stops[j * a.n_stops + c] = st[kStageIds + a.width + c];
  for (int c = tid; c < a.max_blocks; c += kFillThreads)
    a.block_table[j * a.max_blocks + c] = own ? lt[c] : a.reserved;
  const uint8_t* src = a.hidden_cache + (slot_ok ? slot : 0) * a.row_bytes;
  uint8_t* dst = a.draft_hidden + j * a.row_bytes;
  if (a.vec) {
    for (int64_t i = tid; i < a.row_bytes / 16; i += kFillThreads)
      *reinterpret_cast<u32x4_t*>(dst + 16 * i) = slot_ok ? ld16(src + 16 * i) : zero16();
  } else {
    for (int64_t i = tid; i < a.row_bytes; i += kFillThreads) dst[i] = slot_ok ? src[i] : 0;
  }
}

__global__ __launch_bounds__(256) void k_draft_feed(const int64_t* __restrict__ tok, int64_t tok_stride,
                                                   const int64_t* __restrict__ forced_n,
                                                   const int64_t* __restrict__ forced,
                                                   int64_t forced_stride, int64_t step,
                                                   int64_t* __restrict__ out, int64_t out_stride,
                                                   int64_t rows) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= rows) return;
  out[j * out_stride] = forced_n[j] > step ? forced[j * forced_stride] : tok[j * tok_stride];
}

// Row copy through two index lists (the verify step's seed write-back, `scatter_time_active_rows`
// at graph_mtp.py:578-579): dst row dst_idx[j] = src row src_idx[j]; a row whose index lies
// outside its table (a padding row's -1 slot) is skipped. One workgroup per row, 16-byte copies
// when the rows allow them.
__global__ __launch_bounds__(256) void k_copy_rows(const uint8_t* __restrict__ src, int64_t src_rows,
                                                  int64_t src_stride, const int64_t* __restrict__ src_idx,
                                                  uint8_t* __restrict__ dst, int64_t dst_rows,
                                                  int64_t dst_stride, const int64_t* __restrict__ dst_idx,
                                                  int64_t row_bytes, bool vec) {
  const int64_t j = blockIdx.x;
  const int64_t s = src_idx[j], d = dst_idx[j];
  if (s < 0 || s >= src_rows || d < 0 || d >= dst_rows) return;  // uniform over the workgroup
  const uint8_t* a = src + s * src_stride;
  uint8_t* b = dst + d * dst_stride;
  if (vec) {
    for (int64_t i = threadIdx.x; i < row_bytes / 16; i += 256)
      *reinterpret_cast<u32x4_t*>(b + 16 * i) = ld16(a + 16 * i);
  } else {
    for (int64_t i = threadIdx.x; i < row_bytes; i += 256) b[i] = a[i];
  }
}

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int mtpk_round_fill(const int64_t* staging, int64_t rows, int64_t t, int64_t n_stops,
                    const int32_t* lane_tables, int64_t lanes, int64_t max_blocks,
                    int64_t block_size, int32_t reserved_block, const void* hidden_cache,
                    int64_t row_bytes, int64_t* token_matrix, int64_t* pos, int64_t* budget,
                    int64_t* slot_rows, int64_t* forced_n, uint8_t* active, int64_t* forced_ids,
                    int64_t* stops, int32_t* block_table, int32_t* block_valid,
                    int64_t* write_rows, void* draft_hidden, int64_t* pos_grid,
                    int64_t* pos_steps, int64_t* commit_slots, void* stream) {
  if (rows < 0 || rows > INT32_MAX || t < 1 || t > 4096 || n_stops < 0 || n_stops > 4096)
    return MTPK_EINVAL;
  if (lanes < 1 || max_blocks < 1 || max_blocks > INT32_MAX || block_size < 1 || row_bytes < 0)
    return MTPK_EINVAL;
  if (!staging || !lane_tables || !token_matrix || !pos || !budget || !slot_rows || !forced_n ||
      !active || !forced_ids || (n_stops > 0 && !stops) || !block_table || !block_valid ||
      !write_rows || (row_bytes > 0 && (!hidden_cache || !draft_hidden)) || !pos_grid ||
      !pos_steps || !commit_slots)
    return MTPK_EINVAL;
  if (rows == 0) return 0;
  RoundFillArgs a{};
  a.staging = staging;
  a.t = (int)t;
  a.width = t > 1 ? (int)t - 1 : 1;
  a.n_stops = (int)n_stops;
  a.cols = kStageIds + a.width + a.n_stops;
  a.lane_tables = lane_tables;
  a.lanes = lanes;
  a.max_blocks = (int)max_blocks;
  a.block_size = block_size;
  a.reserved = reserved_block;
  a.hidden_cache = static_cast<const uint8_t*>(hidden_cache);
  a.row_bytes = row_bytes;
  a.vec = row_bytes % 16 == 0 && aligned16(hidden_cache) && aligned16(draft_hidden);
  a.token_matrix = token_matrix;
  a.pos = pos;
  a.budget = budget;
  a.slot_rows = slot_rows;
  a.forced_n = forced_n;
  a.active = active;
  a.forced_ids = forced_ids;
  a.stops = stops;
  a.block_table = block_table;
  a.block_valid = block_valid;
  a.write_rows = write_rows;
  a.draft_hidden = static_cast<uint8_t*>(draft_hidden);
  a.pos_grid = pos_grid;
  a.pos_steps = pos_steps;
  a.commit_slots = commit_slots;
  a.rows = rows;
  hipLaunchKernelGGL(k_round_fill, dim3((unsigned)rows), dim3(kFillThreads), 0, (hipStream_t)stream, a);
  return status_of(hipGetLastError());
}

int mtpk_draft_feed(const int64_t* tok, int64_t tok_stride, const int64_t* forced_n,
                    const int64_t* forced, int64_t forced_stride, int64_t step, int64_t* out,
                    int64_t out_stride, int64_t rows, void* stream) {
  if (rows < 0 || !tok || !forced_n || !forced || !out || step < 0) return MTPK_EINVAL;
  if (rows == 0) return 0;
  if ((rows + 255) / 256 > INT32_MAX) return MTPK_EINVAL;
  hipLaunchKernelGGL(k_draft_feed, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, tok, tok_stride, forced_n, forced, forced_stride, step,
                     out, out_stride, rows);
  return status_of(hipGetLastError());
}

int mtpk_copy_rows(const void* src, int64_t src_rows, int64_t src_stride, const int64_t* src_idx,
                   void* dst, int64_t dst_rows, int64_t dst_stride, const int64_t* dst_idx,
                   int64_t rows, int64_t row_bytes, void* stream) {
  if (rows < 0 || rows > INT32_MAX || row_bytes < 0 || src_rows < 0 || dst_rows < 0) return MTPK_EINVAL;
  if (!src_idx || !dst_idx || (row_bytes > 0 && (!src || !dst))) return MTPK_EINVAL;
  if (src_stride < row_bytes || dst_stride < row_bytes) return MTPK_EINVAL;
  if (rows == 0 || row_bytes == 0) return 0;
  const bool vec = row_bytes % 16 == 0 && src_stride % 16 == 0 && dst_stride % 16 == 0 &&
                   aligned16(src) && aligned16(dst);
  hipLaunchKernelGGL(k_copy_rows, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint8_t*>(src), src_rows, src_stride, src_idx,
                     static_cast<uint8_t*>(dst), dst_rows, dst_stride, dst_idx, row_bytes, vec);
  return status_of(hipGetLastError());
}

}  // extern "C"
