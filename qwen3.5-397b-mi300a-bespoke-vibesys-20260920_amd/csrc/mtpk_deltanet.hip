// Gated delta-rule recurrence of the Gated DeltaNet layers for the verify forward and its
// commit (`deltanet_fused.py:274-398` `_delta_rule_verify_exact_kernel`, launched by
// `delta_rule_verify_exact` `:1090-1176`; torch form `model.py:651-697`).
//
// The recurrent state is a pool of fp32 matrices S [slots, heads, dk, dv], row-major (S[k][v]).
// One step for a (row, head) with normalised q, k [dk], v [dv], log-decay g and strength beta:
//   S <- e^g S;   S <- S + k ((v - S^T k) beta)^T;   out = S^T q
// Every column v of S evolves on its own (its update needs only k . s_v), so a lane owns one
// column: its dk (16..128) values stay in registers for all t steps, and one 64-lane wave
// covers 64 columns of one (row, head). q and k are the same for the whole wave and come in through
// LDS; the state is read once (dword loads, 256 contiguous bytes per wave
// instruction) and, in commit mode, written back once in place. At dk = 128 (the real model)
// a lane owns 4 columns over a quarter of the rows instead (16-byte state loads, the column
// sums finished by DPP adds in the lane quad; k_delta_rule_kg below).
//
// Verify mode (lengths == NULL): t steps from the committed state, outputs for every step, the
// state is not written. Commit mode: row j replays its accepted prefix, min(lengths[j], t)
// steps, and stores the advanced state over its slot (outputs optional).

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {


template <int DK, bool OUT, bool COMMIT>
__global__ __launch_bounds__(kWave) void k_delta_rule(
    float* __restrict__ state, int64_t slots_total, const int64_t* __restrict__ slot, int t,
    int heads, int rep, int dv, const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta,
    const int64_t* __restrict__ lengths, float* __restrict__ out) {
  static_assert(DK % 4 == 0, "k and q are read back four values at a time");
  // Workgroup (bh, c) is id bh * nblk + c: the column blocks of one matrix are dispatched
  // together, so the matrix's rows are read whole (its 64-column blocks interleave every
  // 256 bytes) while they are still open in the memory's row buffers.
  const int nblk = (dv + kWave - 1) / kWave;
  const int bh = blockIdx.x / nblk;  // row * heads + head
  const int row = bh / heads, head = bh - row * heads;
  const int col = (blockIdx.x - bh * nblk) * kWave + threadIdx.x;
  const bool live = col < dv;
  const int64_t s_idx = slot ? slot[row] : row;
  if (s_idx < 0 || s_idx >= slots_total) {  // no such slot: zero outputs, no state access
    if (OUT && live)
      for (int st = 0; st < t; ++st) out[((int64_t)row * t + st) * heads * dv + (int64_t)head * dv + col] = 0.f;
    return;  // uniform over the one-wave workgroup
  }
  // the (slot, head) matrix as one buffer: element (i, col) at byte 4 col + 4 dv i, the
  // per-lane part in voffset (out of range for lanes past dv) and the row offset in soffset
  const rsrc_t rsm = make_rsrc(state + ((s_idx * heads + head) * DK) * (int64_t)dv,
                               (uint32_t)(DK * dv * 4));
  const uint32_t vcol = live ? (uint32_t)col * 4u : kOutOfRange, drow = (uint32_t)dv * 4u;
  float s[DK];
#pragma unroll
  for (int i = 0; i < DK; ++i)
    s[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsm, (int)vcol, (int)(drow * i), 0));
  int n = t;
  if (COMMIT) n = (int)min(max(lengths[row], (int64_t)0), (int64_t)t);
  const int qk_heads = heads / rep, kh = head / rep;
  // A step's k and q (the same for the whole wave) pass through LDS: each lane loads one or two
  // of their values, and the product loops read them back four at a time as broadcasts. Step
  // st + 1's k, q, v, g and beta are loaded while step st runs, so no step waits for its
  // inputs after the first.
  constexpr int kPer = (DK + kWave - 1) / kWave;
  __shared__ __attribute__((aligned(16))) float kq[2][2][DK];
  const int lane = threadIdx.x;
  float nk[kPer], nq[kPer], nv = 0.f, ng = 0.f, nbt = 0.f;
  auto step_load = [&](int st) {
    const int64_t rs = (int64_t)row * t + (st < n ? st : 0);
    const int64_t qk_off = (rs * qk_heads + kh) * DK, hv = rs * heads + head;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int i = p * kWave + lane;
      nk[p] = i < DK ? k[qk_off + i] : 0.f;
      nq[p] = OUT && i < DK ? q[qk_off + i] : 0.f;
    }
    nv = live ? v[hv * dv + col] : 0.f;
    ng = g[hv];
    nbt = beta[hv];
  };
  if (n > 0) step_load(0);
  for (int st = 0; st < n; ++st) {
    const int b = st & 1;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int i = p * kWave + lane;
      if (i < DK) {
        kq[b][0][i] = nk[p];
        if (OUT) kq[b][1][i] = nq[p];
      }
    }
    const float decay = __expf(ng), bt = nbt, vv = nv;
    __syncthreads();  // this step's k and q are in LDS (a one-wave workgroup)
    if (st + 1 < n) step_load(st + 1);
    const float4* kk = reinterpret_cast<const float4*>(kq[b][0]);
    const float4* qq = reinterpret_cast<const float4*>(kq[b][1]);
    float mem = 0.f;
#pragma unroll
    for (int i4 = 0; i4 < DK / 4; ++i4) {
      const float4 kv = kk[i4];
      s[4 * i4] *= decay;
      s[4 * i4 + 1] *= decay;
      s[4 * i4 + 2] *= decay;
      s[4 * i4 + 3] *= decay;
      mem = fmaf(s[4 * i4], kv.x, mem);
      mem = fmaf(s[4 * i4 + 1], kv.y, mem);
      mem = fmaf(s[4 * i4 + 2], kv.z, mem);
      mem = fmaf(s[4 * i4 + 3], kv.w, mem);
    }
    const float delta = (vv - mem) * bt;
    // read k again rather than keep all DK values live across both loops: the state already
    // takes DK registers
    asm volatile("" ::: "memory");
    float o = 0.f;
#pragma unroll
    for (int i4 = 0; i4 < DK / 4; ++i4) {
      const float4 kv = kk[i4];
      s[4 * i4] = fmaf(kv.x, delta, s[4 * i4]);
      s[4 * i4 + 1] = fmaf(kv.y, delta, s[4 * i4 + 1]);
      s[4 * i4 + 2] = fmaf(kv.z, delta, s[4 * i4 + 2]);
      s[4 * i4 + 3] = fmaf(kv.w, delta, s[4 * i4 + 3]);
      if (OUT) {
        const float4 qv = qq[i4];
        o = fmaf(s[4 * i4], qv.x, o);
        o = fmaf(s[4 * i4 + 1], qv.y, o);
        o = fmaf(s[4 * i4 + 2], qv.z, o);
        o = fmaf(s[4 * i4 + 3], qv.w, o);
      }
    }
    if (OUT && live) out[((int64_t)row * t + st) * heads * dv + (int64_t)head * dv + col] = o;
  }
  if (COMMIT) {
#pragma unroll
    for (int i = 0; i < DK; ++i)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s[i]), rsm, (int)vcol,
                                            (int)(drow * i), 0);
  }
}

// The k_dim = 128 form (dv a multiple of 64): the rows of a matrix are cut into KG groups of
// 128 / KG and lane (cg = l / KG, kg = l % KG) owns the 4 adjacent columns 4 cg .. 4 cg + 3 of
// its block (64 4 / KG columns) over row group kg, so the state comes in with 16-byte loads
// (128 / KG per lane; every wave instruction reads KG row segments of 16 columns each) instead
// of 128 dword loads, and each step reads only its row group of k and q back from LDS. A
// column's sums over the row groups (S^T k and S^T q) are DPP butterfly adds inside the KG
// adjacent lanes, which leave the same bits in all of them, so every lane applies the same
// delta to its rows. The first 4 lanes of each group write the group's 4 output columns.
template <int CTRL>
__device__ inline float dn_dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
template <int KG>
__device__ inline float group_sum(float x) {
  x += dn_dpp<0xB1>(x);  // quad_perm [1, 0, 3, 2]
  x += dn_dpp<0x4E>(x);  // quad_perm [2, 3, 0, 1]
  if (KG == 8) x += dn_dpp<0x141>(x);  // row_half_mirror: the other quad of the 8 lanes
  return x;
}

template <int KG, bool OUT, bool COMMIT>
__device__ inline void delta_rule_kg_body(
    int bid, float* __restrict__ state, int64_t slots_total, const int64_t* __restrict__ slot, int t,
    int heads, int rep, int dv, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ g, const float* __restrict__ beta,
    const int64_t* __restrict__ lengths, float* __restrict__ out) {
  static_assert(KG == 4 || KG == 8, "row groups of 32 or 16");
  constexpr int DK = 128, QR = DK / KG, CW = 4 * kWave / KG;  // rows per group, columns per wave
  const int nblk = dv / CW;
  const int bh = bid / nblk;  // row * heads + head; a matrix's blocks are adjacent ids
  const int row = bh / heads, head = bh - row * heads;
  const int lane = threadIdx.x, cg = lane / KG, kg = lane % KG;
  const int base = (bid - bh * nblk) * CW;  // the block's first column
  const int col4 = base + 4 * cg;                   // this lane's first state column
  const int64_t s_idx = slot ? slot[row] : row;
  const int64_t o_row = (int64_t)head * dv + col4 + kg;  // kg < 4: the output column it writes
  if (s_idx < 0 || s_idx >= slots_total) {  // no such slot: zero outputs, no state access
    if (OUT && kg < 4)
      for (int st = 0; st < t; ++st) out[((int64_t)row * t + st) * heads * dv + o_row] = 0.f;
    return;  // uniform over the one-wave workgroup
  }
  const rsrc_t rsm = make_rsrc(state + ((s_idx * heads + head) * DK) * (int64_t)dv, (uint32_t)(DK * dv * 4));
  const uint32_t voff = ((uint32_t)(QR * kg) * (uint32_t)dv + (uint32_t)col4) * 4u, drow = (uint32_t)dv * 4u;
  f32x4_t s[QR];  // s[i] = row QR kg + i, columns col4 .. col4 + 3
#pragma unroll
  for (int i = 0; i < QR; ++i) s[i] = __builtin_bit_cast(f32x4_t, buf16(rsm, voff, drow * (uint32_t)i));
  int n = t;
  if (COMMIT) n = (int)min(max(lengths[row], (int64_t)0), (int64_t)t);
  const int qk_heads = heads / rep, kh = head / rep;
  // k and q pass through LDS as in the general form; step st + 1's inputs load while step st runs
  __shared__ __attribute__((aligned(16))) float kq[2][2][DK];
  float nk[2], nq[2], ng = 0.f, nbt = 0.f;
  f32x4_t nv = {0.f, 0.f, 0.f, 0.f};
  auto step_load = [&](int st) {
    const int64_t rs = (int64_t)row * t + (st < n ? st : 0);
    const int64_t qk_off = (rs * qk_heads + kh) * DK, hv = rs * heads + head;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      nk[p] = k[qk_off + p * kWave + lane];
      nq[p] = OUT ? q[qk_off + p * kWave + lane] : 0.f;
    }
    nv = *reinterpret_cast<const f32x4_t*>(v + hv * dv + col4);
    ng = g[hv];
    nbt = beta[hv];
  };
  if (n > 0) step_load(0);
  for (int st = 0; st < n; ++st) {
    const int b = st & 1;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      kq[b][0][p * kWave + lane] = nk[p];
      if (OUT) kq[b][1][p * kWave + lane] = nq[p];
    }
    const float decay = __expf(ng), bt = nbt;
    const f32x4_t vv = nv;
    __syncthreads();  // this step's k and q are in LDS (a one-wave workgroup)
    if (st + 1 < n) step_load(st + 1);
    const float4* kk = reinterpret_cast<const float4*>(&kq[b][0][QR * kg]);
    const float4* qq = reinterpret_cast<const float4*>(&kq[b][1][QR * kg]);
    float m[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i4 = 0; i4 < QR / 4; ++i4) {
      const float4 kv = kk[i4];
      const float kr[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * i4 + e;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          s[i][c] *= decay;
          m[c] = fmaf(s[i][c], kr[e], m[c]);
        }
      }
    }
    float delta[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) delta[c] = (vv[c] - group_sum<KG>(m[c])) * bt;
    asm volatile("" ::: "memory");
    float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i4 = 0; i4 < QR / 4; ++i4) {
      const float4 kv = kk[i4];
      const float kr[4] = {kv.x, kv.y, kv.z, kv.w};
      float qr[4] = {0.f, 0.f, 0.f, 0.f};
      if (OUT) {
        const float4 qv = qq[i4];
        qr[0] = qv.x;
        qr[1] = qv.y;
        qr[2] = qv.z;
        qr[3] = qv.w;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * i4 + e;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          s[i][c] = fmaf(kr[e], delta[c], s[i][c]);
          if (OUT) o[c] = fmaf(s[i][c], qr[e], o[c]);
        }
      }
    }
    if (OUT) {
      float mine = 0.f;  // column col4 + kg (kg < 4), by selects (no indexed registers)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float sum = group_sum<KG>(o[c]);
        if (kg == c) mine = sum;
      }
      if (kg < 4) out[((int64_t)row * t + st) * heads * dv + o_row] = mine;
    }
  }
  if (COMMIT) {
#pragma unroll
    for (int i = 0; i < QR; ++i)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, s[i]), rsm, (int)voff,
                                             (int)(drow * (uint32_t)i), 0);
  }
}

template <int KG, bool OUT, bool COMMIT>
__global__ __launch_bounds__(kWave, KG == 8 ? 4 : (OUT && COMMIT) ? 2 : 3) void k_delta_rule_kg(
    float* __restrict__ state, int64_t slots_total, const int64_t* __restrict__ slot, int t,
    int heads, int rep, int dv, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ g, const float* __restrict__ beta,
    const int64_t* __restrict__ lengths, float* __restrict__ out) {
  delta_rule_kg_body<KG, OUT, COMMIT>((int)blockIdx.x, state, slots_total, slot, t, heads, rep, dv,
                                      q, k, v, g, beta, lengths, out);
}
// Four row groups (164-168 VGPRs, three waves per SIMD): at config 5 (48 rows x 64 heads of
// 128 x 128, t = 4) the verify pass takes 47.4 us against 52.9 us for the dword form; eight row
// groups (four waves per SIMD) took 49.8 us. The commit (a state read and write, 83-88 us) is
// at device-copy speed in every form.
constexpr int kDnKG = 4;

template <int DK, bool OUT, bool COMMIT>
int launch_delta_rule(float* state, int64_t slots_total, const int64_t* slot, int rows, int t, int heads, int rep,
                      int dv, const float* q, const float* k, const float* v, const float* g,
                      const float* beta, const int64_t* lengths, float* out, hipStream_t st) {
  constexpr int kCols = 4 * kWave / kDnKG;  // columns per wave of the k_dim = 128 form
  if (DK == 128 && dv % kCols == 0 && aligned16(state) && aligned16(v)) {
    const int64_t grid = (int64_t)rows * heads * (dv / kCols);
    if (grid > INT32_MAX) return MTPK_EINVAL;
    hipLaunchKernelGGL((k_delta_rule_kg<kDnKG, OUT, COMMIT>), dim3((unsigned)grid), dim3(kWave), 0, st, state, slots_total, slot, t, heads, rep, dv, q, k, v, g, beta, lengths, out);
    return status_of(hipGetLastError());
  }
  const int64_t grid = (int64_t)rows * heads * ((dv + kWave - 1) / kWave);
  if (grid > INT32_MAX) return MTPK_EINVAL;
  hipLaunchKernelGGL((k_delta_rule<DK, OUT, COMMIT>), dim3((unsigned)grid), dim3(kWave), 0, st, state, slots_total, slot, t, heads, rep, dv, q, k, v, g, beta, lengths, out);
  return status_of(hipGetLastError());
}

template <int DK>
int launch_delta_rule_mode(float* state, int64_t slots_total, const int64_t* slot, int rows, int t, int heads, int rep,
                           int dv, const float* q, const float* k, const float* v, const float* g,
                           const float* beta, const int64_t* lengths, float* out, hipStream_t st) {
  if (!lengths)
    return launch_delta_rule<DK, true, false>(state, slots_total, slot, rows, t, heads, rep, dv, q, k, v, g, beta,
                                              nullptr, out, st);
  if (out)
    return launch_delta_rule<DK, true, true>(state, slots_total, slot, rows, t, heads, rep, dv, q, k, v, g, beta,
                                             lengths, out, st);
  return launch_delta_rule<DK, false, true>(state, slots_total, slot, rows, t, heads, rep, dv, q, k, v, g, beta,
                                            lengths, nullptr, st);
}

// ---------------------------------------------------------------- verify-row preparation
// Everything between the DeltaNet in-projection and the delta rule for the verify rows, in one
// launch (`deltanet_verify`, model.py:3738-3905, up to `delta_rule_verify_exact`): the depthwise
// causal conv over the stored window and the new raw columns, SiLU, rounding to the model dtype
// (the conv output is a model-dtype tensor), the q / k / v split, the q and k L2 norms (q also
// scaled by k_dim^-1/2), beta = sigmoid(b) and g = -exp(A_log) softplus(a + dt_bias). One wave
// per (verify row (b, s), head unit), the units being the q heads, then the k heads, then the v
// heads; lane l holds channels l, l + 64, ... A workgroup is 4 units of one row (grid: rows x
// units / 4), so the launch has thousands of workgroups and every wave issues all of its loads
// at once; the workgroups of unit group 0 also write the row's g and beta.
//
// Conv taps run in order j = 0 .. conv_k - 1 as separate products and sums (no fused
// multiply-add), as the torch form does them.
constexpr int kPrepThreadsDn = 256;
constexpr int kConvMaxK1 = 8;  // conv_k - 1 at most
constexpr int kPrepMaxPerLane = 4;  // head dims up to 256

struct DnPrepArgs {
  const void* proj;       // [B * t, proj_stride] model dtype: qkv (C), z, b (vh), a (vh)
  int64_t proj_stride;
  const void* conv;       // conv state [slots, C, k1] model dtype
  const int64_t* slot;    // [B]
  int64_t slots_total;    // conv_state slots; a row whose slot is outside reads a zero window
  const void* conv_w;     // [C, conv_k] model dtype
  const float* a_log;     // [vh] f32
  const float* dt_bias;   // [vh] f32
  int dt, t, kh, kd, vh, vd, conv_k;
  float eps, q_scale;
  float *q, *k, *v, *g, *beta;
};

__global__ __launch_bounds__(kPrepThreadsDn) void k_deltanet_prep(DnPrepArgs a) {
  const int rs = blockIdx.x;  // b * t + s
  const int b = rs / a.t, s = rs - b * a.t;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const int k1 = a.conv_k - 1;
  const int C = 2 * a.kh * a.kd + a.vh * a.vd;
  const int64_t slot = a.slot[b];
  const bool slot_ok = slot >= 0 && slot < a.slots_total;
  const int units = 2 * a.kh + a.vh;
  const int u = blockIdx.y * (kPrepThreadsDn / kWave) + wave;
  if (u < units) {
    const bool is_v = u >= 2 * a.kh;
    const int dim = is_v ? a.vd : a.kd;
    const int c0 = is_v ? 2 * a.kh * a.kd + (u - 2 * a.kh) * a.vd : u * a.kd;
    float x[kPrepMaxPerLane];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kPrepMaxPerLane; ++i) {
      const int ch = lane + kWave * i;
      x[i] = 0.f;
      if (ch >= dim) continue;
      const int c = c0 + ch;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < kConvMaxK1 + 1; ++j) {  // all taps' loads issued together
        if (j >= a.conv_k) break;
        const int p = s + j;  // window column: the stored k1, then the t new ones
        const float win = p < k1 ? (slot_ok ? load_float(a.conv, a.dt, (slot * C + c) * k1 + p) : 0.f)
                                 : load_float(a.proj, a.dt, ((int64_t)b * a.t + p - k1) * a.proj_stride + c);
        const float prod = __fmul_rn(win, load_float(a.conv_w, a.dt, (int64_t)c * a.conv_k + j));
        acc = j == 0 ? prod : __fadd_rn(acc, prod);
      }
      float y = acc / (1.f + expf(-acc));
      if (a.dt == MTPK_BF16) y = bf16_to_f32(f32_to_bf16(y));
      x[i] = y;
      ss += y * y;
    }
    if (is_v) {
      float* dst = a.v + ((int64_t)rs * a.vh + (u - 2 * a.kh)) * a.vd;
#pragma unroll
      for (int i = 0; i < kPrepMaxPerLane; ++i)
        if (lane + kWave * i < dim) dst[lane + kWave * i] = x[i];
    } else {
      const bool is_q = u < a.kh;
      const float inv = rsqrtf(wave_sum(ss) + a.eps);
      const float sc = is_q ? a.q_scale : 1.f;
      float* dst = (is_q ? a.q : a.k) + ((int64_t)rs * a.kh + (is_q ? u : u - a.kh)) * a.kd;
#pragma unroll
      for (int i = 0; i < kPrepMaxPerLane; ++i)
        if (lane + kWave * i < dim) dst[lane + kWave * i] = x[i] * inv * sc;
    }
  }
  for (int h = tid; blockIdx.y == 0 && h < a.vh; h += kPrepThreadsDn) {
    const int64_t base = (int64_t)rs * a.proj_stride + C + a.vh * a.vd;
    const float braw = load_float(a.proj, a.dt, base + h);
    const float araw = load_float(a.proj, a.dt, base + a.vh + h);
    const float x = __fadd_rn(araw, a.dt_bias[h]);
    const float sp = x > 20.f ? x : log1pf(expf(x));
    a.beta[(int64_t)rs * a.vh + h] = 1.f / (1.f + expf(-braw));
    a.g[(int64_t)rs * a.vh + h] = -expf(a.a_log[h]) * sp;
  }
}

// The commit's conv-window update (`deltanet_verify_rollback`, model.py:3907-3972): slot b's
// window becomes columns idx[b][0 .. k1) of [stored window | the t new raw columns]. A thread
// owns one (row, channel) and reads all of its sources before it writes, so the in-place update
// cannot read a value it has already replaced.
struct ConvJob {
  void* conv;
  int dt;
  const int64_t* slot;
  int64_t slots_total;
  const void* proj;
  int64_t proj_stride;
  const int64_t* idx;
  int B, C, k1, t;
};

__device__ inline void conv_commit_one(const ConvJob& j, int64_t i) {
  void* __restrict__ conv = j.conv;
  const int dt = j.dt, C = j.C, k1 = j.k1, t = j.t;
  const int64_t* __restrict__ slot = j.slot;
  const int64_t* __restrict__ idx = j.idx;
  const void* __restrict__ proj = j.proj;
  const int64_t slots_total = j.slots_total, proj_stride = j.proj_stride;
  if (i >= (int64_t)j.B * C) return;
  const int b = (int)(i / C), c = (int)(i - (int64_t)b * C);
  if (slot[b] < 0 || slot[b] >= slots_total) return;  // no such slot: nothing to update
  const int64_t base = (slot[b] * C + c) * k1;
  float v[kConvMaxK1];
  for (int w = 0; w < k1; ++w) {
    int64_t p = idx[(int64_t)b * k1 + w];
    p = p < 0 ? 0 : (p > k1 + t - 1 ? k1 + t - 1 : p);
    v[w] = p < k1 ? load_float(conv, dt, base + p)
                  : load_float(proj, dt, ((int64_t)b * t + p - k1) * proj_stride + c);
  }
  for (int w = 0; w < k1; ++w) store_float(conv, dt, base + w, v[w]);
}

__global__ __launch_bounds__(256) void k_conv_commit(ConvJob j) {
  conv_commit_one(j, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// A DeltaNet layer's whole commit in one launch: the delta rule's commit blocks (k_dim = 128
// form) first, then one-wave blocks of the conv-window update, which run beside the state
// stream instead of in a launch of their own.
__global__ __launch_bounds__(kWave, 3) void k_dn_commit(
    float* __restrict__ state, int64_t slots_total, const int64_t* __restrict__ slot, int t,
    int heads, int rep, int dv, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, const float* __restrict__ g, const float* __restrict__ beta,
    const int64_t* __restrict__ lengths, int dr_blocks, ConvJob cj) {
  if ((int)blockIdx.x >= dr_blocks) {  // uniform over the one-wave workgroup
    conv_commit_one(cj, ((int64_t)blockIdx.x - dr_blocks) * kWave + threadIdx.x);
    return;
  }
  delta_rule_kg_body<kDnKG, false, true>((int)blockIdx.x, state, slots_total, slot, t, heads, rep,
                                         dv, q, k, v, g, beta, lengths, nullptr);
}

}  // namespace mtpk

using namespace mtpk;

extern "C" {

int mtpk_delta_rule(float* state, int64_t slots_total, const int64_t* slot, int64_t rows, int64_t t,
                    int64_t heads, int64_t qk_heads, int64_t k_dim, int64_t v_dim, const float* q,
                    const float* k, const float* v, const float* g, const float* beta,
                    const int64_t* lengths, float* out, void* stream) {
  if (!state || !q || !k || !v || !g || !beta) return MTPK_EINVAL;
  if (rows < 0 || t < 1 || t > INT32_MAX / 2 || heads <= 0 || qk_heads <= 0 || heads % qk_heads)
    return MTPK_EINVAL;
  if (k_dim != 16 && k_dim != 32 && k_dim != 64 && k_dim != 128) return MTPK_EINVAL;
  if (v_dim <= 0 || v_dim > 4096) return MTPK_EINVAL;
  if (slots_total <= 0 || (!slot && slots_total < rows)) return MTPK_EINVAL;
  if (slots_total * heads * k_dim * v_dim >= (int64_t(1) << 40) || rows * heads > INT32_MAX)
    return MTPK_EINVAL;
  if (!lengths && !out) return MTPK_EINVAL;  // nothing to produce
  if (rows == 0) return 0;
  const hipStream_t st = (hipStream_t)stream;
  const int r = (int)rows, tt = (int)t, h = (int)heads, rep = (int)(heads / qk_heads), dv = (int)v_dim;
#define MTPK_DN(DK_) \
  launch_delta_rule_mode<DK_>(state, slots_total, slot, r, tt, h, rep, dv, q, k, v, g, beta, lengths, out, st)
  switch (k_dim) {
    case 16: return MTPK_DN(16);
    case 32: return MTPK_DN(32);
    case 64: return MTPK_DN(64);
    default: return MTPK_DN(128);
  }
#undef MTPK_DN
}

int mtpk_deltanet_prep(const void* proj, int dtype, int64_t proj_stride, const void* conv_state,
                       const int64_t* slot, int64_t slots_total, const void* conv_w, const float* a_log,
                       const float* dt_bias, int64_t batch, int64_t t, int64_t k_heads,
                       int64_t k_dim, int64_t v_heads, int64_t v_dim, int64_t conv_k, float eps,
                       float q_scale, float* q, float* k, float* v, float* g, float* beta,
                       void* stream) {
  if (!proj || !conv_state || !slot || !conv_w || !a_log || !dt_bias || !q || !k || !v || !g || !beta)
    return MTPK_EINVAL;
  if (dtype != MTPK_F32 && dtype != MTPK_BF16) return MTPK_EINVAL;
  if (batch < 0 || t < 1 || k_heads < 1 || v_heads < 1 || conv_k < 2 || conv_k > kConvMaxK1 + 1 ||
      slots_total < 1)
    return MTPK_EINVAL;
  if (k_dim < 1 || k_dim > kWave * kPrepMaxPerLane || v_dim < 1 || v_dim > kWave * kPrepMaxPerLane)
    return MTPK_EINVAL;
  const int64_t C = 2 * k_heads * k_dim + v_heads * v_dim;
  if (proj_stride < C + v_heads * v_dim + 2 * v_heads || batch * t > INT32_MAX) return MTPK_EINVAL;
  if (batch == 0) return 0;
  DnPrepArgs a{proj, proj_stride, conv_state, slot, slots_total, conv_w, a_log, dt_bias, dtype, (int)t,
               (int)k_heads, (int)k_dim, (int)v_heads, (int)v_dim, (int)conv_k, eps, q_scale,
               q, k, v, g, beta};
  const int64_t units = 2 * k_heads + v_heads;
  const int64_t groups = (units + kPrepThreadsDn / kWave - 1) / (kPrepThreadsDn / kWave);
  if (groups > 65535) return MTPK_EINVAL;
  hipLaunchKernelGGL(k_deltanet_prep, dim3((unsigned)(batch * t), (unsigned)groups),
                     dim3(kPrepThreadsDn), 0, (hipStream_t)stream, a);
  return status_of(hipGetLastError());
}

int mtpk_conv_commit(void* conv_state, int dtype, const int64_t* slot, int64_t slots_total,
                     const void* proj,
                     int64_t proj_stride, const int64_t* idx, int64_t batch, int64_t channels,
                     int64_t k1, int64_t t, void* stream) {
  if (!conv_state || !slot || !proj || !idx) return MTPK_EINVAL;
  if (dtype != MTPK_F32 && dtype != MTPK_BF16) return MTPK_EINVAL;
  if (batch < 0 || channels < 1 || k1 < 1 || k1 > kConvMaxK1 || t < 1 || proj_stride < channels ||
      slots_total < 1)
    return MTPK_EINVAL;
  if (batch * channels > INT32_MAX) return MTPK_EINVAL;
  if (batch == 0) return 0;
  const int64_t n = batch * channels;
  const ConvJob cj{conv_state, dtype, slot, slots_total, proj, proj_stride, idx,
                   (int)batch, (int)channels, (int)k1, (int)t};
  hipLaunchKernelGGL(k_conv_commit, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, cj);
  return status_of(hipGetLastError());
}

int mtpk_deltanet_commit(float* state, int64_t slots_total, const int64_t* slot, int64_t rows,
                         int64_t t, int64_t heads, int64_t qk_heads, int64_t k_dim, int64_t v_dim,
                         const float* q, const float* k, const float* v, const float* g,
                         const float* beta, const int64_t* lengths, void* conv_state,
                         int conv_dtype, int64_t conv_slots_total, const void* proj,
                         int64_t proj_stride, const int64_t* conv_idx, int64_t channels, int64_t k1,
                         void* stream) {
  constexpr int kCols = 4 * kWave / kDnKG;
  if (!lengths || !slot) return MTPK_EINVAL;
  const bool fused = k_dim == 128 && v_dim % kCols == 0 && aligned16(state) && aligned16(v) &&
                     rows * heads * (v_dim / kCols) + (rows * channels + kWave - 1) / kWave <= INT32_MAX;
  if (!fused) {  // the two launches
    const int rc = mtpk_delta_rule(state, slots_total, slot, rows, t, heads, qk_heads, k_dim, v_dim,
                                   q, k, v, g, beta, lengths, nullptr, stream);
    if (rc) return rc;
    return mtpk_conv_commit(conv_state, conv_dtype, slot, conv_slots_total, proj, proj_stride,
                            conv_idx, rows, channels, k1, t, stream);
  }
  // the argument checks of both launches
  if (!state || !q || !k || !v || !g || !beta || !conv_state || !proj || !conv_idx) return MTPK_EINVAL;
  if (rows < 0 || t < 1 || t > INT32_MAX / 2 || heads <= 0 || qk_heads <= 0 || heads % qk_heads)
    return MTPK_EINVAL;
  if (v_dim > 4096 || slots_total <= 0) return MTPK_EINVAL;
  if (slots_total * heads * k_dim * v_dim >= (int64_t(1) << 40)) return MTPK_EINVAL;
  if (conv_dtype != MTPK_F32 && conv_dtype != MTPK_BF16) return MTPK_EINVAL;
  if (channels < 1 || k1 < 1 || k1 > kConvMaxK1 || proj_stride < channels || conv_slots_total < 1)
    return MTPK_EINVAL;
  if (rows == 0) return 0;
  const int dr = (int)(rows * heads * (v_dim / kCols));
  const int64_t conv_blocks = (rows * channels + kWave - 1) / kWave;
  const ConvJob cj{conv_state, conv_dtype, slot, conv_slots_total, proj, proj_stride, conv_idx,
                   (int)rows, (int)channels, (int)k1, (int)t};
  hipLaunchKernelGGL(k_dn_commit, dim3((unsigned)(dr + conv_blocks)), dim3(kWave), 0,
                     (hipStream_t)stream, state, slots_total, slot, (int)t, (int)heads,
                     (int)(heads / qk_heads), (int)v_dim, q, k, v, g, beta, lengths, dr, cj);
  return status_of(hipGetLastError());
}

}  // extern "C"
