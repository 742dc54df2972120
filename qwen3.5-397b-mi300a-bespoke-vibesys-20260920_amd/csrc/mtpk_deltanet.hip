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
// scalar loads; the state is read once (dword loads, 256 contiguous bytes per wave
// instruction) and, in commit mode, written back once in place.
//
// Verify mode (lengths == NULL): t steps from the committed state, outputs for every step, the
// state is not written. Commit mode: row j replays its accepted prefix, min(lengths[j], t)
// steps, and stores the advanced state over its slot (outputs optional).

#include "mtpk_device.h"
#include "mtpk_host.h"

namespace mtpk {


// Wave-uniform fp32 reads of data an earlier launch wrote and this one only reads.
typedef const __attribute__((address_space(4))) float* kc_f32_t;
__device__ inline float sloadf(const float* p, int64_t i) { return ((kc_f32_t)p)[i]; }

template <int DK, bool OUT, bool COMMIT>
__global__ __launch_bounds__(kWave) void k_delta_rule(
    float* __restrict__ state, const int64_t* __restrict__ slot, int t, int heads, int rep, int dv,
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta,
    const int64_t* __restrict__ lengths, float* __restrict__ out) {
  const int bh = blockIdx.x;  // row * heads + head
  const int row = bh / heads, head = bh - row * heads;
  const int col = blockIdx.y * kWave + threadIdx.x;
  const bool live = col < dv;
  const int64_t s_idx = slot ? slot[row] : row;
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
  for (int st = 0; st < n; ++st) {
    const int64_t rs = (int64_t)row * t + st;
    const int64_t qk_off = (rs * qk_heads + kh) * DK;
    const int64_t hv = rs * heads + head;
    const float decay = __expf(sloadf(g, hv));
    const float bt = sloadf(beta, hv);
    const float vv = live ? v[hv * dv + col] : 0.f;
    float mem = 0.f;
#pragma unroll
    for (int i = 0; i < DK; ++i) {
      s[i] *= decay;
      mem = fmaf(s[i], sloadf(k, qk_off + i), mem);
    }
    const float delta = (vv - mem) * bt;
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < DK; ++i) {
      s[i] = fmaf(sloadf(k, qk_off + i), delta, s[i]);
      if (OUT) o = fmaf(s[i], sloadf(q, qk_off + i), o);
    }
    if (OUT && live) out[hv * dv + col] = o;
  }
  if (COMMIT) {
#pragma unroll
    for (int i = 0; i < DK; ++i)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s[i]), rsm, (int)vcol,
                                            (int)(drow * i), 0);
  }
}

template <int DK, bool OUT, bool COMMIT>
int launch_delta_rule(float* state, const int64_t* slot, int rows, int t, int heads, int rep,
                      int dv, const float* q, const float* k, const float* v, const float* g,
                      const float* beta, const int64_t* lengths, float* out, hipStream_t st) {
  hipLaunchKernelGGL((k_delta_rule<DK, OUT, COMMIT>), dim3(rows * heads, (dv + kWave - 1) / kWave),
                     dim3(kWave), 0, st, state, slot, t, heads, rep, dv, q, k, v, g, beta, lengths, out);
  return status_of(hipGetLastError());
}

template <int DK>
int launch_delta_rule_mode(float* state, const int64_t* slot, int rows, int t, int heads, int rep,
                           int dv, const float* q, const float* k, const float* v, const float* g,
                           const float* beta, const int64_t* lengths, float* out, hipStream_t st) {
  if (!lengths)
    return launch_delta_rule<DK, true, false>(state, slot, rows, t, heads, rep, dv, q, k, v, g, beta,
                                              nullptr, out, st);
  if (out)
    return launch_delta_rule<DK, true, true>(state, slot, rows, t, heads, rep, dv, q, k, v, g, beta,
                                             lengths, out, st);
  return launch_delta_rule<DK, false, true>(state, slot, rows, t, heads, rep, dv, q, k, v, g, beta,
                                            lengths, nullptr, st);
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
  launch_delta_rule_mode<DK_>(state, slot, r, tt, h, rep, dv, q, k, v, g, beta, lengths, out, st)
  switch (k_dim) {
    case 16: return MTPK_DN(16);
    case 32: return MTPK_DN(32);
    case 64: return MTPK_DN(64);
    default: return MTPK_DN(128);
  }
#undef MTPK_DN
}

}  // extern "C"
