// Host emulation of libmtpk's lane math (built with g++ -DMTPK_HOST_TEST by
// tests/test_host_emulation.py). Each check prints "PASS <name>" or "FAIL <name> ...".
//
//  decode      fp4_to_f32 * e8m0_to_f32 against the closed form, all 256 bytes x 256 scales
//  split       split_bf16 / split3_bf16 reconstruction bounds
//  argmax_key  key order == (value desc, index asc), with -0.0 == +0.0
//  gate_up     the gate_up kernel's wave/trip/lane/slot decomposition (contiguous quarters of
//              the trips per wave, ring steps) covers every K exactly once and reproduces the
//              dot products
//  down        same for the down kernel's loops
//  prep        the prep kernel's phases, emulated thread by thread, give a valid expert-grouped
//              work list with counts <= 16

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "mtpk.h"
#include "mtpk_common.h"

using namespace mtpk;

static uint64_t g_state = 0x9e3779b97f4a7c15ull;
static uint32_t rnd() {
  g_state ^= g_state << 13;
  g_state ^= g_state >> 7;
  g_state ^= g_state << 17;
  return (uint32_t)(g_state >> 11);
}

static int failures = 0;
static void report(bool ok, const char* name, const char* detail = "") {
  std::printf("%s %s %s\n", ok ? "PASS" : "FAIL", name, detail);
  if (!ok) ++failures;
}

static double fp4_closed(int code) {
  const int s = (code >> 3) & 1, e = (code >> 1) & 3, m = code & 1;
  const double mag = e == 0 ? m * 0.5 : std::ldexp(1.0 + m / 2.0, e - 1);
  return s ? -mag : mag;
}

static void check_decode() {
  bool ok = true;
  for (int code = 0; code < 16; ++code) {
    const float v = fp4_to_f32(code);
    if ((double)v != fp4_closed(code) || std::signbit(v) != bool(code & 8)) ok = false;
  }
  for (int s = 0; s < 256 && ok; ++s) {
    const float f = e8m0_to_f32(s);
    const bool want_ok = s == 0 ? (f == 0.f && !std::signbit(f))
                         : s == 255 ? std::isinf(f) && f > 0
                                    : (double)f == std::ldexp(1.0, s - 127);
    if (!want_ok) ok = false;
    for (int code = 0; code < 16; ++code) {
      const float v = fp4_to_f32(code) * f;
      if (s >= 1 && s <= 254) {
        const double want = fp4_closed(code) * std::ldexp(1.0, s - 127);
        if ((double)v != want && !(std::isinf(v) && std::fabs(want) > 3.4e38)) ok = false;
      }
    }
  }
  report(ok, "decode");
}

static void check_split() {
  bool ok = true;
  for (int i = 0; i < 200000; ++i) {
    const uint32_t bits = (rnd() & 0x7fffffffu) % 0x7f000000u + 0x00800000u;  // normal floats
    float v = bits_f32(bits | (rnd() & 0x80000000u));
    uint16_t hi, lo, mid, lo3, hi3;
    // away from the fp32 subnormal range, where lo itself would go subnormal
    if (std::fabs(v) > 1e-30f && std::fabs(v) < 1e30f) {
      split_bf16(v, &hi, &lo);
      const double two = (double)bf16_to_f32(hi) + (double)bf16_to_f32(lo);
      if (std::fabs(two - v) > std::fabs((double)v) * std::ldexp(1.0, -15)) ok = false;
      split3_bf16(v, &hi3, &mid, &lo3);
      const double three = (double)bf16_to_f32(hi3) + (double)bf16_to_f32(mid) + (double)bf16_to_f32(lo3);
      if (three != (double)v) ok = false;
    }
  }
  report(ok, "split");
}

static void check_argmax_key() {
  bool ok = true;
  const float specials[] = {0.f, -0.f, 1.f, -1.f, INFINITY, -INFINITY, 1e-40f, -1e-40f, 3.5f};
  for (float a : specials)
    for (float b : specials)
      for (uint32_t ia = 0; ia < 3; ++ia)
        for (uint32_t ib = 0; ib < 3; ++ib) {
          if (ia == ib) continue;
          const bool want = a > b || (a == b && ia < ib);
          if ((argmax_key(a, ia) > argmax_key(b, ib)) != want) ok = false;
        }
  for (int i = 0; i < 100000; ++i) {
    const float a = bits_f32(rnd() & 0xff7fffffu), b = bits_f32(rnd() & 0xff7fffffu);
    if (std::isnan(a) || std::isnan(b)) continue;
    const uint32_t ia = rnd() % 1000, ib = rnd() % 1000;
    if (ia == ib) continue;
    const bool want = a > b || (a == b && ia < ib);
    if ((argmax_key(a, ia) > argmax_key(b, ib)) != want) ok = false;
    if (argmax_key_index(argmax_key(a, ia)) != ia) ok = false;
  }
  report(ok, "argmax_key");
}

// Weight value of row n at K index k of a packed [rows, K/2] / scale [rows, K/32] matrix, read
// the way a B lane reads it: 16-byte block load at blk*16, dword h, byte j/2, nibble j&1.
static float lane_weight(const uint8_t* packed, const uint8_t* scale, int K, int n, int blk, int h,
                         int j) {
  const uint8_t* load = packed + (size_t)n * (K / 2) + (size_t)blk * 16;
  uint32_t dword;
  std::memcpy(&dword, load + 4 * h, 4);
  const uint32_t byte = (dword >> (8 * (j >> 1))) & 0xffu;
  const uint32_t code = (j & 1) ? (byte >> 4) : (byte & 15u);
  return fp4_to_f32(code) * e8m0_to_f32(scale[(size_t)n * (K / 32) + blk]);
}

static float direct_weight(const uint8_t* packed, const uint8_t* scale, int K, int n, int k) {
  const uint8_t byte = packed[(size_t)n * (K / 2) + k / 2];
  const uint32_t code = (k & 1) ? (byte >> 4) : (byte & 15u);
  return fp4_to_f32(code) * e8m0_to_f32(scale[(size_t)n * (K / 32) + k / 32]);
}

// Emulates one work item of the gate_up kernel (kMoeWaves = 4 waves, chunk C) for the 16
// weight rows [row0, row0 + 16) against 16 activation rows; returns the max relative error
// against the direct dot product, and checks each K is visited once per (m, n).
static bool emulate_tile(const uint8_t* packed, const uint8_t* scale, int K, int row0,
                         const std::vector<float>& act, int cnt, bool split_waves, int C,
                         double* max_rel) {
  const int nb = K >> 5, ntrip = (nb + 3) >> 2;
  const int waves = split_waves ? 4 : 1;
  std::vector<double> acc(16 * 16, 0.0);
  std::vector<int> visits((size_t)K, 0);
  // Split waves take contiguous quarters of the trips (T each); the ring walks trips
  // i = 0..T-1 in steps of C with the same validity test as the kernel's issue step.
  const int T = split_waves ? (ntrip + 3) / 4 : ntrip;
  for (int wave = 0; wave < waves; ++wave) {
    const int tbase = split_waves ? wave * T : 0;
    for (int t0 = 0; t0 < T; t0 += C) {
      for (int cc = 0; cc < C; ++cc) {
        const int i = t0 + cc;
        const int tr = tbase + i;
        if (i >= T) continue;
        for (int lane = 0; lane < 64; ++lane) {
          const MoeLane ln = moe_lane(lane);
          const int blk = moe_block(tr, ln.g);
          if (!(tr < ntrip && blk < nb)) continue;
          for (int h = 0; h < 4; ++h)
            for (int j = 0; j < 8; ++j) {
              const int k = moe_k_index(tr, ln.g, h, j);
              if (ln.c == 0) visits[k]++;
              // lane (g, c) as B lane: row c; as A lane: token slot c. The MFMA pairs A row m
              // with B column n through the same (g, j) slot.
              const float w = lane_weight(packed, scale, K, row0 + ln.c, blk, h, j);
              for (int m = 0; m < 16; ++m) {
                const float a = m < cnt ? act[(size_t)m * K + k] : 0.f;
                acc[m * 16 + ln.c] += (double)a * w;
              }
            }
        }
      }
    }
  }
  bool ok = true;
  for (int k = 0; k < K; ++k)
    if (visits[k] != 1) ok = false;
  double worst = 0;
  for (int m = 0; m < cnt; ++m)
    for (int n = 0; n < 16; ++n) {
      double want = 0, mag = 0;
      for (int k = 0; k < K; ++k) {
        const double p = (double)act[(size_t)m * K + k] * direct_weight(packed, scale, K, row0 + n, k);
        want += p;
        mag += std::fabs(p);
      }
      worst = std::fmax(worst, std::fabs(acc[m * 16 + n] - want) / (mag + 1e-30));
      // output register i of lane group g holds slot m = 4g + i
      const int g = m / 4, i = m % 4;
      if (moe_out_slot(g, i) != m) ok = false;
    }
  *max_rel = worst;
  return ok;
}

static void check_tiles(const char* name, bool split_waves, int C) {
  bool ok = true;
  double worst = 0;
  const int Ks[] = {32, 64, 96, 128, 160, 1024, 4096};
  for (int K : Ks) {
    const int rows = 32;
    std::vector<uint8_t> packed((size_t)rows * K / 2), scale((size_t)rows * K / 32);
    for (auto& b : packed) b = rnd() & 0xff;
    for (auto& s : scale) s = 118 + rnd() % 13;
    std::vector<float> act((size_t)16 * K);
    for (auto& a : act) a = (float)((int)(rnd() % 2001) - 1000) / 512.f;
    for (int cnt : {1, 5, 16}) {
      double rel;
      if (!emulate_tile(packed.data(), scale.data(), K, 16, act, cnt, split_waves, C, &rel)) ok = false;
      worst = std::fmax(worst, rel);
    }
  }
  char detail[64];
  std::snprintf(detail, sizeof detail, "max_rel=%.3g", worst);
  report(ok && worst < 1e-12, name, detail);
}

// The prep kernel, phase by phase (a __syncthreads() separates phases), one thread at a time.
static void check_prep() {
  bool ok = true;
  const int T = 1024, U = MTPK_MOE_UNIT_TOKENS;
  for (int trial = 0; trial < 40 && ok; ++trial) {
    const int E = 1 + rnd() % (trial < 20 ? 600 : 4096);
    const int A = rnd() % 2500;
    const int lo = rnd() % 3;
    std::vector<int> ae(A);
    std::vector<float> aw(A);
    for (int a = 0; a < A; ++a) {
      ae[a] = (int)(rnd() % (E + 4)) - 1;  // includes out-of-range ids
      aw[a] = (rnd() % 7 == 0) ? 0.f : 1.f;
    }
    auto live = [&](int a) {
      const int ex = ae[a] - lo;
      return ex >= 0 && ex < E && aw[a] != 0.f;
    };
    const int max_units = std::min(A, E) + A / U;
    std::vector<int> cnt(E, 0), sorted(A, -1), units(3 * std::max(max_units, 1), -7);
    for (int a = 0; a < A; ++a)
      if (live(a)) cnt[ae[a] - lo]++;
    const int per = (E + T - 1) / T;
    std::vector<int> sc(T, 0), su(T, 0);
    for (int tid = 0; tid < T; ++tid)
      for (int i = 0; i < per; ++i) {
        const int e = tid * per + i;
        if (e < E) {
          sc[tid] += cnt[e];
          su[tid] += (cnt[e] + U - 1) / U;
        }
      }
    // block-wide exclusive scan = wave scans + wave totals, emulated
    std::vector<int> pc(T), pu(T);
    int run_c = 0, run_u = 0;
    for (int tid = 0; tid < T; ++tid) {
      pc[tid] = run_c;
      pu[tid] = run_u;
      run_c += sc[tid];
      run_u += su[tid];
    }
    const int total_units = run_u;
    for (int tid = 0; tid < T; ++tid) {
      int c0 = pc[tid], u0 = pu[tid];
      for (int i = 0; i < per; ++i) {
        const int e = tid * per + i;
        if (e >= E) break;
        const int c = cnt[e], nu = (c + U - 1) / U;
        for (int j = 0; j < nu; ++j) {
          const int u = u0 + j;
          if (u < max_units) {
            units[3 * u] = e;
            units[3 * u + 1] = c0 + j * U;
            units[3 * u + 2] = std::min(U, c - j * U);
          }
        }
        cnt[e] = c0;
        c0 += c;
        u0 += nu;
      }
    }
    const int n_units = std::min(total_units, max_units);
    if (total_units > max_units) ok = false;  // the bound must hold
    for (int a = 0; a < A; ++a)
      if (live(a)) sorted[cnt[ae[a] - lo]++] = a;
    // checks: every live assignment appears once; units partition [0, n_live) by expert
    int n_live = 0;
    for (int a = 0; a < A; ++a) n_live += live(a);
    std::vector<int> seen(A, 0);
    int covered = 0;
    for (int u = 0; u < n_units; ++u) {
      const int e = units[3 * u], first = units[3 * u + 1], c = units[3 * u + 2];
      if (c < 1 || c > U || first != covered) ok = false;
      for (int q = first; q < first + c; ++q) {
        const int a = sorted[q];
        if (a < 0 || a >= A || ae[a] - lo != e || !live(a)) ok = false;
        else seen[a]++;
      }
      covered += c;
    }
    if (covered != n_live) ok = false;
    for (int a = 0; a < A; ++a)
      if (seen[a] != (live(a) ? 1 : 0)) ok = false;
  }
  report(ok, "prep");
}

int main() {
  check_decode();
  check_split();
  check_argmax_key();
  check_tiles("gate_up", true, 2);
  check_tiles("down", false, 2);
  check_prep();
  return failures ? 1 : 0;
}
