// C ABI of libmt_attn.so: argument checks, launch geometry and dispatch to the
// gfx950 kernels in attn_kernels.h.  Declared in include/mt_attention.h.
//
// The validation mirrors the reference's Python checks
// (src/mega_trading/kernels/triton_attention.py:14-23) so a bad call fails
// before any launch, with a message retrievable through mt_last_error().
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/mt_attention.h"
#include "attn_f32_kernels.h"
#include "attn_kernels.h"
#include "decode_kernels.h"
#include "mt_abi.h"

namespace mt_abi {

namespace {
thread_local char g_err[512] = "";
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MT_OK;
}

const char* last_error() { return g_err; }

int device_cus() {
  // per-device cache; concurrent first calls store the same value
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace mt_abi

namespace {

using mt_abi::device_cus;
using mt_abi::fail;
using mt_abi::ok;

// Events armed by mt_time_next_kernel(): attached to the next main kernel
// launch made by this thread (hipExtLaunchKernel stamps them with that
// dispatch's own start and end), then disarmed.
thread_local hipEvent_t g_time_start = nullptr;
thread_local hipEvent_t g_time_stop = nullptr;

// Process-wide queue armed by mt_time_kernel_queue(): event pairs taken in
// launch order by main kernel launches of any thread (after this thread's own
// mt_time_next_kernel arming).
std::mutex g_time_mu;
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_time_queue;
size_t g_time_next = 0;

template <class K>
hipError_t launch_main(K kernel, dim3 grid, dim3 block, hipStream_t st, const mt::AttnParams& p) {
  hipEvent_t a = g_time_start, b = g_time_stop;
  g_time_start = g_time_stop = nullptr;
  if (!a) {
    std::lock_guard<std::mutex> lock(g_time_mu);
    if (g_time_next < g_time_queue.size()) {
      a = g_time_queue[g_time_next].first;
      b = g_time_queue[g_time_next].second;
      ++g_time_next;
    }
  }
  hipExtLaunchKernelGGL(kernel, grid, block, 0, st, a, b, 0, p);
  return hipGetLastError();
}

// One [B,H,T,D] tensor: d stride must be 1, rows 16-byte aligned.
int check_tensor(const char* name, const void* ptr, const int64_t* s) {
  if (!ptr) return fail(MT_E_NULL, "%s is NULL", name);
  if (s[3] != 1) return fail(MT_E_STRIDE, "%s: last-dim stride must be 1 (got %lld)", name, (long long)s[3]);
  if (reinterpret_cast<uintptr_t>(ptr) % 16) return fail(MT_E_STRIDE, "%s: base pointer must be 16-byte aligned", name);
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8) return fail(MT_E_STRIDE, "%s: stride %d (%lld) must be a multiple of 8 elements", name, i, (long long)s[i]);
  // tile staging keeps 64 rows of offsets in 32-bit registers
  if (s[2] > (int64_t(1) << 24)) return fail(MT_E_STRIDE, "%s: row stride %lld too large", name, (long long)s[2]);
  return MT_OK;
}

int check_common(int B, int Hq, int Hkv, int T, int D, int dtype, const float* cs, const float* sn) {
  if (B < 1 || Hq < 1 || Hkv < 1 || T < 1) return fail(MT_E_SHAPE, "B, Hq, Hkv and T must be >= 1 (got %d, %d, %d, %d)", B, Hq, Hkv, T);
  if (Hq % Hkv) return fail(MT_E_SHAPE, "query heads (%d) must equal key/value heads (%d) multiplied by repeats", Hq, Hkv);
  if (D != 32 && D != 64 && D != 128) return fail(MT_E_SHAPE, "head_dim %d unsupported (32, 64 or 128)", D);
  if (dtype != MT_DTYPE_BF16 && dtype != MT_DTYPE_FP16 && dtype != MT_DTYPE_FP32)
    return fail(MT_E_DTYPE, "dtype code %d unsupported", dtype);
  if ((cs == nullptr) != (sn == nullptr)) return fail(MT_E_ROPE, "rope_cos and rope_sin must both be given or both be NULL");
  if (cs && (reinterpret_cast<uintptr_t>(cs) % 16 || reinterpret_cast<uintptr_t>(sn) % 16))
    return fail(MT_E_ROPE, "RoPE tables must be 16-byte aligned");
  return MT_OK;
}

int kv_keys(int) { return mt::kKvKeys; }

// How many workgroups share a key block in the dK/dV pass (each then sums a
// range of the group's heads into fp32 partials that a combine pass adds).
//  * D <= 64: dQ and dK/dV tasks share one grid (attn_bwd_kernel), where the
//    many dQ tasks balance the long causal dK/dV tasks.  At most 4 heads per
//    task (split ceil(R / 4), head ranges as even as R allows), and at least
//    one dK/dV task per CU.  Measured at T = 4096, D = 64 (fwd+bwd TFLOP/s,
//    split 1 / 2): R = 3: 641 / 623, R = 4: 707 / 684, R = 7: 547 / 647,
//    R = 8: 620 / 702; BASELINE config 2 and the config 5 layer are also
//    fastest unsplit (the combine pass costs more than the balance gains).
//  * D = 128: dK/dV runs alone; the smallest divisor of R that gives about
//    four workgroups per CU (two resident, so two rounds) lets the
//    heaviest-first order pair long and short tasks.
#ifndef MT_DKV_FORCE_SPLIT
#define MT_DKV_FORCE_SPLIT 0
#endif
int choose_split(int B, int Hq, int Hkv, int T, int D) {
  const int R = Hq / Hkv;
  if (MT_DKV_FORCE_SPLIT > 0) return MT_DKV_FORCE_SPLIT < R ? MT_DKV_FORCE_SPLIT : R;
  const int nkb = (T + kv_keys(D) - 1) / kv_keys(D);
  const long tasks = (long)nkb * B * Hkv;
  if (D <= 64) {
    int split = (R + 3) / 4;
    while (split < R && tasks * split < device_cus()) ++split;
    return split;
  }
  const long want = 4L * device_cus();
  int split = 1;
  for (int s = 1; s <= R; ++s) {
    if (R % s) continue;
    split = s;
    if (tasks * s >= want) break;
  }
  return split;
}

// workspace layout: -delta [B,Hq,T] fp32 | -lse*log2(e) [B,Hq,T] fp32 | dK/dV partials
size_t vec_bytes(int B, int Hq, int T) { return (((size_t)B * Hq * T * sizeof(float)) + 255) / 256 * 256; }
size_t delta_bytes(int B, int Hq, int T) { return 2 * vec_bytes(B, Hq, T); }

size_t workspace_bytes_split(int B, int Hq, int Hkv, int T, int D, int split) {
  const size_t part = split > 1 ? (size_t)split * 2 * B * Hkv * T * D * sizeof(float) : 0;
  return delta_bytes(B, Hq, T) + part;
}

// the fp32 backward kernels never split a key block's heads (no partials)
int split_for(int B, int Hq, int Hkv, int T, int D, int dtype) {
  return dtype == MT_DTYPE_FP32 ? 1 : choose_split(B, Hq, Hkv, T, D);
}

size_t workspace_bytes(int B, int Hq, int Hkv, int T, int D, int dtype) {
  return workspace_bytes_split(B, Hq, Hkv, T, D, split_for(B, Hq, Hkv, T, D, dtype));
}

// fwd / dQ workgroup geometry for `pairs` (query head, 64-row block) pairs per
// workgroup: the heads of a KV group first (r_sub of them), then row blocks.
void set_pairs(mt::AttnParams& p, int pairs) {
  p.r_sub = (p.R % pairs == 0) ? pairs : (pairs >= 2 && p.R % 2 == 0) ? 2 : 1;
  p.n_hsub = p.R / p.r_sub;
  p.rb = pairs / p.r_sub;
  p.nsb = (p.nqb + p.rb - 1) / p.rb;
}

// Waves per D = 128 dQ workgroup: 8 (one workgroup per CU) or 4 (two per
// CU, each barrier then stalls only half of a CU's waves).  Measured at
// BASELINE config 4 (A/B on one box): 4 waves take the dQ kernel from 0.465
// to 0.433 ms, but the whole fwd+bwd step stays at 1.51 ms (the dK/dV kernel
// that follows runs correspondingly slower), so 8 is kept.
#ifndef MT_DQ128_WAVES
#define MT_DQ128_WAVES 8
#endif
constexpr int kDq128Waves = MT_DQ128_WAVES;

// Waves per D = 128 forward workgroup: 8 with 128-key K / V tiles (one
// workgroup per CU, 128 KB of LDS) or 4 with 64-key tiles (two per CU, so a
// barrier stalls half of a CU's waves).  Measured at BASELINE config 4 (A/B
// on one box): the forward 0.402 -> 0.383 ms with 4, the fwd+bwd step within
// 1 % (the kernels after it run at a lower clock).
#ifndef MT_FWD128_WAVES
#define MT_FWD128_WAVES 4
#endif
constexpr int kFwd128Waves = MT_FWD128_WAVES;

// split = 0: the dK/dV head split of choose_split; else that split (a divisor of R)
void fill_geometry(mt::AttnParams& p, int B, int Hq, int Hkv, int T, int D, float scale, int split = 0) {
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.T = T;
  p.R = Hq / Hkv;
  p.nqb = (T + mt::kBlk - 1) / mt::kBlk;
  set_pairs(p, 4);
  p.nkb = (T + kv_keys(D) - 1) / kv_keys(D);
  p.n_split = split > 0 ? split : choose_split(B, Hq, Hkv, T, D);
  p.scale = scale;
  p.scale_log2 = scale * mt::kLog2e;
}

void copy3(int64_t dst[3], const int64_t* s) {
  dst[0] = s[0];
  dst[1] = s[1];
  dst[2] = s[2];
}

// D <= 64 forward with 8 waves of 32 rows (attn_fwd_w8_kernel) instead of 4 of
// 64: 0 never, 1 when the grid is one resident round, 2 always
#ifndef MT_FWD64_W8
#define MT_FWD64_W8 1
#endif

template <class E, int D, bool ROPE>
hipError_t launch_fwd(mt::AttnParams p, hipStream_t st, int) {
  if (ROPE) {
    // K_rot = rot(K), contiguous; the forward's K tiles and the backward read it
    const int64_t chunks = (int64_t)p.B * p.Hkv * p.T * (D / 8);
    hipLaunchKernelGGL((mt::rope_rows_kernel<E, D>), dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st,
                       p.k, p.sk[0], p.sk[1], p.sk[2], p.dk, p.cos, p.sin, p.Hkv, p.T, chunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    p.k = p.dk;
    p.sk[0] = (int64_t)p.Hkv * p.T * D;
    p.sk[1] = (int64_t)p.T * D;
    p.sk[2] = D;
  }
#ifndef MT_FWD_FOLD
#define MT_FWD_FOLD 1
#endif
  // one resident round (more than one and at most two workgroups per CU):
  // pair heavy and light row blocks on each CU
  const int cus = device_cus();
  auto fold = [&](int grid) { return (MT_FWD_FOLD && grid > cus && grid <= 2 * cus) ? cus : 0; };
  const dim3 grid(p.nsb * p.B * p.Hkv * p.n_hsub);
  p.fwd_fold = fold((int)grid.x);
  if constexpr (D > 64) {
    // kFwd128Waves waves per workgroup (kFwd128Waves / 2 (head, row block) pairs)
    constexpr int keys = kFwd128Waves == 8 ? 128 : 64;
    mt::AttnParams pf = p;
    set_pairs(pf, kFwd128Waves / 2);
    const dim3 grid_w(pf.nsb * pf.B * pf.Hkv * pf.n_hsub), block(64 * kFwd128Waves);
    pf.fwd_fold = fold((int)grid_w.x);
    return pf.rb == 1
               ? launch_main(mt::attn_fwd_w8_kernel<E, D, ROPE, true, kFwd128Waves, keys>, grid_w, block, st, pf)
               : launch_main(mt::attn_fwd_w8_kernel<E, D, ROPE, false, kFwd128Waves, keys>, grid_w, block, st, pf);
  } else {
    if (MT_FWD64_W8 == 2 || (MT_FWD64_W8 == 1 && (int)grid.x <= 2 * cus)) {
      // one resident round: 8 waves of 32 rows, so the longest row blocks
      // run as two waves per SIMD rather than one
      const dim3 block(512);
      return p.rb == 1 ? launch_main(mt::attn_fwd_w8_kernel<E, D, ROPE, true, 8, 128>, grid, block, st, p)
                       : launch_main(mt::attn_fwd_w8_kernel<E, D, ROPE, false, 8, 128>, grid, block, st, p);
    }
    return p.rb == 1 ? launch_main(mt::attn_fwd_kernel<E, D, ROPE, true>, grid, dim3(256), st, p)
                     : launch_main(mt::attn_fwd_kernel<E, D, ROPE, false>, grid, dim3(256), st, p);
  }
}

// Keys per dK/dV task in the one-launch backward (D <= 64): 128, or 64 when
// the launch is bound by its longest tasks rather than by throughput.  The
// task of key block 0 covers every row of its heads; when that work exceeds
// 1.5x the average a workgroup slot (two per CU) has to do, the
// heaviest-first order cannot hide it and the launch ends with those tasks
// running nearly alone (short sequences with few KV groups: BASELINE config
// 2 has 2.1x, config 3 1.1x, the config 5 layer 1.0x).  Work is counted in
// MFMAs per wave: 48 per (64-row block, 64 keys) of a dQ wave, 64 per (32
// keys, 128 rows) of a dK/dV wave.
#ifndef MT_DKV_KEYS
#define MT_DKV_KEYS 0  // 0: by the rule above; 64 or 128: always that
#endif
int merged_dkv_keys(const mt::AttnParams& p) {
  if (MT_DKV_KEYS == 64 || MT_DKV_KEYS == 128) return MT_DKV_KEYS;
  const double steps = (p.T + 127) / 128;                  // 128-row steps of key block 0
  const double hpt = (p.R + p.n_split - 1) / p.n_split;    // heads of the largest task
  const double heavy = 64.0 * hpt * steps;
  const double nqb = p.nqb;
  const double dq = 48.0 * p.B * p.Hq * nqb * (nqb + 1) / 2 / 4;
  const double kv = 64.0 * p.B * p.Hq * steps * (steps + 1) / 2;
  const double mean = (dq + kv) / (2.0 * device_cus());
  return heavy > 1.5 * mean ? 64 : 128;
}

// Longest-first order of the one-launch backward (attn_bwd_kernel): both task
// lists are already sorted by work (MFMAs per wave, as in merged_dkv_keys);
// their merge is described as a head of the kind longer than every task of
// the other, a proportional middle, and a tail of the kind shorter than every
// task of the other.  Measured at BASELINE config 3 against a proportional
// interleave of the whole lists (which starts the medium dK/dV tasks last):
// see the design notes; the end of the launch is its shortest tasks.
void bwd_merge(mt::AttnParams& p, int kvk) {
  const int sh = ((p.n_kv_tasks | p.n_dq_tasks) & 7) == 0 ? 3 : 0;
  const int nk = p.n_kv_tasks >> sh, nd = p.n_dq_tasks >> sh;
  p.mg_mid_kv = p.mg_mid_dq = 0;
  if (nk == 0 || nd == 0) {
    p.mg_head = nk + nd;
    p.mg_head_kv = nk > 0;
    return;
  }
  const long hpt = (p.R + p.n_split - 1) / p.n_split;
  const int kv_groups = p.B * p.Hkv * p.n_split, dq_groups = p.B * p.Hkv * p.n_hsub;
  auto wk = [&](int q) {
    const int kb = (q << sh) / kv_groups;
    return (kvk == 128 ? 64L : 32L) * hpt * ((p.T - kvk * kb + 127) / 128);
  };
  auto wd = [&](int r) {
    const int sb = p.nsb - 1 - (r << sh) / dq_groups;
    return 48L * std::min((sb + 1) * p.rb, p.nqb);
  };
  auto count_k = [&](auto pred) { int c = 0; for (int q = 0; q < nk; ++q) c += pred(wk(q)); return c; };
  auto count_d = [&](auto pred) { int c = 0; for (int r = 0; r < nd; ++r) c += pred(wd(r)); return c; };
  const long k_max = wk(0), k_min = wk(nk - 1), d_max = wd(0), d_min = wd(nd - 1);
  int head_k = 0, head_d = 0, tail_k = 0, tail_d = 0;
  if (k_max > d_max) head_k = count_k([&](long w) { return w > d_max; });
  else if (d_max > k_max) head_d = count_d([&](long w) { return w > k_max; });
  if (k_min > d_min) tail_d = count_d([&](long w) { return w < k_min; });
  else if (d_min > k_min) tail_k = count_k([&](long w) { return w < d_min; });
  p.mg_head_kv = head_k > 0 || head_d == 0;
  p.mg_head = head_k + head_d;
  p.mg_mid_kv = std::max(0, nk - head_k - tail_k);
  p.mg_mid_dq = std::max(0, nd - head_d - tail_d);
}

// stage: 1 = prep (delta, LSE log2 e) + dQ, 2 = dK/dV (reads the prep vectors), 3 = all
template <class E, int D, bool ROPE>
hipError_t launch_bwd(mt::AttnParams p, hipStream_t st, int stage) {
  const int n_dq = p.nsb * p.B * p.Hkv * p.n_hsub;
  const int kvk = D <= 64 ? merged_dkv_keys(p) : mt::kKvKeys;
  const int n_kv = (p.T + kvk - 1) / kvk * p.B * p.Hkv * p.n_split;
  if (D <= 64 && (stage & 1)) {
    // -delta and -LSE log2(e) for both kinds of task (at D = 128 the dQ
    // kernel, which runs first, writes them)
    const int64_t rows = (int64_t)p.B * p.Hq * p.T;
    const int64_t rows_per_block = 256 / (D / 8);
    hipLaunchKernelGGL((mt::attn_bwd_prep_kernel<E, D>), dim3((unsigned)((rows + rows_per_block - 1) / rows_per_block)),
                       dim3(256), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if constexpr (D <= 64) {
    // dQ and dK/dV tasks in one grid
    p.n_dq_tasks = (stage & 1) ? n_dq : 0;
    p.n_kv_tasks = (stage & 2) ? n_kv : 0;
    bwd_merge(p, kvk);
    const dim3 grid(p.n_dq_tasks + p.n_kv_tasks);
    hipError_t e;
    if (kvk == 64)
      e = p.rb == 1 ? launch_main(mt::attn_bwd_kernel<E, D, ROPE, true, 64>, grid, dim3(256), st, p)
                    : launch_main(mt::attn_bwd_kernel<E, D, ROPE, false, 64>, grid, dim3(256), st, p);
    else
      e = p.rb == 1 ? launch_main(mt::attn_bwd_kernel<E, D, ROPE, true, 128>, grid, dim3(256), st, p)
                    : launch_main(mt::attn_bwd_kernel<E, D, ROPE, false, 128>, grid, dim3(256), st, p);
    if (e != hipSuccess) return e;
  } else {
    if (stage & 1) {
      // kDq128Waves waves per workgroup: kDq128Waves / 2 (head, row block) pairs
      mt::AttnParams pq = p;
      set_pairs(pq, kDq128Waves / 2);
      const dim3 grid(pq.nsb * pq.B * pq.Hkv * pq.n_hsub), block(64 * kDq128Waves);
      hipError_t e = pq.rb == 1
                         ? launch_main(mt::attn_bwd_dq_w8_kernel<E, D, ROPE, true, kDq128Waves>, grid, block, st, pq)
                         : launch_main(mt::attn_bwd_dq_w8_kernel<E, D, ROPE, false, kDq128Waves>, grid, block, st, pq);
      if (e != hipSuccess) return e;
    }
    if (stage & 2) {
      hipError_t e = launch_main(mt::attn_bwd_dkv_kernel<E, D, ROPE>, dim3(n_kv), dim3(64 * mt::kKvWaves), st, p);
      if (e != hipSuccess) return e;
    }
  }
  if (stage & 2) {
    if (p.n_split > 1) {
      const int64_t n4 = (int64_t)p.B * p.Hkv * p.T * (D / 4);
      hipLaunchKernelGGL((mt::attn_bwd_combine_kernel<E, D, ROPE>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, p);
      return hipGetLastError();
    }
  }
  return hipSuccess;
}

// fp32 tensors: the fp32-MFMA kernels of attn_f32_kernels.h (K rotated by its
// own pass with RoPE, as for 16-bit; no dK/dV head split)
template <int D, bool ROPE>
hipError_t launch_fwd_f32(mt::AttnParams p, hipStream_t st, int) {
  if (ROPE) {
    const int64_t n4 = (int64_t)p.B * p.Hkv * p.T * (D / 4);
    hipLaunchKernelGGL((mt::rope_f32_kernel<D>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const float*>(p.k), p.sk[0], p.sk[1], p.sk[2], reinterpret_cast<float*>(p.dk),
                       p.cos, p.sin, p.Hkv, p.T, n4);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    p.k = p.dk;
    p.sk[0] = (int64_t)p.Hkv * p.T * D;
    p.sk[1] = (int64_t)p.T * D;
    p.sk[2] = D;
  }
  const int64_t blocks = (int64_t)p.B * p.Hq * ((p.T + 31) / 32);  // one 4-wave workgroup per (batch, head, 32 rows)
  return launch_main(mt::attn_fwd_f32_kernel<D, ROPE>, dim3((unsigned)blocks), dim3(256), st, p);
}

template <int D, bool ROPE>
hipError_t launch_bwd_f32(mt::AttnParams p, hipStream_t st, int stage) {
  const int nblk = (p.T + 31) / 32;
  if (stage & 1) {
    const int64_t rows = (int64_t)p.B * p.Hq * p.T;
    const int64_t rows_per_block = 256 / (D / 4);
    hipLaunchKernelGGL((mt::attn_bwd_prep_f32_kernel<D>), dim3((unsigned)((rows + rows_per_block - 1) / rows_per_block)),
                       dim3(256), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t blocks = (int64_t)p.B * p.Hq * nblk;  // one 4-wave workgroup per (batch, head, 32 rows)
    e = launch_main(mt::attn_bwd_dq_f32_kernel<D, ROPE>, dim3((unsigned)blocks), dim3(256), st, p);
    if (e != hipSuccess) return e;
  }
  if (stage & 2) {
    const int64_t blocks = (int64_t)p.B * p.Hkv * nblk;  // one 4-wave workgroup per (batch, KV head, 32 keys)
    hipError_t e = launch_main(mt::attn_bwd_dkv_f32_kernel<D, ROPE>, dim3((unsigned)blocks), dim3(256), st, p);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

using Launcher = hipError_t (*)(mt::AttnParams, hipStream_t, int);

template <bool FWD, class E, int D>
Launcher pick_rope(bool rope) {
  if (FWD) return rope ? &launch_fwd<E, D, true> : &launch_fwd<E, D, false>;
  return rope ? &launch_bwd<E, D, true> : &launch_bwd<E, D, false>;
}

template <bool FWD, int D>
Launcher pick_f32(bool rope) {
  if (FWD) return rope ? &launch_fwd_f32<D, true> : &launch_fwd_f32<D, false>;
  return rope ? &launch_bwd_f32<D, true> : &launch_bwd_f32<D, false>;
}

template <bool FWD>
Launcher pick(int dtype, int D, bool rope) {
  if (dtype == MT_DTYPE_FP32) {
    if (D == 32) return pick_f32<FWD, 32>(rope);
    if (D == 64) return pick_f32<FWD, 64>(rope);
    return pick_f32<FWD, 128>(rope);
  }
  if (dtype == MT_DTYPE_BF16) {
    if (D == 32) return pick_rope<FWD, mt::BF16, 32>(rope);
    if (D == 64) return pick_rope<FWD, mt::BF16, 64>(rope);
    return pick_rope<FWD, mt::BF16, 128>(rope);
  }
  if (D == 32) return pick_rope<FWD, mt::FP16, 32>(rope);
  if (D == 64) return pick_rope<FWD, mt::FP16, 64>(rope);
  return pick_rope<FWD, mt::FP16, 128>(rope);
}

int bwd_impl(int stage, const void* q, const void* k, const void* v, const void* o, const float* lse,
             const void* dout, void* dq, void* dk, void* dv, void* workspace, size_t workspace_size,
             int B, int Hq, int Hkv, int T, int D, const int64_t* strides, float scale, int dtype,
             const float* rope_cos, const float* rope_sin, void* stream, int split = 0) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, rope_cos, rope_sin);
  if (rc) return rc;
  if (!strides) return fail(MT_E_NULL, "strides is NULL");
  if (!lse) return fail(MT_E_NULL, "lse is NULL");
  if (!workspace) return fail(MT_E_NULL, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(MT_E_STRIDE, "workspace must be 256-byte aligned");
  if (split <= 0) split = split_for(B, Hq, Hkv, T, D, dtype);
  const size_t need = workspace_bytes_split(B, Hq, Hkv, T, D, split);
  if (workspace_size < need)
    return fail(MT_E_WORKSPACE, "workspace too small: %zu bytes given, %zu needed", workspace_size, need);
  if ((rc = check_tensor("q", q, strides + 0))) return rc;
  if ((rc = check_tensor("k", k, strides + 4))) return rc;
  if ((rc = check_tensor("v", v, strides + 8))) return rc;
  if ((rc = check_tensor("o", o, strides + 12))) return rc;
  if ((rc = check_tensor("dout", dout, strides + 16))) return rc;
  if ((rc = check_tensor("dq", dq, strides + 20))) return rc;
  if ((rc = check_tensor("dk", dk, strides + 24))) return rc;
  if ((rc = check_tensor("dv", dv, strides + 28))) return rc;

  mt::AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<const uint16_t*>(o);
  p.dout = static_cast<const uint16_t*>(dout);
  p.out = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.lse = const_cast<float*>(lse);
  p.ndelta = static_cast<float*>(workspace);
  p.nlse2 = reinterpret_cast<float*>(static_cast<char*>(workspace) + vec_bytes(B, Hq, T));
  p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + delta_bytes(B, Hq, T));
  p.cos = rope_cos;
  p.sin = rope_sin;
  copy3(p.sq, strides + 0);
  copy3(p.sk, strides + 4);
  copy3(p.sv, strides + 8);
  copy3(p.so, strides + 12);
  copy3(p.sdo, strides + 16);
  copy3(p.sout, strides + 20);
  copy3(p.sdk, strides + 24);
  copy3(p.sdv, strides + 28);
  fill_geometry(p, B, Hq, Hkv, T, D, scale, split);
  hipError_t e = pick<false>(dtype, D, rope_cos != nullptr)(p, static_cast<hipStream_t>(stream), stage);
  if (e != hipSuccess) return fail(int(e), "backward launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

// ---------------------------------------------------------------------------
// Allocation-free backward: the workspace lives in a fixed device array.
// ---------------------------------------------------------------------------
// Every GPU the library runs on holds its own copy of this array (64 MiB,
// zero-initialised at module load) until the process ends.  In host code
// `scratch` names a host-side stand-in, not device memory: its device address
// is looked up once per device with hipGetSymbolAddress and only that address
// is ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[MT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch` (looked up on the first
// call per device, with that device current).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(int(e), "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MT_E_SHAPE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(e != hipSuccess ? int(e) : MT_E_NULL, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MT_OK;
}

}  // namespace

extern "C" {

int mt_version(void) { return (0 << 16) | 5; }

const char* mt_last_error(void) { return mt_abi::last_error(); }

int mt_time_kernel_queue(void* const* start_events, void* const* stop_events, int n) {
  if (n < 0) return fail(MT_E_SHAPE, "n must be >= 0 (got %d)", n);
  if (n > 0 && (!start_events || !stop_events)) return fail(MT_E_NULL, "event arrays are NULL");
  for (int i = 0; i < n; ++i)
    if (!start_events[i] || !stop_events[i]) return fail(MT_E_NULL, "event pair %d has a NULL event", i);
  std::lock_guard<std::mutex> lock(g_time_mu);
  g_time_queue.clear();
  for (int i = 0; i < n; ++i)
    g_time_queue.emplace_back(static_cast<hipEvent_t>(start_events[i]), static_cast<hipEvent_t>(stop_events[i]));
  g_time_next = 0;
  return ok();
}

int mt_time_next_kernel(void* start_event, void* stop_event) {
  if ((start_event == nullptr) != (stop_event == nullptr))
    return fail(MT_E_NULL, "start_event and stop_event must both be given or both be NULL");
  g_time_start = static_cast<hipEvent_t>(start_event);
  g_time_stop = static_cast<hipEvent_t>(stop_event);
  return ok();
}

size_t mt_gqa_attn_bwd_workspace_size(int B, int Hq, int Hkv, int T, int D) {
  if (B < 1 || Hq < 1 || Hkv < 1 || T < 1 || Hq % Hkv) return 0;
  return workspace_bytes(B, Hq, Hkv, T, D, MT_DTYPE_BF16);  // the 16-bit split: an upper bound for every dtype
}

size_t mt_gqa_attn_bwd_workspace_size_dtype(int B, int Hq, int Hkv, int T, int D, int dtype) {
  if (B < 1 || Hq < 1 || Hkv < 1 || T < 1 || Hq % Hkv) return 0;
  return workspace_bytes(B, Hq, Hkv, T, D, dtype);
}

int mt_gqa_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, void* q_rot, void* k_rot,
                    int B, int Hq, int Hkv, int T, int D,
                    const int64_t* strides, float scale, int dtype,
                    const float* rope_cos, const float* rope_sin, void* stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, rope_cos, rope_sin);
  if (rc) return rc;
  if (!strides) return fail(MT_E_NULL, "strides is NULL");
  if (!lse) return fail(MT_E_NULL, "lse is NULL");
  if ((rc = check_tensor("q", q, strides + 0))) return rc;
  if ((rc = check_tensor("k", k, strides + 4))) return rc;
  if ((rc = check_tensor("v", v, strides + 8))) return rc;
  if ((rc = check_tensor("o", o, strides + 12))) return rc;
  if (rope_cos) {
    if (!q_rot || !k_rot) return fail(MT_E_NULL, "q_rot and k_rot are required with RoPE tables");
    if (reinterpret_cast<uintptr_t>(q_rot) % 16 || reinterpret_cast<uintptr_t>(k_rot) % 16)
      return fail(MT_E_STRIDE, "q_rot / k_rot must be 16-byte aligned");
  }

  mt::AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.out = static_cast<uint16_t*>(o);
  p.qrot = static_cast<uint16_t*>(q_rot);
  p.dk = static_cast<uint16_t*>(k_rot);  // destination of the K RoPE pass
  p.lse = lse;
  p.cos = rope_cos;
  p.sin = rope_sin;
  copy3(p.sq, strides + 0);
  copy3(p.sk, strides + 4);
  copy3(p.sv, strides + 8);
  copy3(p.so, strides + 12);
  fill_geometry(p, B, Hq, Hkv, T, D, scale);
  hipError_t e = pick<true>(dtype, D, rope_cos != nullptr)(p, static_cast<hipStream_t>(stream), 0);
  if (e != hipSuccess) return fail(int(e), "forward launch failed: %s", hipGetErrorString(e));
  return ok();
}

#define MT_BWD_ARGS                                                                                     \
  const void *q, const void *k, const void *v, const void *o, const float *lse, const void *dout,      \
      void *dq, void *dk, void *dv, void *workspace, size_t workspace_size, int B, int Hq, int Hkv,    \
      int T, int D, const int64_t *strides, float scale, int dtype, const float *rope_cos,             \
      const float *rope_sin, void *stream
#define MT_BWD_PASS                                                                                     \
  q, k, v, o, lse, dout, dq, dk, dv, workspace, workspace_size, B, Hq, Hkv, T, D, strides, scale, dtype, \
      rope_cos, rope_sin, stream

int mt_gqa_attn_bwd(MT_BWD_ARGS) { return bwd_impl(3, MT_BWD_PASS); }

int mt_gqa_attn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o, const float* lse,
                            const void* dout, void* dq, void* dk, void* dv, int B, int Hq, int Hkv, int T, int D,
                            const int64_t* strides, float scale, int dtype, const float* rope_cos,
                            const float* rope_sin, void* stream) {
  // shape checks first: a shape whose delta / LSE vectors alone do not fit
  // is rejected before any device call
  int rc = check_common(B, Hq, Hkv, T, D, dtype, rope_cos, rope_sin);
  if (rc) return rc;
  const size_t base = workspace_bytes_split(B, Hq, Hkv, T, D, 1);
  if (base > MT_NOALLOC_SCRATCH_BYTES)
    return fail(MT_E_WORKSPACE,
                "shape B=%d Hq=%d T=%d needs %zu bytes of backward scratch; the allocation-free backward holds "
                "at most %zu (use mt_gqa_attn_bwd with a workspace)",
                B, Hq, T, base, (size_t)MT_NOALLOC_SCRATCH_BYTES);
  if (stream) {
    int sdev = -1, cur = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) == hipSuccess && hipGetDevice(&cur) == hipSuccess &&
        sdev != cur)
      return fail(MT_E_DEVICE, "stream belongs to device %d but device %d is current", sdev, cur);
  }
  // the standard head split when its partials fit, else the largest smaller
  // one that fits (split 1 keeps only delta and LSE, which fit)
  int split = split_for(B, Hq, Hkv, T, D, dtype);
  while (split > 1 && workspace_bytes_split(B, Hq, Hkv, T, D, split) > MT_NOALLOC_SCRATCH_BYTES) --split;
  void* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  return bwd_impl(3, q, k, v, o, lse, dout, dq, dk, dv, ws, MT_NOALLOC_SCRATCH_BYTES, B, Hq, Hkv, T, D, strides,
                  scale, dtype, rope_cos, rope_sin, stream, split);
}
int mt_gqa_attn_bwd_dq(MT_BWD_ARGS) { return bwd_impl(1, MT_BWD_PASS); }
int mt_gqa_attn_bwd_dkv(MT_BWD_ARGS) { return bwd_impl(2, MT_BWD_PASS); }

size_t mt_gqa_attn_decode_workspace_size(int B, int Hq, int L, int D) {
  if (B < 1 || Hq < 1 || L < 1 || D < 1) return 0;
  const size_t nsplit = (size_t)((L + mt::kDecSplit - 1) / mt::kDecSplit);
  return ((size_t)B * Hq * nsplit * (D + 4) * sizeof(float) + 255) / 256 * 256;  // rows of mt::dec_row<D>()
}

namespace {

// A cache of at most kDecWaves splits of 64 keys (its capacity, for
// device-length launches) is decoded by the fused kernel, one workgroup per
// (batch, KV head); longer caches by the split + combine pair, whose grid
// grows with the length.
extern "C++" {
template <class E, int D, int R>
void launch_decode(const mt::DecodeParams& p, dim3 grid_f, dim3 grid_s, dim3 grid_c, hipStream_t st) {
  if (p.nsplit <= mt::kDecWaves) {
    hipLaunchKernelGGL((mt::attn_decode_fused_kernel<E, D, R>), grid_f, dim3(64 * mt::kDecWaves), 0, st, p);
    return;
  }
  hipLaunchKernelGGL((mt::attn_decode_split_kernel<E, D, R>), grid_s, dim3(64), 0, st, p);
  hipLaunchKernelGGL((mt::attn_decode_combine_kernel<E, D>), grid_c, dim3(256), 0, st, p);
}
}  // extern "C++"

int decode_impl(const void* q, const void* k_cache, const void* v_cache, void* o, int B, int Hq, int Hkv, int L,
                const int* length_dev, int D, const int64_t* strides, float scale, int dtype, void* workspace,
                size_t workspace_bytes, void* stream) {
  int rc = check_common(B, Hq, Hkv, L, D, dtype, nullptr, nullptr);
  if (rc) return rc;
  if (dtype == MT_DTYPE_FP32) return fail(MT_E_DTYPE, "decode attention takes bfloat16 or float16 caches");
  if (Hq / Hkv > mt::kDecMaxR)
    return fail(MT_E_SHAPE, "decode supports up to %d query heads per KV head (got %d)", mt::kDecMaxR, Hq / Hkv);
  if (!strides) return fail(MT_E_NULL, "strides is NULL");
  if ((rc = check_tensor("q", q, strides)) || (rc = check_tensor("k_cache", k_cache, strides + 4)) ||
      (rc = check_tensor("v_cache", v_cache, strides + 8)) || (rc = check_tensor("o", o, strides + 12)))
    return rc;
  if (!workspace) return fail(MT_E_NULL, "workspace is NULL");
  if (reinterpret_cast<uintptr_t>(workspace) % 16) return fail(MT_E_STRIDE, "workspace must be 16-byte aligned");
  if (workspace_bytes < mt_gqa_attn_decode_workspace_size(B, Hq, L, D))
    return fail(MT_E_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                mt_gqa_attn_decode_workspace_size(B, Hq, L, D));
  mt::DecodeParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k_cache);
  p.v = static_cast<const uint16_t*>(v_cache);
  p.out = static_cast<uint16_t*>(o);
  p.part = static_cast<float*>(workspace);
  p.sq[0] = strides[0]; p.sq[1] = strides[1];
  p.sk[0] = strides[4]; p.sk[1] = strides[5]; p.sk[2] = strides[6];
  p.sv[0] = strides[8]; p.sv[1] = strides[9]; p.sv[2] = strides[10];
  p.so[0] = strides[12]; p.so[1] = strides[13];
  p.length_dev = length_dev;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.R = Hq / Hkv; p.L = L;
  p.nsplit = (L + mt::kDecSplit - 1) / mt::kDecSplit;
  p.scale_log2 = scale * mt::kLog2e;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid_f((unsigned)(B * Hkv));
  const dim3 grid_s((unsigned)(B * Hkv * p.nsplit));
  const dim3 grid_c((unsigned)(((int64_t)B * Hq * D + 255) / 256));
  // the decode kernels are instantiated per group size R = Hq / Hkv (1..8)
#define MT_DECODE_SPLIT(E, DD, RR) \
  case RR: launch_decode<E, DD, RR>(p, grid_f, grid_s, grid_c, st); break
#define MT_DECODE_LAUNCH(E, DD)                                                                            \
  switch (p.R) {                                                                                           \
    MT_DECODE_SPLIT(E, DD, 1); MT_DECODE_SPLIT(E, DD, 2); MT_DECODE_SPLIT(E, DD, 3); MT_DECODE_SPLIT(E, DD, 4); \
    MT_DECODE_SPLIT(E, DD, 5); MT_DECODE_SPLIT(E, DD, 6); MT_DECODE_SPLIT(E, DD, 7); MT_DECODE_SPLIT(E, DD, 8); \
    default: break;                                                                                        \
  }
  if (dtype == MT_DTYPE_BF16) {
    if (D == 32) { MT_DECODE_LAUNCH(mt::BF16, 32); } else if (D == 64) { MT_DECODE_LAUNCH(mt::BF16, 64); } else { MT_DECODE_LAUNCH(mt::BF16, 128); }
  } else {
    if (D == 32) { MT_DECODE_LAUNCH(mt::FP16, 32); } else if (D == 64) { MT_DECODE_LAUNCH(mt::FP16, 64); } else { MT_DECODE_LAUNCH(mt::FP16, 128); }
  }
#undef MT_DECODE_SPLIT
#undef MT_DECODE_LAUNCH
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "decode launch failed: %s", hipGetErrorString(e));
}

}  // namespace

int mt_gqa_attn_decode(const void* q, const void* k_cache, const void* v_cache, void* o, int B, int Hq, int Hkv, int L,
                       int D, const int64_t* strides, float scale, int dtype, void* workspace, size_t workspace_bytes,
                       void* stream) {
  return decode_impl(q, k_cache, v_cache, o, B, Hq, Hkv, L, nullptr, D, strides, scale, dtype, workspace,
                     workspace_bytes, stream);
}

int mt_gqa_attn_decode_dev(const void* q, const void* k_cache, const void* v_cache, void* o, int B, int Hq, int Hkv,
                           int capacity, const int* length_dev, int D, const int64_t* strides, float scale, int dtype,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (!length_dev) return fail(MT_E_NULL, "length_dev is NULL");
  return decode_impl(q, k_cache, v_cache, o, B, Hq, Hkv, capacity, length_dev, D, strides, scale, dtype, workspace,
                     workspace_bytes, stream);
}

int mt_decode_rope_append(const void* q, const void* k, const void* v, const int64_t* in_strides,
                          const float* rope_cos, const float* rope_sin, int table_rows, int pos, const int* pos_dev,
                          void* q_rot, void* k_cache, void* v_cache, const int64_t* cache_strides, int capacity,
                          int B, int Hq, int Hkv, int D, int in_dtype, int dtype, void* stream) {
  int rc = check_common(B, Hq, Hkv, 1, D, dtype, rope_cos, rope_sin);
  if (rc) return rc;
  if (dtype == MT_DTYPE_FP32) return fail(MT_E_DTYPE, "the KV caches must be bfloat16 or float16");
  if (!q || !k || !v || !q_rot || !k_cache || !v_cache || !rope_cos || !in_strides || !cache_strides)
    return fail(MT_E_NULL, "q, k, v, q_rot, k_cache, v_cache, rope tables and strides must be non-NULL");
  if (in_dtype != MT_DTYPE_BF16 && in_dtype != MT_DTYPE_FP16 && in_dtype != 2)
    return fail(MT_E_DTYPE, "input dtype code %d unsupported", in_dtype);
  if (in_dtype != 2 && in_dtype != dtype) return fail(MT_E_DTYPE, "16-bit inputs must have the cache dtype");
  if (capacity < 1 || table_rows < 1)
    return fail(MT_E_SHAPE, "cache capacity and RoPE table rows must be >= 1 (got %d, %d)", capacity, table_rows);
  // pos is the position written (or, with pos_dev, the largest the device value is clamped to)
  if (pos < 0 || pos >= capacity || pos >= table_rows)
    return fail(MT_E_SHAPE, "pos %d outside the cache (capacity %d) or the RoPE table (%d rows)", pos, capacity,
                table_rows);
  mt::RopeAppendParams p{};
  p.q = q; p.k = k; p.v = v;
  for (int i = 0; i < 2; ++i) {
    p.sq[i] = in_strides[i]; p.sk[i] = in_strides[2 + i]; p.sv[i] = in_strides[4 + i];
  }
  for (int i = 0; i < 3; ++i) { p.skc[i] = cache_strides[i]; p.svc[i] = cache_strides[3 + i]; }
  p.cos = rope_cos; p.sin = rope_sin;
  p.q_out = static_cast<uint16_t*>(q_rot);
  p.kc = static_cast<uint16_t*>(k_cache);
  p.vc = static_cast<uint16_t*>(v_cache);
  p.pos_dev = pos_dev;
  p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.D = D; p.pos = pos;
  const int64_t n = (int64_t)B * (Hq + 2 * Hkv) * (D / 2);
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
#define MT_RA(E, XT) hipLaunchKernelGGL((mt::decode_rope_append_kernel<E, XT>), grid, dim3(256), 0, st, p)
  if (dtype == MT_DTYPE_BF16) {
    if (in_dtype == 2) MT_RA(mt::BF16, 2); else MT_RA(mt::BF16, 0);
  } else {
    if (in_dtype == 2) MT_RA(mt::FP16, 2); else MT_RA(mt::FP16, 1);
  }
#undef MT_RA
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ok() : fail((int)e, "rope append launch failed: %s", hipGetErrorString(e));
}

}  // extern "C"
