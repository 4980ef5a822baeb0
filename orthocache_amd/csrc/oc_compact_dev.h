// Device code of the two-gate mask and stream compaction: the compaction
// kernel (oc_compact.hip) and the ballot prefix that the decode attention
// uses to derive a list from keep flags (oc_attend.hip).  Semantics are
// described in oc_compact.hip.
#pragma once

#include "oc_kernels.h"

namespace oc {

__device__ __forceinline__ bool keep_one(const CompactParams& p, int gj, int h, float tau, float zmax) {
  if (p.mask_in) {
    const int mh = p.mask_in_heads;
    return p.mask_in[(int64_t)gj * mh + (mh == 1 ? 0 : h)] != 0;
  }
  const int64_t e = (int64_t)gj * p.num_kv_heads + h;
  float tm = p.tau_max[e];
  for (int i = 1; i < p.tau_parts; ++i)
    tm = nanmax(tm, p.tau_max[(int64_t)i * p.total_blocks * p.num_kv_heads + e]);
  bool k = tm >= tau;  // false for NaN on either side
  if (p.zeta) k = k & (p.zeta[e] <= zmax);
  return k;
}

// OR over heads without short-circuit, so the loads of all heads are in flight together.
__device__ __forceinline__ bool keep_any(const CompactParams& p, int gj, float tau, float zmax) {
  const int nh = (p.mask_in && p.mask_in_heads == 1) ? 1 : p.num_kv_heads;
  bool a = false;
#pragma unroll 8
  for (int h = 0; h < nh; ++h) a |= keep_one(p, gj, h, tau, zmax);
  return a;
}

// Exclusive prefix of `pred` over the workgroup and the total.  Uniform call.
__device__ __forceinline__ int block_scan_bool(bool pred, int* s_cnt, int& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  const unsigned long long bal = __ballot(pred);
  const int in_wave = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) s_cnt[wave] = __popcll(bal);
  __syncthreads();
  int before = 0, tot = 0;
  for (int w = 0; w < nwaves; ++w) {
    const int c = s_cnt[w];
    before += (w < wave) ? c : 0;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return before + in_wave;
}

template <typename Pred>
__device__ __forceinline__ int stable_partition(int nb, int* out, Pred pred, int* s_cnt) {
  const int t = threadIdx.x;
  int n = 0;
  for (int base = 0; base < nb; base += blockDim.x) {
    const int j = base + t;
    const bool a = (j < nb) && pred(j);
    int tot;
    block_scan_bool(a, s_cnt, tot);
    n += tot;
  }
  int run_act = 0, run_in = 0;
  for (int base = 0; base < nb; base += blockDim.x) {
    const int j = base + t;
    const bool a = (j < nb) && pred(j);
    int tot;
    const int ex = block_scan_bool(a, s_cnt, tot);
    if (j < nb) {
      const int pos = a ? (run_act + ex) : (n + run_in + (t - ex));
      out[pos] = j;
    }
    const int valid = min((int)blockDim.x, nb - base);
    run_act += tot;
    run_in += valid - tot;
  }
  return n;
}

// Mask and compaction of one segment by one workgroup (all threads call it).
// LDS scratch comes from the caller: s_flag (flag_bytes) holds the keep flags
// of a chunk of blocks, s_act (act_cap bytes) the per-block active flags when
// the segment fits (otherwise they are recomputed), s_cnt 16 ints.
__device__ inline void compact_segment(const CompactParams& p, int seg, uint8_t* s_flag, int flag_bytes,
                                uint8_t* s_act, int act_cap, int* s_cnt) {
  const int off = p.cu_blocks ? p.cu_blocks[seg] : 0;
  const int nb = p.cu_blocks ? p.cu_blocks[seg + 1] - off : p.nb_single;
  const float tau = p.tau_arr ? p.tau_arr[seg] : p.tau;
  const float zmax = p.zmax_arr ? p.zmax_arr[seg] : p.zeta_max;
  const int H = p.num_kv_heads;
  const int t = threadIdx.x;
  const bool act_in_lds = nb <= act_cap;
  const int cb = min((int)blockDim.x, flag_bytes / H);  // blocks per chunk

  // Pass 1: every (block, head) predicate in parallel (coalesced), masks,
  // per-block OR through LDS, and the active count.  Each thread first loads
  // kEpt entries into registers (indices clamped, no branches) so the loads
  // are in flight together, then evaluates them.
  constexpr int kEpt = 8;
  int n = 0;
  if (p.indices || p.mask_out || p.active_out) {
    const float* zsrc = p.zeta ? p.zeta : p.tau_max;  // dummy source when gate 2 is off
    for (int b0 = 0; b0 < nb; b0 += cb) {
      const int nbc = min(cb, nb - b0);
      const int ne = nbc * H;
      const int64_t g0 = (int64_t)(off + b0) * H;
      for (int e0 = 0; e0 < ne; e0 += kEpt * (int)blockDim.x) {
        bool kk[kEpt];
        if (p.mask_in) {
          uint8_t mv[kEpt];
#pragma unroll
          for (int u = 0; u < kEpt; ++u) {
            const int e = min(e0 + u * (int)blockDim.x + t, ne - 1);
            const int mh = p.mask_in_heads;
            const int64_t ge = g0 + e;
            mv[u] = p.mask_in[mh == 1 ? (ge / H) : ge];
          }
#pragma unroll
          for (int u = 0; u < kEpt; ++u) kk[u] = mv[u] != 0;
        } else {
          float tv[kEpt], zv[kEpt];
#pragma unroll
          for (int u = 0; u < kEpt; ++u) {
            const int e = min(e0 + u * (int)blockDim.x + t, ne - 1);
            tv[u] = p.tau_max[g0 + e];
            zv[u] = zsrc[g0 + e];
          }
          // Further partial maxima (one per query tile), kPB parts requested
          // together; a clamped repeat of the last part is harmless (max is
          // idempotent).
          constexpr int kPB = 8;
          for (int part = 1; part < p.tau_parts; part += kPB) {
            float pv[kPB][kEpt];
#pragma unroll
            for (int b = 0; b < kPB; ++b) {
              const int pp = min(part + b, p.tau_parts - 1);
              const float* tp = p.tau_max + (int64_t)pp * p.total_blocks * H + g0;
#pragma unroll
              for (int u = 0; u < kEpt; ++u) pv[b][u] = tp[min(e0 + u * (int)blockDim.x + t, ne - 1)];
            }
#pragma unroll
            for (int b = 0; b < kPB; ++b)
#pragma unroll
              for (int u = 0; u < kEpt; ++u) tv[u] = nanmax(tv[u], pv[b][u]);
          }
#pragma unroll
          for (int u = 0; u < kEpt; ++u) kk[u] = (tv[u] >= tau) & ((p.zeta == nullptr) | (zv[u] <= zmax));
        }
#pragma unroll
        for (int u = 0; u < kEpt; ++u) {
          const int e = e0 + u * (int)blockDim.x + t;
          if (e < ne) {
            s_flag[e] = kk[u] ? 1 : 0;
            if (p.mask_out) p.mask_out[g0 + e] = kk[u] ? 1 : 0;
          }
        }
      }
      __syncthreads();
      bool a = false;
      if (t < nbc) {
        for (int h = 0; h < H; ++h) a |= s_flag[t * H + h] != 0;
        if (act_in_lds) s_act[b0 + t] = a ? 1 : 0;
        if (p.active_out) p.active_out[off + b0 + t] = a ? 1 : 0;
      }
      int tot;
      block_scan_bool(a, s_cnt, tot);  // its barriers also retire s_flag
      n += tot;
    }
  }

  // Pass 2: scatter the active-first stable permutation.
  if (p.indices) {
    int run_act = 0, run_in = 0;
    for (int base = 0; base < nb; base += blockDim.x) {
      const int j = base + t;
      bool a = false;
      if (j < nb) a = act_in_lds ? (s_act[j] != 0) : keep_any(p, off + j, tau, zmax);
      int tot;
      const int ex = block_scan_bool(a, s_cnt, tot);
      if (j < nb) {
        const int pos = a ? (run_act + ex) : (n + run_in + (t - ex));
        p.indices[off + pos] = j;
      }
      const int valid = min((int)blockDim.x, nb - base);
      run_act += tot;
      run_in += valid - tot;
    }
    if (t == 0 && p.num_active) p.num_active[seg] = n;
  }

  if (p.head_indices) {
    for (int h = 0; h < H; ++h) {
      int* out = p.head_indices + (int64_t)h * p.total_blocks + off;
      int nh = stable_partition(
          nb, out, [&](int j) { return keep_one(p, off + j, h, tau, zmax); }, s_cnt);
      bool uniform = false;
      if (nh == 0 && p.empty_head_all) {
        for (int j = t; j < nb; j += blockDim.x) out[j] = j;
        nh = nb;
        uniform = true;
      }
      if (t == 0) {
        p.head_num_active[seg * H + h] = nh;
        if (p.head_uniform) p.head_uniform[seg * H + h] = uniform ? 1 : 0;
      }
    }
  }
}

}  // namespace oc
