// Indirect block-sparse attention, decode form (few queries per kv head).
//
// Replaces the attend step of the reference: the loop indirection of
// orthocache_attention / _multihead_loop (src/orthocache/adaptive_attention.py:46-184),
// the Pallas indirect kernel (src/orthocache/indirect_attention.py:29-170) and
// the predicated per-head kernel (src/orthocache/sparse_attention.py:67-138).
// Semantics: softmax(q.k / sqrt(d)) over the tokens of exactly the retained
// blocks, fp32 accumulation; a list with no retained block yields zeros.
//
// The retained blocks come from the compaction kernel as device-side lists:
// one list per (segment, kv head), shared by all heads of a segment
// (unified mask) or one per head (per-head mask).  The list counts stay on
// the device; every workgroup derives the work-item space from them, so no
// host synchronisation or recompilation is needed when the count changes.
//
// Work item = (list, slot i < count, chunk of `chunk` tokens, query group of
// up to 8 queries).  A workgroup streams the chunk's K and V rows once
// (16-byte lane loads, LPR lanes per row), keeps per-row-slot online-softmax
// state (m, l, o) for its queries, merges the slots in LDS and writes one
// partial (m, l, o[D]).  combine_kernel merges the partials of a list in a
// fixed order (log-sum-exp), so results are deterministic.
//
// Logits are kept in the log2 domain: s2 = q.k * log2(e) / sqrt(d), weights
// exp2(s2 - m2); the result is identical in exact arithmetic.
#include "oc_kernels.h"

namespace oc {


__device__ __forceinline__ int list_count(const AttendParams& p, int list) {
  if (p.per_head) return p.counts[list];
  return p.counts[list / p.num_kv_heads];
}

// Exclusive prefix over lists of items per list into s_off[0..nlists].
__device__ int build_item_offsets(const AttendParams& p, int* s_off, int nqg) {
  const int nlists = p.num_segments * p.num_kv_heads;
  const int t = threadIdx.x;
  // Serial scan per thread over a contiguous range, then a scan of range totals.
  __shared__ int s_part[256];
  const int per = (nlists + blockDim.x - 1) / blockDim.x;
  const int lo = t * per;
  const int hi = min(lo + per, nlists);
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += list_count(p, i) * p.nchunk * nqg;
  s_part[t] = sum;
  __syncthreads();
  if (t == 0) {
    int run = 0;
    for (int i = 0; i < (int)blockDim.x; ++i) { const int c = s_part[i]; s_part[i] = run; run += c; }
    s_off[nlists] = run;
  }
  __syncthreads();
  int run = s_part[t];
  for (int i = lo; i < hi; ++i) { s_off[i] = run; run += list_count(p, i) * p.nchunk * nqg; }
  __syncthreads();
  return s_off[nlists];
}

__device__ __forceinline__ int find_list(const int* s_off, int nlists, int item) {
  int lo = 0, hi = nlists - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_off[mid] <= item) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <int DT, int LPR, int NQ>
__global__ __launch_bounds__(256) void attend_decode_kernel(AttendParams p) {
  using E = Elt<DT>;
  constexpr int VEC = E::VEC;
  constexpr int D = LPR * VEC;
  constexpr int NSLOT = 256 / LPR;
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  constexpr int RB = 4;  // rows per sub-batch per slot

  __shared__ int s_off[kMaxLists + 1];
  __shared__ float s_o[NSLOT * NQ * D];
  __shared__ float s_m[NSLOT * NQ];
  __shared__ float s_l[NSLOT * NQ];

  const int nq_total = p.sq * p.group;
  const int nqg = (nq_total + kQG - 1) / kQG;
  const int nlists = p.num_segments * p.num_kv_heads;
  const int total_items = build_item_offsets(p, s_off, nqg);

  const int t = threadIdx.x;
  const int cc = t % LPR;
  const int slot = t / LPR;
  const int rows_per_slot = (p.chunk + NSLOT - 1) / NSLOT;

  for (int item = blockIdx.x; item < total_items; item += gridDim.x) {
    const int list = find_list(s_off, nlists, item);
    int r = item - s_off[list];
    const int qg = r % nqg; r /= nqg;
    const int c = r % p.nchunk;
    const int i = r / p.nchunk;
    const int seg = list / p.num_kv_heads;
    const int h = list - seg * p.num_kv_heads;
    const int off = p.cu_blocks ? p.cu_blocks[seg] : 0;
    const int blk = p.indices[(p.per_head ? (int64_t)h * p.total_blocks : 0) + off + i];
    const bool uni = p.uniform && p.uniform[list];
    const int64_t tok0 = (int64_t)(off + blk) * p.block_size + (int64_t)c * p.chunk;
    const int nrows = min(p.chunk, p.block_size - c * p.chunk);

    // Queries of this item (NQ slots; missing ones are zero and ignored).
    float qv[NQ][VEC];
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
      const int qi = qg * kQG + g;
#pragma unroll
      for (int e = 0; e < VEC; ++e) qv[g][e] = 0.f;
      if (qi < nq_total) {
        const int st = qi / p.group, gg = qi - st * p.group;
        const int64_t qo = (int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                           (int64_t)(h * p.group + gg) * p.q_head_stride + cc * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) qv[g][e] = load_elt(p.q_dtype, p.q, qo + e) * p.logit_scale;
      }
    }

    float m[NQ], l[NQ], o[NQ][VEC];
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
      m[g] = -INFINITY; l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[g][e] = 0.f;
    }

    const char* kb = reinterpret_cast<const char*>(p.k) +
                     (tok0 * p.k_tok_stride + (int64_t)h * p.k_head_stride + (int64_t)cc * VEC) * ESZ;
    const char* vb = reinterpret_cast<const char*>(p.v) +
                     (tok0 * p.v_tok_stride + (int64_t)h * p.v_head_stride + (int64_t)cc * VEC) * ESZ;
    const int64_t krow = p.k_tok_stride * ESZ, vrow = p.v_tok_stride * ESZ;

    for (int r0 = 0; r0 < rows_per_slot; r0 += RB) {
      uint4 kw[RB], vw[RB];
      bool ok[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int row = slot + NSLOT * (r0 + u);
        ok[u] = (r0 + u < rows_per_slot) && (row < nrows);
        if (ok[u]) {
          kw[u] = ld16(kb + row * krow);
          vw[u] = ld16(vb + row * vrow);
        }
      }
      float s[RB][NQ];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        float kx[VEC];
        if (ok[u]) E::unpack(kw[u], kx);
#pragma unroll
        for (int g = 0; g < NQ; ++g) {
          float d = 0.f;
          if (ok[u]) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) d = fmaf(qv[g][e], kx[e], d);
          }
          d = group_sum<LPR>(d);
          s[u][g] = ok[u] ? (uni ? 0.f : d) : -INFINITY;
        }
      }
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        float mb = s[0][g];
#pragma unroll
        for (int u = 1; u < RB; ++u) mb = fmaxf(mb, s[u][g]);
        const float mn = fmaxf(m[g], mb);
        if (mn == -INFINITY) continue;  // nothing valid yet in this slot
        const float alpha = exp2f(m[g] - mn);
        float pw[RB];
        float ls = 0.f;
#pragma unroll
        for (int u = 0; u < RB; ++u) { pw[u] = exp2f(s[u][g] - mn); ls += pw[u]; }
        l[g] = l[g] * alpha + ls;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[g][e] *= alpha;
#pragma unroll
        for (int u = 0; u < RB; ++u) {
          if (ok[u]) {
            float vx[VEC];
            E::unpack(vw[u], vx);
#pragma unroll
            for (int e = 0; e < VEC; ++e) o[g][e] = fmaf(pw[u], vx[e], o[g][e]);
          }
        }
        m[g] = mn;
      }
    }

    // Merge the NSLOT row slots.
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) s_o[(slot * NQ + g) * D + cc * VEC + e] = o[g][e];
      if (cc == 0) { s_m[slot * NQ + g] = m[g]; s_l[slot * NQ + g] = l[g]; }
    }
    __syncthreads();
    float* po = p.part_o + (int64_t)item * kQG * D;
    float* pml = p.part_ml + (int64_t)item * kQG * 2;
    for (int e = t; e < NQ * D; e += blockDim.x) {
      const int g = e / D, d = e - g * D;
      float mm = -INFINITY;
#pragma unroll
      for (int s2 = 0; s2 < NSLOT; ++s2) mm = fmaxf(mm, s_m[s2 * NQ + g]);
      float acc = 0.f, ll = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < NSLOT; ++s2) {
        const float ms = s_m[s2 * NQ + g];
        const float w = (ms == -INFINITY) ? 0.f : exp2f(ms - mm);
        acc = fmaf(s_o[(s2 * NQ + g) * D + d], w, acc);
        ll = fmaf(s_l[s2 * NQ + g], w, ll);
      }
      po[g * D + d] = acc;
      if (d == 0) { pml[2 * g] = mm; pml[2 * g + 1] = ll; }
    }
    __syncthreads();
  }
}

// One workgroup per output row (segment, query token, query head): merge the
// list's partials in item order, o / l, cast to the output dtype.  Zero rows
// for an empty list.
__global__ __launch_bounds__(256) void combine_kernel(AttendParams p) {
  __shared__ int s_off[kMaxLists + 1];
  const int nq_total = p.sq * p.group;
  const int nqg = (nq_total + kQG - 1) / kQG;
  const int nlists = p.num_segments * p.num_kv_heads;
  build_item_offsets(p, s_off, nqg);
  const int hq_count = p.num_kv_heads * p.group;
  int id = blockIdx.x;
  const int hq = id % hq_count; id /= hq_count;
  const int st = id % p.sq;
  const int seg = id / p.sq;
  const int h = hq / p.group, g = hq - h * p.group;
  const int qi = st * p.group + g;
  const int qg = qi / kQG, ql = qi - qg * kQG;
  const int list = seg * p.num_kv_heads + h;
  const int n = list_count(p, list) * p.nchunk;  // items of this query group
  const int base = s_off[list];
  const int D = p.head_dim;
  const int64_t orow = (int64_t)seg * p.out_seg_stride + (int64_t)st * p.out_tok_stride +
                       (int64_t)hq * p.out_head_stride;
  float mm = -INFINITY;
  for (int j = 0; j < n; ++j) {
    const int item = base + j * nqg + qg;
    mm = fmaxf(mm, p.part_ml[((int64_t)item * kQG + ql) * 2]);
  }
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f, ll = 0.f;
    for (int j = 0; j < n; ++j) {
      const int item = base + j * nqg + qg;
      const float mi = p.part_ml[((int64_t)item * kQG + ql) * 2];
      const float w = (mi == -INFINITY) ? 0.f : exp2f(mi - mm);
      acc = fmaf(p.part_o[((int64_t)item * kQG + ql) * D + d], w, acc);
      ll = fmaf(p.part_ml[((int64_t)item * kQG + ql) * 2 + 1], w, ll);
    }
    const float r = (n == 0) ? 0.f : acc / ll;
    store_elt(p.out_dtype, p.out, orow + d, r);
  }
}

template <int DT, int LPR, int NQ>
static hipError_t launch_attend_t(const AttendParams& p, int grid, hipStream_t s) {
  hipLaunchKernelGGL((attend_decode_kernel<DT, LPR, NQ>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int DT, int LPR>
static hipError_t launch_attend_nq(const AttendParams& p, int grid, hipStream_t s) {
  const int nq = p.sq * p.group;
  if (nq <= 1) return launch_attend_t<DT, LPR, 1>(p, grid, s);
  if (nq <= 2) return launch_attend_t<DT, LPR, 2>(p, grid, s);
  if (nq <= 4) return launch_attend_t<DT, LPR, 4>(p, grid, s);
  return launch_attend_t<DT, LPR, 8>(p, grid, s);
}

template <int DT>
static hipError_t launch_attend_dt(const AttendParams& p, int grid, hipStream_t s) {
  switch (p.head_dim / Elt<DT>::VEC) {
    case 8: return launch_attend_nq<DT, 8>(p, grid, s);
    case 16: return launch_attend_nq<DT, 16>(p, grid, s);
    case 32: return launch_attend_nq<DT, 32>(p, grid, s);
    case 64: return launch_attend_nq<DT, 64>(p, grid, s);
    default: return hipErrorInvalidValue;
  }
}

bool attend_supported(int dt, int head_dim) {
  const int vec = (dt == kF32) ? 4 : 8;
  if (head_dim % vec) return false;
  const int lpr = head_dim / vec;
  return lpr == 8 || lpr == 16 || lpr == 32 || lpr == 64;
}

// Upper bound on work items (and partial slots) for a launch.
int64_t attend_max_items(const AttendParams& p) {
  const int nq_total = p.sq * p.group;
  const int nqg = (nq_total + kQG - 1) / kQG;
  return (int64_t)p.num_kv_heads * p.total_blocks * p.nchunk * nqg;
}

hipError_t launch_attend(const AttendParams& p, hipStream_t s) {
  const int64_t max_items = attend_max_items(p);
  if (max_items > 0) {
    const int grid = (int)(max_items < 2048 ? max_items : 2048);
    hipError_t e;
    switch (p.kv_dtype) {
      case kF32: e = launch_attend_dt<kF32>(p, grid, s); break;
      case kBF16: e = launch_attend_dt<kBF16>(p, grid, s); break;
      case kF16: e = launch_attend_dt<kF16>(p, grid, s); break;
      default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
  }
  const int rows = p.num_segments * p.sq * p.num_kv_heads * p.group;
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3(rows), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace oc
