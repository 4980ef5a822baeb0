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
// Work item = (list, slot i < count, chunk of tokens, query group of up to 8
// queries).  A workgroup (256 threads) takes one item:
//   - LPR lanes per token row (16-byte loads along head_dim, coalesced),
//     NSLOT = 256/LPR row slots, R rows per slot; every K and V row of the
//     item is requested before any arithmetic, so one HBM round trip covers
//     the item;
//   - the R x NQ partial dot products of a lane are reduced across its LPR
//     lanes with a halving butterfly (V - 1 shuffles for V values instead of
//     V log2(LPR)), leaving each lane one logit;
//   - per-slot softmax from LDS, P.V in registers, slots merged by shuffles
//     inside a wave and through LDS across waves; one partial (m, l, o[D]).
// combine_kernel merges a list's partials in item order (log-sum-exp), so the
// result is deterministic.
//
// Logits are kept in the log2 domain: s2 = q.k * log2(e) / sqrt(d), weights
// exp2(s2 - m2); identical to the natural-log form in exact arithmetic.
//
// Keep-flag mode (one segment, unified list): instead of a compacted list,
// the kernel gets the (block, kv head) keep flags of the two-gate mask and
// every workgroup derives the active list itself -- the OR over heads, a
// ballot prefix, the list in LDS (one round trip for 1-2 KB of flags, no
// compaction launch, no dependent load of the count and then the list).
// Workgroup 0 also writes the active-first permutation and the count, the
// outputs the compaction would have written.
//
// Logits variant (LG): inside the fused decode layer the scoring kernel has
// already formed every key row's logits while streaming the keys
// (ScoreParams::logits), so an item reads its rows' logits (NQ floats per
// row) and the value rows only -- half the bytes of K + V -- and skips the
// dot products, the butterfly and the LDS logit exchange.
#include "oc_compact_dev.h"

#ifndef OC_ATTEND_THREADS
#define OC_ATTEND_THREADS 256
#endif

namespace oc {

// Blocks of segment `seg`.
__device__ __forceinline__ int segment_blocks(const AttendParams& p, int seg) {
  return p.cu_blocks ? p.cu_blocks[seg + 1] - p.cu_blocks[seg] : p.total_blocks;
}

// Entries of a block list, clamped to [0, blocks of its segment] so that a
// malformed count never indexes outside the list arrays.
__device__ __forceinline__ int list_count(const AttendParams& p, int list) {
  const int seg = list / p.num_kv_heads;
  const int c = p.per_head ? p.counts[list] : p.counts[seg];
  return min(max(c, 0), segment_blocks(p, seg));
}

// Exclusive scan of one int per thread over a 256-thread workgroup.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave, int& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  int incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int u = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += u;
  }
  if (lane == kWave - 1) s_wave[wave] = incl;
  __syncthreads();
  int before = 0, tot = 0;
  const int nw = blockDim.x / kWave;
  for (int w = 0; w < nw; ++w) {
    const int c = s_wave[w];
    before += (w < wave) ? c : 0;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return before + incl - v;
}

// Work-item offsets of the enumeration units: with unified lists (one list
// per segment, shared by its kv heads) a unit is a segment and its items run
// head-fastest; with per-head lists a unit is one (segment, head) list.
// s_off[u] = first item of unit u, s_off[units] = total items.
__device__ __forceinline__ int num_units(const AttendParams& p) {
  return p.per_head ? p.num_segments * p.num_kv_heads : p.num_segments;
}

__device__ __forceinline__ int unit_items(const AttendParams& p, int u, int nqg) {
  if (p.per_head) return list_count(p, u) * p.nchunk * nqg;
  return list_count(p, u * p.num_kv_heads) * p.nchunk * nqg * p.num_kv_heads;
}

__device__ int build_item_offsets(const AttendParams& p, int* s_off, int nqg) {
  __shared__ int s_wave[16];
  const int nu = num_units(p);
  const int t = threadIdx.x;
  const int per = (nu + blockDim.x - 1) / blockDim.x;
  const int lo = min(t * per, nu);
  const int hi = min(lo + per, nu);
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += unit_items(p, i, nqg);
  int total;
  int run = block_exclusive_scan(sum, s_wave, total);
  for (int i = lo; i < hi; ++i) {
    s_off[i] = run;
    run += unit_items(p, i, nqg);
  }
  if (t == 0) s_off[nu] = total;
  __syncthreads();
  return total;
}

__device__ __forceinline__ int find_list(const int* s_off, int nlists, int item) {
  int lo = 0, hi = nlists - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_off[mid] <= item) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// OR of a block's H keep flags (16-, 4- or 1-byte loads, all in flight
// together).  kp is 16-byte aligned when H is a multiple of 16, 4-byte
// aligned when H is a multiple of 4.
__device__ __forceinline__ bool any_flag(const uint8_t* kp, int H) {
  uint32_t acc = 0;
  if ((H & 15) == 0) {
    for (int h = 0; h < H; h += 16) {
      const uint4 w = *reinterpret_cast<const uint4*>(kp + h);
      acc |= w.x | w.y | w.z | w.w;
    }
  } else if ((H & 3) == 0) {
    for (int h = 0; h < H; h += 4) acc |= *reinterpret_cast<const uint32_t*>(kp + h);
  } else {
    for (int h = 0; h < H; ++h) acc |= kp[h];
  }
  return acc != 0;
}

// The unified active list of one segment from its keep flags, into s_list
// (ascending block ids); returns the count.  Workgroup 0 also writes the
// full active-first stable permutation to p.list_out and the count to
// p.count_out.  s_act holds one flag per block.  Uniform call.
__device__ int list_from_keep(const AttendParams& p, int* s_list, uint8_t* s_act, int* s_cnt) {
  const int nb = p.total_blocks, H = p.num_kv_heads;
  const int t = threadIdx.x;
  int n = 0;
  for (int b0 = 0; b0 < nb; b0 += blockDim.x) {
    const int j = b0 + t;
    const bool a = j < nb && any_flag(p.keep + (int64_t)j * H, H);
    int tot;
    const int ex = block_scan_bool(a, s_cnt, tot);
    if (a) s_list[n + ex] = j;
    if (j < nb) s_act[j] = a ? 1 : 0;
    n += tot;
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    int run = 0;
    for (int b0 = 0; b0 < nb; b0 += blockDim.x) {
      const int j = b0 + t;
      const bool a = j < nb && s_act[j] != 0;
      int tot;
      const int ex = block_scan_bool(a, s_cnt, tot);
      // Active blocks before j: run + ex; inactive ones: j - run - ex.
      if (j < nb) p.list_out[a ? run + ex : n + (j - run - ex)] = j;
      run += tot;
    }
    if (t == 0) p.count_out[0] = n;
  }
  return n;
}

// Threads per attention workgroup: NSLOT = kAttendThreads / LPR token rows
// are in flight per load instruction, R per slot per item.
constexpr int kAttendThreads = OC_ATTEND_THREADS;
constexpr int kAttendGrid = 2048 * 256 / kAttendThreads;

template <int NQ>
__host__ __device__ constexpr int rows_per_slot() {
  return NQ <= 4 ? 8 : 4;
}

template <int DT, int LPR, int NQ, int QDT, bool LG>
__global__ __launch_bounds__(kAttendThreads) void attend_decode_kernel(AttendParams p) {
  using E = Elt<DT>;
  using EQ = Elt<QDT>;
  constexpr int VEC = E::VEC;
  constexpr int D = LPR * VEC;
  constexpr int NSLOT = kAttendThreads / LPR;
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  constexpr int R = rows_per_slot<NQ>();
  constexpr int V = R * NQ;                       // logits per slot
  constexpr int PER_LANE = V >= LPR ? V / LPR : 1;
  constexpr int SPW = kWave / LPR;                // slots per wave
  constexpr int NWAVE = kAttendThreads / kWave;

  static_assert(!LG || NQ <= kLogitsMaxQ, "logits carry at most kLogitsMaxQ queries");
  __shared__ int s_off[kMaxLists + 1];  // item offsets, or the active list in keep-flag mode
  __shared__ uint8_t s_act[kMaxLists];
  __shared__ int s_cnt[16];
  __shared__ float s_log[LG ? 1 : NSLOT * V];
  __shared__ float s_o[NWAVE * NQ * D];
  __shared__ float s_m[NWAVE * NQ];
  __shared__ float s_l[NWAVE * NQ];

  const int nq_total = p.sq * p.group;
  const int nqg = (nq_total + kQG - 1) / kQG;
  const int H = p.num_kv_heads;
  // One segment with one list shared by the heads: no prefix is needed.
  const bool one_unit = !p.per_head && p.num_segments == 1;
  const bool from_keep = p.keep != nullptr;  // one_unit holds (checked on the host)
  int total_items;
  if (from_keep) total_items = list_from_keep(p, s_off, s_act, s_cnt) * p.nchunk * nqg * H;
  else if (one_unit) total_items = min(max(p.counts[0], 0), p.total_blocks) * p.nchunk * nqg * H;
  else total_items = build_item_offsets(p, s_off, nqg);

  const int t = threadIdx.x;
  const int cc = t % LPR;
  const int slot = t / LPR;
  const int wave = t / kWave;

  for (int item = blockIdx.x; item < total_items; item += gridDim.x) {
    // Unified lists are enumerated head-fastest within their segment, so
    // concurrently running workgroups read the other heads' pieces of the
    // same token rows (whole rows of the (seq, heads, dim) layout, as the
    // scoring kernel does).  Per-head lists go list by list.
    int list, r0;
    if (!p.per_head) {
      int seg0 = 0, r = item;
      if (!one_unit) {
        seg0 = find_list(s_off, p.num_segments, item);
        r = item - s_off[seg0];
      }
      list = seg0 * H + r % H;
      r0 = r / H;
    } else {
      list = find_list(s_off, p.num_segments * H, item);
      r0 = item - s_off[list];
    }
    const int qg = r0 % nqg; r0 /= nqg;
    const int c = r0 % p.nchunk;
    const int i = r0 / p.nchunk;
    const int seg = list / p.num_kv_heads;
    const int h = list - seg * p.num_kv_heads;
    const int off = p.cu_blocks ? p.cu_blocks[seg] : 0;
    const int nbs = p.cu_blocks ? p.cu_blocks[seg + 1] - off : p.total_blocks;
    const int blk = from_keep ? s_off[i]
                              : min(max(p.indices[(p.per_head ? (int64_t)h * p.total_blocks : 0) + off + i], 0), nbs - 1);
    const int64_t page = page_of(p.pages, p.num_pages, (int64_t)off + blk);
    const int64_t tok0 = page * p.block_size + (int64_t)c * p.chunk;
    const int nrows = min(p.chunk, p.block_size - c * p.chunk);

    const char* vb = reinterpret_cast<const char*>(p.v) +
                     (tok0 * p.v_tok_stride + (int64_t)h * p.v_head_stride + (int64_t)cc * VEC) * ESZ;
    const int64_t vrow = p.v_tok_stride * ESZ;
    // Uniform per workgroup: a scalar load, which does not wait on the vector loads.
    const bool uni = (p.uniform != nullptr) && (p.uniform[list] != 0);

    // Logits of the lane's R rows (log2 domain): sl[r][g].
    float sl[R][NQ];
    uint4 vw[R];
    if constexpr (LG) {
      // From the scoring pass: NQ floats per row of the block's 512 x NQ
      // tile, rows clamped into the chunk (masked below), then the V rows.
      const float* lb = p.logits + (((int64_t)(off + blk) * p.num_kv_heads + h) * kBlock +
                                    (int64_t)c * p.chunk) * NQ;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float* lp = lb + (int64_t)min(slot + NSLOT * r, nrows - 1) * NQ;
        if constexpr (NQ == 4) {
          const float4 w = *reinterpret_cast<const float4*>(lp);
          sl[r][0] = w.x; sl[r][1] = w.y; sl[r][2] = w.z; sl[r][3] = w.w;
        } else if constexpr (NQ == 2) {
          const float2 w = *reinterpret_cast<const float2*>(lp);
          sl[r][0] = w.x; sl[r][1] = w.y;
        } else {
          sl[r][0] = lp[0];
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) vw[r] = ld16_nt(vb + min(slot + NSLOT * r, nrows - 1) * vrow);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool ok = slot + NSLOT * r < nrows;
#pragma unroll
        for (int g = 0; g < NQ; ++g) sl[r][g] = ok ? (uni ? 0.f : sl[r][g]) : -INFINITY;
      }
    } else {
      const char* kb = reinterpret_cast<const char*>(p.k) +
                       (tok0 * p.k_tok_stride + (int64_t)h * p.k_head_stride + (int64_t)cc * VEC) * ESZ;
      const int64_t krow = p.k_tok_stride * ESZ;

      // Queries (pre-scaled by log2(e)/sqrt(d)); 16-byte loads of the lane's
      // VEC elements, query index clamped and missing queries zeroed.  They are
      // requested before K and V: loads retire in order, so the dot products
      // then wait only for K while V is still arriving.
      float qv[NQ][VEC];
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        const int qi = qg * kQG + g;
        const int qc = min(qi, nq_total - 1);
        const int st = qc / p.group, gg = qc - st * p.group;
        constexpr int QSZ = (QDT == kF32) ? 4 : 2;
        const char* qp = reinterpret_cast<const char*>(p.q) +
                         ((int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                          (int64_t)(h * p.group + gg) * p.q_head_stride + (int64_t)cc * VEC) * QSZ;
        const float sc = qi < nq_total ? p.logit_scale : 0.f;
#pragma unroll
        for (int e0 = 0; e0 < VEC; e0 += EQ::VEC) {
          float tmp[EQ::VEC];
          EQ::unpack(ld16(qp + e0 * QSZ), tmp);
#pragma unroll
          for (int e = 0; e < EQ::VEC && e0 + e < VEC; ++e) qv[g][e0 + e] = tmp[e] * sc;
        }
      }

      // Every K and V load of the item, before any arithmetic.  Row indices are clamped
      // into the block (loads stay unconditional, so none waits behind a
      // branch) and rows past nrows are masked afterwards.
      uint4 kw[R];
#pragma unroll
      for (int r = 0; r < R; ++r) kw[r] = ld16_nt(kb + min(slot + NSLOT * r, nrows - 1) * krow);
#pragma unroll
      for (int r = 0; r < R; ++r) vw[r] = ld16_nt(vb + min(slot + NSLOT * r, nrows - 1) * vrow);

      // Partial dot products, value index r*NQ + g.
      float part[V];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float kx[VEC];
        E::unpack(kw[r], kx);
#pragma unroll
        for (int g = 0; g < NQ; ++g) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) d = fmaf(qv[g][e], kx[e], d);
          part[r * NQ + g] = d;
        }
      }
      Butterfly<V, V, LPR / 2, LPR>::run(part, cc);

      // Logits to LDS (invalid rows -inf, uniform lists 0).
      if constexpr (V >= LPR) {
#pragma unroll
        for (int u = 0; u < PER_LANE; ++u) {
          const int idx = cc * PER_LANE + u;
          const int row = slot + NSLOT * (idx / NQ);
          s_log[slot * V + idx] = row < nrows ? (uni ? 0.f : part[u]) : -INFINITY;
        }
      } else {
        constexpr int REP = LPR / V;
        if (cc % REP == 0) {
          const int idx = cc / REP;
          const int row = slot + NSLOT * (idx / NQ);
          s_log[slot * V + idx] = row < nrows ? (uni ? 0.f : part[0]) : -INFINITY;
        }
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int g = 0; g < NQ; ++g) sl[r][g] = s_log[slot * V + r * NQ + g];
    }

    // Per-slot softmax state and P.V.
    float m[NQ], l[NQ], o[NQ][VEC];
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < R; ++r) mx = fmaxf(mx, sl[r][g]);
      m[g] = mx;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[g][e] = 0.f;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = slot + NSLOT * r;
      if (row < nrows) {
        float vx[VEC];
        E::unpack(vw[r], vx);
#pragma unroll
        for (int g = 0; g < NQ; ++g) {
          const float pw = __builtin_amdgcn_exp2f(sl[r][g] - m[g]);  // v_exp_f32; below 2^-126 flushes to 0
          l[g] += pw;
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[g][e] = fmaf(pw, vx[e], o[g][e]);
        }
      }
    }

    // Merge the slots of this wave (lanes LPR apart) with shuffles.
#pragma unroll
    for (int b = LPR; b < kWave; b <<= 1) {
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        const float m2 = __shfl_xor(m[g], b, kWave);
        const float l2 = __shfl_xor(l[g], b, kWave);
        const float mm = fmaxf(m[g], m2);
        const float w1 = (m[g] == -INFINITY) ? 0.f : exp2f(m[g] - mm);
        const float w2 = (m2 == -INFINITY) ? 0.f : exp2f(m2 - mm);
        l[g] = l[g] * w1 + l2 * w2;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float o2 = __shfl_xor(o[g][e], b, kWave);
          o[g][e] = o[g][e] * w1 + o2 * w2;
        }
        m[g] = mm;
      }
    }
    if ((t & (kWave - 1)) < LPR) {
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) s_o[(wave * NQ + g) * D + cc * VEC + e] = o[g][e];
        if (cc == 0) { s_m[wave * NQ + g] = m[g]; s_l[wave * NQ + g] = l[g]; }
      }
    }
    __syncthreads();

    // Merge the waves and write the item's partial.
    float* po = p.part_o + (int64_t)item * kQG * D;
    float* pml = p.part_ml + (int64_t)item * kQG * 2;
    for (int e = t; e < NQ * D; e += blockDim.x) {
      const int g = e / D, d = e - g * D;
      float mm = -INFINITY;
#pragma unroll
      for (int w = 0; w < NWAVE; ++w) mm = fmaxf(mm, s_m[w * NQ + g]);
      float acc = 0.f, ll = 0.f;
#pragma unroll
      for (int w = 0; w < NWAVE; ++w) {
        const float ms = s_m[w * NQ + g];
        const float wt = (ms == -INFINITY) ? 0.f : exp2f(ms - mm);
        acc = fmaf(s_o[(w * NQ + g) * D + d], wt, acc);
        ll = fmaf(s_l[w * NQ + g], wt, ll);
      }
      po[g * D + d] = acc;
      if (d == 0) { pml[2 * g] = mm; pml[2 * g + 1] = ll; }
    }
    __syncthreads();
    (void)SPW;
  }
}

// Chunk offsets of the lists for the streaming form: list L = seg * Hkv + h
// (unified lists share their segment's count, per-head lists have their own)
// has count_L * nchunk chunks; s_off[L] = chunks of lists before L,
// s_off[nlists] = total.  keep_n >= 0: one segment whose list has keep_n
// blocks for every head.  Uniform call; returns the total.
__device__ int build_list_offsets(const AttendParams& p, int* s_off, int keep_n) {
  __shared__ int s_wave[16];
  const int nl = p.num_segments * p.num_kv_heads;
  const int t = threadIdx.x;
  const int per = (nl + blockDim.x - 1) / blockDim.x;
  const int lo = min(t * per, nl);
  const int hi = min(lo + per, nl);
  auto chunks = [&](int L) { return (keep_n >= 0 ? keep_n : list_count(p, L)) * p.nchunk; };
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += chunks(i);
  int total;
  int run = block_exclusive_scan(sum, s_wave, total);
  for (int i = lo; i < hi; ++i) {
    s_off[i] = run;
    run += chunks(i);
  }
  if (t == 0) s_off[nl] = total;
  __syncthreads();
  return total;
}

constexpr float kStreamLazy = 8.f;  // log2 headroom before a streaming query's reference moves

// Pieces shared by the streaming forms: a chunk is `chunk` rows of one block
// and kv head; a lane holds R rows of its slot and VEC columns, and a row
// slot's online softmax state (m, l, o) for NQ query rows.  KV = false: the
// chunk's logits come from the scoring pass (values and logits are read);
// KV = true: keys and values are read and the logits formed here (the lane's
// partial dot products summed over the row's LPR lanes with the halving
// butterfly, then gathered to every lane of the slot with shuffles, so no
// LDS barrier interrupts the loads in flight).
template <int DT, int LPR, int NQ, bool KV = false, int QDT = DT>
struct Stream {
  using E = Elt<DT>;
  using EQ = Elt<QDT>;
  static constexpr int VEC = E::VEC;
  static constexpr int D = LPR * VEC;
  static constexpr int NSLOT = kAttendThreads / LPR;
  static constexpr int ESZ = (DT == kF32) ? 4 : 2;
  static constexpr int R = rows_per_slot<NQ>();
  static constexpr int NWAVE = kAttendThreads / kWave;
  // Chunk buffers in flight: chunk g + NB - 1 is requested before chunk g is
  // consumed (about one workgroup per CU, so registers go to loads in flight;
  // with logits NB = 3 measured best against 2 and 4; keys and values take
  // twice the registers per chunk).  Four query rows with logits take two:
  // 242 VGPRs, two workgroups per CU, where three buffers
  // needed AGPR spill space and ran one.
  static constexpr int NB = (KV || NQ == 4) ? 2 : 3;
  static_assert(KV ? NQ <= 2 * kLogitsMaxQ : NQ <= kLogitsMaxQ,
                "the streaming forms carry at most kLogitsMaxQ queries with logits, twice that reading keys");

  struct State {
    float m[NQ], l[NQ], o[NQ][VEC];
  };
  // One chunk in flight: value rows, and logits (KV = false) or key rows.
  struct Buf {
    uint4 vw[R];
    float sl[KV ? 1 : R][NQ];
    uint4 kw[KV ? R : 1];
  };
  // The lane's query columns (KV = true).  With 16-bit keys and queries of
  // the same type they stay packed (DOT2: packed dot products on the raw key
  // words, the sums scaled by log2(e)/sqrt(d) after the lane reduction);
  // otherwise they are widened and pre-scaled.
  static constexpr bool DOT2 = KV && DT != kF32 && QDT == DT;
  struct Query {
    float q[KV && !DOT2 ? NQ : 1][VEC];
    uint32_t qw[DOT2 ? NQ : 1][VEC / 2];
    float scale;
  };

  __device__ __forceinline__ static void reset(State& st) {
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
      st.m[g] = -INFINITY;
      st.l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) st.o[g][e] = 0.f;
    }
  }

  // Chunk c of flattened block `flat` (physical page `page`), kv head h:
  // logits (NQ floats per row) or key rows, then value rows.
  __device__ __forceinline__ static void load(const AttendParams& p, int64_t flat, int64_t page, int h, int c,
                                              int slot, int cc, Buf& b) {
    const int64_t tok0 = page * kBlock + (int64_t)c * p.chunk;
    if constexpr (KV) {
      const int64_t krow = p.k_tok_stride * ESZ;
      const char* kb = reinterpret_cast<const char*>(p.k) +
                       (tok0 * p.k_tok_stride + (int64_t)h * p.k_head_stride + (int64_t)cc * VEC) * ESZ;
#pragma unroll
      for (int r = 0; r < R; ++r) b.kw[r] = ld16_nt(kb + (int64_t)(slot + NSLOT * r) * krow);
    } else {
      const float* lb = p.logits + ((flat * p.num_kv_heads + h) * kBlock + (int64_t)c * p.chunk) * NQ;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float* lp = lb + (slot + NSLOT * r) * NQ;
        if constexpr (NQ == 4) {
          const float4 x = *reinterpret_cast<const float4*>(lp);
          b.sl[r][0] = x.x; b.sl[r][1] = x.y; b.sl[r][2] = x.z; b.sl[r][3] = x.w;
        } else if constexpr (NQ == 2) {
          const float2 x = *reinterpret_cast<const float2*>(lp);
          b.sl[r][0] = x.x; b.sl[r][1] = x.y;
        } else {
          b.sl[r][0] = lp[0];
        }
      }
    }
    const int64_t vrow = p.v_tok_stride * ESZ;
    const char* vb = reinterpret_cast<const char*>(p.v) +
                     (tok0 * p.v_tok_stride + (int64_t)h * p.v_head_stride + (int64_t)cc * VEC) * ESZ;
#pragma unroll
    for (int r = 0; r < R; ++r) b.vw[r] = ld16_nt(vb + (int64_t)(slot + NSLOT * r) * vrow);
  }

  // The query rows of list (seg, h), this lane's VEC columns (KV = true).
  // q0: the first of the NQ query rows (the split form's query group).
  __device__ __forceinline__ static void load_query(const AttendParams& p, int seg, int h, int cc, Query& qr,
                                                    int q0 = 0) {
    if constexpr (KV) {
      constexpr int QSZ = (QDT == kF32) ? 4 : 2;
      const int nq = p.sq * p.group - q0;  // rows of this group and after it
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        const int qc = q0 + min(g, nq - 1);
        const int st = qc / p.group, gg = qc - st * p.group;
        const char* qp = reinterpret_cast<const char*>(p.q) +
                         ((int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                          (int64_t)(h * p.group + gg) * p.q_head_stride + (int64_t)cc * VEC) * QSZ;
        if constexpr (DOT2) {
          const uint4 w = ld16(qp);
#pragma unroll
          for (int i = 0; i < VEC / 2; ++i) qr.qw[g][i] = g < nq ? word_of(w, i) : 0u;
        } else {
          const float sc = g < nq ? p.logit_scale : 0.f;
#pragma unroll
          for (int e0 = 0; e0 < VEC; e0 += EQ::VEC) {
            float tmp[EQ::VEC];
            EQ::unpack(ld16(qp + e0 * QSZ), tmp);
#pragma unroll
            for (int e = 0; e < EQ::VEC && e0 + e < VEC; ++e) qr.q[g][e0 + e] = tmp[e] * sc;
          }
        }
      }
      qr.scale = p.logit_scale;
    }
  }

  // The chunk's logits in the log2 domain, every row of the lane's slot:
  // given (KV = false) or formed from the keys (KV = true).
  __device__ __forceinline__ static void logits(const Buf& b, const Query& qr, int cc, float (&lg)[R][NQ]) {
    if constexpr (!KV) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int g = 0; g < NQ; ++g) lg[r][g] = b.sl[r][g];
    } else {
      constexpr int V = R * NQ;  // value index r * NQ + g
      float part[V];
      if constexpr (DOT2) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int g = 0; g < NQ; ++g) {
            float d = 0.f;
#pragma unroll
            for (int w = 0; w < VEC / 2; ++w) d = dot2_acc<DT>(word_of(b.kw[r], w), qr.qw[g][w], d);
            part[r * NQ + g] = d;
          }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float kx[VEC];
          E::unpack(b.kw[r], kx);
#pragma unroll
          for (int g = 0; g < NQ; ++g) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) d = fmaf(qr.q[g][e], kx[e], d);
            part[r * NQ + g] = d;
          }
        }
      }
      Butterfly<V, V, LPR / 2, LPR>::run(part, cc);
      if constexpr (DOT2) {
#pragma unroll
        for (int i = 0; i < V; ++i) part[i] *= qr.scale;
      }
      // Gather the V sums to every lane of the slot (width-LPR shuffles).
      if constexpr (V >= LPR) {
        constexpr int PL = V / LPR;  // lane s holds indices s * PL .. + PL
#pragma unroll
        for (int u = 0; u < PL; ++u)
#pragma unroll
          for (int src = 0; src < LPR; ++src) {
            const int idx = src * PL + u;
            lg[idx / NQ][idx % NQ] = __shfl(part[u], src, LPR);
          }
      } else {
        constexpr int REP = LPR / V;  // lanes idx * REP .. hold index idx
#pragma unroll
        for (int idx = 0; idx < V; ++idx) lg[idx / NQ][idx % NQ] = __shfl(part[0], idx * REP, LPR);
      }
    }
  }

  // Online softmax update with one chunk (all R rows are in the block: the
  // chunk divides the 512-token block).  Uniform lists take equal logits.
  // Lazy rescale: the reference point m of a query moves only when the
  // chunk's max exceeds it by more than 2^kStreamLazy (weights stay below
  // 2^kStreamLazy, exact in fp32); l and o share the reference, so o / l is
  // unchanged, and most chunks skip the rescale of o.  Weights are v_exp_f32
  // directly: a weight below 2^-126 of the reference's flushes to zero.
  __device__ __forceinline__ static void consume(State& st, const Buf& b, const Query& qr, int cc, bool uni) {
    float sl[R][NQ];
    logits(b, qr, cc, sl);
    if (uni) {  // wave-uniform and rare
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int g = 0; g < NQ; ++g) sl[r][g] = 0.f;
    }
    const uint4 (&vw)[R] = b.vw;
    float mt[NQ], sc[NQ];
    bool any_move = false;
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
      float mx = sl[0][g];
#pragma unroll
      for (int r = 1; r < R; ++r) mx = fmaxf(mx, sl[r][g]);
      const bool move = !(mx <= st.m[g] + kStreamLazy);  // also true while m = -inf
      mt[g] = move ? fmaxf(st.m[g], mx) : st.m[g];
      sc[g] = (st.m[g] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(st.m[g] - mt[g]);
      any_move |= move;
    }
    if (__ballot(any_move)) {  // wave-uniform
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        st.l[g] *= sc[g];
#pragma unroll
        for (int e = 0; e < VEC; ++e) st.o[g][e] *= sc[g];
      }
    }
#pragma unroll
    for (int g = 0; g < NQ; ++g) st.m[g] = mt[g];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float vx[VEC];
      E::unpack(vw[r], vx);
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        const float pw = __builtin_amdgcn_exp2f(sl[r][g] - mt[g]);
        st.l[g] += pw;
#pragma unroll
        for (int e = 0; e < VEC; ++e) st.o[g][e] = fmaf(pw, vx[e], st.o[g][e]);
      }
    }
  }

  // Merge the slots of a wave (lanes LPR apart) with shuffles: lanes
  // 0..LPR-1 end with the wave's state for their columns.
  __device__ __forceinline__ static void merge_wave(State& st) {
#pragma unroll
    for (int b = LPR; b < kWave; b <<= 1) {
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        const float m2 = __shfl_xor(st.m[g], b, kWave);
        const float l2 = __shfl_xor(st.l[g], b, kWave);
        const float mm = fmaxf(st.m[g], m2);
        const float w1 = (st.m[g] == -INFINITY) ? 0.f : exp2f(st.m[g] - mm);
        const float w2 = (m2 == -INFINITY) ? 0.f : exp2f(m2 - mm);
        st.l[g] = st.l[g] * w1 + l2 * w2;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float o2 = __shfl_xor(st.o[g][e], b, kWave);
          st.o[g][e] = st.o[g][e] * w1 + o2 * w2;
        }
        st.m[g] = mm;
      }
    }
  }
};

// Split form (kStreamSplit): one segment, a unified list (the one-segment
// decode layer).  Workgroup (split, h) takes a contiguous range of kv head
// h's chunks, so concurrently running workgroups read the other heads'
// pieces of the same token rows; the list is derived from the keep flags or
// copied to LDS once per workgroup.  At the end the slots merge across waves
// through LDS into one partial per (head, split), item split * Hkv + h.
template <int DT, int LPR, int NQ, bool KV, int QDT>
__global__ __launch_bounds__(kAttendThreads) void attend_split_kernel(AttendParams p) {
  using S = Stream<DT, LPR, NQ, KV, QDT>;
  constexpr int R = S::R, NB = S::NB, D = S::D, VEC = S::VEC, NWAVE = S::NWAVE;
  __shared__ int s_list[kMaxLists];
  __shared__ uint8_t s_act[kMaxLists];
  __shared__ int s_cnt[16];
  __shared__ float s_o[NWAVE * NQ * D];
  __shared__ float s_m[NWAVE * NQ];
  __shared__ float s_l[NWAVE * NQ];

  const int H = p.num_kv_heads;
  const int h = blockIdx.x % H;
  // Query group (more than kLogitsMaxQ rows per kv head): rows qg * NQ ...
  constexpr bool kGroups = NQ > kLogitsMaxQ;
  const int split = kGroups ? (blockIdx.x / H) % p.splits : blockIdx.x / H;
  const int qg = kGroups ? blockIdx.x / (H * p.splits) : 0;
  const int t = threadIdx.x;
  const int cc = t % LPR;
  const int slot = t / LPR;
  const int wave = t / kWave;
  const int nb = p.total_blocks;

  int n;
  if (p.keep) {
    n = list_from_keep(p, s_list, s_act, s_cnt);
  } else {
    n = min(max(p.counts[0], 0), nb);
    for (int i = t; i < n; i += blockDim.x) s_list[i] = min(max(p.indices[i], 0), nb - 1);
    __syncthreads();
  }
  n = __builtin_amdgcn_readfirstlane(n);
  const int nu = n * p.nchunk;
  const int per = (nu + p.splits - 1) / p.splits;
  const int u0 = min(split * per, nu);
  const int u1 = min(u0 + per, nu);

  auto load = [&](int u, typename S::Buf& b) {
    const int i = u / p.nchunk, c = u - i * p.nchunk;
    const int blk = __builtin_amdgcn_readfirstlane(s_list[i]);
    int64_t page = blk;
    if (p.pages) {
      const int pg = ld_const(p.pages + blk);
      page = (unsigned)pg < (unsigned)p.num_pages ? pg : (pg < 0 ? 0 : p.num_pages - 1);
    }
    S::load(p, blk, page, h, c, slot, cc, b);
  };

  typename S::State st;
  S::reset(st);
  typename S::Query qr;
  S::load_query(p, 0, h, cc, qr, qg * NQ);
  typename S::Buf buf[NB];
#pragma unroll
  for (int j = 0; j < NB - 1; ++j)
    if (u0 + j < u1) load(u0 + j, buf[j]);
  for (int u = u0; u < u1; u += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (u + j < u1) {
        if (u + j + NB - 1 < u1) load(u + j + NB - 1, buf[(j + NB - 1) % NB]);
        S::consume(st, buf[j], qr, cc, false);
      }
    }
  }

  S::merge_wave(st);
  if ((t & (kWave - 1)) < LPR) {
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) s_o[(wave * NQ + g) * D + cc * VEC + e] = st.o[g][e];
      if (cc == 0) { s_m[wave * NQ + g] = st.m[g]; s_l[wave * NQ + g] = st.l[g]; }
    }
  }
  __syncthreads();
  const int64_t item = ((int64_t)qg * p.splits + split) * H + h;
  float* po = p.part_o + item * kQG * D;
  float* pml = p.part_ml + item * kQG * 2;
  for (int e = t; e < NQ * D; e += blockDim.x) {
    const int g = e / D, d = e - g * D;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) mm = fmaxf(mm, s_m[w * NQ + g]);
    float acc = 0.f, ll = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const float ms = s_m[w * NQ + g];
      const float wt = (ms == -INFINITY) ? 0.f : exp2f(ms - mm);
      acc = fmaf(s_o[(w * NQ + g) * D + d], wt, acc);
      ll = fmaf(s_l[w * NQ + g], wt, ll);
    }
    po[g * D + d] = acc;
    if (d == 0) { pml[2 * g] = mm; pml[2 * g + 1] = ll; }
  }
}

// Ranges form (kStreamRanges): any lists -- several segments, per-head lists,
// uniform flags.  The chunks of all lists, in list order (list L = seg * Hkv
// + h; chunk u of a list: list slot u / nchunk, rows (u % nchunk) * chunk ..),
// form one index space; workgroup w takes the contiguous range
// [w P, (w + 1) P) of it, P = ceil(total / grid), so every workgroup streams
// the same number of chunks whatever the lists' lengths.  It keeps the slot
// states while the chunks belong to one list; when the list changes (and at
// the end) each wave merges its slots with shuffles, the waves merge through
// LDS behind LDS-only barriers (the chunks in flight are not waited for; all
// waves walk the same chunks, so they reach a list change together), and the
// workgroup writes one partial, slot w + L.  Slots are distinct for distinct
// (w, L) because ranges are monotone in w; the combine finds a list's pieces
// from the same offsets.  (One partial per wave instead, merged by the
// combine: C3 combine 12.3 us.)  List entries and offsets are read wave-uniformly (readfirstlane,
// constant-address loads), so the next chunk's list entry is a scalar load
// that does not wait for the vector loads in flight.
template <int DT, int LPR, int NQ, bool KV, int QDT>
__global__ __launch_bounds__(kAttendThreads) void attend_stream_kernel(AttendParams p) {
  using S = Stream<DT, LPR, NQ, KV, QDT>;
  constexpr int R = S::R, NB = S::NB, D = S::D, VEC = S::VEC, NWAVE = S::NWAVE;
  __shared__ int s_off[kMaxLists + 1];
  __shared__ float s_fo[NWAVE * NQ * D];
  __shared__ float s_fm[NWAVE * NQ], s_fl[NWAVE * NQ];

  const int H = p.num_kv_heads;
  const int nl = p.num_segments * H;
  const int w = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int cc = t % LPR;
  const int slot = t / LPR;
  const int wave = t / kWave;

  // Values read back from LDS are the same in every lane: readfirstlane
  // makes that visible to the compiler, so the chunk loop and the addresses
  // derived from it stay scalar.
  const int total = __builtin_amdgcn_readfirstlane(build_list_offsets(p, s_off, -1));
  const int per = (total + (int)gridDim.x - 1) / (int)gridDim.x;
  const int g0 = min(w * per, total);
  const int g1 = min(g0 + per, total);
  if (g0 >= g1) return;  // uniform per workgroup; after the prologue's barriers

  auto uoff = [&](int L) { return __builtin_amdgcn_readfirstlane(s_off[L]); };
  auto load = [&](int g, int L, typename S::Buf& b) {
    const int seg = L / H, h = L - seg * H;
    const int u = g - uoff(L);
    const int i = u / p.nchunk, c = u - i * p.nchunk;
    const int off = p.cu_blocks ? ld_const(p.cu_blocks + seg) : 0;
    const int nbs = p.cu_blocks ? ld_const(p.cu_blocks + seg + 1) - off : p.total_blocks;
    const int blk = min(max(ld_const(p.indices + (p.per_head ? (int64_t)h * p.total_blocks : 0) + off + i), 0), nbs - 1);
    const int64_t flat = (int64_t)off + blk;
    int64_t page = flat;
    if (p.pages) {
      const int pg = ld_const(p.pages + flat);
      page = (unsigned)pg < (unsigned)p.num_pages ? pg : (pg < 0 ? 0 : p.num_pages - 1);
    }
    S::load(p, flat, page, h, c, slot, cc, b);
  };

  typename S::State st;
  typename S::Query qr;
  // The workgroup's partial of list L's piece: each wave merges its slots
  // (lanes 0..LPR-1 hold the result), then the waves merge through LDS.
  auto flush = [&](int L) {
    S::merge_wave(st);
    if (lane < LPR) {
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) s_fo[(wave * NQ + g) * D + cc * VEC + e] = st.o[g][e];
        if (lane == 0) { s_fm[wave * NQ + g] = st.m[g]; s_fl[wave * NQ + g] = st.l[g]; }
      }
    }
    lds_barrier();
    const int64_t item = (int64_t)w + L;
    float* po = p.part_o + item * kQG * D;
    float* pml = p.part_ml + item * kQG * 2;
    for (int e = t; e < NQ * D; e += kAttendThreads) {
      const int g = e / D, d = e - g * D;
      float mm = -INFINITY;
#pragma unroll
      for (int v = 0; v < NWAVE; ++v) mm = fmaxf(mm, s_fm[v * NQ + g]);
      float acc = 0.f, ll = 0.f;
#pragma unroll
      for (int v = 0; v < NWAVE; ++v) {
        const float ms = s_fm[v * NQ + g];
        const float wt = (ms == -INFINITY) ? 0.f : exp2f(ms - mm);
        acc = fmaf(s_fo[(v * NQ + g) * D + d], wt, acc);
        ll = fmaf(s_fl[v * NQ + g], wt, ll);
      }
      po[g * D + d] = acc;
      if (d == 0) { pml[2 * g] = mm; pml[2 * g + 1] = ll; }
    }
    lds_barrier();  // every wave has read the staging before the next flush
  };
  auto is_uniform = [&](int L) { return p.uniform != nullptr && ld_const(p.uniform + L) != 0; };
  // List of chunk g, from a pointer that only moves forward.
  auto advance = [&](int L, int g) {
    while (uoff(L + 1) <= g) ++L;
    return L;
  };

  typename S::Buf buf[NB];
  const int L0 = advance(__builtin_amdgcn_readfirstlane(find_list(s_off, nl, g0)), g0);
  int Lc = L0;  // list being accumulated
  S::load_query(p, Lc / H, Lc - (Lc / H) * H, cc, qr);
  int Ll = L0;  // list of the next chunk to load
  int gl = g0;
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) {
    if (gl < g1) {
      Ll = advance(Ll, gl);
      load(gl, Ll, buf[j]);
      ++gl;
    }
  }
  bool uni = is_uniform(Lc);
  S::reset(st);
  for (int g = g0; g < g1; g += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (g + j < g1) {
        if (gl < g1) {
          Ll = advance(Ll, gl);
          load(gl, Ll, buf[(j + NB - 1) % NB]);
          ++gl;
        }
        const int Ln = advance(Lc, g + j);
        if (Ln != Lc) {
          flush(Lc);
          S::reset(st);
          Lc = Ln;
          uni = is_uniform(Lc);
          S::load_query(p, Lc / H, Lc - (Lc / H) * H, cc, qr);  // keys need the new list's queries
        }
        S::consume(st, buf[j], qr, cc, uni);
      }
    }
  }
  flush(Lc);
}

// Combine (per-item and split forms; the ranges form has combine_lists_kernel
// below): one workgroup per (output row, 64-wide head_dim slice).  Wave w
// takes the list's items w, w+4, ... in rounds of kCombineBatch items: each
// lane requests the partial outputs of the round's items for its column and
// lane u the (m, l) of item u, all before any arithmetic, so one round trip
// serves a round (lists of up to 4 * kCombineBatch partials take one).
// Within a wave the rounds merge online (running max, rescaled sums); the
// four waves merge through LDS.  The order is fixed, so the result is
// deterministic.  kCombineBatch is 32 for per-item lists (lanes 0..31 hold
// their m, l); the split form, whose partial count is known on the host,
// takes the smallest batch that covers its splits in one round, so a wave
// does not issue clamped duplicate loads (C2, 16 splits: batch 4, layer
// 108.0 -> 106.6 us).
template <int kCombineBatch>
__global__ __launch_bounds__(256) void combine_kernel(AttendParams p) {
  __shared__ int s_off[kMaxLists + 1];
  __shared__ float s_ml[2 * 4];
  __shared__ float s_acc[4 * 64];
  const int nq_total = p.sq * p.group;
  const int nqg = (nq_total + kQG - 1) / kQG;
  if (p.stream == kStreamNone && (p.per_head || p.num_segments != 1)) build_item_offsets(p, s_off, nqg);
  const int D = p.head_dim;
  const int ndc = (D + 63) / 64;
  int id = blockIdx.x;
  const int dc = id % ndc; id /= ndc;
  const int hq_count = p.num_kv_heads * p.group;
  const int hq = id % hq_count; id /= hq_count;
  const int st = id % p.sq;
  const int seg = id / p.sq;
  const int h = hq / p.group, g = hq - h * p.group;
  const int qi = st * p.group + g;
  const int qg = qi / kQG, ql = qi - qg * kQG;
  const int list = seg * p.num_kv_heads + h;
  const int H = p.num_kv_heads;
  // Split form: one partial per split (empty splits hold m = -inf, l = 0);
  // per-item form: one partial per (slot, chunk) of the list.
  const int n = p.stream == kStreamSplit ? p.splits : list_count(p, list) * p.nchunk;
  // Item of the list's j-th partial, i0 + j * istr: split partials are
  // split * Hkv + h; per-item partials are enumerated head-fastest within the
  // segment for unified lists and list by list for per-head lists.
  const bool one_unit = !p.per_head && p.num_segments == 1;
  const int base = (one_unit || p.stream != kStreamNone) ? 0 : s_off[p.per_head ? list : seg];
  int64_t i0, istr;
  if (p.stream == kStreamSplit) { i0 = (int64_t)qg * p.splits * H + h; istr = H; }
  else if (p.per_head) { i0 = base + qg; istr = nqg; }
  else { i0 = (int64_t)base + (int64_t)qg * H + h; istr = (int64_t)nqg * H; }
  auto item_of = [&](int j) -> int64_t { return i0 + (int64_t)j * istr; };
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int d = min(dc * 64 + lane, D - 1);
  const int64_t orow = (int64_t)seg * p.out_seg_stride + (int64_t)st * p.out_tok_stride +
                       (int64_t)hq * p.out_head_stride;

  float m_run = -INFINITY, l_run = 0.f, acc = 0.f;
  const int last = max(n - 1, 0);
  for (int b0 = 0; b0 < n; b0 += 4 * kCombineBatch) {
    // Requests first: partial outputs (clamped indices) and lane u's (m, l).
    float ov[kCombineBatch];
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const int j = min(b0 + wave + 4 * u, last);
      ov[u] = p.part_o[(item_of(j) * kQG + ql) * D + d];
    }
    const int ju = b0 + wave + 4 * (lane % kCombineBatch);
    const float2 ml = *reinterpret_cast<const float2*>(p.part_ml + (item_of(min(ju, last)) * kQG + ql) * 2);
    const bool valid = lane < kCombineBatch && ju < n;
    const float mi = valid ? ml.x : -INFINITY;

    const float m_new = fmaxf(m_run, wave_max(mi));
    const float scale = (m_run == -INFINITY) ? 0.f : exp2f(m_run - m_new);
    const float w = (mi == -INFINITY) ? 0.f : exp2f(mi - m_new);
    l_run = l_run * scale + wave_sum(valid ? w * ml.y : 0.f);
    acc *= scale;
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
      if (b0 + wave + 4 * u < n) acc = fmaf(wu, ov[u], acc);
    }
    m_run = m_new;
  }
  if (lane == 0) { s_ml[2 * wave] = m_run; s_ml[2 * wave + 1] = l_run; }
  s_acc[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0 && dc * 64 + lane < D) {
    float mm = -INFINITY;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) mm = fmaxf(mm, s_ml[2 * w2]);
    float a = 0.f, ll = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      const float mw = s_ml[2 * w2];
      const float sw = (mw == -INFINITY) ? 0.f : exp2f(mw - mm);
      a = fmaf(s_acc[w2 * 64 + lane], sw, a);
      ll = fmaf(s_ml[2 * w2 + 1], sw, ll);
    }
    // No retained token (an empty list, or only empty splits): zeros.
    store_elt(p.out_dtype, p.out, orow + dc * 64 + lane, ll == 0.f ? 0.f : a / ll);
  }
}

// Ranges form: one workgroup per list (segment, kv head) merges the list's
// partials for all of its query rows and columns, so the list offsets are
// scanned once per list (combine_kernel scans them once per query row and 64
// columns: C3 has 8 times as many workgroups; C3 layer 346 -> 341 us).  The
// split form keeps combine_kernel: with one list per kv head (C2: 16) this
// kernel's few workgroups each walk a long chain of loads (C2 layer 108.0 ->
// 111.3 us).  Lists of at most kListRegMax pieces merge in registers,
// kListFast pieces per round: each thread requests the round's (m, l) and its
// own elements' partials together, then folds them in with a running maximum
// (C3, one round: combine 10.45 -> 9.40 -> 8.8 us; eight segments of 32
// retained blocks, 8 kv heads, 8-9 pieces per list: 9.3 -> 8.3 us).  Each
// further round waits for its own loads, which the staged form below
// overlaps (16-17 and 33 pieces per list: 11.4 -> 12.6 and 12.8 -> 18.0 us
// in rounds), so longer lists are staged: first the row maxima M of the
// pieces' references m, then, a batch of partials at a time, the weights
// exp2(m_j - M) staged in LDS (and l = sum w_j l_j), and each thread
// accumulates its output elements over the batch.  Either way the pieces are
// taken in partial order, so the result is deterministic.  An empty list (or
// only empty pieces, m = -inf) gives zeros.
constexpr int kListBatch = 256;  // partials whose weights are staged per round
constexpr int kListFast = 8;     // pieces per register round
constexpr int kListRegMax = 12;  // lists of at most this many pieces merge in registers

__global__ __launch_bounds__(256) void combine_lists_kernel(AttendParams p) {
  constexpr int NWS = 1;                        // partials per piece (one per workgroup)
  constexpr int MQ = kLogitsMaxQ;              // the ranges form carries at most 4 query rows
  constexpr int EPT = MQ * 512 / 256;          // output elements per thread (head_dim <= 512)
  __shared__ int s_off[kMaxLists + 1];
  __shared__ float s_w[kListBatch * MQ];
  __shared__ float s_red[MQ * 4];
  const int H = p.num_kv_heads;
  const int L = blockIdx.x;
  const int seg = L / H, h = L - seg * H;
  const int nq = min(p.sq * p.group, MQ);
  const int D = p.head_dim;
  const int total = build_list_offsets(p, s_off, -1);
  const int per = (total + p.splits - 1) / p.splits;
  const int c0 = s_off[L], c1 = s_off[L + 1];
  const int fw = c1 > c0 ? c0 / per : 0;
  const int n = c1 > c0 ? ((c1 - 1) / per - fw + 1) * NWS : 0;
  const int64_t i0 = ((int64_t)fw + L) * NWS;  // partial j is item i0 + j
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1), wave = t / kWave;
  auto ml_at = [&](int j, int g) {
    return *reinterpret_cast<const float2*>(p.part_ml + ((i0 + j) * kQG + g) * 2);
  };
  auto store_out = [&](int e, float v) {
    const int g = e / D, d = e - g * D;
    const int st = g / p.group, gg = g - st * p.group;
    const int64_t orow = (int64_t)seg * p.out_seg_stride + (int64_t)st * p.out_tok_stride +
                         (int64_t)(h * p.group + gg) * p.out_head_stride;
    store_elt(p.out_dtype, p.out, orow + d, v);
  };

  // Few pieces (the common case; C3 takes one round of kListFast): per round
  // every thread requests the pieces' (m, l) and its own output elements'
  // partials at once and merges them in registers (running maximum, sums
  // rescaled when it moves), with no barrier after the list offsets.
  if (n <= kListRegMax) {
    float M[MQ], lsum[MQ], acc[EPT];
#pragma unroll
    for (int g = 0; g < MQ; ++g) { M[g] = -INFINITY; lsum[g] = 0.f; }
#pragma unroll
    for (int k = 0; k < EPT; ++k) acc[k] = 0.f;
    // Query row of each of the thread's output elements.
    int gk[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) gk[k] = min(t + 256 * k, nq * D - 1) / D;
    for (int r0 = 0; r0 < n; r0 += kListFast) {
      float mv[kListFast][MQ], lv[kListFast][MQ], ov[kListFast][EPT];
#pragma unroll
      for (int j = 0; j < kListFast; ++j) {
        const int jc = min(r0 + j, n - 1);
#pragma unroll
        for (int g = 0; g < MQ; ++g) {
          const float2 ml = ml_at(jc, min(g, nq - 1));
          mv[j][g] = ml.x;
          lv[j][g] = ml.y;
        }
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
          const int e = min(t + 256 * k, nq * D - 1);
          const int g = e / D, d = e - g * D;
          ov[j][k] = p.part_o[((i0 + jc) * kQG + g) * D + d];
        }
      }
      float bm[MQ], sc[MQ];
#pragma unroll
      for (int g = 0; g < MQ; ++g) {
        bm[g] = M[g];
#pragma unroll
        for (int j = 0; j < kListFast; ++j) bm[g] = fmaxf(bm[g], r0 + j < n ? mv[j][g] : -INFINITY);
        sc[g] = (M[g] == -INFINITY) ? 0.f : exp2f(M[g] - bm[g]);
        lsum[g] *= sc[g];
        M[g] = bm[g];
      }
#pragma unroll
      for (int k = 0; k < EPT; ++k) {
        float s = sc[0];
#pragma unroll
        for (int gg = 1; gg < MQ; ++gg) s = gk[k] == gg ? sc[gg] : s;
        acc[k] *= s;
      }
#pragma unroll
      for (int j = 0; j < kListFast; ++j) {
        if (r0 + j < n) {
          float w[MQ];
#pragma unroll
          for (int g = 0; g < MQ; ++g) {
            w[g] = (mv[j][g] == -INFINITY) ? 0.f : exp2f(mv[j][g] - M[g]);
            lsum[g] = fmaf(w[g], lv[j][g], lsum[g]);
          }
#pragma unroll
          for (int k = 0; k < EPT; ++k) {
            float wg = w[0];
#pragma unroll
            for (int gg = 1; gg < MQ; ++gg) wg = gk[k] == gg ? w[gg] : wg;
            acc[k] = fmaf(wg, ov[j][k], acc[k]);
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = t + 256 * k;
      if (e < nq * D) {
        float lg = lsum[0];
#pragma unroll
        for (int gg = 1; gg < MQ; ++gg) lg = gk[k] == gg ? lsum[gg] : lg;
        store_out(e, lg == 0.f ? 0.f : acc[k] / lg);
      }
    }
    return;
  }

  float mx[MQ];
#pragma unroll
  for (int g = 0; g < MQ; ++g) mx[g] = -INFINITY;
  for (int j = t; j < n; j += blockDim.x)
#pragma unroll
    for (int g = 0; g < MQ; ++g)
      if (g < nq) mx[g] = fmaxf(mx[g], ml_at(j, g).x);
#pragma unroll
  for (int g = 0; g < MQ; ++g) {
    const float w = wave_max(mx[g]);
    if (lane == 0) s_red[g * 4 + wave] = w;
  }
  __syncthreads();
  float M[MQ];
#pragma unroll
  for (int g = 0; g < MQ; ++g)
    M[g] = fmaxf(fmaxf(s_red[g * 4], s_red[g * 4 + 1]), fmaxf(s_red[g * 4 + 2], s_red[g * 4 + 3]));

  float lsum[MQ], acc[EPT];
#pragma unroll
  for (int g = 0; g < MQ; ++g) lsum[g] = 0.f;
#pragma unroll
  for (int k = 0; k < EPT; ++k) acc[k] = 0.f;
  for (int b0 = 0; b0 < n; b0 += kListBatch) {
    __syncthreads();  // the previous batch's weights have been used
    const int j = b0 + t;
#pragma unroll
    for (int g = 0; g < MQ; ++g) {
      float w = 0.f;
      if (j < n && g < nq) {
        const float2 ml = ml_at(j, g);
        w = (ml.x == -INFINITY) ? 0.f : exp2f(ml.x - M[g]);
        lsum[g] = fmaf(w, ml.y, lsum[g]);
      }
      if (t < kListBatch) s_w[t * MQ + g] = w;
    }
    __syncthreads();
    const int nb = min(kListBatch, n - b0);
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = t + 256 * k;
      if (e < nq * D) {
        const int g = e / D, d = e - g * D;
        const float* po = p.part_o + ((i0 + b0) * kQG + g) * D + d;
        float a = acc[k];
#pragma unroll 4
        for (int jj = 0; jj < nb; ++jj) a = fmaf(s_w[jj * MQ + g], po[(int64_t)jj * kQG * D], a);
        acc[k] = a;
      }
    }
  }
  block_sum<MQ>(lsum, s_red);
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = t + 256 * k;
    if (e < nq * D) {
      const int g = e / D;
      store_out(e, lsum[g] == 0.f ? 0.f : acc[k] / lsum[g]);
    }
  }
}

// Row-wise combine with its batch: one round of 4 x batch partials covers the
// split form's `splits`; per-item lists take 32.
static void launch_combine(const AttendParams& p, dim3 grid, hipStream_t s) {
  const int n = p.stream == kStreamSplit ? p.splits : 1 << 30;
  if (n <= 16) hipLaunchKernelGGL(combine_kernel<4>, grid, dim3(256), 0, s, p);
  else if (n <= 32) hipLaunchKernelGGL(combine_kernel<8>, grid, dim3(256), 0, s, p);
  else if (n <= 64) hipLaunchKernelGGL(combine_kernel<16>, grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL(combine_kernel<32>, grid, dim3(256), 0, s, p);
}

template <int DT, int LPR, int NQ>
static hipError_t launch_attend_t(const AttendParams& p, int grid, hipStream_t s) {
  if (p.logits) {
    // The queries are already folded into the logits.
    if constexpr (NQ <= kLogitsMaxQ) {
      hipLaunchKernelGGL((attend_decode_kernel<DT, LPR, NQ, DT, true>), dim3(grid), dim3(kAttendThreads), 0, s, p);
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  if (p.q_dtype == DT) {
    hipLaunchKernelGGL((attend_decode_kernel<DT, LPR, NQ, DT, false>), dim3(grid), dim3(kAttendThreads), 0, s, p);
  } else if (p.q_dtype == kF32) {
    hipLaunchKernelGGL((attend_decode_kernel<DT, LPR, NQ, kF32, false>), dim3(grid), dim3(kAttendThreads), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DT, int LPR>
static hipError_t launch_attend_nq(const AttendParams& p, int grid, hipStream_t s) {
  switch (attend_nq_bucket(p.sq * p.group)) {
    case 1: return launch_attend_t<DT, LPR, 1>(p, grid, s);
    case 2: return launch_attend_t<DT, LPR, 2>(p, grid, s);
    case 4: return launch_attend_t<DT, LPR, 4>(p, grid, s);
    default: return launch_attend_t<DT, LPR, 8>(p, grid, s);
  }
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

int attend_nq_bucket(int nq_total) {
  if (nq_total <= 1) return 1;
  if (nq_total <= 2) return 2;
  if (nq_total <= 4) return 4;
  return 8;
}

int attend_chunk(int dt, int head_dim, int nq_total) {
  const int vec = (dt == kF32) ? 4 : 8;
  const int lpr = head_dim / vec;
  const int nslot = kAttendThreads / lpr;
  const int nqb = attend_nq_bucket(nq_total);
  const int r = nqb <= 2 ? rows_per_slot<2>() : (nqb == 4 ? rows_per_slot<4>() : rows_per_slot<8>());
  return r * nslot;
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

// Query groups of the split form: kQG rows each above kLogitsMaxQ rows per
// kv head (every group's workgroups read the same keys and values, the second
// time mostly from the infinity cache), one group otherwise.
constexpr int kSplitMaxRows = 2 * kQG;
static int split_qgroups(const AttendParams& p) {
  const int nq = p.sq * p.group;
  return nq > kLogitsMaxQ ? (nq + kQG - 1) / kQG : 1;
}

template <int DT, int LPR, int NQ, bool KV, int QDT>
static void launch_stream_k(const AttendParams& p, hipStream_t s) {
  if (p.stream == kStreamSplit) {
    hipLaunchKernelGGL((attend_split_kernel<DT, LPR, NQ, KV, QDT>), dim3(p.num_kv_heads * p.splits * split_qgroups(p)),
                       dim3(kAttendThreads), 0, s, p);
  } else if constexpr (NQ <= kLogitsMaxQ) {  // the ranges form carries at most kLogitsMaxQ rows
    hipLaunchKernelGGL((attend_stream_kernel<DT, LPR, NQ, KV, QDT>), dim3(p.splits), dim3(kAttendThreads), 0, s, p);
  }
}

template <int DT, int LPR, int NQ>
static hipError_t launch_stream_nq(const AttendParams& p, hipStream_t s) {
  if (p.logits) {
    if constexpr (NQ <= kLogitsMaxQ) launch_stream_k<DT, LPR, NQ, false, DT>(p, s);
    else return hipErrorInvalidValue;
  } else if (p.q_dtype == DT) {
    launch_stream_k<DT, LPR, NQ, true, DT>(p, s);
  } else if (p.q_dtype == kF32) {
    launch_stream_k<DT, LPR, NQ, true, kF32>(p, s);
  } else {
    return hipErrorInvalidValue;
  }
  return hipSuccess;
}

template <int DT, int LPR>
static hipError_t launch_stream_dt(const AttendParams& p, hipStream_t s) {
  hipError_t e;
  switch (attend_nq_bucket(p.sq * p.group)) {
    case 1: e = launch_stream_nq<DT, LPR, 1>(p, s); break;
    case 2: e = launch_stream_nq<DT, LPR, 2>(p, s); break;
    case 4: e = launch_stream_nq<DT, LPR, 4>(p, s); break;
    case 8: e = launch_stream_nq<DT, LPR, 8>(p, s); break;
    default: return hipErrorInvalidValue;
  }
  return e != hipSuccess ? e : hipGetLastError();
}

template <int DT>
static hipError_t launch_stream(const AttendParams& p, hipStream_t s) {
  switch (p.head_dim / Elt<DT>::VEC) {
    case 8: return launch_stream_dt<DT, 8>(p, s);
    case 16: return launch_stream_dt<DT, 16>(p, s);
    case 32: return launch_stream_dt<DT, 32>(p, s);
    case 64: return launch_stream_dt<DT, 64>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// Which streaming form applies and its `splits`: about one workgroup per CU,
// two where the kernel fits two.  C2 at 90%, split form with logits,
// attention + combine: 128, 256, 512, 1024 and 2048 workgroups gave 26.1,
// 19.1, 19.7, 21.4 and 23.2 us (a two-chunk ring).  Four query rows with
// logits fit two workgroups per CU, and both forms then take 512: one segment
// of 425 blocks, 8 kv heads, head_dim 128, split form with 256 workgroups
// 100.1 + 5.0 us (attention + combine), with 512 85.9 + 5.0 us.  Whole
// 512-token blocks and at most 4 query rows per kv head, or 5-16 in the split
// form reading keys and values, in groups of 8 rows (8 rows, one segment of
// 256 blocks, 8 kv heads, head_dim 128, as per-item work: 52.2 us at 26
// retained blocks and 200.8 us at 128; split form 29.8 and 92.3 us; 16 rows at
// 26 blocks 84.4 -> 40.8 us); keys and values (no logits)
// also need a block of whole chunks.  The split form needs one segment and a
// unified list (its list fits LDS); the ranges form takes any lists, with few
// enough workgroups that its w + L partial slots fit the per-item workspace.
void attend_stream_plan(AttendParams& p) {
  p.stream = kStreamNone;
  p.splits = 0;
  const int64_t nl = (int64_t)p.num_segments * p.num_kv_heads;
  // 5-16 query rows per kv head: the split form reading keys and values
  // only, in groups of kQG rows.
  const bool wide = p.sq * p.group > kLogitsMaxQ;
  if (p.prefill || p.block_size != kBlock || p.total_blocks < 1 || nl > kMaxLists ||
      p.sq * p.group > kSplitMaxRows || (wide && p.logits) || (p.keep && p.total_blocks > kMaxLists) ||
      kBlock % p.chunk != 0)
    return;
  const int64_t chunks = (int64_t)p.total_blocks * p.nchunk;
  // Workgroups: one per CU, two where the kernel fits two (four query rows
  // with logits).
  const int64_t cap = (p.logits && attend_nq_bucket(p.sq * p.group) == 4) ? 512 : 256;
  if (!p.cu_blocks && !p.per_head && !p.uniform && p.total_blocks <= kMaxLists) {
    int64_t sp = cap / ((int64_t)p.num_kv_heads * split_qgroups(p));
    sp = sp < 1 ? 1 : (sp > 64 ? 64 : sp);
    p.stream = kStreamSplit;
    p.splits = (int)(sp < chunks ? sp : chunks);
    return;
  }
  if (wide) return;
  // Ranges form (two workgroups per CU for four query rows with logits: C3
  // layer 350.5 -> 345.5 us).
  const int64_t room = attend_max_items(p) - nl;
  const int64_t g = room < cap ? room : cap;
  if (g >= 1 && !p.keep) {
    p.stream = kStreamRanges;
    p.splits = (int)g;
  }
}

// Partial slots the decode launch of these parameters writes (the workspace
// holds this many (kQG x D) + (kQG x 2) partials).  The split form writes
// item split * Hkv + h for split < splits; the ranges form writes w + L for
// workgroup w < splits and list L < segments * Hkv; the per-item form writes
// at most one per work item, bounded by attend_max_items.  The plan depends
// on whether logits and keep flags are given, so callers size with those
// fields set as they will be at launch.
int64_t attend_partial_slots(const AttendParams& p_in) {
  AttendParams p = p_in;
  attend_stream_plan(p);
  if (p.stream == kStreamSplit) return (int64_t)p.num_kv_heads * p.splits * split_qgroups(p);
  if (p.stream == kStreamRanges) return (int64_t)p.splits + (int64_t)p.num_segments * p.num_kv_heads;
  return attend_max_items(p);
}

hipError_t launch_attend(const AttendParams& p_in, hipStream_t s) {
  if (p_in.prefill) return launch_prefill(p_in, s);
  AttendParams p = p_in;
  attend_stream_plan(p);
  if (p.stream != kStreamNone) {
    hipError_t e;
    switch (p.kv_dtype) {
      case kF32: e = launch_stream<kF32>(p, s); break;
      case kBF16: e = launch_stream<kBF16>(p, s); break;
      case kF16: e = launch_stream<kF16>(p, s); break;
      default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    if (p.stream == kStreamRanges) {
      hipLaunchKernelGGL(combine_lists_kernel, dim3(p.num_segments * p.num_kv_heads), dim3(256), 0, s, p);
      return hipGetLastError();
    }
    const int rows = p.num_segments * p.sq * p.num_kv_heads * p.group;
    const int ndc = (p.head_dim + 63) / 64;
    launch_combine(p, dim3(rows * ndc), s);
    return hipGetLastError();
  }
  const int64_t max_items = attend_max_items(p);
  if (max_items > 0) {
    const int grid = (int)(max_items < kAttendGrid ? max_items : kAttendGrid);
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
  const int ndc = (p.head_dim + 63) / 64;
  launch_combine(p, dim3(rows * ndc), s);
  return hipGetLastError();
}

}  // namespace oc
