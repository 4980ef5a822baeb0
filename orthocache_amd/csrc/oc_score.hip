// Block scoring: spectral bands, zeta, block mean and the query-aware bound.
//
// Replaces the reference's compute_spectral_bands / compute_spectral_decay_ratio
// / compute_query_aware_bounds / compute_query_aware_mask
// (src/orthocache/spectral_energy.py:69-196), which materialise the full
// 512-point FWHT of every (block, head, dim) column.  The bands are ranges of
// natural (Hadamard) coefficient indices: DC = {0}, low = [1,64),
// mid = [64,256), high = [256,512), i.e. cosets of the top three index bits.
// By Parseval, the energy of a coset only needs the butterflies over token
// bits 6, 7 and 8.  Write a token index as i = 64*k + l (k in 0..7, l in 0..63)
// and, per column and per l, x_k = K[64k + l]:
//   E_high = 1/2 * sum_l sum_{k<4} (x_k - x_{k+4})^2            (index bit 8 set)
//   u_k    = x_k + x_{k+4},  y = WHT4(u)
//   E_mid  = 1/8 * sum_l (y1^2 + y2^2 + y3^2)                    (bits 6/7 set, 8 clear)
//          = 1/8 * sum_l (2 a1^2 + 2 a3^2 + y2^2), with a1 = u0 - u1, a3 = u2 - u3,
//            since y1^2 + y3^2 = (a1 + a3)^2 + (a1 - a3)^2
//   E_low  = 1/8 * sum_l (y0_l - mean_l y0)^2                    (coset 0 minus DC)
//   DC     = sum_l y0_l / sqrt(512),  kbar = DC / sqrt(512)
// so one pass over the keys, ~4 VALU ops per element, gives every score the
// reference derives from the full spectrum.  E_low is formed as a centred sum
// of squares (shifted sums per thread, Chan merge across threads), so a large
// block mean does not cancel it away.
//
// One workgroup (256 threads) scores one tile: 512 token rows of one kv head,
// or of two adjacent kv heads side by side when a head's row is 128 or 256
// bytes (HPT = 2; per-head sums are kept apart).  Lanes are laid out LPR per
// tile row (16-byte loads along D, coalesced); NSLOT = 256/LPR row slots each
// walk 64/NSLOT values of l, loading the eight rows 64k + l together.
//
// Optionally (NQL > 0, decode with at most 4 query rows per kv head) the same
// pass also forms the attention logits q.k of every key row it streams: the
// lane's VEC-element partial dot products of its eight rows are summed over
// the row's LPR lanes with a halving butterfly, staged in LDS and written as
// one contiguous 512 x NQL fp32 tile.  The attention then reads only the
// values of the retained blocks, not their keys a second time.
#include "oc_kernels.h"

namespace oc {

// Rows 64k + l (k = 0..7) of the tile: a wave-uniform base (tile start plus
// 64k rows, scalar registers) and the lane's 32-bit offset l * row_bytes +
// column bytes, so each load takes one address VGPR (global_load saddr form).
// The host guarantees 64 * row_bytes < 2^31.
__device__ __forceinline__ void load_rows(const char* tbase, int64_t stride64, uint32_t loff, uint4 (&r)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) r[k] = ld16_nt(tbase + k * stride64 + loff);
}

constexpr int kMaxSegLds = 4096;  // segments whose offsets are staged in LDS
template <int N> struct IntTag { static constexpr int value = N; };  // a row count as a type
template <bool B> struct BoolTag { static constexpr bool value = B; };
constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }
constexpr int kScoreRed = 256;  // floats of the epilogue's reduction scratch
constexpr int kWideBoundRows = 16;  // query rows per kv head of the single-reduction inline bound

// Segment holding flattened block gb (binary search over cu staged in LDS).
__device__ __forceinline__ int find_segment(const int* s_cu, int num_segments, int gb) {
  int lo = 0, hi = num_segments - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_cu[mid] <= gb) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Occupancy floor of the logits variants whose registers fit three
// workgroups per CU without spilling (168 VGPRs): packed dot products
// (16-bit keys and queries) with 32 lanes per row and two query rows, or bf16
// with 16 lanes per row and four query rows.  Measured: the C2 shape (bf16,
// head_dim 256) 90 us at three workgroups per CU against 97 us at two; the C3 layer (head_dim 128, four query rows per kv
// head) 363 us against 377 us.
// The other bf16 logits variants are held to at least two.  (Some fp16
// logits variants need more than 256 VGPRs as scheduled and would spill under
// a floor; they keep the compiler's choice.)  LPR counts the lanes of a tile
// row, LPR / HPT those of one head.
template <int DT, int LPR, int QDT, int NQL, int HPT>
constexpr int score_min_waves() {
  return (DT != kF32 && QDT == DT &&
          ((NQL == 2 && LPR == 32 && HPT == 1) || (NQL == 4 && LPR / HPT == 16 && DT == kBF16)))
             ? 3
             : ((NQL > 0 && DT == kBF16) ? 2 : 1);
}

template <int DT, int LPR, int QDT, int NQL, int HPT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(score_min_waves<DT, LPR, QDT, NQL, HPT>())))
void score_kernel(ScoreParams p) {
  using E = Elt<DT>;
  using EQ = Elt<QDT>;
  constexpr int VEC = E::VEC;
  constexpr int DW = LPR * VEC;   // columns of a tile row: HPT heads side by side
  constexpr int D = DW / HPT;     // head_dim
  constexpr int LPH = LPR / HPT;  // lanes per head within a row
  constexpr int NSLOT = 256 / LPR;
  constexpr int NLO = 64 / NSLOT;
  static_assert(NLO >= 2 && (NLO % 2) == 0, "unsupported lane layout");
  static_assert(HPT == 1 || HPT == 2, "one or two kv heads per tile");
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  constexpr int QSZ = (QDT == kF32) ? 4 : 2;

  constexpr int NI = (DW + 255) / 256;  // tile columns per thread in the epilogue
  __shared__ float s_mean[NSLOT * DW];
  __shared__ float s_m2[NSLOT * DW];
  __shared__ float s_red[kScoreRed];
  __shared__ int s_cu[kMaxSegLds + 1];
  __shared__ __attribute__((aligned(16))) float s_lg[NQL > 0 ? HPT * kBlock * NQL : 4];

  // Tile = (block gb, kv heads h0 .. h0 + HPT - 1); its per-head outputs are
  // items tile0 + hh, hh < HPT.
  const int H = p.num_kv_heads;
  const int bid = blockIdx.x;
  const int gb = bid / (H / HPT);
  const int h0 = (bid - gb * (H / HPT)) * HPT;
  const int64_t tile0 = HPT == 1 ? (int64_t)bid : (int64_t)gb * H + h0;
  const int t = threadIdx.x;
  const int cc = t % LPR;
  const int slot = t / LPR;
  const int hh = HPT == 1 ? 0 : cc / LPH;              // the lane's head within the tile
  const int cw = HPT == 1 ? cc * VEC : (cc % LPH) * VEC;  // its first column within that head

  const int64_t row_bytes = p.k_tok_stride * ESZ;
  const int64_t stride64 = 64 * row_bytes;
  // Paged caches: the block's keys live in physical page pages[gb].
  const int64_t page = page_of(p.pages, p.num_pages, gb);
  const char* tbase = reinterpret_cast<const char*>(p.k) +
                      (page * kBlock * p.k_tok_stride + (int64_t)h0 * p.k_head_stride) * ESZ;
  // Lane offset of row l within the 64-row group: l * row_bytes + column bytes.
  const uint32_t col_off =
      HPT == 1 ? (uint32_t)(cc * VEC * ESZ) : (uint32_t)(((int64_t)hh * p.k_head_stride + cw) * ESZ);
  auto lane_off = [&](int l) -> uint32_t { return (uint32_t)(l * (uint32_t)row_bytes) + col_off; };
  // 16-bit variants with logits and one kv head per tile request their first
  // eight rows before anything else (query prefetch, segment table, address
  // set-up), so every workgroup's key stream starts as early as it can.  C2's
  // variant then takes 130 VGPRs and three workgroups per CU instead of 124
  // and four, and is still faster: scoring 86.4 -> 85.4 us (forcing four
  // workgroups spills: 88.3 us).  The other variants keep the later request:
  // several of them would lose a workgroup per CU, and neither C3's (two heads
  // per tile: 197.1 -> 197.7 us) nor C5's (823.3 -> 824.2 us) gained.
  constexpr bool kEarlyRows = NQL > 0 && DT != kF32 && HPT == 1;
  uint4 ra[8], rb[8];
  if constexpr (kEarlyRows) load_rows(tbase, stride64, lane_off(slot), ra);
  // Query element offset of tile column dcol (head h0 + dcol / D, dim dcol % D).
  auto qcol_off = [&](int dcol) -> int64_t {
    if constexpr (HPT == 1) return dcol;
    return (int64_t)(dcol / D) * p.group * p.q_head_stride + dcol % D;
  };

  // Query-aware bound inputs, requested before the key stream so their
  // latency overlaps it: the segment table (ragged batches) goes to LDS, the
  // first four queries' values of this thread's columns go to registers
  // (one segment; a ragged batch needs the segment id first).
  const bool want_bound = p.q != nullptr && p.tau_max != nullptr;
  const int nq = p.sq * p.group;
  const bool need_seg = p.cu_blocks != nullptr && (want_bound || NQL > 0);
  if (need_seg) {
    for (int i = t; i <= p.num_segments; i += 256) s_cu[i] = p.cu_blocks[i];
  }
  float qpre[4][NI];
  const bool prefetch = want_bound && p.cu_blocks == nullptr && nq > 0;
  if (prefetch) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int qi = min(u, nq - 1);
      const int st = qi / p.group, g = qi - st * p.group;
      const int64_t qoff = (int64_t)st * p.q_tok_stride + (int64_t)(h0 * p.group + g) * p.q_head_stride;
#pragma unroll
      for (int i = 0; i < NI; ++i) qpre[u][i] = EQ::load1(p.q, qoff + qcol_off(min(t + 256 * i, DW - 1)));
    }
  }

  float acc_hi[VEC], acc_mid[VEC], acc_mid2[VEC], piv[VEC], ssum[VEC], ssq[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) { acc_hi[c] = 0.f; acc_mid[c] = 0.f; acc_mid2[c] = 0.f; ssum[c] = 0.f; ssq[c] = 0.f; piv[c] = 0.f; }

  // Logit queries: this lane's VEC columns of each of the kv head's query
  // rows (rows past nq are zero).  With 16-bit keys and queries of the same
  // type they stay packed (DOT2: packed dot products on the raw key words,
  // scaled by log2(e)/sqrt(d) after the lane reduction); otherwise they are
  // widened and pre-scaled.
  constexpr bool DOT2 = NQL > 0 && DT != kF32 && QDT == DT;
  float lq[NQL > 0 && !DOT2 ? NQL : 1][VEC];
  uint32_t lqw[DOT2 ? NQL : 1][VEC / 2];

  // Band statistics of column c from its values in the eight rows 64k + l.
  auto stats = [&](float x0, float x1, float x2, float x3, float x4, float x5, float x6, float x7, bool first,
                   int c) {
    const float d0 = x0 - x4, d1 = x1 - x5;
    const float d2 = x2 - x6, d3 = x3 - x7;
    float ah = acc_hi[c];
    ah = fmaf(d0, d0, ah); ah = fmaf(d1, d1, ah); ah = fmaf(d2, d2, ah); ah = fmaf(d3, d3, ah);
    acc_hi[c] = ah;
    const float u0 = x0 + x4, u1 = x1 + x5;
    const float u2 = x2 + x6, u3 = x3 + x7;
    const float a0 = u0 + u1, a1 = u0 - u1, a2 = u2 + u3, a3 = u2 - u3;
    const float y0 = a0 + a2, y2 = a0 - a2;
    float am = acc_mid[c], am2 = acc_mid2[c];
    am2 = fmaf(a1, a1, am2); am2 = fmaf(a3, a3, am2); am = fmaf(y2, y2, am);
    acc_mid[c] = am; acc_mid2[c] = am2;
    if (first) {
      piv[c] = y0;
    } else {
      const float dv = y0 - piv[c];
      ssum[c] += dv;
      ssq[c] = fmaf(dv, dv, ssq[c]);
    }
  };

  // With logits: column c's statistics and the rows' partial dot products
  // with the queries (value index k * NQL + g), column by column so that
  // only eight widened values are live next to the partial sums.
  auto column = [&](const uint4 (&r)[8], bool first, int c, float* part) {
    float x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = E::get(r[k], c);
    stats(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7], first, c);
    if constexpr (NQL > 0 && !DOT2) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int g = 0; g < NQL; ++g) part[k * NQL + g] = fmaf(lq[g][c], x[k], part[k * NQL + g]);
    }
  };

  // Sum each row's partial dots over its LPR lanes, then stage them (packed
  // dot products are scaled once, after the sum).
  auto reduce_store = [&](auto& part, int l) {
    constexpr int V = NQL > 0 ? 8 * NQL : LPH;  // (unused without logits)
    Butterfly<V, V, LPH / 2, LPH>::run(part, cc);
    const float sc = DOT2 ? p.logit_scale : 1.f;
    float* lg = s_lg + (HPT > 1 ? hh * kBlock * NQL : 0);
    const int ch = HPT == 1 ? cc : cc % LPH;
    if constexpr (V >= LPH) {
      constexpr int PER_LANE = V / LPH;
#pragma unroll
      for (int u = 0; u < PER_LANE; ++u) {
        const int idx = ch * PER_LANE + u;
        lg[(64 * (idx / NQL) + l) * NQL + idx % NQL] = part[u] * sc;
      }
    } else {
      // REP = LPH / V lanes hold each complete sum; all of them store it
      // (same address, same value), which keeps the loop free of branches.
      constexpr int REP = LPH / V;
      const int idx = ch / REP;
      lg[(64 * (idx / NQL) + l) * NQL + idx % NQL] = part[0] * sc;
    }
  };

  auto consume = [&](const uint4 (&r)[8], bool first, int l) {
    constexpr int V = NQL > 0 ? 8 * NQL : 1;
    float part[V];
#pragma unroll
    for (int i = 0; i < V; ++i) part[i] = 0.f;
    if constexpr (DOT2) {
      // Packed dot products of the raw key words (two columns each).
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int w = 0; w < VEC / 2; ++w)
#pragma unroll
          for (int g = 0; g < NQL; ++g) part[k * NQL + g] = dot2_acc<DT>(word_of(r[k], w), lqw[g][w], part[k * NQL + g]);
    }
    if constexpr (DOT2 && DT == kBF16) {
      // bf16: the partial sums are reduced and staged before the statistics,
      // which then widen one column at a time, so the sums and the widened
      // rows are never live together.  C2's variant (head_dim 256, two query
      // rows) needed 125 VGPRs, four workgroups per CU, against 136 and three
      // (scoring 90.8 -> 89.2 us); four query rows 162 against 172-198.
      reduce_store(part, l);
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        float x[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = E::get(r[k], c);
        stats(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7], first, c);
      }
      return;
    }
    if constexpr (NQL == 0 || DOT2) {
      // Statistics: widen the eight rows at once.
      float x[8][VEC];
#pragma unroll
      for (int k = 0; k < 8; ++k) E::unpack(r[k], x[k]);
#pragma unroll
      for (int c = 0; c < VEC; ++c)
        stats(x[0][c], x[1][c], x[2][c], x[3][c], x[4][c], x[5][c], x[6][c], x[7][c], first, c);
    } else {
#pragma unroll
      for (int c = 0; c < VEC; ++c) column(r, first, c, part);
    }
    if constexpr (NQL > 0) reduce_store(part, l);
  };

  if constexpr (!kEarlyRows) load_rows(tbase, stride64, lane_off(slot), ra);
  int seg = 0;
  if constexpr (NQL > 0) {
    // The logits need this block's queries before the first rows arrive: in
    // a ragged batch, find the segment now (s_cu was requested above).
    if (need_seg) {
      __syncthreads();
      seg = find_segment(s_cu, p.num_segments, gb);
    }
#pragma unroll
    for (int g = 0; g < NQL; ++g) {
      const int qc = min(g, nq - 1);
      const int st = qc / p.group, gg = qc - st * p.group;
      const char* qp = reinterpret_cast<const char*>(p.q) +
                       ((int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                        (int64_t)((h0 + hh) * p.group + gg) * p.q_head_stride +
                        (HPT == 1 ? (int64_t)cc * VEC : (int64_t)cw)) * QSZ;
      if constexpr (DOT2) {
        const uint4 w = ld16(qp);
#pragma unroll
        for (int i = 0; i < VEC / 2; ++i) lqw[g][i] = g < nq ? word_of(w, i) : 0u;
      } else {
        const float sc = g < nq ? p.logit_scale : 0.f;
#pragma unroll
        for (int e0 = 0; e0 < VEC; e0 += EQ::VEC) {
          float tmp[EQ::VEC];
          EQ::unpack(ld16(qp + e0 * QSZ), tmp);
#pragma unroll
          for (int e = 0; e < EQ::VEC && e0 + e < VEC; ++e) lq[g][e0 + e] = tmp[e] * sc;
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NLO; j += 2) {
    load_rows(tbase, stride64, lane_off(slot + NSLOT * (j + 1)), rb);
    consume(ra, j == 0, slot + NSLOT * j);
    if (j + 2 < NLO) load_rows(tbase, stride64, lane_off(slot + NSLOT * (j + 2)), ra);
    consume(rb, false, slot + NSLOT * (j + 1));
  }

  float hi = 0.f, mid = 0.f;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    hi += acc_hi[c];
    mid += acc_mid[c] + 2.f * acc_mid2[c];
    const float mean_t = piv[c] + ssum[c] * (1.f / NLO);
    // Clamp rounding below zero without dropping NaN (fmaxf would).
    const float m2_raw = ssq[c] - ssum[c] * ssum[c] * (1.f / NLO);
    const float m2_t = m2_raw < 0.f ? 0.f : m2_raw;
    s_mean[slot * DW + cc * VEC + c] = mean_t;
    s_m2[slot * DW + cc * VEC + c] = m2_t;
  }
  __syncthreads();

  if constexpr (NQL > 0) {
    // The tile's logits: HPT x 512 x NQL fp32, contiguous, 16 bytes per thread.
    float* dst = p.logits + tile0 * kBlock * NQL;
#pragma unroll
    for (int i = 4 * t; i < HPT * kBlock * NQL; i += 4 * 256)
      st16_nt(dst + i, *reinterpret_cast<const float4*>(s_lg + i));
  }

  // Per column: merge the NSLOT partial (mean, M2) pairs (equal counts NLO).
  // Column d of the tile row is dim d % D of head h0 + d / D; the dc rows of
  // the tile's heads are adjacent, so column d goes to dc[tile0 * D + d].
  float elow[HPT];
#pragma unroll
  for (int k = 0; k < HPT; ++k) elow[k] = 0.f;
  float kbar_r[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = t + 256 * i;
    kbar_r[i] = 0.f;
    if (d < DW) {
      float m = 0.f;
#pragma unroll
      for (int s = 0; s < NSLOT; ++s) m += s_mean[s * DW + d];
      m *= (1.f / NSLOT);
      float m2 = 0.f;
#pragma unroll
      for (int s = 0; s < NSLOT; ++s) {
        const float dm = s_mean[s * DW + d] - m;
        m2 += s_m2[s * DW + d] + (float)NLO * dm * dm;
      }
      if constexpr (HPT == 1) {
        elow[0] += m2;
      } else {
#pragma unroll
        for (int k = 0; k < HPT; ++k) elow[k] += (d / D == k) ? m2 : 0.f;
      }
      const float dcv = (64.f * m) / kSqrt512;  // sum over l of y0, over sqrt(512)
      if (p.dc) p.dc[tile0 * D + d] = dcv;
      kbar_r[i] = dcv / kSqrt512;                // spectral_energy.py:166
    }
  }

  // Band totals per head: a lane's columns all belong to head hh.
  float tot[3 * HPT];
#pragma unroll
  for (int k = 0; k < HPT; ++k) {
    tot[3 * k] = (HPT == 1 || hh == k) ? hi : 0.f;
    tot[3 * k + 1] = (HPT == 1 || hh == k) ? mid : 0.f;
    tot[3 * k + 2] = elow[k];
  }
  // The segment of this block (s_cu was filled before the key stream; the
  // barrier after the statistics has made it visible).
  if (NQL == 0 && need_seg) seg = find_segment(s_cu, p.num_segments, gb);

  // Up to 16 query rows per kv head take the inline bound in one reduction
  // (WQ = 4 for 1-4 rows, 16 for 5-16 in the variants without logits; those
  // with logits carry at most 4 rows).  With one kv head per tile, or 1-4
  // rows, the band totals ride in that same reduction (fused), so the tile
  // has one reduction barrier in all; otherwise they take block_sum first.
  const bool wide = want_bound && nq > 0 && nq <= kWideBoundRows && (NQL == 0 || nq <= 4);
  const bool fused = want_bound && nq > 0 && (nq <= 4 || (wide && HPT == 1));
  float e_ac[HPT], zeta[HPT], sqrt_eac[HPT], best[HPT];
#pragma unroll
  for (int k = 0; k < HPT; ++k) best[k] = -INFINITY;
  // Energies, E_AC and zeta of head k from its three band totals; thread 0
  // stores them.
  auto finish_bands = [&](int k, float t_high, float t_mid, float t_low) {
    const float e_high = 0.5f * t_high;
    const float e_mid = 0.125f * t_mid;
    const float e_low = 0.125f * t_low;
    e_ac[k] = e_low + e_mid + e_high;
    zeta[k] = e_high / (e_low + 1e-6f);  // spectral_energy.py:138
    sqrt_eac[k] = sqrtf(e_ac[k]);
    if (t == 0) {
      if (p.e_low) p.e_low[tile0 + k] = e_low;
      if (p.e_mid) p.e_mid[tile0 + k] = e_mid;
      if (p.e_high) p.e_high[tile0 + k] = e_high;
      if (p.e_ac) p.e_ac[tile0 + k] = e_ac[k];
      if (p.zeta) p.zeta[tile0 + k] = zeta[k];
    }
  };
  if (!fused) {
    block_sum<3 * HPT>(tot, s_red);
#pragma unroll
    for (int k = 0; k < HPT; ++k) finish_bands(k, tot[3 * k], tot[3 * k + 1], tot[3 * k + 2]);
  }

  // Inline query-aware bound: tau_j = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d),
  // max over the segment's queries of every query head sharing kv head h.
  if (want_bound) {
    const float sqrt_d = sqrtf((float)D);
    // WQ query rows at once: every row's q.kbar and |q|^2 partials (and with
    // FUSE the band totals) in one halving butterfly per wave (V - 1
    // exchanges for V values), one barrier, and the per-head maximum over the
    // rows in wave 0 (instead of a two-barrier workgroup sum per four rows:
    // C2's scoring 88.5 -> 86.5 us, 16 rows per kv head 80.6 -> 45 us).  The
    // per-wave sums pair lanes in the order wave_sum does and the waves are
    // added in block_sum's order, so fused band totals are bit-identical to
    // block_sum's.
    auto bound_rows = [&](auto wq_tag, auto fuse_tag) {
      constexpr int WQ = decltype(wq_tag)::value;
      constexpr bool FUSE = decltype(fuse_tag)::value;
      constexpr int NBV = 2 * WQ * HPT;  // value (k * WQ + u) * 2 + {0: q.kbar, 1: |q|^2}
      constexpr int NV = FUSE ? NBV + 3 * HPT : NBV;  // then head k's band totals at NBV + 3 k
      constexpr int V = pow2_at_least(NV);
      static_assert(V <= kWave && V * (256 / kWave) <= kScoreRed, "one value per lane after the butterfly");
      float qv[WQ][NI];
#pragma unroll
      for (int u = 0; u < WQ; ++u) {
        const int qi = min(u, nq - 1);
        const int st = qi / p.group, g = qi - st * p.group;
        const int64_t qoff = (int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                             (int64_t)(h0 * p.group + g) * p.q_head_stride;
#pragma unroll
        for (int i = 0; i < NI; ++i)
          qv[u][i] = (prefetch && u < 4) ? qpre[u][i] : EQ::load1(p.q, qoff + qcol_off(min(t + 256 * i, DW - 1)));
      }
      float val[V];
#pragma unroll
      for (int k = 0; k < HPT; ++k)
#pragma unroll
        for (int u = 0; u < WQ; ++u) {
          float a = 0.f, b = 0.f;
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            const int d = t + 256 * i;
            const float v = (d < DW && (HPT == 1 || d / D == k)) ? qv[u][i] : 0.f;
            a = fmaf(v, kbar_r[i], a);
            b = fmaf(v, v, b);
          }
          val[(k * WQ + u) * 2] = a;
          val[(k * WQ + u) * 2 + 1] = b;
        }
#pragma unroll
      for (int i = NBV; i < V; ++i) val[i] = (FUSE && i < NV) ? tot[i - NBV] : 0.f;
      const int lane = t & (kWave - 1), wave = t / kWave;
      Butterfly<V, V, kWave / 2, kWave>::run(val, lane);
      // Lane l now holds the wave's sum of value l / (64 / V).  (Unfused,
      // block_sum's second barrier has released s_red.)
      constexpr int REPV = kWave / V;
      if (lane % REPV == 0) s_red[wave * V + lane / REPV] = val[0];
      __syncthreads();
      if (wave == 0) {
        if constexpr (FUSE) {
#pragma unroll
          for (int k = 0; k < HPT; ++k) {
            float tt[3];
#pragma unroll
            for (int j = 0; j < 3; ++j) {
              float s = 0.f;
#pragma unroll
              for (int w = 0; w < 256 / kWave; ++w) s += s_red[w * V + NBV + 3 * k + j];
              tt[j] = s;
            }
            finish_bands(k, tt[0], tt[1], tt[2]);
          }
        }
        float bnd = -INFINITY;
        if (lane < NBV && (lane & 1) == 0) {
          float a = 0.f, b = 0.f;
#pragma unroll
          for (int w = 0; w < 256 / kWave; ++w) {
            a += s_red[w * V + lane];
            b += s_red[w * V + lane + 1];
          }
          const int k = (lane >> 1) / WQ, u = (lane >> 1) % WQ;
          float se = sqrt_eac[0];
#pragma unroll
          for (int kk = 1; kk < HPT; ++kk) se = k == kk ? sqrt_eac[kk] : se;
          if (u < nq) bnd = a / sqrt_d + (sqrtf(b) * se) / sqrt_d;
        }
        // The rows of head k sit at lanes 2 WQ k + 2 u: maximum over u
        // (NaN-propagating) within each 2 WQ-lane window.
#pragma unroll
        for (int o = 2; o < 2 * WQ; o <<= 1) bnd = nanmax(bnd, __shfl_xor(bnd, o, kWave));
#pragma unroll
        for (int k = 0; k < HPT; ++k) best[k] = __shfl(bnd, 2 * WQ * k, kWave);
      }
    };
    if (fused) {
      if (nq <= 4) {
        bound_rows(IntTag<4>{}, BoolTag<true>{});
      } else if constexpr (NQL == 0 && HPT == 1) {
        bound_rows(IntTag<kWideBoundRows>{}, BoolTag<true>{});
      }
    } else if (wide) {
      if constexpr (NQL == 0) bound_rows(IntTag<kWideBoundRows>{}, BoolTag<false>{});
    }
    for (int q0 = 0; q0 < (wide ? 0 : nq); q0 += 4) {
      float qv[4][NI];
      if (prefetch && q0 == 0) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < NI; ++i) qv[u][i] = qpre[u][i];
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int qi = min(q0 + u, nq - 1);
          const int st = qi / p.group, g = qi - st * p.group;
          const int64_t qoff = (int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                               (int64_t)(h0 * p.group + g) * p.q_head_stride;
#pragma unroll
          for (int i = 0; i < NI; ++i) qv[u][i] = EQ::load1(p.q, qoff + qcol_off(min(t + 256 * i, DW - 1)));
        }
      }
      // Per query and head: q.kbar and |q|^2 over the head's columns.
      float part[8 * HPT];
#pragma unroll
      for (int k = 0; k < HPT; ++k)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float a = 0.f, b = 0.f;
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            const int d = t + 256 * i;
            const float v = (d < DW && (HPT == 1 || d / D == k)) ? qv[u][i] : 0.f;
            a = fmaf(v, kbar_r[i], a);
            b = fmaf(v, v, b);
          }
          part[8 * k + 2 * u] = a;
          part[8 * k + 2 * u + 1] = b;
        }
      block_sum<8 * HPT>(part, s_red);
#pragma unroll
      for (int k = 0; k < HPT; ++k) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (q0 + u < nq) {
            const float align = part[8 * k + 2 * u] / sqrt_d;
            const float resid = (sqrtf(part[8 * k + 2 * u + 1]) * sqrt_eac[k]) / sqrt_d;
            best[k] = nanmax(align + resid, best[k]);
          }
        }
      }
    }
    if (t == 0) {
#pragma unroll
      for (int k = 0; k < HPT; ++k) {
        p.tau_max[tile0 + k] = best[k];
        // The two-gate mask of this tile (compute_multiband_mask,
        // spectral_energy.py:199-234), from the same fp32 scores.
        if (p.gate.keep) {
          const uint8_t kf = gate_keep(p.gate, seg, best[k], zeta[k]);
          p.gate.keep[tile0 + k] = kf;
          if (p.gate.mask_out) p.gate.mask_out[tile0 + k] = kf;
        }
      }
    }
  }
}

// Query-aware bound for many queries (prefill): one workgroup per
// (64 queries, 64 blocks, kv head).  Needs kbar (from dc) and E_AC from
// score_kernel.  Writes the full bound tensor (Sq*G, nb, Hkv) and/or the
// per-query-tile NaN-propagating max (ntiles, nb, Hkv), ntiles = ceil(Sq*G/64).
//
// The q.kbar products are a small GEMM per kv head, done on the fp32 matrix
// cores (v_mfma_f32_32x32x2_f32, fp32 inputs and accumulation): each wave
// computes a 32 x 32 (query x block) tile.  Lane l supplies query row l % 32
// and block row l % 32; its k index runs over its own half of head_dim (the
// contraction order is free as long as A and B agree), so each lane reads two
// contiguous half-rows.  The lane's squared query norm comes from the same
// values.  Output lane l, i: query 8(i/4) + 4(l/32) + i%4, block l % 32.
constexpr int kBoundQT = 64;
constexpr int kBoundBT = 64;
constexpr int kBoundKC = 32;  // head_dim elements per lane per chunk

// VECLD: q and dc rows are 16-byte aligned and each half-row is a whole number
// of 16-byte chunks (checked on the host), so a chunk takes 16-byte loads.
template <int QDT, bool VECLD>
__global__ __launch_bounds__(256) void bound_kernel(BoundParams p) {
  using EQ = Elt<QDT>;
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  __shared__ float s_m[2][2][32];
  const int D = p.head_dim;
  const int H = p.num_kv_heads;
  const int nb = p.num_blocks;
  const int nq = p.sq * p.group;
  const int nbt = (nb + kBoundBT - 1) / kBoundBT;
  int id = blockIdx.x;
  const int h = id % H; id /= H;
  const int bt = id % nbt;
  const int qt = id / nbt;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = t / kWave;
  const int wq = wave & 1, wb = wave >> 1;
  const int r = lane & 31, hf = lane >> 5;

  const int qrow = qt * kBoundQT + wq * 32 + r;
  const int qc = min(qrow, nq - 1);
  const int st = qc / p.group, gq = qc - st * p.group;
  const int64_t qoff = (int64_t)st * p.q_tok_stride + (int64_t)(h * p.group + gq) * p.q_head_stride;
  const int brow = bt * kBoundBT + wb * 32 + r;
  const float* dcrow = p.dc + ((int64_t)min(brow, nb - 1) * H + h) * D;
  const float eac = p.e_ac[(int64_t)min(brow, nb - 1) * H + h];

  // Reciprocals instead of divisions in the hot loop and the epilogue (a
  // divide is a ten-instruction sequence; the products differ from the
  // quotients by at most one rounding).
  constexpr float kInv = 1.f / kSqrt512;
  const int half = (D + 1) / 2;
  const int d0 = hf * half;
  const int d1 = min(d0 + half, D);
  f32x16 acc, acc2;  // two interleaved chains (even / odd k), summed at the end
#pragma unroll
  for (int i = 0; i < 16; ++i) { acc[i] = 0.f; acc2[i] = 0.f; }
  float qq = 0.f;
  for (int c0 = 0; c0 < half; c0 += kBoundKC) {
    float qa[kBoundKC], kb[kBoundKC];
    if constexpr (VECLD) {
      // Chunks of 16 bytes; the last chunk of a half-row may run past it
      // (clamped to the row's last chunk and zeroed).
      constexpr int QV = EQ::VEC;  // q elements per 16-byte load
      constexpr int QSZ = (QDT == kF32) ? 4 : 2;
      const char* qb = reinterpret_cast<const char*>(p.q) + qoff * QSZ;
#pragma unroll
      for (int j = 0; j < kBoundKC; j += QV) {
        const int d = d0 + c0 + j;
        const int dd = d < d1 ? d : d1 - QV;
        float tmp[QV];
        EQ::unpack(ld16(qb + (int64_t)dd * QSZ), tmp);
#pragma unroll
        for (int e = 0; e < QV; ++e) qa[j + e] = d < d1 ? tmp[e] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kBoundKC; j += 4) {
        const int d = d0 + c0 + j;
        const int dd = d < d1 ? d : d1 - 4;
        const float4 kv = *reinterpret_cast<const float4*>(dcrow + dd);
        const float kvv[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) kb[j + e] = d < d1 ? kvv[e] * kInv : 0.f;  // kbar, spectral_energy.py:166
      }
    } else {
#pragma unroll
      for (int j = 0; j < kBoundKC; ++j) {
        const int d = d0 + c0 + j;
        const bool ok = d < d1;
        const int dd = ok ? d : D - 1;
        const float qv = EQ::load1(p.q, qoff + dd);
        const float kv = dcrow[dd];
        qa[j] = ok ? qv : 0.f;
        kb[j] = ok ? kv * kInv : 0.f;  // kbar, spectral_energy.py:166
      }
    }
#pragma unroll
    for (int j = 0; j < kBoundKC; j += 2) {
      qq = fmaf(qa[j], qa[j], qq);
      qq = fmaf(qa[j + 1], qa[j + 1], qq);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[j], kb[j], acc, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[j + 1], kb[j + 1], acc2, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] += acc2[i];
  qq += __shfl_xor(qq, 32, kWave);  // full squared norm of query row r

  // tau_j(q) = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d) (spectral_energy.py:170-176).
  const float inv_sqrt_d = 1.f / sqrtf((float)D);
  const float sqrt_eac = sqrtf(eac);
  const int b = bt * kBoundBT + wb * 32 + r;
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rr = 8 * (i >> 2) + 4 * hf + (i & 3);
    const float qn = __shfl(qq, rr, kWave);
    const int qi = qt * kBoundQT + wq * 32 + rr;
    if (qi < nq && b < nb) {
      const float bound = acc[i] * inv_sqrt_d + (sqrtf(qn) * sqrt_eac) * inv_sqrt_d;
      if (p.bounds) p.bounds[((int64_t)qi * nb + b) * H + h] = bound;
      m = nanmax(m, bound);
    }
  }
  if (p.tau_part) {
    // NaN-propagating max over the tile's 64 queries: the two lane halves,
    // then the two query-half waves through LDS.
    m = nanmax(m, __shfl_xor(m, 32, kWave));
    if (hf == 0) s_m[wb][wq][r] = m;
    __syncthreads();
    if (wq == 0 && hf == 0 && b < nb)
      p.tau_part[((int64_t)qt * nb + b) * H + h] = nanmax(s_m[wb][0][r], s_m[wb][1][r]);
  }
}

// Exact three-term bf16 split of an fp32 value: x = hi + mid + lo, each term
// a bf16 value (returned as fp32 bit patterns whose low 16 bits are zero).
// hi keeps the top 8 of x's 24 significant bits, mid the top 8 of the
// remainder, and lo the rest (at most 8 bits), so the sum is exact for every
// finite x above the subnormal range; +-inf gives (inf, 0, 0) and NaN a NaN hi.
__device__ __forceinline__ void split_bf16x3(float x, uint32_t& hb, uint32_t& mb, uint32_t& lb) {
  hb = (x != x) ? 0x7FC00000u : (__float_as_uint(x) & 0xFFFF0000u);
  const float r1 = __builtin_isinf(x) ? 0.f : x - __uint_as_float(hb);
  mb = __float_as_uint(r1) & 0xFFFF0000u;
  const float r2 = r1 - __uint_as_float(mb);
  lb = __float_as_uint(r2) & 0xFFFF0000u;
}

// bound_kernel for bf16 queries on the bf16 matrix cores.  q is exact in bf16
// and kbar = dc / sqrt(512) (fp32) is split exactly into three bf16 terms, so
// q.kbar is the sum of three bf16 products, each exact, accumulated in fp32
// by v_mfma_f32_32x32x16_bf16 -- the fp32 kernel's arithmetic, at three
// 8-pass products per 16 dims instead of eight 16-pass fp32 ones.  A
// workgroup covers NQT query tiles of 64 rows against 64 blocks of one kv
// head; each wave splits its 32 blocks' kbar chunk once per 16 dims and uses
// it for all NQT tiles.  MFMA lane l supplies row l % 32 and k indices
// 8 (l / 32) .. + 8, which map to dims hf * D/2 + s .. + 8 of both operands
// (the contraction order is free as long as A and B agree).  |q|^2 comes
// from packed dot products of the same query words.  Output lane l, i:
// query 8(i/4) + 4(l/32) + i%4, block l % 32, as in bound_kernel.
template <int NQT, int HALF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void bound_bf16_kernel(BoundParams p) {
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  __shared__ float s_m[NQT][2][2][32];
  constexpr int D = 2 * HALF;
  const int H = p.num_kv_heads;
  const int nb = p.num_blocks;
  const int nq = p.sq * p.group;
  const int nbt = (nb + kBoundBT - 1) / kBoundBT;
  int id = blockIdx.x;
  const int h = id % H; id /= H;
  const int bt = id % nbt;
  const int qb = id / nbt;  // query tiles qb * NQT .. + NQT
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = t / kWave;
  const int wq = wave & 1, wb = wave >> 1;
  const int r = lane & 31, hf = lane >> 5;

  const int brow = bt * kBoundBT + wb * 32 + r;
  const float* dcrow = p.dc + ((int64_t)min(brow, nb - 1) * H + h) * D;
  const float eac = p.e_ac[(int64_t)min(brow, nb - 1) * H + h];
  const int d0 = hf * HALF;
  const uint16_t* qrow[NQT];
#pragma unroll
  for (int k = 0; k < NQT; ++k) {
    const int qc = min((qb * NQT + k) * kBoundQT + wq * 32 + r, nq - 1);
    const int st = qc / p.group, gq = qc - st * p.group;
    qrow[k] = reinterpret_cast<const uint16_t*>(p.q) + (int64_t)st * p.q_tok_stride +
              (int64_t)(h * p.group + gq) * p.q_head_stride + d0;
  }
  constexpr float kInv = 1.f / kSqrt512;
  f32x16 acc[NQT];
  float qq[NQT];
#pragma unroll
  for (int k = 0; k < NQT; ++k) {
    qq[k] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[k][i] = 0.f;
  }
  // Rounds of 32 dims of the lane's half: all of a round's loads are issued
  // before its products, so a wave waits for memory once per round, and the
  // registers (96 at head_dim 128) leave room for every wave of the launch
  // at once (C4: 7.75 -> 7.56 us against 64-dim rounds at 120 registers).
  constexpr int kSteps = HALF / 8 < 4 ? HALF / 8 : 4;  // 8 dims per product step
#pragma unroll
  for (int s0 = 0; s0 < HALF; s0 += 8 * kSteps) {
    uint4 qa[kSteps][NQT];
    float4 c[kSteps][2];
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const int s = s0 + 8 * j;
#pragma unroll
      for (int k = 0; k < NQT; ++k) qa[j][k] = ld16(qrow[k] + s);
      c[j][0] = *reinterpret_cast<const float4*>(dcrow + d0 + s);
      c[j][1] = *reinterpret_cast<const float4*>(dcrow + d0 + s + 4);
    }
    // Keep the compiler from sinking the loads to their uses (it would wait
    // for memory once per step).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
      const float kb[8] = {c[j][0].x * kInv, c[j][0].y * kInv, c[j][0].z * kInv, c[j][0].w * kInv,  // kbar, spectral_energy.py:166
                           c[j][1].x * kInv, c[j][1].y * kInv, c[j][1].z * kInv, c[j][1].w * kInv};
      uint4 bh, bm, bl;
      uint32_t* ph = &bh.x;
      uint32_t* pm = &bm.x;
      uint32_t* pl = &bl.x;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t h0, m0, l0, h1, m1, l1;
        split_bf16x3(kb[2 * i], h0, m0, l0);
        split_bf16x3(kb[2 * i + 1], h1, m1, l1);
        ph[i] = (h0 >> 16) | h1;
        pm[i] = (m0 >> 16) | m1;
        pl[i] = (l0 >> 16) | l1;
      }
      const bf16x8 vh = __builtin_bit_cast(bf16x8, bh);
      const bf16x8 vm = __builtin_bit_cast(bf16x8, bm);
      const bf16x8 vl = __builtin_bit_cast(bf16x8, bl);
#pragma unroll
      for (int k = 0; k < NQT; ++k) {
        const bf16x8 va = __builtin_bit_cast(bf16x8, qa[j][k]);
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, vh, acc[k], 0, 0, 0);
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, vm, acc[k], 0, 0, 0);
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, vl, acc[k], 0, 0, 0);
        qq[k] = dot2_acc<kBF16>(qa[j][k].x, qa[j][k].x, qq[k]);
        qq[k] = dot2_acc<kBF16>(qa[j][k].y, qa[j][k].y, qq[k]);
        qq[k] = dot2_acc<kBF16>(qa[j][k].z, qa[j][k].z, qq[k]);
        qq[k] = dot2_acc<kBF16>(qa[j][k].w, qa[j][k].w, qq[k]);
      }
    }
  }

  // tau_j(q) = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d) (spectral_energy.py:170-176).
  const float inv_sqrt_d = 1.f / sqrtf((float)D);
  const float sqrt_eac = sqrtf(eac);
#pragma unroll
  for (int k = 0; k < NQT; ++k) {
    const float qf = qq[k] + __shfl_xor(qq[k], 32, kWave);  // full squared norm of query row r
    const int q0 = (qb * NQT + k) * kBoundQT + wq * 32;
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = 8 * (i >> 2) + 4 * hf + (i & 3);
      const float qn = __shfl(qf, rr, kWave);
      if (q0 + rr < nq && brow < nb) {
        const float bound = acc[k][i] * inv_sqrt_d + (sqrtf(qn) * sqrt_eac) * inv_sqrt_d;
        if (p.bounds) p.bounds[((int64_t)(q0 + rr) * nb + brow) * H + h] = bound;
        m = nanmax(m, bound);
      }
    }
    if (p.tau_part) {
      m = nanmax(m, __shfl_xor(m, 32, kWave));
      if (hf == 0) s_m[k][wb][wq][r] = m;
    }
  }
  if (p.tau_part) {
    // NaN-propagating max over each tile's 64 queries: the two query-half
    // waves through LDS.
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NQT; ++k) {
      const int qt = qb * NQT + k;
      if (wq == 0 && hf == 0 && brow < nb && qt * kBoundQT < nq)
        p.tau_part[((int64_t)qt * nb + brow) * H + h] = nanmax(s_m[k][wb][0][r], s_m[k][wb][1][r]);
    }
  }
}

// Query-aware bound from write-time block statistics: with kbar, E_AC and
// zeta computed once when a block enters the cache (oc_score_blocks without
// queries), a decode step only needs tau_j(q) = q.kbar/sqrt(d) +
// ||q|| sqrt(E_AC)/sqrt(d) per (block, kv head), max over the query rows
// sharing the kv head -- the hoisting of docs/mathematical_framework.md:242-250.
// One wave per (block, kv head) tile: lane l holds dims l*DPL .. +DPL of dc
// (kbar = dc / sqrt(512), as the scoring kernel forms it) and of each query;
// dot products and squared norms are wave sums.  Reads Hkv*D*4 B per block
// instead of the block's keys.
template <int QDT, int DPL>
__global__ __launch_bounds__(256) void cached_bound_kernel(CachedBoundParams p) {
  using EQ = Elt<QDT>;
  constexpr int D = DPL * kWave;
  const int H = p.num_kv_heads;
  const int tile = blockIdx.x * (256 / kWave) + (int)(threadIdx.x / kWave);
  if (tile >= p.total_blocks * H) return;  // whole waves exit together
  const int lane = threadIdx.x & (kWave - 1);
  const int gb = tile / H, h = tile - gb * H;
  int seg = 0;
  if (p.cu_blocks) {
    int lo = 0, hi = p.num_segments - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.cu_blocks[mid] <= gb) lo = mid; else hi = mid - 1;
    }
    seg = lo;
  }
  float kb[DPL];
  const float* dcp = p.dc + (int64_t)tile * D + lane * DPL;
#pragma unroll
  for (int j = 0; j < DPL; ++j) kb[j] = dcp[j] / kSqrt512;  // spectral_energy.py:166
  const float sqrt_d = sqrtf((float)D);
  const float sqrt_eac = sqrtf(p.e_ac[tile]);
  const int nq = p.sq * p.group;
  float best = -INFINITY;
  for (int qi = 0; qi < nq; ++qi) {
    const int st = qi / p.group, g = qi - st * p.group;
    const int64_t qoff = (int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                         (int64_t)(h * p.group + g) * p.q_head_stride + lane * DPL;
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float v = EQ::load1(p.q, qoff + j);
      a = fmaf(v, kb[j], a);
      b = fmaf(v, v, b);
    }
    a = wave_sum(a);
    b = wave_sum(b);
    const float align = a / sqrt_d;
    const float resid = (sqrtf(b) * sqrt_eac) / sqrt_d;
    best = nanmax(align + resid, best);
  }
  if (lane == 0) {
    p.tau_max[tile] = best;
    if (p.gate.keep) {
      const uint8_t k = gate_keep(p.gate, seg, best, p.zeta[tile]);
      p.gate.keep[tile] = k;
      if (p.gate.mask_out) p.gate.mask_out[tile] = k;
    }
  }
}

template <int QDT>
static hipError_t launch_cached_bound_q(const CachedBoundParams& p, hipStream_t s) {
  const dim3 grid((unsigned)(((int64_t)p.total_blocks * p.num_kv_heads + 3) / 4));
  switch (p.head_dim) {
    case 64: hipLaunchKernelGGL((cached_bound_kernel<QDT, 1>), grid, dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL((cached_bound_kernel<QDT, 2>), grid, dim3(256), 0, s, p); break;
    case 256: hipLaunchKernelGGL((cached_bound_kernel<QDT, 4>), grid, dim3(256), 0, s, p); break;
    case 512: hipLaunchKernelGGL((cached_bound_kernel<QDT, 8>), grid, dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_cached_bound(const CachedBoundParams& p, hipStream_t s) {
  if ((int64_t)p.total_blocks * p.num_kv_heads == 0) return hipSuccess;
  switch (p.q_dtype) {
    case kF32: return launch_cached_bound_q<kF32>(p, s);
    case kBF16: return launch_cached_bound_q<kBF16>(p, s);
    case kF16: return launch_cached_bound_q<kF16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// Spatial energy sum k^2 per (block, head) for any block size
// (spectral_energy.py:21-35).  One workgroup per (block, head).
__global__ __launch_bounds__(256) void block_energy_kernel(EnergyParams p) {
  __shared__ float s_red[8];
  const int tile = blockIdx.x;
  const int b = tile / p.num_kv_heads, h = tile - b * p.num_kv_heads;
  const int n = p.block_size * p.head_dim;
  float acc = 0.f;
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const int r = e / p.head_dim, d = e - r * p.head_dim;
    const float v = load_elt(p.k_dtype, p.k, ((int64_t)b * p.block_size + r) * p.k_tok_stride +
                                              (int64_t)h * p.k_head_stride + d);
    acc = fmaf(v, v, acc);
  }
  float v1[1] = {acc};
  block_sum<1>(v1, s_red);
  if (threadIdx.x == 0) p.out[tile] = v1[0];
}

}  // namespace oc

// ---------------------------------------------------------------- launchers
namespace oc {

template <int DT, int LPR, int QDT, int HPT>
static hipError_t launch_score_q(const ScoreParams& p, hipStream_t s) {
  const int tiles = p.total_blocks * (p.num_kv_heads / HPT);
  if (!p.logits) {
    hipLaunchKernelGGL((score_kernel<DT, LPR, QDT, 0, HPT>), dim3(tiles), dim3(256), 0, s, p);
    return hipGetLastError();
  }
  // Logits: lanes per head row of the attention's value loads (<= 64).
  if constexpr (LPR / HPT <= 64) {
    switch (logits_nq_pad(p.sq * p.group)) {
      case 1: hipLaunchKernelGGL((score_kernel<DT, LPR, QDT, 1, HPT>), dim3(tiles), dim3(256), 0, s, p); break;
      case 2: hipLaunchKernelGGL((score_kernel<DT, LPR, QDT, 2, HPT>), dim3(tiles), dim3(256), 0, s, p); break;
      default: hipLaunchKernelGGL((score_kernel<DT, LPR, QDT, 4, HPT>), dim3(tiles), dim3(256), 0, s, p); break;
    }
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

template <int DT, int LPR, int HPT = 1>
static hipError_t launch_score_t(const ScoreParams& p, hipStream_t s) {
  // Without queries the query type is irrelevant: use the key type.
  const int qdt = p.q ? p.q_dtype : DT;
  if (qdt == DT) return launch_score_q<DT, LPR, DT, HPT>(p, s);
  if (qdt == kF32) return launch_score_q<DT, LPR, kF32, HPT>(p, s);
  return hipErrorInvalidValue;
}

// Heads with 128- or 256-byte rows (8 or 16 lanes of 16 bytes: bf16/fp16
// head_dim 64 or 128, fp32 32 or 64) are scored two per tile when the head
// count is even, so a tile row is twice as long; head_dim 128 then reads as
// head_dim 256 does: C3's scoring pass with logits 208 -> 190 us, without 176 ->
// 165 us at the same bytes (the per-tile merge, reductions and bound are
// shared by twice the keys).
// The second head's lane offset (its head stride plus the lane's column, in
// bytes) must fit the 32-bit lane offset next to 64 token rows (< 2^31, checked
// by the API), so pairs are formed only for head strides under 2^30 bytes.
template <int DT>
static hipError_t launch_score_dt(const ScoreParams& p, hipStream_t s) {
  const int lpr = p.head_dim / Elt<DT>::VEC;
  const bool pairs = p.num_kv_heads % 2 == 0 && p.k_head_stride >= 0 &&
                     p.k_head_stride * (int64_t)(16 / Elt<DT>::VEC) < ((int64_t)1 << 30);
  switch (lpr) {
    case 8: return pairs ? launch_score_t<DT, 16, 2>(p, s) : launch_score_t<DT, 8>(p, s);
    case 16: return pairs ? launch_score_t<DT, 32, 2>(p, s) : launch_score_t<DT, 16>(p, s);
    case 32: return launch_score_t<DT, 32>(p, s);
    case 64: return launch_score_t<DT, 64>(p, s);
    case 128: return launch_score_t<DT, 128>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// True when score_kernel has an instantiation for (dtype, head_dim).
bool score_supported(int dt, int head_dim) {
  const int vec = (dt == kF32) ? 4 : 8;
  if (head_dim % vec) return false;
  const int lpr = head_dim / vec;
  return lpr == 8 || lpr == 16 || lpr == 32 || lpr == 64 || lpr == 128;
}

// True when score_kernel can also write the attention logits of nq query
// rows per kv head.
bool score_logits_supported(int dt, int head_dim, int nq) {
  const int vec = (dt == kF32) ? 4 : 8;
  return score_supported(dt, head_dim) && head_dim / vec <= 64 && nq >= 1 && nq <= kLogitsMaxQ;
}

hipError_t launch_score(const ScoreParams& p, hipStream_t s) {
  if (p.total_blocks == 0) return hipSuccess;
  switch (p.k_dtype) {
    case kF32: return launch_score_dt<kF32>(p, s);
    case kBF16: return launch_score_dt<kBF16>(p, s);
    case kF16: return launch_score_dt<kF16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <int QDT>
static void launch_bound_q(const BoundParams& p, dim3 grid, bool vec, hipStream_t s) {
  if (vec) {
    hipLaunchKernelGGL((bound_kernel<QDT, true>), grid, dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((bound_kernel<QDT, false>), grid, dim3(256), 0, s, p);
  }
}

hipError_t launch_bound(const BoundParams& p, hipStream_t s) {
  const int nq = p.sq * p.group;
  if (nq == 0 || p.num_blocks == 0) return hipSuccess;
  const int nqt = (nq + kBoundQT - 1) / kBoundQT;
  const int nbt = (p.num_blocks + kBoundBT - 1) / kBoundBT;
  const dim3 grid(nqt * nbt * p.num_kv_heads);
  const int qsz = p.q_dtype == kF32 ? 4 : 2;
  const int half = (p.head_dim + 1) / 2;
  const bool vec = (reinterpret_cast<uintptr_t>(p.q) % 16 == 0) && (reinterpret_cast<uintptr_t>(p.dc) % 16 == 0) &&
                   (p.q_tok_stride * qsz) % 16 == 0 && (p.q_head_stride * qsz) % 16 == 0 &&
                   p.head_dim % 2 == 0 && (half * qsz) % 16 == 0 && (half * 4) % 16 == 0;
  if (p.q_dtype == kBF16 && vec) {
    // bf16 queries, head_dim 64 / 128 / 256: the bf16 matrix cores with kbar
    // split into three bf16 terms, one query tile per workgroup (C4, 2048
    // rows x 256 blocks x 8 kv heads: 7.8 us against 8.5 us for the fp32
    // kernel; two or four tiles per workgroup, sharing each split: 11.1 and
    // 17.6 us).
    constexpr int kNqt = 1;
    const dim3 g2(((nqt + kNqt - 1) / kNqt) * nbt * p.num_kv_heads);
    switch (p.head_dim) {
      case 64: hipLaunchKernelGGL((bound_bf16_kernel<kNqt, 32>), g2, dim3(256), 0, s, p); return hipGetLastError();
      case 128: hipLaunchKernelGGL((bound_bf16_kernel<kNqt, 64>), g2, dim3(256), 0, s, p); return hipGetLastError();
      case 256: hipLaunchKernelGGL((bound_bf16_kernel<kNqt, 128>), g2, dim3(256), 0, s, p); return hipGetLastError();
      default: break;  // other head dims: the fp32 kernel
    }
  }
  switch (p.q_dtype) {
    case kF32: launch_bound_q<kF32>(p, grid, vec, s); break;
    case kBF16: launch_bound_q<kBF16>(p, grid, vec, s); break;
    case kF16: launch_bound_q<kF16>(p, grid, vec, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int bound_query_tile() { return kBoundQT; }
int bound_block_tile() { return kBoundBT; }

hipError_t launch_block_energy(const EnergyParams& p, hipStream_t s) {
  if (p.num_blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(block_energy_kernel, dim3(p.num_blocks * p.num_kv_heads), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace oc
