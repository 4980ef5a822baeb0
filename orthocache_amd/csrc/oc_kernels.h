// Internal kernel parameter blocks and launchers shared by the kernel
// translation units and the C ABI (oc_api.hip).
#pragma once

#include "oc_common.h"

namespace oc {

// ------------------------------------------------------------ oc_fwht.hip
struct FwhtParams {
  const void* x;
  int x_dtype;
  int64_t x_batch_stride, x_row_stride;  // elements
  void* y;
  int y_dtype;
  int64_t y_batch_stride, y_row_stride;
  int64_t n_cols;
  int64_t n_batch;
};

struct BandParams {
  const float* spec;  // (nb, 512, H, D) fp32
  int num_blocks, num_heads, head_dim;
  int s0, s1;
  float* out;
};

hipError_t launch_fwht(const FwhtParams& p, hipStream_t s);
hipError_t launch_band_energy(const BandParams& p, hipStream_t s);

// Two-gate keep flags written by a scoring kernel: the predicate of the
// mask + compaction step, keep = (tau_max >= tau) & (zeta <= zeta_max) with
// fp32 compares (NaN -> false), per segment thresholds when given.
struct GateParams {
  uint8_t* keep;          // (total_blocks, Hkv) or null: no flags
  uint8_t* mask_out;      // (total_blocks, Hkv) or null: a second copy (any alignment)
  const float* tau_arr;   // (num_segments) or null: tau
  float tau;
  const float* zmax_arr;  // (num_segments) or null: zeta_max
  float zeta_max;
};

__device__ __forceinline__ uint8_t gate_keep(const GateParams& g, int seg, float tau_max, float zeta) {
  const float tau = g.tau_arr ? g.tau_arr[seg] : g.tau;
  const float zm = g.zmax_arr ? g.zmax_arr[seg] : g.zeta_max;
  return ((tau_max >= tau) & (zeta <= zm)) ? 1 : 0;
}

// ----------------------------------------------------------- oc_score.hip

struct BoundParams {
  const float* dc;     // (nb, Hkv, D)
  const float* e_ac;   // (nb, Hkv)
  const void* q;
  int q_dtype;
  int64_t q_tok_stride, q_head_stride;
  int sq, group, head_dim, num_kv_heads, num_blocks;
  float* bounds;       // (sq*group, nb, Hkv) or null
  float* tau_part;     // (ceil(sq*group/64), nb, Hkv) or null
};

// Bound from write-time block statistics (dc, E_AC of oc_score_blocks), for
// few queries per kv head: tau_max[j, h] = NaN-propagating max over the
// segment's query rows.
struct CachedBoundParams {
  const float* dc;     // (total_blocks, Hkv, D)
  const float* e_ac;   // (total_blocks, Hkv)
  const void* q;
  int q_dtype;
  int64_t q_seg_stride, q_tok_stride, q_head_stride;
  int sq, group, head_dim, num_kv_heads, total_blocks;
  const int* cu_blocks;  // (num_segments + 1) or null
  int num_segments;
  float* tau_max;      // (total_blocks, Hkv)
  const float* zeta;   // (total_blocks, Hkv) cached zeta, read for gate.keep
  GateParams gate;
};

struct EnergyParams {
  const void* k;
  int k_dtype;
  int64_t k_tok_stride, k_head_stride;
  int head_dim, num_kv_heads, num_blocks, block_size;
  float* out;
};

hipError_t launch_cached_bound(const CachedBoundParams& p, hipStream_t s);
int bound_query_tile();  // queries per partial maximum of the bound kernel
int bound_block_tile();
hipError_t launch_bound(const BoundParams& p, hipStream_t s);
hipError_t launch_block_energy(const EnergyParams& p, hipStream_t s);

// --------------------------------------------------------- oc_compact.hip
struct CompactParams {
  const float* tau_max;    // (tau_parts, total_blocks, Hkv)
  int tau_parts;
  const float* zeta;       // (total_blocks, Hkv) or null: gate 2 off
  const uint8_t* mask_in;  // (total_blocks, mask_in_heads): use instead of scores when non-null
  int mask_in_heads;
  const float* tau_arr;    // per-segment thresholds, or null to use tau
  float tau;
  const float* zmax_arr;
  float zeta_max;
  const int* cu_blocks;    // (num_segments + 1) or null for one segment of nb_single blocks
  int num_segments;
  int nb_single;
  int num_kv_heads;
  int total_blocks;
  uint8_t* mask_out;       // (total_blocks, Hkv) or null
  uint8_t* active_out;     // (total_blocks) or null
  int* indices;            // (total_blocks) or null: local block ids per segment
  int* num_active;         // (num_segments) or null
  int* head_indices;       // (Hkv, total_blocks) or null
  int* head_num_active;    // (num_segments, Hkv)
  int* head_uniform;       // (num_segments, Hkv) or null
  int empty_head_all;
};

struct CopyParams {
  const void* src;
  void* dst;
  const int* indices;
  const int* num_active;
  int num_blocks;
  int64_t block_bytes;  // multiple of 16
  int scatter;
};

hipError_t launch_compact(const CompactParams& p, hipStream_t s);

struct ScoreParams {
  const void* k;
  int64_t k_tok_stride;   // elements between consecutive tokens
  int64_t k_head_stride;  // elements between kv heads
  int k_dtype;
  int head_dim;
  int num_kv_heads;
  int total_blocks;
  const int* cu_blocks;   // (num_segments + 1) block offsets, or null for one segment
  int num_segments;
  // Queries for the inline bound (may be null): segment s, query t, head hq
  // at q + s*q_seg_stride + t*q_tok_stride + hq*q_head_stride.
  const void* q;
  int q_dtype;
  int64_t q_seg_stride, q_tok_stride, q_head_stride;
  int sq;      // queries per segment
  int group;   // query heads per kv head
  // Outputs, each optional.
  float* tau_max;  // (total_blocks, Hkv): NaN-propagating max over queries
  float* zeta;     // (total_blocks, Hkv)
  float* dc;       // (total_blocks, Hkv, D): FWHT coefficient 0
  float* e_low;
  float* e_mid;
  float* e_high;
  float* e_ac;
  const int* pages;  // (total_blocks) physical 512-token page of each block, or null (pages = blocks)
  int num_pages;     // pool size in pages (page numbers are clamped into it)
  // Attention logits of the segment's queries, written while the keys stream
  // (or null): logits[((gb * Hkv + h) * 512 + row) * nq_pad + i] =
  // q_i . k_row * logit_scale for query row i < sq*group of kv head h
  // (0 for i >= sq*group); nq_pad = logits_nq_pad(sq * group) <= kLogitsMaxQ.
  float* logits;
  float logit_scale;  // log2(e) / sqrt(head_dim)
  GateParams gate;    // keep flags from tau_max and zeta (needs q)
};

constexpr int kLogitsMaxQ = 4;  // query rows per kv head with scoring-pass logits
__host__ __device__ inline int logits_nq_pad(int nq) { return nq <= 1 ? 1 : (nq <= 2 ? 2 : 4); }

bool score_supported(int dt, int head_dim);
bool score_logits_supported(int dt, int head_dim, int nq);
hipError_t launch_score(const ScoreParams& p, hipStream_t s);
hipError_t launch_copy_blocks(const CopyParams& p, hipStream_t s);

// Physical page of flattened block j: pages[j] clamped into [0, num_pages),
// or j itself for a contiguous cache.
__device__ __forceinline__ int64_t page_of(const int* pages, int num_pages, int64_t j) {
  if (!pages) return j;
  const int pg = pages[j];
  return (int64_t)((unsigned)pg < (unsigned)num_pages ? pg : (pg < 0 ? 0 : num_pages - 1));
}

// ---------------------------------------------------------- oc_attend.hip
constexpr int kQG = 8;           // queries per attention work item
enum StreamForm : int { kStreamNone = 0, kStreamSplit = 1, kStreamRanges = 2 };
constexpr int kMaxLists = 2048;  // (segments x kv heads) per launch

struct AttendParams {
  const void* q;
  int q_dtype;
  int64_t q_seg_stride, q_tok_stride, q_head_stride;
  const void* k;
  const void* v;
  int kv_dtype;
  int64_t k_tok_stride, k_head_stride, v_tok_stride, v_head_stride;
  int head_dim, num_kv_heads, group, sq;
  int block_size, total_blocks;
  const int* cu_blocks;  // (num_segments + 1) or null
  int num_segments;
  const int* indices;    // unified (total_blocks) or per head (Hkv, total_blocks)
  const int* counts;     // unified (num_segments) or per head (num_segments, Hkv)
  int per_head;
  const int* uniform;      // (num_segments, Hkv) or null: equal weights on every token
  float logit_scale;       // log2(e) / sqrt(head_dim)
  int chunk, nchunk;
  float* part_o;    // decode: (max_items, kQG, D); prefill: (nsplit, segments, Hkv, D, rows_pad)
  float* part_ml;   // decode: (max_items, kQG, 2); prefill: (nsplit, segments, Hkv, rows_pad, 2)
  int prefill;      // 1: matrix-core prefill kernels (oc_prefill.hip)
  int nsplit;       // prefill: ways the tile range of a list is split
  void* out;
  int out_dtype;
  int64_t out_seg_stride, out_tok_stride, out_head_stride;
  const int* pages;  // (total_blocks) physical page of each block (block_size tokens), or null
  int num_pages;     // pool size in pages (page numbers are clamped into it)
  // Logits from the scoring pass (ScoreParams::logits layout) or null.  When
  // set, the decode kernel reads them instead of the keys (block_size 512,
  // sq*group <= kLogitsMaxQ); k is not read.
  const float* logits;
  // Keep flags (total_blocks, Hkv) of one segment instead of a compacted
  // list (or null): every decode workgroup derives the unified active list
  // itself; workgroup 0 writes the permutation and count to list_out and
  // count_out, which the combine then reads (counts must equal count_out).
  const uint8_t* keep;
  int* list_out;
  int* count_out;
  // Streaming forms (with logits): kStreamSplit (one segment, unified list):
  // each kv head's chunks split `splits` ways, one partial per (head, split);
  // kStreamRanges: the chunks of all lists cut into `splits` equal ranges,
  // one partial per (range, list piece, wave).  kStreamNone: one partial per
  // work item.
  int stream;
  int splits;
};

bool attend_supported(int dt, int head_dim);
int attend_nq_bucket(int nq_total);
int attend_chunk(int dt, int head_dim, int nq_total);  // tokens per work item
int64_t attend_max_items(const AttendParams& p);
int64_t attend_partial_slots(const AttendParams& p);  // partials the decode launch writes
hipError_t launch_attend(const AttendParams& p, hipStream_t s);

// ---------------------------------------------------------- oc_prefill.hip
constexpr int kPrefillMinRows = 32;   // query rows per kv head from which the MFMA path is used
constexpr int kPrefillMaxSplit = 16;

// Waves per prefill workgroup, one 32-row MFMA tile each: 8 for head_dim 128
// (each staged K / V^T tile serves 256 query rows), 4 for head_dim 64.
__host__ __device__ constexpr int prefill_waves(int head_dim) { return head_dim >= 128 ? 8 : 4; }
__host__ __device__ constexpr int prefill_tile_rows(int head_dim) { return prefill_waves(head_dim) * 32; }

__host__ __device__ inline int prefill_rows(const AttendParams& p) { return p.sq * p.group; }
__host__ __device__ inline int prefill_qtiles(const AttendParams& p) {
  const int tr = prefill_tile_rows(p.head_dim);
  return (prefill_rows(p) + tr - 1) / tr;
}
// Partial rows per (split, segment, kv head): the query tiles padded to whole tiles.
__host__ __device__ inline int64_t prefill_rows_pad(const AttendParams& p) {
  return (int64_t)prefill_qtiles(p) * prefill_tile_rows(p.head_dim);
}

bool prefill_supported(int kv_dtype, int q_dtype, int head_dim, int nq_rows, int block_size);
int prefill_nsplit(const AttendParams& p);
int64_t prefill_partial_floats(const AttendParams& p);
hipError_t launch_prefill(const AttendParams& p, hipStream_t s);

}  // namespace oc
