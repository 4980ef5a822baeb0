/*
 * orthocache_hip.h - C ABI of liborthocache_hip.so, the MI355X (gfx950)
 * implementation of OrthoCache's block-eviction attention path:
 *   FWHT-512 -> band energies / zeta / block mean / query-aware bound
 *   -> two-gate mask -> stream compaction -> indirect block-sparse attention.
 *
 * Conventions
 *  - Every pointer argument named as data is a DEVICE pointer (HIP global
 *    memory), except the argument structs themselves, which live on the host.
 *  - Layouts follow the reference: keys/values (seq, kv_heads, head_dim),
 *    queries (seq_q, q_heads, head_dim), head_dim contiguous.  Strides are in
 *    elements.  Query head hq reads kv head hq / group (GQA; group 1 is the
 *    reference's equal-heads case).
 *  - A "segment" is one sequence of a ragged batch (or one layer of a
 *    multi-layer sweep): cu_blocks[s]..cu_blocks[s+1] are its blocks in the
 *    flattened block space, whose token range is [cu*512, ...).  cu_blocks ==
 *    NULL means one segment of total_blocks blocks.
 *  - Calls are asynchronous on `stream` (a hipStream_t; NULL = default
 *    stream), never synchronise the host, and never allocate: outputs and
 *    workspaces are caller-owned.  Counts such as num_active stay on device.
 *  - Return 0 on success or a negative OC_ERR_* code; oc_last_error() gives
 *    a message (thread-local).  Entry points are stateless and reentrant.
 *  - Workspaces must be 256-byte aligned (hipMalloc and torch allocations
 *    are); an unaligned one is rejected with OC_ERR_INVALID_ARGUMENT.
 *  - Paged caches: the argument structs of scoring, attention and the layer
 *    take `pages`, an int32 device array (total_blocks): the block with
 *    flattened index j (segment offsets included) lives in physical page
 *    pages[j] of the key/value pool, i.e. at token pages[j] * block_size.
 *    NULL means block j is at token j * block_size (contiguous cache).  Masks,
 *    scores and block lists stay in logical block numbering.  num_pages is the
 *    pool size in pages; page numbers outside [0, num_pages) are clamped into
 *    it (the kernels never read outside the pool), as are block-list entries
 *    outside their segment.  (ABI version 2 appended these fields.)
 *  - ABI version 3 appended to oc_score_args and oc_attend_args:
 *    scoring-pass logits (with at most 4 query rows per kv head the scoring
 *    pass can also write the attention logits of every key row it streams,
 *    and the decode attention can read them instead of the keys), and the
 *    two-gate mask written by the scoring pass, which the decode attention
 *    of one segment can take instead of a compacted list.
 */
#ifndef ORTHOCACHE_HIP_H
#define ORTHOCACHE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OC_ABI_VERSION 3

#define OC_OK 0
#define OC_ERR_INVALID_ARGUMENT (-1)
#define OC_ERR_UNSUPPORTED (-2)
#define OC_ERR_HIP (-3)
#define OC_ERR_WORKSPACE (-4)

/* Element types. */
#define OC_F32 0
#define OC_BF16 1
#define OC_F16 2

#define OC_BLOCK 512 /* FWHT length: tokens per scored block */

/* Thread-local message for the last failing call on this thread. */
const char* oc_last_error(void);
int oc_abi_version(void);

/* ---------------------------------------------------------------- FWHT
 * Replaces fwht_512 (src/orthocache/fwht.py:4-65) and, with n_batch = nb and
 * strides of (seq, heads*dim), _run_fwht_on_blocks
 * (src/orthocache/spectral_energy.py:38-66).  y[b, :, c] = H_512 x[b, :, c]
 * / sqrt(512) in natural (Hadamard) order, fp32 arithmetic.  512 rows per
 * batch entry, n_cols contiguous columns. */
typedef struct oc_fwht_args {
  const void* x;
  int32_t x_dtype;
  int64_t x_batch_stride, x_row_stride;
  void* y;
  int32_t y_dtype;
  int64_t y_batch_stride, y_row_stride;
  int64_t n_cols;
  int64_t n_batch;
} oc_fwht_args;
int oc_fwht512(const oc_fwht_args* a, void* stream);

/* Energy of a coefficient band over a materialised fp32 spectrum
 * (nb, 512, heads, dim): out[b, h] = sum_{s in [s0, s1)} sum_d spec^2.
 * Replaces the band sums of compute_spectral_bands for non-default bands
 * (src/orthocache/spectral_energy.py:100-104). */
int oc_band_energy(const float* spec, int32_t num_blocks, int32_t num_heads, int32_t head_dim,
                   int32_t s0, int32_t s1, float* out, void* stream);

/* Spatial block energy sum k^2 per (block, head), any block size.
 * Replaces compute_block_energy_jax (src/orthocache/spectral_energy.py:21-35). */
int oc_block_energy(const void* keys, int32_t keys_dtype, int64_t tok_stride, int64_t head_stride,
                    int32_t head_dim, int32_t num_kv_heads, int32_t num_blocks, int32_t block_size,
                    float* out, void* stream);

/* ---------------------------------------------------------------- scores
 * One pass over the keys per (block, kv head): band energies (natural-index
 * bands DC, [1,64), [64,256), [256,512)), zeta = E_high / (E_low + 1e-6),
 * DC coefficient, E_AC, and - when q is given - the NaN-propagating max over
 * the segment's queries (sq tokens x group heads) of the query-aware bound
 * tau_j = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d).
 * Replaces compute_spectral_bands, compute_spectral_decay_ratio,
 * compute_query_aware_bounds + the max of compute_query_aware_mask
 * (src/orthocache/spectral_energy.py:69-196).  Block size is 512.
 * Every output pointer may be NULL.  Requirements: head_dim * esize a multiple
 * of 16 and head_dim / (16 / esize) in {8,16,32,64,128}; 16-byte aligned keys,
 * strides multiples of 16 bytes.
 * logits (optional, needs q, 1 <= sq*group <= 4, head_dim / (16 / esize) <=
 * 64, 16-byte aligned q rows): fp32 (total_blocks, Hkv, 512, nq_pad) with
 * nq_pad = 1, 2 or 4 (sq*group rounded up to a power of two); entry
 * [j, h, r, i] = q_i . k_{512 j + r, h} * log2(e) / sqrt(head_dim) for query
 * row i = t*group + g of kv head h (zero for i >= sq*group).  The logits of
 * softmax(q.k / sqrt(d)) (src/orthocache/adaptive_attention.py:60-61, :103-104) in the
 * base-2 form, formed while the keys stream so that oc_attend need not read
 * the keys again.  No counterpart in the reference.
 * mask (optional, needs q and tau_max): the two-gate mask of each (block, kv
 * head), (tau_max >= tau) & (zeta <= zeta_max) in fp32 with NaN -> 0, as
 * uint8 (total_blocks, Hkv) -- compute_multiband_mask
 * (src/orthocache/spectral_energy.py:199-234) from the same scores, with
 * per-segment thresholds tau_arr / zeta_max_arr when given (as in
 * oc_mask_compact). */
typedef struct oc_score_args {
  const void* keys;
  int32_t keys_dtype;
  int64_t keys_tok_stride, keys_head_stride;
  int32_t head_dim, num_kv_heads, total_blocks;
  const int32_t* cu_blocks; /* device, num_segments + 1, or NULL */
  int32_t num_segments;
  const void* q; /* NULL: no bound */
  int32_t q_dtype;
  int64_t q_seg_stride, q_tok_stride, q_head_stride;
  int32_t sq, group;
  float* tau_max; /* (total_blocks, Hkv) */
  float* zeta;    /* (total_blocks, Hkv) */
  float* dc;      /* (total_blocks, Hkv, head_dim) */
  float* e_low;
  float* e_mid;
  float* e_high;
  float* e_ac;
  const int32_t* pages; /* (total_blocks) physical page per block, or NULL */
  int32_t num_pages;    /* pages in the key pool (used when pages != NULL) */
  float* logits;        /* (total_blocks, Hkv, 512, nq_pad), or NULL (ABI 3) */
  uint8_t* mask;        /* (total_blocks, Hkv) two-gate mask, or NULL (ABI 3) */
  const float* tau_arr; /* device, per segment, or NULL -> tau (ABI 3) */
  float tau;
  const float* zeta_max_arr;
  float zeta_max;
} oc_score_args;
int oc_score_blocks(const oc_score_args* a, void* stream);

/* Query-aware bound for many queries of one segment (prefill), from the dc
 * and e_ac outputs of oc_score_blocks.  bounds: (sq*group, nb, Hkv) with query
 * row t*group + g (the GQA-folded layout); tau_part: (ceil(sq*group/64), nb,
 * Hkv) partial maxima for oc_mask_compact (tau_parts = that count).
 * Replaces compute_query_aware_bounds (src/orthocache/spectral_energy.py:141-177). */
typedef struct oc_bound_args {
  const float* dc;
  const float* e_ac;
  const void* q;
  int32_t q_dtype;
  int64_t q_tok_stride, q_head_stride;
  int32_t sq, group, head_dim, num_kv_heads, num_blocks;
  float* bounds;
  float* tau_part;
} oc_bound_args;
int oc_query_bounds(const oc_bound_args* a, void* stream);
int32_t oc_query_bound_tiles(int32_t sq, int32_t group);

/* ---------------------------------------------------------------- mask + compaction
 * keep[j,h] = (max_p tau_max[p,j,h] >= tau) & (zeta[j,h] <= zeta_max), NaN ->
 * false, thresholds compared in fp32 (compute_multiband_mask,
 * src/orthocache/spectral_energy.py:199-234), or keep = mask_in when given.
 * active[j] = OR_h keep[j,h]; indices = per segment the active-first stable
 * permutation of local block ids, num_active = popcount (stream_compact,
 * src/orthocache/compaction.py:65-82; src/orthocache/adaptive_attention.py:29-40).
 * head_indices / head_num_active: the same partition per kv head; with
 * empty_head_all, a head keeping nothing lists every block and gets
 * head_uniform = 1 (the all-masked softmax of jax_block_sparse_attention,
 * src/orthocache/sparse_attention.py:49-57). */
typedef struct oc_compact_args {
  const float* tau_max;
  int32_t tau_parts;
  const float* zeta;       /* NULL: gate 2 off */
  const uint8_t* mask_in;  /* (total_blocks, mask_in_heads), instead of scores */
  int32_t mask_in_heads;
  const float* tau_arr;    /* device, per segment, or NULL -> tau */
  float tau;
  const float* zeta_max_arr;
  float zeta_max;
  const int32_t* cu_blocks;
  int32_t num_segments;
  int32_t num_kv_heads, total_blocks;
  uint8_t* mask_out;       /* (total_blocks, Hkv) */
  uint8_t* active_out;     /* (total_blocks) */
  int32_t* indices;        /* (total_blocks) */
  int32_t* num_active;     /* (num_segments) */
  int32_t* head_indices;   /* (Hkv, total_blocks) */
  int32_t* head_num_active;/* (num_segments, Hkv) */
  int32_t* head_uniform;   /* (num_segments, Hkv) */
  int32_t empty_head_all;
} oc_compact_args;
int oc_mask_compact(const oc_compact_args* a, void* stream);

/* Materialised compaction / decompaction of whole blocks
 * (stream_compact's gather, src/orthocache/compaction.py:86-98;
 * stream_decompact, :103-154).  scatter = 0: dst[i] = src[indices[i]] for
 * i < *num_active, zero otherwise; scatter = 1: dst[indices[i]] = src[i] for
 * i < *num_active, zero for every block no such i names.  block_bytes must
 * be a multiple of 16.  Every one of the num_blocks destination blocks is
 * written exactly once, whatever the list holds: entries in [-num_blocks, 0)
 * count from the end (NumPy indexing); other entries outside [0, num_blocks)
 * are clamped into it by the gather and dropped by the scatter (JAX's
 * gather / scatter rules); if several positions i < *num_active name one
 * block, the scatter takes the last of them; *num_active is clamped into
 * [0, num_blocks]. */
int oc_copy_blocks(const void* src, void* dst, const int32_t* indices, const int32_t* num_active,
                   int32_t num_blocks, int64_t block_bytes, int32_t scatter, void* stream);

/* ---------------------------------------------------------------- attention
 * Softmax attention over the tokens of the retained blocks listed by
 * oc_mask_compact (unified lists, or per-head lists with per_head = 1), fp32
 * accumulation, output cast to out_dtype; an empty list gives zeros, a
 * uniform-flagged list gives equal weights over its blocks.
 * Replaces orthocache_attention / _multihead_loop
 * (src/orthocache/adaptive_attention.py:46-184), indirect_attention
 * (src/orthocache/indirect_attention.py:127-170) and the kernel of
 * compile_pallas_sparse_attention (src/orthocache/sparse_attention.py:67-180).
 * Two kernel families, chosen per call (oc_attend_plan reports which):
 *  - decode: any sq*group (work split in groups of 8 queries; large query
 *    counts re-read K/V once per group); head_dim/(16/esize) in {8,16,32,64};
 *  - prefill (matrix cores): bf16 or fp16 q, K and V of one dtype,
 *    head_dim 64 or 128, block_size a multiple of 64 and at least 32 query
 *    rows (sq * group) per kv head; Q K^T and P V on bf16/fp16 MFMA tiles with
 *    fp32 softmax state, P rounded to the input dtype for the P V product.
 * logits (ABI 3, optional): the oc_score_blocks logits of the same q, keys
 * and segments; the decode kernel then reads them and the values only (k may
 * be NULL).  Needs block_size 512 and 1 <= sq*group <= 4.
 * mask (ABI 3, optional): a (total_blocks, Hkv) uint8 block mask of one
 * segment (cu_blocks NULL, per_head 0, 1 <= total_blocks <= 2048, decode
 * family) instead of indices/counts, which are then ignored: the attention
 * takes the blocks kept by any head (the unified list of
 * orthocache_attention, src/orthocache/adaptive_attention.py:29-40) and
 * writes the active-first permutation to indices_out and the count to
 * num_active_out (both required), as oc_mask_compact would.
 * workspace >= oc_attend_workspace_size(...). */
typedef struct oc_attend_args {
  const void* q;
  int32_t q_dtype;
  int64_t q_seg_stride, q_tok_stride, q_head_stride;
  const void* k;
  const void* v;
  int32_t kv_dtype;
  int64_t k_tok_stride, k_head_stride, v_tok_stride, v_head_stride;
  int32_t head_dim, num_kv_heads, group, sq;
  int32_t block_size, total_blocks;
  const int32_t* cu_blocks;
  int32_t num_segments;
  const int32_t* indices;
  const int32_t* counts;
  int32_t per_head;
  const int32_t* uniform;  /* (num_segments, Hkv), per-head lists only */
  void* out;
  int32_t out_dtype;
  int64_t out_seg_stride, out_tok_stride, out_head_stride;
  const int32_t* pages;    /* (total_blocks) physical page per block, or NULL */
  int32_t num_pages;       /* pages in the key/value pools (used when pages != NULL) */
  const float* logits;     /* scoring-pass logits, or NULL (ABI 3) */
  const uint8_t* mask;     /* (total_blocks, Hkv) block mask instead of a list, or NULL (ABI 3) */
  int32_t* indices_out;    /* (total_blocks), written when mask is given */
  int32_t* num_active_out; /* (1), written when mask is given */
} oc_attend_args;
size_t oc_attend_workspace_size(const oc_attend_args* a);
int oc_attend(const oc_attend_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* Which kernel family oc_attend uses for these arguments, and for the prefill
 * kernels the number of ways each list's tile range is split.  No
 * counterpart in the reference (its dispatch is the Python-side `path`
 * label of adaptive_attention.py:172-183); it lets callers and tests check
 * the choice without a device. */
#define OC_ATTEND_DECODE 0
#define OC_ATTEND_PREFILL_MFMA 1
int oc_attend_plan(const oc_attend_args* a, int32_t* kernel, int32_t* nsplit);

/* ---------------------------------------------------------------- one layer
 * The hot path in one call: oc_score_blocks -> oc_mask_compact -> oc_attend
 * (what orthocache_forward(mode='compact') does with a given tau and
 * zeta_max, src/orthocache/pipeline.py:96-145), for a batch of segments with
 * per-segment thresholds.  Optional outputs (tau_max, zeta, mask, indices,
 * num_active) may be NULL, in which case the workspace holds them.
 * Launches scoring, mask + compaction, attention and its combine on the
 * stream.  At most 16 queries per kv head (sq * group).  With at most 4
 * (and head_dim / (16 / esize) <= 64) the scoring pass also writes the
 * attention logits into the workspace and the attention reads only the
 * values of the retained blocks.  For one segment of at most 2048 blocks the
 * scoring pass also writes the two-gate mask and the attention derives the
 * list from it (no separate compaction launch); the outputs are the same.
 * workspace >= oc_decode_layer_workspace_size(...). */
typedef struct oc_layer_args {
  const void* q;
  int32_t q_dtype;
  int64_t q_seg_stride, q_tok_stride, q_head_stride;
  const void* k;
  const void* v;
  int32_t kv_dtype;
  int64_t k_tok_stride, k_head_stride, v_tok_stride, v_head_stride;
  int32_t head_dim, num_kv_heads, group, sq;
  int32_t total_blocks;
  const int32_t* cu_blocks;
  int32_t num_segments;
  const float* tau_arr;
  float tau;
  const float* zeta_max_arr;
  float zeta_max;
  void* out;
  int32_t out_dtype;
  int64_t out_seg_stride, out_tok_stride, out_head_stride;
  float* tau_max;
  float* zeta;
  uint8_t* mask;
  int32_t* indices;
  int32_t* num_active;
  const int32_t* pages;    /* (total_blocks) physical page per block, or NULL */
  int32_t num_pages;       /* pages in the key/value pools (used when pages != NULL) */
} oc_layer_args;
size_t oc_decode_layer_workspace_size(const oc_layer_args* a);
int oc_decode_layer(const oc_layer_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------- write-time block statistics
 * The decode step with the scoring hoisted to cache-write time
 * (docs/mathematical_framework.md:242-250, docs/technical_report.md:74: zeta
 * is query-independent and computed once when a block enters the KV cache).
 * When blocks are written, oc_score_blocks without queries (keys and outputs
 * offset to the first new block) yields their statistics: dc (FWHT
 * coefficient 0 per column, kbar = dc / sqrt(512)), e_ac and zeta.  A decode
 * step then reads those instead of the keys: the bound
 * tau_j(q) = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d) per (block, kv head)
 * (spectral_energy.py:141-177), the two-gate mask on the cached zeta, the
 * compaction and the attention -- the same results as oc_decode_layer on the
 * same keys, up to fp32 rounding of the bound.  `zeta` in oc_layer_args is
 * not written.  head_dim 64, 128, 256 or 512.  No counterpart entry point in
 * the reference (it recomputes the FWHT on every call, pipeline.py:96-145).
 * workspace >= oc_decode_layer_cached_workspace_size(...). */
typedef struct oc_block_stats {
  const float* dc;     /* (total_blocks, Hkv, head_dim) */
  const float* e_ac;   /* (total_blocks, Hkv) */
  const float* zeta;   /* (total_blocks, Hkv) */
} oc_block_stats;
size_t oc_decode_layer_cached_workspace_size(const oc_layer_args* a);
int oc_decode_layer_cached(const oc_layer_args* a, const oc_block_stats* stats, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------- allocation-free decode layer
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc: oc_decode_layer without a workspace argument.  The
 * library keeps OC_NOALLOC_SCRATCH_BYTES of scratch memory on every GPU it
 * runs on (a static device array, loaded with the library and held until the
 * process ends) and runs the layer there; inputs and outputs are the
 * caller's, as for oc_decode_layer, with the same results.  The call
 * allocates nothing; its first call on a device looks up that device's
 * scratch address.  A layer whose oc_decode_layer_workspace_size() exceeds
 * the scratch is rejected with OC_ERR_WORKSPACE before any launch (C2 --
 * 64K tokens, 16 kv heads, head_dim 256, two query rows per kv head -- needs
 * 10 MiB; 128K tokens 18 MiB).  The stream must belong to the current
 * device.  Every call on one GPU uses that GPU's scratch: calls that overlap
 * on one GPU (several streams or threads) race, and the caller must
 * serialise them.  Each call writes every scratch byte it reads, so nothing
 * has to be cleared between calls. */
#define OC_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int oc_decode_layer_noalloc(const oc_layer_args* a, void* stream);

/* ---------------------------------------------------- reference custom call
 * The reference's own C entry point for its compacted attention, under its
 * name and signature (notebooks/phase_d_kaggle.py:211-222, the XLA custom
 * call orthocache_compacted_attention(void* out, const void** inputs) and its
 * five-int32 CompactedAttentionDescriptor, same field order), so a caller
 * bound to that symbol links against this library unchanged.  Here the
 * buffers are device memory: inputs[0] q fp32 (seq_len_q, head_dim),
 * inputs[1] keys and inputs[2] values fp32 (num_blocks * block_size,
 * head_dim), inputs[3] block_mask int32 (num_blocks; nonzero = active);
 * inputs[4] points to the descriptor in host memory; out fp32 (seq_len_q,
 * head_dim).  Softmax attention of each query over the tokens of the active
 * blocks only, with scale 1/sqrt(head_dim); rows are zero when no block is
 * active.  Runs on the null stream and returns when out is written (the
 * reference's function is synchronous); allocates its workspace per call.
 * Supported: head_dim 32, 64, 128 or 256, any number of blocks (the
 * reference's own function holds at most 4096), seq_len_k = num_blocks *
 * block_size.  There is no return value, as
 * in the reference: on an error out is left unchanged and oc_last_error()
 * names it (it is not cleared on success). */
typedef struct oc_compacted_attention_desc {
  int32_t seq_len_q, seq_len_k, head_dim, block_size, num_blocks;
} oc_compacted_attention_desc;
void orthocache_compacted_attention(void* out, const void** inputs);

#ifdef __cplusplus
}
#endif

#endif /* ORTHOCACHE_HIP_H */
