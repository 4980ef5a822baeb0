// C ABI of liborthocache_hip.so: argument validation, workspace layout and
// kernel launches.  Declarations and semantics: include/orthocache_hip.h.
#include "oc_api_internal.h"
#include "oc_kernels.h"
#include "orthocache_hip.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>


namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(OC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return OC_OK;
}

bool valid_dtype(int dt) { return dt == OC_F32 || dt == OC_BF16 || dt == OC_F16; }
int esize(int dt) { return dt == OC_F32 ? 4 : 2; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// Workspaces are carved at 256-byte offsets and read with 16-byte vector loads.
bool aligned256(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 255u) == 0; }
size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

int check_kv(const char* name, const void* p, int dt, int64_t tok_stride, int64_t head_stride, int head_dim) {
  if (!p) return fail(OC_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (!valid_dtype(dt)) return fail(OC_ERR_INVALID_ARGUMENT, "%s: unknown dtype %d", name, dt);
  const int es = esize(dt);
  if (!aligned16(p) || (tok_stride * es) % 16 || (head_stride * es) % 16 || (head_dim * es) % 16)
    return fail(OC_ERR_INVALID_ARGUMENT,
                "%s must be 16-byte aligned with 16-byte multiple strides (tok %lld, head %lld, dim %d)",
                name, (long long)tok_stride, (long long)head_stride, head_dim);
  return OC_OK;
}

// The scoring kernel addresses a 64-row group of a tile with 32-bit lane
// offsets: 64 key rows must span less than 2 GiB.
bool score_rows_fit(int64_t tok_stride, int dt) { return tok_stride >= 0 && tok_stride * esize(dt) * 64 < (1LL << 31); }

float logit_scale_for(int head_dim) { return (float)(1.4426950408889634 / std::sqrt((double)head_dim)); }

// q as the 16-byte row loads of the logits and attention kernels read it.
int check_q16(const void* q, int dt, int64_t seg_stride, int64_t tok_stride, int64_t head_stride) {
  const int qs = esize(dt);
  if (!aligned16(q) || (tok_stride * qs) % 16 || (head_stride * qs) % 16 || (seg_stride * qs) % 16)
    return fail(OC_ERR_INVALID_ARGUMENT, "q must be 16-byte aligned with 16-byte multiple strides");
  return OC_OK;
}

}  // namespace

extern "C" {

const char* oc_last_error(void) { return g_err; }
int oc_abi_version(void) { return OC_ABI_VERSION; }

int oc_fwht512(const oc_fwht_args* a, void* stream) {
  if (!a) return fail(OC_ERR_INVALID_ARGUMENT, "args is NULL");
  if (!a->x || !a->y) return fail(OC_ERR_INVALID_ARGUMENT, "x or y is NULL");
  if (!valid_dtype(a->x_dtype) || !valid_dtype(a->y_dtype))
    return fail(OC_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (a->n_cols < 0 || a->n_batch < 0) return fail(OC_ERR_INVALID_ARGUMENT, "negative size");
  if ((a->n_cols + 31) / 32 * a->n_batch > 0x7fffffffLL) return fail(OC_ERR_UNSUPPORTED, "too many tiles");
  oc::FwhtParams p{a->x, a->x_dtype, a->x_batch_stride, a->x_row_stride, a->y, a->y_dtype,
                   a->y_batch_stride, a->y_row_stride, a->n_cols, a->n_batch};
  return hip_check(oc::launch_fwht(p, (hipStream_t)stream), "oc_fwht512");
}

int oc_band_energy(const float* spec, int32_t num_blocks, int32_t num_heads, int32_t head_dim,
                   int32_t s0, int32_t s1, float* out, void* stream) {
  if (!spec || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (num_blocks < 0 || num_heads <= 0 || head_dim <= 0 || s0 < 0 || s1 > OC_BLOCK || s0 > s1)
    return fail(OC_ERR_INVALID_ARGUMENT, "bad band [%d, %d) or shape", s0, s1);
  oc::BandParams p{spec, num_blocks, num_heads, head_dim, s0, s1, out};
  return hip_check(oc::launch_band_energy(p, (hipStream_t)stream), "oc_band_energy");
}

int oc_block_energy(const void* keys, int32_t keys_dtype, int64_t tok_stride, int64_t head_stride,
                    int32_t head_dim, int32_t num_kv_heads, int32_t num_blocks, int32_t block_size,
                    float* out, void* stream) {
  if (!keys || !out) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (!valid_dtype(keys_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (head_dim <= 0 || num_kv_heads <= 0 || num_blocks < 0 || block_size <= 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "bad shape");
  oc::EnergyParams p{keys, keys_dtype, tok_stride, head_stride, head_dim, num_kv_heads, num_blocks,
                     block_size, out};
  return hip_check(oc::launch_block_energy(p, (hipStream_t)stream), "oc_block_energy");
}

int oc_score_blocks(const oc_score_args* a, void* stream) {
  if (!a) return fail(OC_ERR_INVALID_ARGUMENT, "args is NULL");
  int rc = check_kv("keys", a->keys, a->keys_dtype, a->keys_tok_stride, a->keys_head_stride, a->head_dim);
  if (rc) return rc;
  if (!oc::score_supported(a->keys_dtype, a->head_dim))
    return fail(OC_ERR_UNSUPPORTED, "head_dim %d unsupported for dtype %d (need head_dim/(16/esize) in {8..128} power of 2)",
                a->head_dim, a->keys_dtype);
  if (a->num_kv_heads <= 0 || a->total_blocks < 0) return fail(OC_ERR_INVALID_ARGUMENT, "bad shape");
  if ((int64_t)a->total_blocks * a->num_kv_heads > 0x7fffffffLL) return fail(OC_ERR_UNSUPPORTED, "too many tiles");
  if (!score_rows_fit(a->keys_tok_stride, a->keys_dtype))
    return fail(OC_ERR_UNSUPPORTED, "keys token stride %lld too large (64 rows must span < 2 GiB)",
                (long long)a->keys_tok_stride);
  if (a->cu_blocks && a->num_segments <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "cu_blocks needs num_segments > 0");
  if (a->q) {
    if (!valid_dtype(a->q_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "q: unknown dtype");
    if (a->q_dtype != a->keys_dtype && a->q_dtype != OC_F32)
      return fail(OC_ERR_UNSUPPORTED, "q dtype must equal the key dtype or be fp32");
    if (a->sq < 0 || a->group <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "bad sq/group");
    if (a->cu_blocks && a->num_segments > 4096)
      return fail(OC_ERR_UNSUPPORTED, "at most 4096 segments per call");
  }
  if (a->pages && a->num_pages <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "pages given with num_pages %d", a->num_pages);
  if (a->logits) {
    if (!a->q) return fail(OC_ERR_INVALID_ARGUMENT, "logits need q");
    if (!oc::score_logits_supported(a->keys_dtype, a->head_dim, a->sq * a->group))
      return fail(OC_ERR_UNSUPPORTED, "logits: %d query rows per kv head, head_dim %d unsupported (1..%d rows)",
                  a->sq * a->group, a->head_dim, oc::kLogitsMaxQ);
    if (!aligned16(a->logits)) return fail(OC_ERR_INVALID_ARGUMENT, "logits must be 16-byte aligned");
    rc = check_q16(a->q, a->q_dtype, a->cu_blocks ? a->q_seg_stride : 0, a->q_tok_stride, a->q_head_stride);
    if (rc) return rc;
  }
  if (a->mask && (!a->q || !a->tau_max))
    return fail(OC_ERR_INVALID_ARGUMENT, "the two-gate mask needs q and tau_max");
  oc::ScoreParams p{a->keys, a->keys_tok_stride, a->keys_head_stride, a->keys_dtype, a->head_dim,
                    a->num_kv_heads, a->total_blocks, a->cu_blocks, a->cu_blocks ? a->num_segments : 1,
                    a->q, a->q_dtype, a->q_seg_stride, a->q_tok_stride, a->q_head_stride, a->sq, a->group,
                    a->tau_max, a->zeta, a->dc, a->e_low, a->e_mid, a->e_high, a->e_ac, a->pages,
                    a->num_pages, a->logits, logit_scale_for(a->head_dim),
                    oc::GateParams{a->mask, nullptr, a->tau_arr, a->tau, a->zeta_max_arr, a->zeta_max}};
  return hip_check(oc::launch_score(p, (hipStream_t)stream), "oc_score_blocks");
}

int32_t oc_query_bound_tiles(int32_t sq, int32_t group) {
  const int qt = oc::bound_query_tile();
  return (sq * group + qt - 1) / qt;
}

int oc_query_bounds(const oc_bound_args* a, void* stream) {
  if (!a) return fail(OC_ERR_INVALID_ARGUMENT, "args is NULL");
  if (!a->dc || !a->e_ac || !a->q) return fail(OC_ERR_INVALID_ARGUMENT, "NULL input");
  if (!valid_dtype(a->q_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "q: unknown dtype");
  if (a->head_dim <= 0 || a->head_dim > 1024 || a->num_kv_heads <= 0 || a->num_blocks < 0 || a->sq < 0 || a->group <= 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "bad shape");
  const int bbt = oc::bound_block_tile();
  const int64_t grid = (int64_t)oc_query_bound_tiles(a->sq, a->group) * ((a->num_blocks + bbt - 1) / bbt) * a->num_kv_heads;
  if (grid > 0x7fffffffLL) return fail(OC_ERR_UNSUPPORTED, "too many tiles");
  oc::BoundParams p{a->dc, a->e_ac, a->q, a->q_dtype, a->q_tok_stride, a->q_head_stride, a->sq, a->group,
                    a->head_dim, a->num_kv_heads, a->num_blocks, a->bounds, a->tau_part};
  return hip_check(oc::launch_bound(p, (hipStream_t)stream), "oc_query_bounds");
}

int oc_mask_compact(const oc_compact_args* a, void* stream) {
  if (!a) return fail(OC_ERR_INVALID_ARGUMENT, "args is NULL");
  if (!a->mask_in && !a->tau_max) return fail(OC_ERR_INVALID_ARGUMENT, "need tau_max or mask_in");
  if (a->mask_in && a->mask_in_heads != 1 && a->mask_in_heads != a->num_kv_heads)
    return fail(OC_ERR_INVALID_ARGUMENT, "mask_in_heads must be 1 or num_kv_heads");
  if (a->num_kv_heads <= 0 || a->num_kv_heads > 16384 || a->total_blocks < 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "bad shape");
  if (a->tau_max && a->tau_parts <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "tau_parts must be > 0");
  if (a->cu_blocks && a->num_segments <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "cu_blocks needs num_segments > 0");
  if (a->indices && !a->num_active) return fail(OC_ERR_INVALID_ARGUMENT, "indices needs num_active");
  if (a->head_indices && !a->head_num_active) return fail(OC_ERR_INVALID_ARGUMENT, "head_indices needs head_num_active");
  oc::CompactParams p{a->tau_max, a->tau_parts, a->zeta, a->mask_in, a->mask_in_heads,
                      a->tau_arr, a->tau, a->zeta_max_arr, a->zeta_max,
                      a->cu_blocks, a->cu_blocks ? a->num_segments : 1, a->total_blocks,
                      a->num_kv_heads, a->total_blocks,
                      a->mask_out, a->active_out, a->indices, a->num_active,
                      a->head_indices, a->head_num_active, a->head_uniform, a->empty_head_all};
  return hip_check(oc::launch_compact(p, (hipStream_t)stream), "oc_mask_compact");
}

int oc_copy_blocks(const void* src, void* dst, const int32_t* indices, const int32_t* num_active,
                   int32_t num_blocks, int64_t block_bytes, int32_t scatter, void* stream) {
  if (!src || !dst || !indices || !num_active) return fail(OC_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (num_blocks < 0 || block_bytes <= 0 || block_bytes % 16 || !aligned16(src) || !aligned16(dst))
    return fail(OC_ERR_INVALID_ARGUMENT, "blocks must be 16-byte aligned multiples of 16 bytes");
  if (num_blocks > 65535) return fail(OC_ERR_UNSUPPORTED, "more than 65535 blocks");
  oc::CopyParams p{src, dst, indices, num_active, num_blocks, block_bytes, scatter};
  return hip_check(oc::launch_copy_blocks(p, (hipStream_t)stream), "oc_copy_blocks");
}

}  // extern "C"

namespace {

int make_attend_params(const oc_attend_args* a, oc::AttendParams& p) {
  // With scoring-pass logits the keys are not read.
  int rc = a->logits ? OC_OK : check_kv("k", a->k, a->kv_dtype, a->k_tok_stride, a->k_head_stride, a->head_dim);
  if (rc) return rc;
  rc = check_kv("v", a->v, a->kv_dtype, a->v_tok_stride, a->v_head_stride, a->head_dim);
  if (rc) return rc;
  if (!oc::attend_supported(a->kv_dtype, a->head_dim))
    return fail(OC_ERR_UNSUPPORTED, "attention: head_dim %d unsupported for dtype %d", a->head_dim, a->kv_dtype);
  if (!a->q || !a->out) return fail(OC_ERR_INVALID_ARGUMENT, "q or out is NULL");
  if (!valid_dtype(a->q_dtype) || !valid_dtype(a->out_dtype)) return fail(OC_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (a->q_dtype != a->kv_dtype && a->q_dtype != OC_F32)
    return fail(OC_ERR_UNSUPPORTED, "q dtype must equal the kv dtype or be fp32");
  rc = check_q16(a->q, a->q_dtype, a->q_seg_stride, a->q_tok_stride, a->q_head_stride);
  if (rc) return rc;
  if (a->logits) {
    if (a->block_size != OC_BLOCK)
      return fail(OC_ERR_INVALID_ARGUMENT, "logits: block_size must be %d", OC_BLOCK);
    if (a->sq * a->group < 1 || a->sq * a->group > oc::kLogitsMaxQ)
      return fail(OC_ERR_UNSUPPORTED, "logits: %d query rows per kv head (1..%d)", a->sq * a->group, oc::kLogitsMaxQ);
    if (!aligned16(a->logits)) return fail(OC_ERR_INVALID_ARGUMENT, "logits must be 16-byte aligned");
  }
  if (a->num_kv_heads <= 0 || a->group <= 0 || a->sq < 0 || a->block_size <= 0 || a->total_blocks < 0)
    return fail(OC_ERR_INVALID_ARGUMENT, "bad shape");
  const int nseg = a->cu_blocks ? a->num_segments : 1;
  if (nseg <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "num_segments must be > 0");
  if ((int64_t)nseg * a->num_kv_heads > oc::kMaxLists)
    return fail(OC_ERR_UNSUPPORTED, "segments x kv heads = %lld exceeds %d", (long long)nseg * a->num_kv_heads, oc::kMaxLists);
  if (a->mask) {
    if (a->cu_blocks)
      return fail(OC_ERR_UNSUPPORTED, "mask input: one segment without cu_blocks (use oc_mask_compact lists for several)");
    if (a->per_head || a->uniform) return fail(OC_ERR_UNSUPPORTED, "mask input: unified lists only");
    if (a->total_blocks < 1 || a->total_blocks > oc::kMaxLists)
      return fail(OC_ERR_UNSUPPORTED, "mask input: 1..%d blocks, got %d", oc::kMaxLists, a->total_blocks);
    if (!a->indices_out || !a->num_active_out)
      return fail(OC_ERR_INVALID_ARGUMENT, "mask input needs indices_out and num_active_out");
    const int H = a->num_kv_heads;
    const int al = (H % 16 == 0) ? 16 : ((H % 4 == 0) ? 4 : 1);
    if ((reinterpret_cast<uintptr_t>(a->mask) % al) != 0)
      return fail(OC_ERR_INVALID_ARGUMENT, "mask must be %d-byte aligned for %d kv heads", al, H);
  } else if (!a->indices || !a->counts) {
    return fail(OC_ERR_INVALID_ARGUMENT, "indices/counts are NULL");
  }
  if (a->pages && a->num_pages <= 0) return fail(OC_ERR_INVALID_ARGUMENT, "pages given with num_pages %d", a->num_pages);
  const int chunk = oc::attend_chunk(a->kv_dtype, a->head_dim, a->sq * a->group);
  p = oc::AttendParams{};
  p.q = a->q; p.q_dtype = a->q_dtype;
  p.q_seg_stride = a->q_seg_stride; p.q_tok_stride = a->q_tok_stride; p.q_head_stride = a->q_head_stride;
  p.k = a->k; p.v = a->v; p.kv_dtype = a->kv_dtype;
  p.k_tok_stride = a->k_tok_stride; p.k_head_stride = a->k_head_stride;
  p.v_tok_stride = a->v_tok_stride; p.v_head_stride = a->v_head_stride;
  p.head_dim = a->head_dim; p.num_kv_heads = a->num_kv_heads; p.group = a->group; p.sq = a->sq;
  p.block_size = a->block_size; p.total_blocks = a->total_blocks;
  p.cu_blocks = a->cu_blocks; p.num_segments = nseg;
  p.indices = a->indices; p.counts = a->counts; p.per_head = a->per_head; p.uniform = a->uniform;
  p.logit_scale = logit_scale_for(a->head_dim);
  p.chunk = chunk; p.nchunk = (a->block_size + chunk - 1) / chunk;
  p.part_o = nullptr; p.part_ml = nullptr;
  p.out = a->out; p.out_dtype = a->out_dtype;
  p.out_seg_stride = a->out_seg_stride; p.out_tok_stride = a->out_tok_stride; p.out_head_stride = a->out_head_stride;
  p.pages = a->pages; p.num_pages = a->num_pages;
  p.logits = a->logits;
  p.keep = a->mask;
  p.list_out = a->indices_out;
  p.count_out = a->num_active_out;
  if (a->mask) {
    p.indices = a->indices_out;
    p.counts = a->num_active_out;  // the combine reads the count the attention wrote
  }
  p.prefill = oc::prefill_supported(a->kv_dtype, a->q_dtype, a->head_dim, a->sq * a->group, a->block_size) ? 1 : 0;
  // The prefill kernel keeps per-thread offsets inside a 64-token tile in 32 bits.
  if (a->k_tok_stride >= (1 << 24) || a->v_tok_stride >= (1 << 24) || a->logits) p.prefill = 0;
  if (a->mask && p.prefill)
    return fail(OC_ERR_UNSUPPORTED, "mask input: decode shapes only (%d query rows per kv head take the matrix-core "
                "kernels; compact with oc_mask_compact)", a->sq * a->group);
  p.nsplit = p.prefill ? oc::prefill_nsplit(p) : 0;
  return OC_OK;
}

// Partial-result bytes: [o | (m, l)], for the partials the launch of these
// parameters writes (decode: one (kQG x D) + (kQG x 2) pair per slot).
size_t attend_part_o_bytes(const oc::AttendParams& p) {
  if (p.prefill) return align256((size_t)oc::prefill_partial_floats(p) * sizeof(float));
  return align256((size_t)oc::attend_partial_slots(p) * oc::kQG * p.head_dim * sizeof(float));
}

size_t attend_part_ml_bytes(const oc::AttendParams& p) {
  if (p.prefill) return align256((size_t)oc::prefill_partial_floats(p) / p.head_dim * 2 * sizeof(float));
  return align256((size_t)oc::attend_partial_slots(p) * oc::kQG * 2 * sizeof(float));
}

size_t attend_ws(const oc::AttendParams& p) { return attend_part_o_bytes(p) + attend_part_ml_bytes(p); }

void attend_bind_ws(oc::AttendParams& p, void* ws) {
  char* w = static_cast<char*>(ws);
  p.part_o = reinterpret_cast<float*>(w);
  p.part_ml = reinterpret_cast<float*>(w + attend_part_o_bytes(p));
}

}  // namespace

extern "C" {

size_t oc_attend_workspace_size(const oc_attend_args* a) {
  oc::AttendParams p;
  if (!a || make_attend_params(a, p)) return 0;
  return attend_ws(p);
}

int oc_attend_plan(const oc_attend_args* a, int32_t* kernel, int32_t* nsplit) {
  if (!a || !kernel || !nsplit) return fail(OC_ERR_INVALID_ARGUMENT, "NULL argument");
  oc::AttendParams p;
  const int rc = make_attend_params(a, p);
  if (rc) return rc;
  *kernel = p.prefill ? OC_ATTEND_PREFILL_MFMA : OC_ATTEND_DECODE;
  *nsplit = p.prefill ? p.nsplit : 0;
  return OC_OK;
}

int oc_attend(const oc_attend_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  if (!a) return fail(OC_ERR_INVALID_ARGUMENT, "args is NULL");
  oc::AttendParams p;
  int rc = make_attend_params(a, p);
  if (rc) return rc;
  const size_t need = attend_ws(p);
  if (need && (!workspace || workspace_bytes < need))
    return fail(OC_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", workspace_bytes, need);
  if (need && !aligned256(workspace)) return fail(OC_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  attend_bind_ws(p, workspace);
  return hip_check(oc::launch_attend(p, (hipStream_t)stream), "oc_attend");
}

}  // extern "C"

namespace {

struct LayerWs {
  size_t tau, zeta, idx, cnt, keep, logits, attend, total;
};

// True when the layer's scoring pass writes the two-gate keep flags and the
// attention derives the list from them (one segment of at most kMaxLists
// blocks): no compaction launch.
bool layer_uses_keep(const oc_layer_args* a) {
  return a->cu_blocks == nullptr && a->total_blocks >= 1 && a->total_blocks <= oc::kMaxLists;
}

// True when the layer's scoring pass also writes the attention logits (the
// attention then reads values only).  fp16 keys with one query row at
// head_dim 256, or with fp32 queries and 3-4 rows at head_dim 128, are left
// out: those logit variants of the scoring kernel hold one wave per SIMD, and
// the layer measured faster with the attention reading the keys itself
// (150.7 -> 106.4 us and 74.0 -> 45.4 us for 64K tokens on one MI355X).
bool layer_uses_logits(const oc_layer_args* a) {
  const int nq = a->sq * a->group;
  if (a->kv_dtype == OC_F16 &&
      ((a->head_dim == 256 && nq == 1) || (a->q_dtype == OC_F32 && a->head_dim == 128 && nq > 2)))
    return false;
  return oc::score_logits_supported(a->kv_dtype, a->head_dim, nq);
}

// Workspace: [tau_max | zeta | indices | num_active | keep | logits | attention partials].
LayerWs layer_ws_layout(const oc_layer_args* a, size_t attend_bytes, bool logits) {
  LayerWs w{};
  const size_t tiles = (size_t)a->total_blocks * a->num_kv_heads;
  const int nseg = a->cu_blocks ? a->num_segments : 1;
  size_t off = 0;
  w.tau = off; off += a->tau_max ? 0 : align256(tiles * 4);
  w.zeta = off; off += a->zeta ? 0 : align256(tiles * 4);
  w.idx = off; off += a->indices ? 0 : align256((size_t)a->total_blocks * 4);
  w.cnt = off; off += a->num_active ? 0 : align256((size_t)nseg * 4);
  w.keep = off; off += layer_uses_keep(a) ? align256(tiles) : 0;
  w.logits = off;
  off += logits ? align256(tiles * OC_BLOCK * oc::logits_nq_pad(a->sq * a->group) * sizeof(float)) : 0;
  w.attend = off; off += attend_bytes;
  w.total = off;
  return w;
}

oc_attend_args layer_attend_args(const oc_layer_args* a) {
  oc_attend_args t{};
  t.q = a->q; t.q_dtype = a->q_dtype;
  t.q_seg_stride = a->q_seg_stride; t.q_tok_stride = a->q_tok_stride; t.q_head_stride = a->q_head_stride;
  t.k = a->k; t.v = a->v; t.kv_dtype = a->kv_dtype;
  t.k_tok_stride = a->k_tok_stride; t.k_head_stride = a->k_head_stride;
  t.v_tok_stride = a->v_tok_stride; t.v_head_stride = a->v_head_stride;
  t.head_dim = a->head_dim; t.num_kv_heads = a->num_kv_heads; t.group = a->group; t.sq = a->sq;
  t.block_size = OC_BLOCK; t.total_blocks = a->total_blocks;
  t.cu_blocks = a->cu_blocks; t.num_segments = a->num_segments;
  t.indices = reinterpret_cast<const int32_t*>(16);  // placeholder: validated before binding
  t.counts = reinterpret_cast<const int32_t*>(16);
  t.per_head = 0; t.uniform = nullptr;
  t.out = a->out; t.out_dtype = a->out_dtype;
  t.out_seg_stride = a->out_seg_stride; t.out_tok_stride = a->out_tok_stride; t.out_head_stride = a->out_head_stride;
  t.pages = a->pages; t.num_pages = a->num_pages;
  return t;
}

// The layer's attention parameters, with the scoring-pass logits and the
// keep flags marked present exactly when the layer will pass them: the
// attention's form, and with it the partial count and the workspace, depends
// on both.  The markers are never dereferenced; decode_layer_impl replaces
// them with the workspace addresses before launching.
int layer_attend_params(const oc_layer_args* a, bool logits, oc::AttendParams& p) {
  oc_attend_args t = layer_attend_args(a);
  const int rc = make_attend_params(&t, p);
  if (rc) return rc;
  static const float marker = 0.f;
  p.logits = logits ? &marker : nullptr;
  p.keep = layer_uses_keep(a) ? reinterpret_cast<const uint8_t*>(&marker) : nullptr;
  return OC_OK;
}

}  // namespace

extern "C" {

size_t oc_decode_layer_workspace_size(const oc_layer_args* a) {
  if (!a) return 0;
  const bool logits = layer_uses_logits(a);
  oc::AttendParams p;
  if (layer_attend_params(a, logits, p)) return 0;
  return layer_ws_layout(a, attend_ws(p), logits).total;
}

}  // extern "C"

namespace {

// The layer body shared by oc_decode_layer (scores from the keys) and
// oc_decode_layer_cached (bounds from write-time block statistics).
int decode_layer_impl(const oc_layer_args* a, const oc_block_stats* st, void* workspace, size_t workspace_bytes,
                      void* stream, const char* name) {
  if (!a) return fail(OC_ERR_INVALID_ARGUMENT, "args is NULL");
  const bool use_logits = !st && layer_uses_logits(a);
  oc::AttendParams ap;
  int rc = layer_attend_params(a, use_logits, ap);
  if (rc) return rc;
  if (st) {
    if (!st->dc || !st->e_ac || !st->zeta) return fail(OC_ERR_INVALID_ARGUMENT, "%s: NULL block statistics", name);
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256 && a->head_dim != 512)
      return fail(OC_ERR_UNSUPPORTED, "%s: head_dim %d unsupported (64, 128, 256 or 512)", name, a->head_dim);
  } else if (!oc::score_supported(a->kv_dtype, a->head_dim)) {
    return fail(OC_ERR_UNSUPPORTED, "scores: head_dim %d unsupported", a->head_dim);
  } else if (!score_rows_fit(a->k_tok_stride, a->kv_dtype)) {
    return fail(OC_ERR_UNSUPPORTED, "keys token stride %lld too large (64 rows must span < 2 GiB)",
                (long long)a->k_tok_stride);
  }
  if (a->q_dtype != a->kv_dtype && a->q_dtype != OC_F32)
    return fail(OC_ERR_UNSUPPORTED, "q dtype must equal the kv dtype or be fp32");
  if (a->sq * a->group > 16)
    return fail(OC_ERR_UNSUPPORTED, "decode layer takes at most 16 queries per kv head (sq * group)");
  const int nseg = a->cu_blocks ? a->num_segments : 1;
  if (a->cu_blocks && nseg > 4096) return fail(OC_ERR_UNSUPPORTED, "at most 4096 segments per call");
  const LayerWs w = layer_ws_layout(a, attend_ws(ap), use_logits);
  if (w.total && (!workspace || workspace_bytes < w.total))
    return fail(OC_ERR_WORKSPACE, "workspace %zu bytes < %zu needed", workspace_bytes, w.total);
  if (w.total && !aligned256(workspace)) return fail(OC_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned", name);
  char* ws = static_cast<char*>(workspace);
  float* tau_max = a->tau_max ? a->tau_max : reinterpret_cast<float*>(ws + w.tau);
  const float* zeta_in;
  int32_t* idx = a->indices ? a->indices : reinterpret_cast<int32_t*>(ws + w.idx);
  int32_t* cnt = a->num_active ? a->num_active : reinterpret_cast<int32_t*>(ws + w.cnt);
  const hipStream_t s = (hipStream_t)stream;
  // One segment: the scoring pass writes the keep flags and the attention
  // derives the list (and writes indices / num_active) itself.
  const bool use_keep = layer_uses_keep(a);
  const oc::GateParams gate{use_keep ? reinterpret_cast<uint8_t*>(ws + w.keep) : nullptr, a->mask,
                            a->tau_arr, a->tau, a->zeta_max_arr, a->zeta_max};

  // 1. Scores: from the keys, or bounds from the cached statistics.
  if (st) {
    oc::CachedBoundParams cp{};
    cp.dc = st->dc; cp.e_ac = st->e_ac;
    cp.q = a->q; cp.q_dtype = a->q_dtype;
    cp.q_seg_stride = a->q_seg_stride; cp.q_tok_stride = a->q_tok_stride; cp.q_head_stride = a->q_head_stride;
    cp.sq = a->sq; cp.group = a->group; cp.head_dim = a->head_dim; cp.num_kv_heads = a->num_kv_heads;
    cp.total_blocks = a->total_blocks; cp.cu_blocks = a->cu_blocks; cp.num_segments = nseg;
    cp.tau_max = tau_max;
    cp.zeta = st->zeta;
    if (use_keep) cp.gate = gate;
    rc = hip_check(oc::launch_cached_bound(cp, s), "oc_decode_layer_cached bounds");
    if (rc) return rc;
    zeta_in = st->zeta;
  } else {
    float* zeta = a->zeta ? a->zeta : reinterpret_cast<float*>(ws + w.zeta);
    oc::ScoreParams sp{};
    sp.k = a->k; sp.k_tok_stride = a->k_tok_stride; sp.k_head_stride = a->k_head_stride; sp.k_dtype = a->kv_dtype;
    sp.head_dim = a->head_dim; sp.num_kv_heads = a->num_kv_heads; sp.total_blocks = a->total_blocks;
    sp.cu_blocks = a->cu_blocks; sp.num_segments = nseg;
    sp.q = a->q; sp.q_dtype = a->q_dtype;
    sp.q_seg_stride = a->q_seg_stride; sp.q_tok_stride = a->q_tok_stride; sp.q_head_stride = a->q_head_stride;
    sp.sq = a->sq; sp.group = a->group;
    sp.tau_max = tau_max; sp.zeta = zeta;
    sp.pages = a->pages; sp.num_pages = a->num_pages;
    if (use_logits) {
      sp.logits = reinterpret_cast<float*>(ws + w.logits);
      sp.logit_scale = ap.logit_scale;
      ap.logits = sp.logits;
    }
    if (use_keep) sp.gate = gate;
    rc = hip_check(oc::launch_score(sp, s), "oc_decode_layer scores");
    if (rc) return rc;
    zeta_in = zeta;
  }

  // 2. Mask + compaction (several segments; one segment takes the keep flags).
  if (use_keep) {
    ap.keep = gate.keep;
    ap.list_out = idx;
    ap.count_out = cnt;
  } else {
    ap.keep = nullptr;
    oc::CompactParams cp{};
    cp.tau_max = tau_max; cp.tau_parts = 1; cp.zeta = zeta_in;
    cp.tau_arr = a->tau_arr; cp.tau = a->tau; cp.zmax_arr = a->zeta_max_arr; cp.zeta_max = a->zeta_max;
    cp.cu_blocks = a->cu_blocks; cp.num_segments = nseg; cp.nb_single = a->total_blocks;
    cp.num_kv_heads = a->num_kv_heads; cp.total_blocks = a->total_blocks;
    cp.mask_out = a->mask; cp.indices = idx; cp.num_active = cnt;
    rc = hip_check(oc::launch_compact(cp, s), "oc_decode_layer compaction");
    if (rc) return rc;
  }

  // 3. Attention (+ combine).
  ap.indices = idx;
  ap.counts = cnt;
  attend_bind_ws(ap, ws + w.attend);
  return hip_check(oc::launch_attend(ap, s), name);
}

}  // namespace

extern "C" {

int oc_decode_layer(const oc_layer_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  return decode_layer_impl(a, nullptr, workspace, workspace_bytes, stream, "oc_decode_layer");
}

size_t oc_decode_layer_cached_workspace_size(const oc_layer_args* a) {
  if (!a) return 0;
  oc::AttendParams p;
  if (layer_attend_params(a, false, p)) return 0;
  return layer_ws_layout(a, attend_ws(p), false).total;
}

int oc_decode_layer_cached(const oc_layer_args* a, const oc_block_stats* stats, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!stats) return fail(OC_ERR_INVALID_ARGUMENT, "stats is NULL");
  return decode_layer_impl(a, stats, workspace, workspace_bytes, stream, "oc_decode_layer_cached");
}

}  // extern "C"

namespace oc {

int api_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int api_hip_check(hipError_t e, const char* what) { return hip_check(e, what); }

int decode_layer_run(const oc_layer_args* a, void* workspace, size_t workspace_bytes, void* stream,
                     const char* name) {
  return decode_layer_impl(a, nullptr, workspace, workspace_bytes, stream, name);
}

}  // namespace oc
