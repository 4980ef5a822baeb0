// The reference's custom-call entry point, on the GPU.
//
// The reference binds its compacted attention into XLA as a C function
// (notebooks/phase_d_kaggle.py:211-222, orthocache_compacted_attention): one
// fp32 head, q (seq_len_q, head_dim), keys and values (num_blocks *
// block_size, head_dim), an int32 block mask, and a five-int32 descriptor;
// softmax attention over the tokens of the active blocks only, zeros when no
// block is active.  This is the same function over device buffers: the mask
// becomes one-byte flags (a one-pass conversion kernel), oc_mask_compact
// turns them into the active list and its count, and oc_attend attends it.
// It runs on the null stream and returns when out is written, as the
// reference's CPU function does, and it allocates its workspace per call.
#include "oc_api_internal.h"
#include "oc_kernels.h"

namespace {

__global__ __launch_bounds__(256) void mask_flags_kernel(const int32_t* in, uint8_t* out, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = in[i] != 0 ? 1 : 0;
}

size_t round256(size_t n) { return (n + 255) & ~size_t(255); }

int run(void* out, const void** inputs) {
  if (!out || !inputs) return oc::api_fail(OC_ERR_INVALID_ARGUMENT, "out and inputs must not be NULL");
  const auto* d = static_cast<const oc_compacted_attention_desc*>(inputs[4]);
  if (!d) return oc::api_fail(OC_ERR_INVALID_ARGUMENT, "inputs[4] (descriptor) is NULL");
  const int sq = d->seq_len_q, dim = d->head_dim, bs = d->block_size, nb = d->num_blocks;
  if (sq < 0 || dim <= 0 || bs <= 0 || nb < 0)
    return oc::api_fail(OC_ERR_INVALID_ARGUMENT, "descriptor: seq_len_q %d, head_dim %d, block_size %d, num_blocks %d",
                        sq, dim, bs, nb);
  if ((int64_t)d->seq_len_k != (int64_t)nb * bs)
    return oc::api_fail(OC_ERR_INVALID_ARGUMENT, "descriptor: seq_len_k %d != num_blocks * block_size (%lld)",
                        d->seq_len_k, (long long)nb * bs);
  hipStream_t s = nullptr;
  if (sq == 0) return OC_OK;
  if (nb == 0) {  // no block: every output row is zero
    int rc = oc::api_hip_check(hipMemsetAsync(out, 0, (size_t)sq * dim * sizeof(float), s), "memset");
    return rc ? rc : oc::api_hip_check(hipStreamSynchronize(s), "synchronize");
  }
  for (int i = 0; i < 4; ++i)
    if (!inputs[i]) return oc::api_fail(OC_ERR_INVALID_ARGUMENT, "inputs[%d] is NULL", i);
  if (reinterpret_cast<uintptr_t>(inputs[3]) % 4 != 0)
    return oc::api_fail(OC_ERR_INVALID_ARGUMENT, "block_mask (inputs[3]) must be 4-byte aligned");

  // Workspace: [flags | active list | count | attention partials].
  const size_t off_idx = round256((size_t)nb);
  const size_t off_cnt = off_idx + round256((size_t)nb * 4);
  const size_t off_att = off_cnt + 256;
  // One head, contiguous rows, the list that the compaction writes.
  static const int32_t marker = 0;  // stands in for the workspace while sizing
  oc_attend_args a{};
  a.q = inputs[0]; a.q_dtype = OC_F32;
  a.q_seg_stride = 0; a.q_tok_stride = dim; a.q_head_stride = dim;
  a.k = inputs[1]; a.v = inputs[2]; a.kv_dtype = OC_F32;
  a.k_tok_stride = dim; a.k_head_stride = dim; a.v_tok_stride = dim; a.v_head_stride = dim;
  a.head_dim = dim; a.num_kv_heads = 1; a.group = 1; a.sq = sq;
  a.block_size = bs; a.total_blocks = nb;
  a.num_segments = 1;
  a.out = out; a.out_dtype = OC_F32;
  a.out_seg_stride = 0; a.out_tok_stride = dim; a.out_head_stride = dim;
  a.indices = &marker; a.counts = &marker;
  const size_t att = oc_attend_workspace_size(&a);
  if (att == 0) {
    int32_t kernel = 0, nsplit = 0;
    const int rc = oc_attend_plan(&a, &kernel, &nsplit);  // the reason, when the arguments are refused
    if (rc) return rc;
  }
  char* ws = nullptr;
  int rc = oc::api_hip_check(hipMalloc(&ws, off_att + att), "hipMalloc");
  if (rc) return rc;
  int32_t* idx = reinterpret_cast<int32_t*>(ws + off_idx);
  int32_t* cnt = reinterpret_cast<int32_t*>(ws + off_cnt);
  hipLaunchKernelGGL(mask_flags_kernel, dim3((nb + 255) / 256), dim3(256), 0, s,
                     static_cast<const int32_t*>(inputs[3]), reinterpret_cast<uint8_t*>(ws), nb);
  rc = oc::api_hip_check(hipGetLastError(), "mask_flags_kernel");
  if (!rc) {
    oc_compact_args c{};
    c.mask_in = reinterpret_cast<const uint8_t*>(ws);
    c.mask_in_heads = 1;
    c.num_segments = 1;
    c.num_kv_heads = 1;
    c.total_blocks = nb;
    c.indices = idx;
    c.num_active = cnt;
    rc = oc_mask_compact(&c, s);
  }
  a.indices = idx;
  a.counts = cnt;
  if (!rc) rc = oc_attend(&a, ws + off_att, att, s);
  const int rs = oc::api_hip_check(hipStreamSynchronize(s), "synchronize");
  const hipError_t ef = hipFree(ws);
  if (rc) return rc;
  if (rs) return rs;
  return oc::api_hip_check(ef, "hipFree");
}

}  // namespace

extern "C" void orthocache_compacted_attention(void* out, const void** inputs) { (void)run(out, inputs); }
