/*
 * lmcache_amd.h — C ABI of the MI355X (gfx950) KV-transfer, CacheGen and
 * fused K-RoPE library (liblmcache_amd.so).
 *
 * Every entry point takes plain pointers, sizes and a hipStream_t passed as
 * `void *`; there are no torch types in any signature.  Tensors cross the
 * boundary as `lmc_tensor` descriptors (data pointer, dtype, device, sizes,
 * strides — the same facts the reference host code reads from a
 * torch::Tensor).  Work is enqueued asynchronously on `stream`; callers keep
 * every buffer alive until the stream has drained, exactly as the reference's
 * ops require (csrc/mem_kernels.cpp:96-108 captures raw pointers in the
 * launch lambda).
 *
 * Return value of every function: one of the LMC_* status codes below.  On a
 * non-zero status `lmc_last_error()` returns a thread-local message.  The
 * Python layer raises ValueError / RuntimeError / NotImplementedError for
 * LMC_ERR_VALUE / LMC_ERR_RUNTIME (and LMC_ERR_HIP) / LMC_ERR_NOT_IMPLEMENTED,
 * the exception types the reference raises (csrc/utils.cpp:903-966,
 * TORCH_CHECK sites, csrc/mem_kernels.cpp:255-263).
 */
#ifndef LMCACHE_AMD_H
#define LMCACHE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum lmc_status {
  LMC_OK = 0,
  LMC_ERR_VALUE = 1,           /* bad argument value (Python ValueError)        */
  LMC_ERR_RUNTIME = 2,         /* failed check (Python RuntimeError)            */
  LMC_ERR_NOT_IMPLEMENTED = 3, /* Python NotImplementedError                    */
  LMC_ERR_HIP = 4              /* HIP runtime error (Python RuntimeError)       */
};

enum lmc_dtype {
  LMC_U8 = 0,
  LMC_I8 = 1,
  LMC_I16 = 2,
  LMC_I32 = 3,
  LMC_I64 = 4,
  LMC_F16 = 5,
  LMC_BF16 = 6,
  LMC_F32 = 7
};

/* KV cache storage formats; the integer values are the reference's
 * KVCacheFormat contract (lmcache_ascend/v1/kv_format.py:13-83). */
enum lmc_kv_format {
  LMC_FMT_UNDEFINED = 0,
  LMC_FMT_MERGED_KV = 1,
  LMC_FMT_SEPARATE_KV = 2,
  LMC_FMT_MLA_KV = 3,
  LMC_FMT_DSA_KV = 4,
  LMC_FMT_MLA_LATENT = 5,
  LMC_FMT_DSA_INDEX = 6
};

#define LMC_MAX_DIMS 6

/* A strided tensor.  `data` is the address of element 0: a device address
 * when device >= 0, a host address when device == -1 (pinned host memory is
 * translated to its device mapping by the library, like the reference's
 * get_kernel_ptr, csrc/utils.h:32-51).  Strides are in elements. */
typedef struct lmc_tensor {
  void *data;
  int32_t dtype;
  int32_t device;
  int32_t ndim;
  int32_t reserved;
  int64_t sizes[LMC_MAX_DIMS];
  int64_t strides[LMC_MAX_DIMS];
} lmc_tensor;

/* Thread-local text of the last error raised on this thread. */
const char *lmc_last_error(void);

/* Library version string. */
const char *lmc_version(void);

/* ------------------------------------------------------------------------
 * Paged-KV gather / scatter
 * ------------------------------------------------------------------------ */

/* Replaces multi_layer_kv_transfer (csrc/mem_kernels.cpp:75-111; planner
 * csrc/utils.cpp:29-154; pybind csrc/pybind.cpp:364).
 * key_value: LMCache memory object, [kv, L, T, W] (device or pinned host).
 * key_value_ptrs: device int64 table of paged-cache base addresses.
 * direction != 0: paged -> key_value (store); 0: key_value -> paged. */
int lmc_multi_layer_kv_transfer(const lmc_tensor *key_value,
                                const lmc_tensor *key_value_ptrs,
                                const lmc_tensor *slot_mapping,
                                int32_t paged_device, int64_t page_buffer_size,
                                int32_t direction, int32_t use_mla,
                                int32_t kvcache_format, int64_t k_hidden_dims,
                                int64_t v_hidden_dims, int64_t dsa_hidden_dims,
                                void *stream);

/* Batched form of lmc_multi_layer_kv_transfer: `n_chunks` memory objects
 * (`chunks[i]`, each [kv, L, T_i, W]) that cover the token ranges
 * [token_starts[i], token_starts[i] + T_i) of `slot_mapping`, moved by one
 * kernel launch per 64 chunks.  It replaces the per-chunk launch loop of the
 * reference's caller (lmcache_ascend/v1/npu_connector/npu_connectors.py:
 * 1278-1284 and 1465-1469); each chunk's bytes are identical to a
 * lmc_multi_layer_kv_transfer call on that chunk.  token_starts is a host
 * array. */
int lmc_multi_layer_kv_transfer_batched(
    const lmc_tensor *chunks, int32_t n_chunks, const int64_t *token_starts,
    const lmc_tensor *key_value_ptrs, const lmc_tensor *slot_mapping,
    int32_t paged_device, int64_t page_buffer_size, int32_t direction,
    int32_t use_mla, int32_t kvcache_format, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream);

/* Replaces fused_multi_layer_kv_transfer (csrc/mem_kernels.cpp:113-213;
 * pybind csrc/pybind.cpp:365): the gather/scatter runs against the device
 * `staging_cache`, and one DMA copy moves required_size bytes between the
 * staging buffer and the host buffer `key_value` (after the kernel for
 * direction != 0, before it for direction == 0). */
int lmc_fused_multi_layer_kv_transfer(
    const lmc_tensor *key_value, const lmc_tensor *staging_cache,
    const lmc_tensor *key_value_ptrs, const lmc_tensor *slot_mapping,
    int32_t paged_device, int64_t page_buffer_size, int32_t direction,
    int32_t use_mla, int32_t kvcache_format, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream);

/* No counterpart in the reference.  lmc_fused_multi_layer_kv_transfer for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc): the staging buffer is the library's
 * own static device area of LMC_NOALLOC_STAGING_BYTES per GPU (resolved once
 * per device on the first call), so the call allocates nothing; a transfer
 * needing more staging than that is refused with LMC_ERR_RUNTIME.  The
 * staging device is `paged_device` (the current device when negative).  A
 * store zeroes the staging bytes first (a fill kernel), so rows of skipped
 * slots arrive in `key_value` as zeros, as with a zeroed staging_cache.
 * Every call on one GPU shares that GPU's area.  Eager calls are ordered:
 * each call's stream waits for the previous call's work (an event recorded
 * per GPU), whatever stream or thread made it.  Calls enqueued under HIP
 * graph capture skip that wait, so a graph replay that overlaps another
 * call on the same GPU races with it.  The area lives in its own code
 * object, reserved on a GPU only once this entry point has run there. */
#define LMC_NOALLOC_STAGING_BYTES (64ll << 20)
int lmc_fused_multi_layer_kv_transfer_noalloc(
    const lmc_tensor *key_value, const lmc_tensor *key_value_ptrs,
    const lmc_tensor *slot_mapping, int32_t paged_device,
    int64_t page_buffer_size, int32_t direction, int32_t use_mla,
    int32_t kvcache_format, int64_t k_hidden_dims, int64_t v_hidden_dims,
    int64_t dsa_hidden_dims, void *stream);

/* Replaces single_layer_kv_transfer (csrc/mem_kernels.cpp:265-334; planner
 * csrc/utils.cpp:212-406; validation csrc/utils.cpp:903-966; pybind
 * csrc/pybind.cpp:467-472).  `caches` holds the n_caches paged tensors of
 * one layer (MERGED: 1; SEPARATE: K, V; MLA: K, V; DSA_KV: K, V, DSA;
 * DSA_INDEX: indexer). */
int lmc_single_layer_kv_transfer(const lmc_tensor *lmc_key_value_cache,
                                 const lmc_tensor *caches, int32_t n_caches,
                                 const lmc_tensor *slot_mapping,
                                 int32_t direction, int32_t kvcache_format,
                                 int32_t token_major, int32_t vllm_two_major,
                                 int64_t k_hidden_dims, int64_t v_hidden_dims,
                                 int64_t dsa_hidden_dims, void *stream);

/* Replaces load_and_reshape_flash (csrc/mem_kernels.cpp:1341-1389; pybind
 * csrc/pybind.cpp:475): layer `layer_idx` of key_value [2, L, T, W] is
 * filled from key_cache / value_cache rows slot_mapping[t]. */
int lmc_load_and_reshape_flash(const lmc_tensor *key_value,
                               const lmc_tensor *key_cache,
                               const lmc_tensor *value_cache,
                               const lmc_tensor *slot_mapping,
                               int32_t layer_idx, void *stream);

/* Replaces reshape_and_cache_back_flash (csrc/mem_kernels.cpp:1391-1440;
 * pybind csrc/pybind.cpp:476): the inverse of lmc_load_and_reshape_flash. */
int lmc_reshape_and_cache_back_flash(const lmc_tensor *key_value,
                                     const lmc_tensor *key_cache,
                                     const lmc_tensor *value_cache,
                                     const lmc_tensor *slot_mapping,
                                     int32_t layer_idx, void *stream);

/* ------------------------------------------------------------------------
 * Sparse, direct and staged-batch single-layer transfers
 * ------------------------------------------------------------------------ */

/* Replaces sparse_single_layer_kv_transfer (csrc/mem_kernels.cpp:418-497;
 * pybind csrc/pybind.cpp:381-387): retrieve only, for each i
 * paged[slot_mapping_packed[i]] = LMC token selected_token_idx[i] of the
 * single-layer buffer (layout as lmc_single_layer_kv_transfer).  Both index
 * tensors are 1-D or both 2-D of the same shape; selected_token_idx is
 * int32.  Entries with an out-of-range slot or token are skipped. */
int lmc_sparse_single_layer_kv_transfer(
    const lmc_tensor *lmc_key_value_cache, const lmc_tensor *caches,
    int32_t n_caches, const lmc_tensor *slot_mapping_packed,
    const lmc_tensor *selected_token_idx, int32_t kvcache_format,
    int32_t token_major, int32_t vllm_two_major, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream);

/* Replaces sparse_mla_dsa_batched_direct_kv_transfer and its _fast /
 * _prepared forms (csrc/mem_kernels.cpp:588-752, 833-976; pybind csrc/pybind.cpp:
 * 397-436): retrieve from memory objects reached through the device table
 * chunk_ptrs (int64, one kernel-visible address per chunk).  Entry i moves
 * token selected_token_idx[i] (chunk = token / chunk_size, n_c = min(
 * chunk_size, total_tokens - chunk * chunk_size)) to slot
 * slot_mapping_packed[i].  MLA/DSA chunks are stacked planes
 * [K: n_c*kH | V: n_c*vH | DSA: n_c*dsaH] or, with lmc_host_interleaved,
 * per-token [K | V | DSA] rows; MERGED/SEPARATE chunks have the layout of
 * lmc_layout_sample ([n, 2, W] when token_major, else [2, n, W]).
 * selected_token_counts (nullable, int32): entries form numel(counts) rows
 * of equal width and row r holds counts[r * stride(0)] valid entries.
 * validate_inputs adds the reference's argument checks. */
int lmc_sparse_direct_kv_transfer(
    const lmc_tensor *chunk_ptrs, const lmc_tensor *lmc_layout_sample,
    const lmc_tensor *caches, int32_t n_caches,
    const lmc_tensor *slot_mapping_packed, const lmc_tensor *selected_token_idx,
    const lmc_tensor *selected_token_counts, int64_t chunk_size,
    int64_t total_tokens, int32_t kvcache_format, int32_t token_major,
    int32_t vllm_two_major, int64_t k_hidden_dims, int64_t v_hidden_dims,
    int64_t dsa_hidden_dims, int32_t lmc_host_interleaved,
    int32_t validate_inputs, void *stream);

/* Replaces dense_mla_dsa_batched_direct_kv_transfer and its _fast /
 * _prepared / group forms (csrc/mem_kernels.cpp:978-1306; pybind
 * csrc/pybind.cpp:441-472, 312-327), MLA/DSA formats: token g in
 * [0, numel(slot_mapping_full)) belongs to chunk g / fixed_chunk_size, or
 * (fixed_chunk_size == 0) to the chunk c with chunk_offsets[c] <= g <
 * chunk_offsets[c] + chunk_sizes[c] (int32 device tables, ascending
 * offsets); its rows move between that chunk and slot_mapping_full[g]
 * (direction != 0: paged -> chunk).  Chunk layout as in
 * lmc_sparse_direct_kv_transfer. */
int lmc_dense_direct_kv_transfer(
    const lmc_tensor *chunk_ptrs, const lmc_tensor *caches, int32_t n_caches,
    const lmc_tensor *slot_mapping_full, const lmc_tensor *chunk_offsets,
    const lmc_tensor *chunk_sizes, int64_t total_tokens,
    int64_t fixed_chunk_size, int32_t kvcache_format, int32_t vllm_two_major,
    int64_t k_hidden_dims, int64_t v_hidden_dims, int64_t dsa_hidden_dims,
    int32_t lmc_host_interleaved, int32_t direction, int32_t validate_inputs,
    void *stream);

/* Replaces batched_fused_single_layer_kv_transfer (csrc/mem_kernels.cpp:
 * 336-413; pybind csrc/pybind.cpp:373-380): a single-layer transfer between
 * the paged caches and the device staging_cache, and one DMA copy per plane
 * and chunk between staging tokens [chunk_offsets[i], + chunk_sizes[i]) and
 * memory object lmc_tensors[i] (host chunk offsets and sizes; layouts as
 * csrc/utils.cpp:500-733).  direction != 0: paged -> staging -> objects. */
int lmc_batched_fused_single_layer_kv_transfer(
    const lmc_tensor *lmc_tensors, int32_t n_chunks,
    const lmc_tensor *staging_cache, const lmc_tensor *caches, int32_t n_caches,
    const lmc_tensor *slot_mapping_full, const int64_t *chunk_offsets,
    const int64_t *chunk_sizes, int32_t direction, int32_t kvcache_format,
    int32_t token_major, int32_t vllm_two_major, int64_t k_hidden_dims,
    int64_t v_hidden_dims, int64_t dsa_hidden_dims, void *stream);

/* Replaces batched_fused_sparse_single_layer_kv_transfer
 * (csrc/mem_kernels.cpp:1308-1339; pybind csrc/pybind.cpp:388-396):
 * objects -> staging, then lmc_sparse_single_layer_kv_transfer from the
 * staging buffer. */
int lmc_batched_fused_sparse_single_layer_kv_transfer(
    const lmc_tensor *lmc_tensors, int32_t n_chunks,
    const lmc_tensor *staging_cache, const lmc_tensor *caches, int32_t n_caches,
    const lmc_tensor *slot_mapping_packed, const lmc_tensor *selected_token_idx,
    const int64_t *chunk_offsets, const int64_t *chunk_sizes,
    int32_t kvcache_format, int32_t token_major, int32_t vllm_two_major,
    int64_t k_hidden_dims, int64_t v_hidden_dims, int64_t dsa_hidden_dims,
    void *stream);

/* Replaces sparse_graph_kv_transfer and its sfa_copy kernels
 * (csrc/mem_kernels.cpp:754-831; csrc/graph/sparse_graph_kernel.cpp:6-132;
 * pybind csrc/pybind.cpp:437-440): entry (r, j) of the packed
 * [requests, row_width] `selected` / `slots` matrices, active for j <
 * min(counts[r * stride(0)], row_width) when counts and limits[r] are > 0,
 * copies token selected[r, j] in [0, limits[r]) from the chunk sources
 * ptrs[0 | 1, r * chunks_per_request + token / chunk_size] (K, PE; null
 * skips) into row slots[r, j] of k_cache / pe_cache.  k_hidden_dims /
 * pe_hidden_dims <= 0 take the caches' last two dims.  max_aiv_cores is
 * accepted and does not change the result. */
int lmc_sparse_graph_kv_transfer(const lmc_tensor *k_cache, const lmc_tensor *pe_cache,
                                 int64_t k_hidden_dims, int64_t pe_hidden_dims,
                                 const lmc_tensor *slots, const lmc_tensor *selected,
                                 const lmc_tensor *counts, const lmc_tensor *ptrs,
                                 const lmc_tensor *limits, int64_t chunk_size,
                                 int64_t max_aiv_cores, void *stream);

/* IndexerC8State's checks (csrc/indexer_c8.cpp:13-50): keys
 * [NB, 128, 1, 128] float16/bfloat16 alone, or int8 with float16 scales
 * [NB, 128, 1, 1]; slot_factor 1 (or 2 for int8); optional int32 block_map
 * [NB] (int8, factor 1).  scales and block_map may be NULL. */
int lmc_indexer_c8_check_state(const lmc_tensor *keys, const lmc_tensor *scales,
                               int64_t slot_factor, const lmc_tensor *block_map);

/* Replaces indexer_c8_transfer_prepared and indexer_c8_group_transfer_prepared
 * (csrc/indexer_c8.cpp:52-185; csrc/indexer_c8/kernel.cpp:29-121; pybind
 * csrc/pybind.cpp:243-262): for each of n_layers layers (per-layer keys,
 * scales, block_maps entries may be NULL, slot_factors[l]) and each chunk c
 * (packet packet_ptrs[l, c]; tokens [start, start + count) of slot_mapping,
 * start / count from chunk_offsets / chunk_counts or, with fixed_chunks, c *
 * chunk_capacity and the rest of the mapping), token t's key row and scale
 * move between the packet ([count key rows | count scales]) and the cache's
 * physical slot (block_map[s / 128] * 128 + s % 128, or s + (s / 128) *
 * (slot_factor - 1) * 128).  from_npu != 0: cache -> packet. */
int lmc_indexer_c8_transfer(const lmc_tensor *const *keys, const lmc_tensor *const *scales,
                            const lmc_tensor *const *block_maps, const int64_t *slot_factors,
                            int32_t n_layers, const lmc_tensor *packet_ptrs,
                            const lmc_tensor *chunk_offsets, const lmc_tensor *chunk_counts,
                            const lmc_tensor *slot_mapping, int64_t chunk_capacity,
                            int32_t from_npu, int32_t fixed_chunks, void *stream);

/* The cache checks of prepare_sparse_direct_layer_state /
 * prepare_sparse_direct_destination_state (csrc/utils.cpp:408-498,
 * 903-966): LMC_ERR_VALUE with the reference's message on a bad format or
 * cache tuple. */
int lmc_check_kv_caches(const lmc_tensor *caches, int32_t n_caches,
                        int32_t kvcache_format, int32_t vllm_two_major,
                        int64_t k_hidden_dims, int64_t v_hidden_dims,
                        int64_t dsa_hidden_dims);

/* ------------------------------------------------------------------------
 * CacheGen codec
 * ------------------------------------------------------------------------ */

/* Replaces calculate_cdf (csrc/cachegen_kernels.cpp:119-155; pybind
 * csrc/pybind.cpp:480).  input: [L, T, C] u8/i8 symbols.  output: a
 * caller-allocated int16 [L, C, n_bins + 1] tensor, every entry of which is
 * written (the reference allocates it with torch::zeros; the Python layer
 * allocates it without a fill).  Each row is a CDF of aligned power-of-two
 * intervals in symbol order with the code length in the low 4 bits: the
 * lengths of an optimal alphabetic code (Garsia-Wachs) when the longest
 * fits 8 bits (at most 256 counted symbols) or 12 (more), else Shannon
 * lengths clamped to [1, 12]. */
int lmc_calculate_cdf(const lmc_tensor *input, int32_t n_bins,
                      const lmc_tensor *output, void *stream);

/* Replaces encode_fast_new (csrc/cachegen_kernels.cpp:17-58; pybind
 * csrc/pybind.cpp:477). */
int lmc_encode_fast_new(const lmc_tensor *cdf, const lmc_tensor *input_sym,
                        const lmc_tensor *output_buffer,
                        const lmc_tensor *output_lengths, void *stream);

/* Replaces decode_fast_new (csrc/cachegen_kernels.cpp:60-65; pybind
 * csrc/pybind.cpp:478); like the reference it always returns
 * LMC_ERR_NOT_IMPLEMENTED. */
int lmc_decode_fast_new(const lmc_tensor *cdf, const lmc_tensor *bytestreams,
                        const lmc_tensor *lengths, const lmc_tensor *output,
                        void *stream);

/* Replaces decode_fast_prefsum (csrc/cachegen_kernels.cpp:67-112; pybind
 * csrc/pybind.cpp:479). */
int lmc_decode_fast_prefsum(const lmc_tensor *cdf,
                            const lmc_tensor *bytestreams,
                            const lmc_tensor *lengths,
                            const lmc_tensor *output, void *stream);

/* ------------------------------------------------------------------------
 * Fused K re-rotation (CacheBlend)
 * ------------------------------------------------------------------------ */

/* No counterpart in the reference: the CacheBlend connector's per-layer
 * retrieve (lmcache_ascend/v1/npu_connector/npu_connectors.py:556-689) in one
 * kernel.  The bytes written to the paged `caches` (MERGED_KV or SEPARATE_KV,
 * one layer) equal the connector's sequence: a zeroed [2, N, W] buffer
 * (N = slot_mapping.size(0)) receives each KV_2TD memory object
 * `objects[i]` ([2, n_i, W]) at tokens [token_starts[i], token_starts[i] + n_i)
 * (objects must not overlap); when positions are given, its K half is
 * re-rotated as lmc_rotary_embedding_k_fused(old_positions, new_positions,
 * K, head_size, cos_sin_cache, is_neox) would; the buffer is then scattered
 * as lmc_single_layer_kv_transfer(buffer, caches, slot_mapping, 0, fmt, 0,
 * vllm_two_major).  No buffer is allocated.  old_positions and
 * new_positions are both null (no re-rotation) or both [N] device tensors.
 * Objects may be device tensors or page-locked host memory (read in place).
 * Geometry outside the kernel's (keys other than bf16/fp16, rows or heads
 * not in 16-byte pieces, rotary halves not a multiple of 8 dims) returns
 * LMC_ERR_NOT_IMPLEMENTED before any work. */
int lmc_blend_layer_to_paged(const lmc_tensor *objects, int32_t n_objects,
                             const int64_t *token_starts, const lmc_tensor *caches,
                             int32_t n_caches, const lmc_tensor *slot_mapping,
                             const lmc_tensor *old_positions, const lmc_tensor *new_positions,
                             const lmc_tensor *cos_sin_cache, int64_t head_size, int32_t is_neox,
                             int32_t kvcache_format, int32_t vllm_two_major, void *stream);

/* Replaces rotary_embedding_k_fused (csrc/pos_kernels.cpp:158-196; pybind
 * csrc/pybind.cpp:481): key [T, H*head_size] is rotated in place from
 * old_positions to new_positions with the [max_pos, rot] cos|sin cache. */
int lmc_rotary_embedding_k_fused(const lmc_tensor *old_positions,
                                 const lmc_tensor *new_positions,
                                 const lmc_tensor *key, int64_t head_size,
                                 const lmc_tensor *cos_sin_cache,
                                 int32_t is_neox, void *stream);

/* ------------------------------------------------------------------------
 * Pinned host memory and device address translation
 * ------------------------------------------------------------------------ */

/* Replaces get_device_ptr (csrc/common/managed_mem.cpp:189-236; pybind
 * csrc/pybind.cpp:330-336): device address of host address `host_ptr`
 * valid for `required_size` bytes, or 0 when the range is not mapped. */
int lmc_get_device_ptr(uintptr_t host_ptr, size_t required_size,
                       uintptr_t *out_device_ptr);

/* Replaces register_mapping (csrc/common/managed_mem.cpp:395-407; pybind
 * csrc/pybind.cpp:337-342): records host->device for `size` bytes. */
int lmc_register_mapping(uintptr_t host_ptr, uintptr_t dev_ptr, size_t size,
                         uintptr_t *out_device_ptr);

/* Replaces unregister_ptr (csrc/common/managed_mem.cpp:409-422; pybind
 * csrc/pybind.cpp:343-345).  *out_status is
 * 0 when a mapping was removed, -1 when none existed. */
int lmc_unregister_ptr(uintptr_t host_ptr, int32_t *out_status);

/* Replaces alloc_pinned_ptr (csrc/common/mem_alloc.cpp:19-44; pybind
 * csrc/pybind.cpp:346-347): page-locked host memory mapped into the device
 * address space and recorded for lmc_get_device_ptr. */
int lmc_alloc_pinned_ptr(size_t size, uint32_t flags, uintptr_t *out_ptr);

/* Replaces free_pinned_ptr (csrc/common/mem_alloc.cpp:46-52; pybind
 * csrc/pybind.cpp:348). */
int lmc_free_pinned_ptr(uintptr_t ptr);

/* Replaces alloc_pinned_numa_ptr (csrc/common/mem_alloc.cpp:56-92; pybind
 * csrc/pybind.cpp:349-350): zeroed page-locked host memory placed on NUMA
 * node `node` (the calling thread's policy is bound to it for the
 * allocation and restored afterwards), mapped into the device address space
 * and recorded for lmc_get_device_ptr. */
int lmc_alloc_pinned_numa_ptr(size_t size, int32_t node, uintptr_t *out_ptr);

/* Replaces free_pinned_numa_ptr (csrc/common/mem_alloc.cpp:94-106; pybind
 * csrc/pybind.cpp:351).  `size` is accepted for the reference's
 * signature; the runtime knows the allocation's extent. */
int lmc_free_pinned_numa_ptr(uintptr_t ptr, size_t size);

/* Replaces alloc_shm_pinned_ptr (csrc/common/mem_alloc.cpp:252-321; pybind
 * csrc/pybind.cpp:352-355): creates POSIX shared-memory segment `shm_name`
 * (exclusive create, mode 0600) of `size` bytes, reserves it in full and
 * prefaults it, interleaved over nodes[0..n_nodes) when n_nodes > 0 (which
 * requires the default thread memory policy).  The mapping is host memory
 * that transfers reach through staged copies; it is not device-mapped. */
int lmc_alloc_shm_pinned_ptr(size_t size, const char *shm_name, const int32_t *nodes,
                             int32_t n_nodes, uintptr_t *out_ptr);

/* Replaces attach_shm_pinned_ptr (csrc/common/mem_alloc.cpp:323-357; pybind
 * csrc/pybind.cpp:356-358): maps an existing segment, read-only when
 * writable == 0.  A segment smaller than `size` is an error. */
int lmc_attach_shm_pinned_ptr(size_t size, const char *shm_name, int32_t writable,
                              uintptr_t *out_ptr);

/* Replaces free_shm_pinned_ptr (csrc/common/mem_alloc.cpp:359-381; pybind
 * csrc/pybind.cpp:359-360): unmaps and unlinks the creator's mapping. */
int lmc_free_shm_pinned_ptr(uintptr_t ptr, size_t size, const char *shm_name);

/* Replaces detach_shm_pinned_ptr (csrc/common/mem_alloc.cpp:383-403; pybind
 * csrc/pybind.cpp:361-362): unmaps a peer's mapping. */
int lmc_detach_shm_pinned_ptr(uintptr_t ptr, size_t size);

/* Replaces unlink_shm (csrc/common/mem_alloc.cpp:405-410; pybind
 * csrc/pybind.cpp:363): removes a segment name; a missing name is not an
 * error. */
int lmc_unlink_shm(const char *shm_name);

/* One host<->device copy row: `bytes` bytes from `src` to `dst` (host
 * addresses for the host side, device addresses for the device side). */
typedef struct lmc_dma_segment {
  uint64_t dst;
  uint64_t src;
  uint64_t bytes;
} lmc_dma_segment;

/* Replaces layerwise_prefill_dma_copy (csrc/pybind.cpp:295-310): submits
 * copies[0..n) on `stream` (device-to-host when device_to_host != 0, else
 * host-to-device) on the copy engines.  Rows of zero bytes are skipped.
 * When no two destinations overlap, rows are reordered by destination,
 * adjacent rows merged and equal-stride runs issued as one rectangular
 * copy; otherwise rows go in the given order. */
int lmc_layerwise_prefill_dma_copy(const lmc_dma_segment *copies, int64_t n, int32_t device_to_host,
                                   void *stream);

/* Replaces layerwise_prefill_dma_copy_diagnose (csrc/pybind.cpp:263-294):
 * submits every row as given, one copy each, and writes each submission's
 * host-side duration in microseconds to copy_us[i]. */
int lmc_layerwise_prefill_dma_copy_diagnose(const lmc_dma_segment *copies, int64_t n,
                                            int32_t device_to_host, void *stream, double *copy_us);

/* Replaces get_gpu_pci_bus_id (pybind csrc/pybind.cpp:482): the PCI bus id
 * string of `device`, written NUL-terminated into buf[0..buf_len). */
int lmc_get_gpu_pci_bus_id(int32_t device, char *buf, int32_t buf_len);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* LMCACHE_AMD_H */
