// The staged multi-layer transfer shared by lmc_fused_multi_layer_kv_transfer
// (kv_transfer.hip) and lmc_fused_multi_layer_kv_transfer_noalloc
// (kv_noalloc.hip), which differ only in where the staging bytes live.
#pragma once

#include "common.h"

namespace lmc {

// fused_multi_layer_kv_transfer (csrc/mem_kernels.cpp:113-213) through a
// staging buffer of `capacity` bytes at `stg_data` on device `stg_device`:
// an H2D copy into the staging buffer before a load, the gather/scatter
// against it, a D2H copy out of it after a store, all enqueued on `s`.
// `too_small` prefixes the error when the transfer needs more than
// `capacity`; `clear_before_store` zeroes the staging bytes of a store
// first (a fill kernel), so rows of skipped slots leave as zeros.
void fused_transfer(const lmc_tensor &kv, uint8_t *stg_data, int stg_device,
                    int64_t capacity, const char *too_small,
                    bool clear_before_store, const lmc_tensor *key_value_ptrs,
                    const lmc_tensor *slot_mapping, int32_t paged_device,
                    int64_t page_buffer_size, bool direction, bool use_mla,
                    int32_t kvcache_format, int64_t k_hidden_dims,
                    int64_t v_hidden_dims, int64_t dsa_hidden_dims,
                    hipStream_t s);

} // namespace lmc
