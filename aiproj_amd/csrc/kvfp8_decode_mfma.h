// FP8 paged decode on the gfx950 matrix cores (declarations).
#pragma once

#include "kvfp8_decode_common.h"

namespace kvfp8 {

// Shapes the MFMA kernel handles; everything else goes to the generic kernel.
bool mfma_decode_supported(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int kv_dtype);

// Tokens per work item, chosen from shapes only.
int32_t mfma_chunk_tokens(int32_t batch, int32_t num_kv_heads, int64_t bt_width, int32_t block_size);

template <int QT>
hipError_t launch_mfma_decode(const DecodeArgs& a, int64_t units_total, hipStream_t stream);

}  // namespace kvfp8
