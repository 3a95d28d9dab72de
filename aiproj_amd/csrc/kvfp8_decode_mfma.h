// FP8 paged decode on the gfx950 matrix cores (declarations).
#pragma once

#include "kvfp8_decode_common.h"

namespace kvfp8 {

// Shapes the MFMA kernel handles (e4m3fn, bf16 or f16 cache, D in {64, 128}, page
// size a multiple of 16, group size <= 16; an f16 cache also needs f16 q, which the
// caller checks); everything else goes to the VALU kernels.
bool mfma_decode_supported(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int64_t bt_width, int32_t block_size, int kv_dtype);

// Workspace bytes of the MFMA path (tile prefix, then two partial softmax states
// per workgroup); offsets[0..3] receive the byte offsets of plan, m, l and acc.
int64_t mfma_workspace_layout(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                              int64_t offsets[4]);

// phases: kPhaseSplit (the decode kernel), kPhaseReduce (the combine kernel), or both.
template <int QT>
hipError_t launch_mfma_decode(const DecodeArgs& a, int kv_dtype, void* workspace, hipStream_t stream, int phases);

}  // namespace kvfp8
