// FP8 paged decode on the gfx950 matrix cores.
#include "kvfp8_decode_mfma.h"

namespace kvfp8 {

bool mfma_decode_supported(int32_t, int32_t, int32_t, int) { return false; }

int32_t mfma_chunk_tokens(int32_t, int32_t, int64_t, int32_t) { return 256; }

template <int QT>
hipError_t launch_mfma_decode(const DecodeArgs&, int64_t, hipStream_t) { return hipErrorNotSupported; }

template hipError_t launch_mfma_decode<KVFP8_F32>(const DecodeArgs&, int64_t, hipStream_t);
template hipError_t launch_mfma_decode<KVFP8_F16>(const DecodeArgs&, int64_t, hipStream_t);
template hipError_t launch_mfma_decode<KVFP8_BF16>(const DecodeArgs&, int64_t, hipStream_t);

}  // namespace kvfp8
