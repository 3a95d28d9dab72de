// SwiGLU activation of the feed-forward block (gfx950):
//   out[r, j] = silu(x[r, j]) * x[r, n + j],  silu(g) = g * (1 / (1 + exp(-g)))
// with gate and up the two halves of each row of x (the fused gate/up projection's
// output), computed in float32 and rounded once to the output dtype, as the
// reference's fused grouped_swiglu_up kernel does from its float32 accumulators
// (reference src/torch_llm/kernals/moe/grouped_swiglu_up.py:239).
//
// One launch replaces the two elementwise launches of silu(gate) and its product
// with up. Rows are independent; a lane handles 16 bytes of gate and of up when the
// row starts, strides and n allow 16-byte vectors, one element otherwise.
#include "kvfp8_common.h"

namespace kvfp8 {

constexpr int kSwigluThreads = 256;

__device__ __forceinline__ float swiglu(float g, float u) {
    const float s = 1.0f / (1.0f + expf(-g));
    return (g * s) * u;
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kSwigluThreads)
silu_mul_kernel(const void* x, int64_t rows, int32_t n, int64_t x_stride, void* out, int64_t out_stride) {
    using T = typename Elem<DT>::T;
    constexpr int kPer = VEC ? 16 / (int)sizeof(T) : 1;
    const int64_t per_row = n / kPer;
    const int64_t total = rows * per_row;
    for (int64_t i = (int64_t)blockIdx.x * kSwigluThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kSwigluThreads) {
        const int64_t r = i / per_row;
        const int64_t j = (i - r * per_row) * kPer;
        const T* gate = reinterpret_cast<const T*>(x) + r * x_stride + j;
        const T* up = gate + n;
        T* dst = reinterpret_cast<T*>(out) + r * out_stride + j;
        if constexpr (VEC) {
            const uint4 gv = *reinterpret_cast<const uint4*>(gate);
            const uint4 uv = *reinterpret_cast<const uint4*>(up);
            const T* ge = reinterpret_cast<const T*>(&gv);
            const T* ue = reinterpret_cast<const T*>(&uv);
            uint4 ov;
            T* oe = reinterpret_cast<T*>(&ov);
#pragma unroll
            for (int e = 0; e < kPer; ++e) oe[e] = Elem<DT>::store(swiglu(Elem<DT>::load(ge[e]), Elem<DT>::load(ue[e])));
            *reinterpret_cast<uint4*>(dst) = ov;
        } else {
            dst[0] = Elem<DT>::store(swiglu(Elem<DT>::load(gate[0]), Elem<DT>::load(up[0])));
        }
    }
}

}  // namespace kvfp8

using namespace kvfp8;

namespace {

template <int DT>
hipError_t launch_silu_mul(const void* x, int64_t rows, int32_t n, int64_t xs, void* out, int64_t os, hipStream_t s) {
    using T = typename Elem<DT>::T;
    constexpr int kPer = 16 / (int)sizeof(T);
    const bool vec = n % kPer == 0 && xs % kPer == 0 && os % kPer == 0 &&
                     ((uintptr_t)x % 16) == 0 && ((uintptr_t)out % 16) == 0;
    const int64_t items = rows * (vec ? n / kPer : n);
    int64_t blocks = (items + kSwigluThreads - 1) / kSwigluThreads;
    blocks = blocks > 65536 ? 65536 : (blocks < 1 ? 1 : blocks);
    if (vec)
        hipLaunchKernelGGL((silu_mul_kernel<DT, true>), dim3((unsigned)blocks), dim3(kSwigluThreads), 0, s, x, rows, n, xs, out, os);
    else
        hipLaunchKernelGGL((silu_mul_kernel<DT, false>), dim3((unsigned)blocks), dim3(kSwigluThreads), 0, s, x, rows, n, xs, out, os);
    return hipGetLastError();
}

}  // namespace

extern "C" int kvfp8_silu_mul(const void* x, int dtype, int64_t rows, int32_t n, int64_t x_row_stride, void* out,
                              int64_t out_row_stride, void* stream) {
    if (dtype != KVFP8_F32 && dtype != KVFP8_F16 && dtype != KVFP8_BF16) return KVFP8_EDTYPE;
    if (rows < 0 || n <= 0 || x_row_stride < 2 * (int64_t)n || out_row_stride < n) return KVFP8_ESHAPE;
    if (rows == 0) return KVFP8_OK;
    if (!x || !out) return KVFP8_ENULL;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (dtype) {
        case KVFP8_F32: return (int)launch_silu_mul<KVFP8_F32>(x, rows, n, x_row_stride, out, out_row_stride, s);
        case KVFP8_F16: return (int)launch_silu_mul<KVFP8_F16>(x, rows, n, x_row_stride, out, out_row_stride, s);
        default: return (int)launch_silu_mul<KVFP8_BF16>(x, rows, n, x_row_stride, out, out_row_stride, s);
    }
}
