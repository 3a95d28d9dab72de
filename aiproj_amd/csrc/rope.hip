// Interleaved-pair rotary embedding applied in place to the q and k heads of a
// packed projection output (gfx950).
//
// Replaces the PyTorch op sequence of reference src/torch_llm/model/rope.py:46-55
// with one kernel. For every row t, head h < heads and pair i < head_dim / 2:
//   c = cos_table[pos[t], i], s = sin_table[pos[t], i]     (cast to the dtype)
//   x0' = c x0 - s x1,  x1' = s x0 + c x1
// Each multiply, add and subtract is rounded to the tensor dtype, as the
// reference's elementwise operations on a bf16/f16 tensor are, so the result is
// bit-identical to that sequence. Rows whose position lies outside the tables are
// left unrotated (the reference's table lookup would fault on them).
#include "kvfp8_common.h"

namespace kvfp8 {

constexpr int kRopeThreads = 256;

struct RopeArgs {
    void* x;
    int64_t rows;
    int32_t heads, head_dim;
    int64_t row_stride, head_stride;     // elements
    const void* positions;
    int32_t pos64;
    const void* cos_table;
    const void* sin_table;
    int64_t table_rows;
};

template <int DT>
__device__ __forceinline__ float rnd(float x) { return Elem<DT>::load(Elem<DT>::store(x)); }

template <int DT, int TT>
__global__ void __launch_bounds__(kRopeThreads)
rope_kernel(RopeArgs a) {
    // Separate multiplies and adds, like the reference's elementwise operations.
#pragma clang fp contract(off)
    using T = typename Elem<DT>::T;
    const int half = a.head_dim / 2;
    const int64_t pairs_per_row = (int64_t)a.heads * half;
    const int64_t total = a.rows * pairs_per_row;
    for (int64_t p = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x; p < total;
         p += (int64_t)gridDim.x * kRopeThreads) {
        const int64_t r = p / pairs_per_row;
        const int64_t rem = p - r * pairs_per_row;
        const int h = (int)(rem / half);
        const int i = (int)(rem - (int64_t)h * half);
        const int64_t pos = a.pos64 ? reinterpret_cast<const int64_t*>(a.positions)[r]
                                    : (int64_t)reinterpret_cast<const int32_t*>(a.positions)[r];
        if (pos < 0 || pos >= a.table_rows) continue;
        using TabT = typename Elem<TT>::T;
        const float c = rnd<DT>(Elem<TT>::load(reinterpret_cast<const TabT*>(a.cos_table)[pos * half + i]));
        const float s = rnd<DT>(Elem<TT>::load(reinterpret_cast<const TabT*>(a.sin_table)[pos * half + i]));
        T* e = reinterpret_cast<T*>(a.x) + r * a.row_stride + (int64_t)h * a.head_stride + 2 * i;
        const float x0 = Elem<DT>::load(e[0]), x1 = Elem<DT>::load(e[1]);
        const float y0 = rnd<DT>(rnd<DT>(c * x0) - rnd<DT>(s * x1));
        const float y1 = rnd<DT>(rnd<DT>(s * x0) + rnd<DT>(c * x1));
        e[0] = Elem<DT>::store(y0);
        e[1] = Elem<DT>::store(y1);
    }
}

}  // namespace kvfp8

using namespace kvfp8;

namespace {

template <int DT>
hipError_t launch_rope(const RopeArgs& a, int table_dtype, dim3 grid, hipStream_t s) {
    switch (table_dtype) {
        case KVFP8_F32: hipLaunchKernelGGL((rope_kernel<DT, KVFP8_F32>), grid, dim3(kRopeThreads), 0, s, a); break;
        case KVFP8_F16: hipLaunchKernelGGL((rope_kernel<DT, KVFP8_F16>), grid, dim3(kRopeThreads), 0, s, a); break;
        default: hipLaunchKernelGGL((rope_kernel<DT, KVFP8_BF16>), grid, dim3(kRopeThreads), 0, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

extern "C" int kvfp8_rope_inplace(void* x, int dtype, int64_t rows, int32_t heads, int32_t head_dim,
                                  int64_t row_stride, int64_t head_stride, const void* positions, int pos_dtype,
                                  const void* cos_table, const void* sin_table, int table_dtype,
                                  int64_t table_rows, void* stream) {
    auto is_float = [](int d) { return d == KVFP8_F32 || d == KVFP8_F16 || d == KVFP8_BF16; };
    if (!is_float(dtype) || !is_float(table_dtype)) return KVFP8_EDTYPE;
    if (pos_dtype != KVFP8_I32 && pos_dtype != KVFP8_I64) return KVFP8_EDTYPE;
    if (rows < 0 || heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || table_rows <= 0) return KVFP8_ESHAPE;
    if (rows == 0) return KVFP8_OK;
    if (!x || !positions || !cos_table || !sin_table) return KVFP8_ENULL;
    RopeArgs a{x, rows, heads, head_dim, row_stride, head_stride, positions, pos_dtype == KVFP8_I64,
               cos_table, sin_table, table_rows};
    const int64_t total = rows * heads * (head_dim / 2);
    int64_t blocks = (total + kRopeThreads - 1) / kRopeThreads;
    blocks = blocks > 65536 ? 65536 : blocks;
    const dim3 grid((unsigned)blocks);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (dtype) {
        case KVFP8_F32: return (int)launch_rope<KVFP8_F32>(a, table_dtype, grid, s);
        case KVFP8_F16: return (int)launch_rope<KVFP8_F16>(a, table_dtype, grid, s);
        default: return (int)launch_rope<KVFP8_BF16>(a, table_dtype, grid, s);
    }
}
