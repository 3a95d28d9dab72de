// Quantize-and-scatter append of new K/V tokens into the paged cache (gfx950).
//
// Replaces the Triton `quantize_append` kernel of reference
// src/torch_llm/kernals/kv_cache/quantized_append.py:74-133 and the unquantized
// indexed store of src/torch_llm/inference/paged_kv_cache.py:77-79.
//
// Work layout: one "row" is the D values of one (token, kv head) for K or for V.
// A row is owned by LPR lanes (a power of two, LPR * 16 >= D); each lane holds
// 16 consecutive elements, so for D = 128 eight lanes cover a row and a wave64
// covers eight rows. The absmax is a lane-local integer max of |x| bit patterns
// followed by an xor-butterfly across the LPR lanes of the row; the codes leave
// as one 16-byte store per lane. K and V rows of one (token, head) are adjacent
// rows, so their block/offset loads share cache lines.
#include "kvfp8_common.h"

namespace kvfp8 {

constexpr int kAppendThreads = 256;
constexpr int kElemsPerLane = 16;

__device__ __forceinline__ int64_t load_index(const void* p, int is64, int64_t i) {
    return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

struct AppendArgs {
    const void* k;
    const void* v;
    int64_t k_stride_t, k_stride_h, v_stride_t, v_stride_h;
    const void* blocks;
    const void* offsets;
    int blocks64, offsets64;
    int64_t num_tokens;
    int32_t num_kv_heads, head_dim;
    int64_t num_blocks;
    int32_t block_size;
    void* k_cache;
    void* v_cache;
    float* k_scales;
    float* v_scales;
};

// Loads this lane's 16 elements of a row (zeros past D). VEC: the row start and
// the lane offset are 16-byte aligned and D is a multiple of 16, so a lane's
// 16 elements are either all inside the row or all past its end.
template <int DT, bool VEC>
__device__ __forceinline__ void load_lane(const typename Elem<DT>::T* row, int d0, int D, float (&x)[kElemsPerLane]) {
    using T = typename Elem<DT>::T;
    if constexpr (VEC) {
        if (d0 >= D) {
#pragma unroll
            for (int i = 0; i < kElemsPerLane; ++i) x[i] = 0.0f;
            return;
        }
        constexpr int kPer16B = 16 / sizeof(T);
        static_assert(kElemsPerLane % kPer16B == 0, "lane width must be whole 16-byte vectors");
#pragma unroll
        for (int c = 0; c < kElemsPerLane / kPer16B; ++c) {
            const uint4 raw = *reinterpret_cast<const uint4*>(row + d0 + c * kPer16B);
            const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
            for (int i = 0; i < kPer16B; ++i) x[c * kPer16B + i] = Elem<DT>::load(e[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < kElemsPerLane; ++i) {
            const int d = d0 + i;
            x[i] = d < D ? Elem<DT>::load(row[d]) : 0.0f;
        }
    }
}

template <int DT, int LPR, bool VEC>
__global__ void __launch_bounds__(kAppendThreads)
quantize_append_kernel(AppendArgs a) {
    using T = typename Elem<DT>::T;
    constexpr int kRowsPerBlock = kAppendThreads / LPR;
    const int lane_in_row = threadIdx.x % LPR;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / LPR;
    const int64_t num_rows = a.num_tokens * a.num_kv_heads * 2;
    // Rows past the end still take part in the butterfly below with zeros; they
    // only skip the stores. (Every lane of a row shares the row index.)
    const bool live = row < num_rows;
    const int64_t r = live ? row : 0;
    const int is_v = (int)(r & 1);
    const int64_t th = r >> 1;
    const int64_t t = th / a.num_kv_heads;
    const int h = (int)(th - t * a.num_kv_heads);
    const int D = a.head_dim;
    const int d0 = lane_in_row * kElemsPerLane;

    // Page indices first: their latency overlaps the row load and the math.
    const int64_t block = load_index(a.blocks, a.blocks64, t);
    const int64_t offset = load_index(a.offsets, a.offsets64, t);
    const T* src = reinterpret_cast<const T*>(is_v ? a.v : a.k) +
                   t * (is_v ? a.v_stride_t : a.k_stride_t) + h * (is_v ? a.v_stride_h : a.k_stride_h);
    float x[kElemsPerLane];
    load_lane<DT, VEC>(src, d0, D, x);

    uint32_t amax = 0;
#pragma unroll
    for (int i = 0; i < kElemsPerLane; ++i) amax = max(amax, abs_bits(x[i]));
#pragma unroll
    for (int s = 1; s < LPR; s <<= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, s, LPR));

    const float scale = row_scale(amax);
    const RowDivider div(scale);
    uint32_t packed[kElemsPerLane / 4];
    if (div.fast && amax < 0x7F800000u) {
        // Finite row, scale in the corrected-division range: |x / scale| <=
        // 448 (1 + 2^-23), which needs no clamp and is never NaN, so the
        // hardware round-to-nearest-even converter gives the oracle's codes
        // (checked over every such float32 by kvfp8_selftest_fp8_encoder).
#pragma unroll
        for (int i = 0; i < kElemsPerLane / 4; ++i) {
            int w = __builtin_amdgcn_cvt_pk_fp8_f32(div.corrected(x[4 * i]), div.corrected(x[4 * i + 1]), 0, false);
            w = __builtin_amdgcn_cvt_pk_fp8_f32(div.corrected(x[4 * i + 2]), div.corrected(x[4 * i + 3]), w, true);
            packed[i] = (uint32_t)w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kElemsPerLane / 4; ++i) {
            packed[i] = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) packed[i] |= (uint32_t)clamp_encode(x[4 * i + e] / scale) << (8 * e);
        }
    }
    const uint8_t* codes = reinterpret_cast<const uint8_t*>(packed);

    if (!live || block < 0 || block >= a.num_blocks || offset < 0 || offset >= a.block_size) return;

    const int64_t slot = (block * a.block_size + offset) * a.num_kv_heads + h;
    uint8_t* dst = reinterpret_cast<uint8_t*>(is_v ? a.v_cache : a.k_cache) + slot * D;
    if constexpr (VEC) {
        if (d0 < D) *reinterpret_cast<uint4*>(dst + d0) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    } else {
#pragma unroll
        for (int i = 0; i < kElemsPerLane; ++i)
            if (d0 + i < D) dst[d0 + i] = codes[i];
    }
    if (lane_in_row == 0) (is_v ? a.v_scales : a.k_scales)[slot] = scale;
}

// Plain cast-and-scatter for unquantized caches (one lane per 16 elements).
template <int DT_IN, int DT_OUT>
__global__ void __launch_bounds__(kAppendThreads)
store_append_kernel(AppendArgs a, int lanes_per_row) {
    using TI = typename Elem<DT_IN>::T;
    using TO = typename Elem<DT_OUT>::T;
    const int64_t gid = (int64_t)blockIdx.x * kAppendThreads + threadIdx.x;
    const int64_t row = gid / lanes_per_row;
    const int lane_in_row = (int)(gid - row * lanes_per_row);
    if (row >= a.num_tokens * a.num_kv_heads * 2) return;
    const int is_v = (int)(row & 1);
    const int64_t th = row >> 1;
    const int64_t t = th / a.num_kv_heads;
    const int h = (int)(th - t * a.num_kv_heads);
    const int64_t block = load_index(a.blocks, a.blocks64, t);
    const int64_t offset = load_index(a.offsets, a.offsets64, t);
    if (block < 0 || block >= a.num_blocks || offset < 0 || offset >= a.block_size) return;
    const TI* src = reinterpret_cast<const TI*>(is_v ? a.v : a.k) +
                    t * (is_v ? a.v_stride_t : a.k_stride_t) + h * (is_v ? a.v_stride_h : a.k_stride_h);
    TO* dst = reinterpret_cast<TO*>(is_v ? a.v_cache : a.k_cache) +
              ((block * a.block_size + offset) * a.num_kv_heads + h) * a.head_dim;
    const int d0 = lane_in_row * kElemsPerLane;
#pragma unroll
    for (int i = 0; i < kElemsPerLane; ++i) {
        const int d = d0 + i;
        if (d < a.head_dim) dst[d] = Elem<DT_OUT>::store(Elem<DT_IN>::load(src[d]));
    }
}

// Every float32 bit pattern m with |x| <= 448 (1 + 2^-19) (sign from the grid's
// y index): hardware converter vs the software encoder; counts mismatches.
__global__ void __launch_bounds__(256) fp8_encoder_selftest_kernel(uint32_t limit, unsigned long long* mismatches) {
    unsigned long long local = 0;
    const uint32_t sign = blockIdx.y ? 0x80000000u : 0u;
    for (uint32_t m = blockIdx.x * 256u + threadIdx.x; m <= limit; m += gridDim.x * 256u) {
        const float a = bits_f32(m | sign);
        const float b = bits_f32((limit - m) | sign);
        const uint32_t hw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
        local += (hw & 0xFFu) != encode_e4m3fn(a);
        local += ((hw >> 8) & 0xFFu) != encode_e4m3fn(b);
    }
    if (local) atomicAdd(mismatches, local);
}

}  // namespace kvfp8

using namespace kvfp8;

namespace {

int element_size(int dtype) {
    switch (dtype) {
        case KVFP8_F32: return 4;
        case KVFP8_F16:
        case KVFP8_BF16: return 2;
        case KVFP8_E4M3FN: return 1;
        case KVFP8_I32: return 4;
        case KVFP8_I64: return 8;
        default: return 0;
    }
}

bool is_float_in(int dtype) { return dtype == KVFP8_F32 || dtype == KVFP8_F16 || dtype == KVFP8_BF16; }
bool is_index(int dtype) { return dtype == KVFP8_I32 || dtype == KVFP8_I64; }

int check_append(const void* k, const void* v, int in_dtype, const void* blocks, int blocks_dtype,
                 const void* offsets, int offsets_dtype, int64_t num_tokens, int32_t num_kv_heads,
                 int32_t head_dim, int64_t num_blocks, int32_t block_size, const void* kc, const void* vc) {
    if (!is_float_in(in_dtype)) return KVFP8_EDTYPE;
    if (!is_index(blocks_dtype) || !is_index(offsets_dtype)) return KVFP8_EDTYPE;
    if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0 || block_size <= 0)
        return KVFP8_ESHAPE;
    if (head_dim > 64 * kElemsPerLane) return KVFP8_ELIMIT;
    if (num_tokens > 0 && (!k || !v || !blocks || !offsets || !kc || !vc)) return KVFP8_ENULL;
    return KVFP8_OK;
}

int lanes_for(int head_dim) {
    int lpr = 1;
    while (lpr * kElemsPerLane < head_dim) lpr <<= 1;
    return lpr;
}

template <int DT, int LPR>
hipError_t launch_quantize(const AppendArgs& a, bool vec, hipStream_t stream) {
    constexpr int kRowsPerBlock = kAppendThreads / LPR;
    const int64_t rows = a.num_tokens * a.num_kv_heads * 2;
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    if (vec)
        hipLaunchKernelGGL((quantize_append_kernel<DT, LPR, true>), grid, dim3(kAppendThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((quantize_append_kernel<DT, LPR, false>), grid, dim3(kAppendThreads), 0, stream, a);
    return hipGetLastError();
}

template <int DT>
hipError_t dispatch_quantize_lpr(const AppendArgs& a, bool vec, hipStream_t stream) {
    switch (lanes_for(a.head_dim)) {
        case 1: return launch_quantize<DT, 1>(a, vec, stream);
        case 2: return launch_quantize<DT, 2>(a, vec, stream);
        case 4: return launch_quantize<DT, 4>(a, vec, stream);
        case 8: return launch_quantize<DT, 8>(a, vec, stream);
        case 16: return launch_quantize<DT, 16>(a, vec, stream);
        case 32: return launch_quantize<DT, 32>(a, vec, stream);
        default: return launch_quantize<DT, 64>(a, vec, stream);
    }
}

template <int DI, int DO>
hipError_t launch_store(const AppendArgs& a, hipStream_t stream) {
    const int lpr = (a.head_dim + kElemsPerLane - 1) / kElemsPerLane;
    const int64_t threads = a.num_tokens * a.num_kv_heads * 2 * lpr;
    const dim3 grid((unsigned)((threads + kAppendThreads - 1) / kAppendThreads));
    hipLaunchKernelGGL((store_append_kernel<DI, DO>), grid, dim3(kAppendThreads), 0, stream, a, lpr);
    return hipGetLastError();
}

template <int DI>
hipError_t dispatch_store_out(const AppendArgs& a, int cache_dtype, hipStream_t stream) {
    switch (cache_dtype) {
        case KVFP8_F32: return launch_store<DI, KVFP8_F32>(a, stream);
        case KVFP8_F16: return launch_store<DI, KVFP8_F16>(a, stream);
        default: return launch_store<DI, KVFP8_BF16>(a, stream);
    }
}

bool aligned16(const void* p, int64_t byte_stride_t, int64_t byte_stride_h) {
    return ((uintptr_t)p % 16 == 0) && (byte_stride_t % 16 == 0) && (byte_stride_h % 16 == 0);
}

}  // namespace

extern "C" int kvfp8_quantize_append(const void* k, const void* v, int in_dtype, int64_t k_stride_t,
                                     int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h,
                                     const void* blocks, int blocks_dtype, const void* offsets,
                                     int offsets_dtype, int64_t num_tokens, int32_t num_kv_heads,
                                     int32_t head_dim, int64_t num_blocks, int32_t block_size,
                                     void* k_cache, void* v_cache, float* k_scales, float* v_scales,
                                     void* stream) {
    int rc = check_append(k, v, in_dtype, blocks, blocks_dtype, offsets, offsets_dtype, num_tokens,
                          num_kv_heads, head_dim, num_blocks, block_size, k_cache, v_cache);
    if (rc != KVFP8_OK) return rc;
    if (num_tokens > 0 && (!k_scales || !v_scales)) return KVFP8_ENULL;
    if (num_tokens == 0) return KVFP8_OK;
    AppendArgs a{k, v, k_stride_t, k_stride_h, v_stride_t, v_stride_h, blocks, offsets,
                 blocks_dtype == KVFP8_I64, offsets_dtype == KVFP8_I64, num_tokens, num_kv_heads,
                 head_dim, num_blocks, block_size, k_cache, v_cache, k_scales, v_scales};
    const int es = element_size(in_dtype);
    const bool vec = head_dim % kElemsPerLane == 0 && aligned16(k, k_stride_t * es, k_stride_h * es) &&
                     aligned16(v, v_stride_t * es, v_stride_h * es) && (uintptr_t)k_cache % 16 == 0 &&
                     (uintptr_t)v_cache % 16 == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t err;
    switch (in_dtype) {
        case KVFP8_F32: err = dispatch_quantize_lpr<KVFP8_F32>(a, vec, s); break;
        case KVFP8_F16: err = dispatch_quantize_lpr<KVFP8_F16>(a, vec, s); break;
        default: err = dispatch_quantize_lpr<KVFP8_BF16>(a, vec, s); break;
    }
    return (int)err;
}

extern "C" int kvfp8_store_append(const void* k, const void* v, int in_dtype, int64_t k_stride_t,
                                  int64_t k_stride_h, int64_t v_stride_t, int64_t v_stride_h,
                                  const void* blocks, int blocks_dtype, const void* offsets,
                                  int offsets_dtype, int64_t num_tokens, int32_t num_kv_heads,
                                  int32_t head_dim, int64_t num_blocks, int32_t block_size,
                                  void* k_cache, void* v_cache, int cache_dtype, void* stream) {
    int rc = check_append(k, v, in_dtype, blocks, blocks_dtype, offsets, offsets_dtype, num_tokens,
                          num_kv_heads, head_dim, num_blocks, block_size, k_cache, v_cache);
    if (rc != KVFP8_OK) return rc;
    if (!is_float_in(cache_dtype)) return KVFP8_EDTYPE;
    if (num_tokens == 0) return KVFP8_OK;
    AppendArgs a{k, v, k_stride_t, k_stride_h, v_stride_t, v_stride_h, blocks, offsets,
                 blocks_dtype == KVFP8_I64, offsets_dtype == KVFP8_I64, num_tokens, num_kv_heads,
                 head_dim, num_blocks, block_size, k_cache, v_cache, nullptr, nullptr};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t err;
    switch (in_dtype) {
        case KVFP8_F32: err = dispatch_store_out<KVFP8_F32>(a, cache_dtype, s); break;
        case KVFP8_F16: err = dispatch_store_out<KVFP8_F16>(a, cache_dtype, s); break;
        default: err = dispatch_store_out<KVFP8_BF16>(a, cache_dtype, s); break;
    }
    return (int)err;
}

extern "C" void kvfp8_host_encode_e4m3fn(const float* x, uint8_t* codes, int64_t n) {
    for (int64_t i = 0; i < n; ++i) codes[i] = encode_e4m3fn(x[i]);
}

extern "C" void kvfp8_host_quantize_rows(const float* x, int64_t rows, int32_t head_dim, uint8_t* codes,
                                         float* scales) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = x + r * head_dim;
        uint32_t amax = 0;
        for (int d = 0; d < head_dim; ++d) amax = amax > abs_bits(row[d]) ? amax : abs_bits(row[d]);
        const float scale = row_scale(amax);
        const RowDivider div(scale);
        scales[r] = scale;
        for (int d = 0; d < head_dim; ++d) codes[r * head_dim + d] = clamp_encode(div.divide(row[d]));
    }
}

extern "C" void kvfp8_host_row_quotients(const float* x, int64_t rows, int32_t head_dim, float* q) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = x + r * head_dim;
        uint32_t amax = 0;
        for (int d = 0; d < head_dim; ++d) amax = amax > abs_bits(row[d]) ? amax : abs_bits(row[d]);
        const RowDivider div(row_scale(amax));
        for (int d = 0; d < head_dim; ++d) q[r * head_dim + d] = div.divide(row[d]);
    }
}

extern "C" int kvfp8_selftest_fp8_encoder(unsigned long long* mismatches_dev, void* stream) {
    if (!mismatches_dev) return KVFP8_ENULL;
    const uint32_t limit = 0x43E00010u;    // 448 (1 + 2^-19): every quotient the fast path makes
    hipLaunchKernelGGL(fp8_encoder_selftest_kernel, dim3(8192, 2), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), limit, mismatches_dev);
    return (int)hipGetLastError();
}
