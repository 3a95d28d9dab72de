// RMSNorm forward for the decode and prefill steps (gfx950), optionally fused with
// the residual add that precedes it.
//
// Replaces the Triton `rmsnorm_kernal` of reference
// src/torch_llm/model/rmsnorm.py:60-113 (forward only):
//   inv_rms = 1 / sqrt(mean(x^2) + eps)        (float32)
//   out     = (x * inv_rms) * weight           (float32, stored in x's dtype)
// The fused form first forms the residual sum s = x + update in float32, rounds
// it to the state dtype (what `state + update` stores, reference
// model/residual.py:33-35) and normalizes that rounded value.
//
// One wave per row, rows grid-strided over the launch. A lane holds 8 elements
// (one 16-byte vector of a 16-bit dtype) per 512-element chunk of the row, so a
// row of up to 4096 elements stays in registers between the reduction and the
// scaling; longer rows are read twice.
#include "kvfp8_common.h"

namespace kvfp8 {

constexpr int kNormThreads = 256;
constexpr int kNormVec = 8;          // elements per lane per chunk
constexpr int kNormChunks = 8;       // chunks kept in registers (4096 elements)

struct NormArgs {
    const void* x;
    const void* update;     // null: plain RMSNorm
    const void* weight;
    void* out;
    void* state_out;        // fused form: x + update in x's dtype
    float* inv_rms;         // may be null
    int64_t rows;
    int32_t d_model;
    int64_t x_stride, update_stride, out_stride, state_stride;   // elements
    float eps;
};

template <int DT>
__device__ __forceinline__ void load8(const typename Elem<DT>::T* p, bool vec, int n, float (&v)[kNormVec]) {
    using T = typename Elem<DT>::T;
    if (vec && n == kNormVec) {
        if constexpr (sizeof(T) == 2) {
            const uint4 raw = *reinterpret_cast<const uint4*>(p);
            const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
            for (int i = 0; i < kNormVec; ++i) v[i] = Elem<DT>::load(e[i]);
        } else {
            const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kNormVec; ++i) v[i] = i < n ? Elem<DT>::load(p[i]) : 0.0f;
    }
}

template <int DT>
__device__ __forceinline__ void store8(typename Elem<DT>::T* p, bool vec, int n, const float (&v)[kNormVec]) {
    using T = typename Elem<DT>::T;
    if (vec && n == kNormVec) {
        if constexpr (sizeof(T) == 2) {
            T e[kNormVec];
#pragma unroll
            for (int i = 0; i < kNormVec; ++i) e[i] = Elem<DT>::store(v[i]);
            *reinterpret_cast<uint4*>(p) = *reinterpret_cast<const uint4*>(e);
        } else {
            reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
            reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < kNormVec; ++i)
            if (i < n) p[i] = Elem<DT>::store(v[i]);
    }
}

// Row element of the (possibly fused) input: x, or round(x + update) to x's dtype.
template <int DT, bool kFused>
__device__ __forceinline__ void row_chunk(const NormArgs& a, int64_t r, int d0, int n, bool vec, float (&v)[kNormVec]) {
    using T = typename Elem<DT>::T;
    load8<DT>(reinterpret_cast<const T*>(a.x) + r * a.x_stride + d0, vec, n, v);
    if constexpr (kFused) {
        float u[kNormVec];
        load8<DT>(reinterpret_cast<const T*>(a.update) + r * a.update_stride + d0, vec, n, u);
#pragma unroll
        for (int i = 0; i < kNormVec; ++i) v[i] = Elem<DT>::load(Elem<DT>::store(v[i] + u[i]));
    }
}

template <int DT, int WT, bool kFused>
__global__ void __launch_bounds__(kNormThreads)
rmsnorm_kernel(NormArgs a, int vec_ok) {
    using T = typename Elem<DT>::T;
    using W = typename Elem<WT>::T;
    const int lane = threadIdx.x & 63;
    const int64_t wave0 = ((int64_t)blockIdx.x * kNormThreads + threadIdx.x) >> 6;
    const int64_t waves = ((int64_t)gridDim.x * kNormThreads) >> 6;
    const int D = a.d_model;
    const int chunk = 64 * kNormVec;
    const int nchunks = (D + chunk - 1) / chunk;
    const bool cached = nchunks <= kNormChunks;
    const bool vec = vec_ok != 0;

    for (int64_t r = wave0; r < a.rows; r += waves) {
        float ss = 0.0f;
        if (cached) {
            // Every load of the row (x, update, weight) is issued before the first
            // store, so no store can order the loads behind it (outputs may alias).
            float v[kNormChunks][kNormVec], w[kNormChunks][kNormVec];
#pragma unroll
            for (int c = 0; c < kNormChunks; ++c) {
                const int d0 = c * chunk + lane * kNormVec;
                const int n = c < nchunks ? max(0, min(kNormVec, D - d0)) : 0;
                if (n > 0) {
                    row_chunk<DT, kFused>(a, r, d0, n, vec, v[c]);
                    load8<WT>(reinterpret_cast<const W*>(a.weight) + d0, vec, n, w[c]);
                } else {
#pragma unroll
                    for (int i = 0; i < kNormVec; ++i) v[c][i] = w[c][i] = 0.0f;
                }
            }
#pragma unroll
            for (int c = 0; c < kNormChunks; ++c) {
#pragma unroll
                for (int i = 0; i < kNormVec; ++i) ss += v[c][i] * v[c][i];
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
            if (lane == 0 && a.inv_rms) a.inv_rms[r] = inv;
#pragma unroll
            for (int c = 0; c < kNormChunks; ++c) {
                const int d0 = c * chunk + lane * kNormVec;
                const int n = c < nchunks ? max(0, min(kNormVec, D - d0)) : 0;
                if (n <= 0) continue;
                if constexpr (kFused) store8<DT>(reinterpret_cast<T*>(a.state_out) + r * a.state_stride + d0, vec, n, v[c]);
                float o[kNormVec];
#pragma unroll
                for (int i = 0; i < kNormVec; ++i) o[i] = (v[c][i] * inv) * w[c][i];
                store8<DT>(reinterpret_cast<T*>(a.out) + r * a.out_stride + d0, vec, n, o);
            }
        } else {
            for (int c = 0; c < nchunks; ++c) {
                const int d0 = c * chunk + lane * kNormVec;
                const int n = max(0, min(kNormVec, D - d0));
                float t[kNormVec];
                row_chunk<DT, kFused>(a, r, d0, n, vec, t);
                if constexpr (kFused) {
                    if (n > 0) store8<DT>(reinterpret_cast<T*>(a.state_out) + r * a.state_stride + d0, vec, n, t);
                }
#pragma unroll
                for (int i = 0; i < kNormVec; ++i) ss += t[i] * t[i];
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
            if (lane == 0 && a.inv_rms) a.inv_rms[r] = inv;
            for (int c = 0; c < nchunks; ++c) {
                const int d0 = c * chunk + lane * kNormVec;
                const int n = max(0, min(kNormVec, D - d0));
                if (n <= 0) continue;
                float t[kNormVec], w[kNormVec];
                // The fused form re-reads the rounded sum it stored above.
                if constexpr (kFused)
                    load8<DT>(reinterpret_cast<const T*>(a.state_out) + r * a.state_stride + d0, vec, n, t);
                else
                    row_chunk<DT, false>(a, r, d0, n, vec, t);
                load8<WT>(reinterpret_cast<const W*>(a.weight) + d0, vec, n, w);
#pragma unroll
                for (int i = 0; i < kNormVec; ++i) t[i] = (t[i] * inv) * w[i];
                store8<DT>(reinterpret_cast<T*>(a.out) + r * a.out_stride + d0, vec, n, t);
            }
        }
    }
}

// One workgroup per row (grid-strided over the rows) for aligned rows of up to
// 256 x 8 x VPT elements: thread t owns the 16-byte vectors t, t + 256, ... of the
// row in every tensor, so the row is read once, with 256 independent loads in
// flight per tensor. The sum of squares is reduced across the wave (shuffles)
// and then across the four waves through LDS, with one barrier per row (the LDS
// slot alternates by row parity, so a fast wave writing row r + 2 cannot overwrite
// values a slow wave still reads for row r: the barrier of row r + 1 lies between).
// A decode step's 64 rows then run as 64 workgroups instead of 64 waves.
template <int DT, int WT, bool kFused, int VPT>
__global__ void __launch_bounds__(kNormThreads)
rmsnorm_row_kernel(NormArgs a) {
    using T = typename Elem<DT>::T;
    using W = typename Elem<WT>::T;
    __shared__ float partial[2][kNormThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int D = a.d_model;
    float w[VPT][kNormVec];
#pragma unroll
    for (int k = 0; k < VPT; ++k) {
        const int d0 = (tid + kNormThreads * k) * kNormVec;
        load8<WT>(reinterpret_cast<const W*>(a.weight) + d0, true, d0 < D ? kNormVec : 0, w[k]);
    }
    int parity = 0;
    for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x, parity ^= 1) {
        float v[VPT][kNormVec];
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int d0 = (tid + kNormThreads * k) * kNormVec;
            if (d0 < D) {
                row_chunk<DT, kFused>(a, r, d0, kNormVec, true, v[k]);
            } else {
#pragma unroll
                for (int i = 0; i < kNormVec; ++i) v[k][i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < kNormVec; ++i) ss += v[k][i] * v[k][i];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
        if (lane == 0) partial[parity][wave] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < kNormThreads / 64; ++i) total += partial[parity][i];
        const float inv = 1.0f / sqrtf(total / (float)D + a.eps);
        if (tid == 0 && a.inv_rms) a.inv_rms[r] = inv;
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
            const int d0 = (tid + kNormThreads * k) * kNormVec;
            if (d0 >= D) continue;
            if constexpr (kFused) store8<DT>(reinterpret_cast<T*>(a.state_out) + r * a.state_stride + d0, true, kNormVec, v[k]);
            float o[kNormVec];
#pragma unroll
            for (int i = 0; i < kNormVec; ++i) o[i] = (v[k][i] * inv) * w[k][i];
            store8<DT>(reinterpret_cast<T*>(a.out) + r * a.out_stride + d0, true, kNormVec, o);
        }
    }
}

}  // namespace kvfp8

using namespace kvfp8;

namespace {

int esize(int dt) { return dt == KVFP8_F32 ? 4 : 2; }

bool is_float(int dt) { return dt == KVFP8_F32 || dt == KVFP8_F16 || dt == KVFP8_BF16; }

bool aligned(const void* p, int64_t stride_elems, int es) {
    return p == nullptr || (((uintptr_t)p % 16) == 0 && (stride_elems * es) % 16 == 0);
}

template <int DT, int WT, bool F>
hipError_t launch_norm(const NormArgs& a, hipStream_t s) {
    const int es = esize(DT);
    const bool vec = a.d_model % kNormVec == 0 && aligned(a.x, a.x_stride, es) && aligned(a.out, a.out_stride, es) &&
                     aligned(a.update, a.update_stride, es) && aligned(a.state_out, a.state_stride, es) &&
                     aligned(a.weight, 0, esize(WT));
    // Aligned rows of up to 8192 elements: a workgroup per row (at most 4096
    // workgroups in flight, each then loops over rows).
    const int vectors = (a.d_model + kNormVec - 1) / kNormVec;
    if (vec && vectors <= 4 * kNormThreads) {
        const int vpt = (vectors + kNormThreads - 1) / kNormThreads;
        const dim3 grid((unsigned)(a.rows < 4096 ? a.rows : 4096)), block(kNormThreads);
        if (vpt == 1) hipLaunchKernelGGL((rmsnorm_row_kernel<DT, WT, F, 1>), grid, block, 0, s, a);
        else if (vpt == 2) hipLaunchKernelGGL((rmsnorm_row_kernel<DT, WT, F, 2>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((rmsnorm_row_kernel<DT, WT, F, 4>), grid, block, 0, s, a);
        return hipGetLastError();
    }
    int64_t blocks = (a.rows + 3) / 4;
    blocks = blocks < 1 ? 1 : (blocks > 65536 ? 65536 : blocks);
    hipLaunchKernelGGL((rmsnorm_kernel<DT, WT, F>), dim3((unsigned)blocks), dim3(kNormThreads), 0, s, a, (int)vec);
    return hipGetLastError();
}

template <int DT, bool F>
hipError_t dispatch_weight(const NormArgs& a, int w_dtype, hipStream_t s) {
    switch (w_dtype) {
        case KVFP8_F32: return launch_norm<DT, KVFP8_F32, F>(a, s);
        case KVFP8_F16: return launch_norm<DT, KVFP8_F16, F>(a, s);
        default: return launch_norm<DT, KVFP8_BF16, F>(a, s);
    }
}

template <bool F>
hipError_t dispatch_norm(const NormArgs& a, int dtype, int w_dtype, hipStream_t s) {
    switch (dtype) {
        case KVFP8_F32: return dispatch_weight<KVFP8_F32, F>(a, w_dtype, s);
        case KVFP8_F16: return dispatch_weight<KVFP8_F16, F>(a, w_dtype, s);
        default: return dispatch_weight<KVFP8_BF16, F>(a, w_dtype, s);
    }
}

int check_norm(const void* x, int dtype, int64_t rows, int32_t d_model, const void* weight, int w_dtype,
               const void* out) {
    if (!is_float(dtype) || !is_float(w_dtype)) return KVFP8_EDTYPE;
    if (rows < 0 || d_model <= 0) return KVFP8_ESHAPE;
    if (rows > 0 && (!x || !weight || !out)) return KVFP8_ENULL;
    return KVFP8_OK;
}

}  // namespace

extern "C" int kvfp8_rmsnorm_forward(const void* x, int dtype, int64_t x_stride, int64_t rows, int32_t d_model,
                                     const void* weight, int w_dtype, float eps, void* out, int64_t out_stride,
                                     float* inv_rms, void* stream) {
    const int rc = check_norm(x, dtype, rows, d_model, weight, w_dtype, out);
    if (rc != KVFP8_OK || rows == 0) return rc;
    NormArgs a{x, nullptr, weight, out, nullptr, inv_rms, rows, d_model, x_stride, 0, out_stride, 0, eps};
    return (int)dispatch_norm<false>(a, dtype, w_dtype, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int kvfp8_add_rmsnorm_forward(const void* x, const void* update, int dtype, int64_t x_stride,
                                         int64_t update_stride, int64_t rows, int32_t d_model, const void* weight,
                                         int w_dtype, float eps, void* state_out, int64_t state_stride, void* out,
                                         int64_t out_stride, float* inv_rms, void* stream) {
    int rc = check_norm(x, dtype, rows, d_model, weight, w_dtype, out);
    if (rc != KVFP8_OK || rows == 0) return rc;
    if (!update || !state_out) return KVFP8_ENULL;
    NormArgs a{x, update, weight, out, state_out, inv_rms, rows, d_model, x_stride, update_stride, out_stride,
               state_stride, eps};
    return (int)dispatch_norm<true>(a, dtype, w_dtype, reinterpret_cast<hipStream_t>(stream));
}
