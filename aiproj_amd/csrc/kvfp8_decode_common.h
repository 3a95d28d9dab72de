// Shared pieces of the paged decode kernels: argument block, the sequence
// scheduler that maps a flat work index to (sequence, chunk, head unit) without
// any host synchronization, and the split-K partial layout.
#pragma once

#include "kvfp8_common.h"

#include <hip/hip_ext.h>

namespace kvfp8 {

constexpr float kLog2e = 1.4426950408889634f;

// The two launches of one decode call: the split kernel (partial softmax states,
// and the output rows of sequences it finishes whole) and the reduce kernel (the
// merge of the partial states, zeros for empty sequences).
constexpr int kPhaseSplit = 1;
constexpr int kPhaseReduce = 2;
constexpr float kNegInf = -__builtin_huge_valf();

struct DecodeArgs {
    const void* q;
    int64_t q_stride_b, q_stride_h;
    int32_t batch, num_q_heads, num_kv_heads, head_dim;
    const void* k_cache;
    const void* v_cache;
    const float* k_scales;
    const float* v_scales;
    int64_t num_blocks;
    int32_t block_size;
    int32_t bs_shift;         // log2(block_size)
    const int32_t* block_table;
    int64_t bt_rows, bt_width;
    const void* slots;
    const void* ctx;
    int32_t slots64, ctx64;
    float score_scale;        // sm_scale * log2(e): scores live in the base-2 domain
    void* out;
    // Split-K partial states, one per (sequence, chunk, q head):
    //   part_m/part_l [batch * max_chunks * Hq], part_acc [... * head_dim].
    float* part_m;
    float* part_l;
    float* part_acc;
    int32_t chunk_tokens;     // tokens per work item (a multiple of 16)
    int32_t max_chunks;       // ceil(bt_width * block_size / chunk_tokens)
    int32_t kv_dwords;        // generic kernel: a lane's slice of a K/V row is read as whole dwords
    int32_t q_dtype;          // grouped kernel: element type of q and out (kvfp8_dtype)
    int32_t group_heads;      // grouped kernel: q heads per work unit (of one KV head's group)
    // Fused append (kvfp8_append_paged_decode; new_k is null otherwise): the new
    // token of every sequence, rows [batch, Hkv, D] with element strides (row
    // stride, D, 1), quantized into the cache at (new_blocks[b], new_offsets[b])
    // when that is the sequence's last attended position, before it is attended.
    // Any other location is refused: no write, 1 stored to *new_refused (when not
    // null). Read only by the kernels built for the fused call.
    const void* new_k;
    const void* new_v;
    int32_t new_dtype;
    int32_t new_k_sb, new_v_sb;
    const void* new_blocks;
    const void* new_offsets;
    int32_t new_blocks64, new_offsets64;
    int32_t* new_refused;
};

__device__ __forceinline__ int64_t load_i(const void* p, int is64, int64_t i) {
    return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

// Attended tokens of sequence b: context_lengths[b] clipped to what the block
// table can address (reference decode_attention.py:293-297 masks logical blocks
// at or past the table width), and 0 for a slot outside the table.
__device__ __forceinline__ int64_t seq_tokens(const DecodeArgs& a, int b, int64_t* slot_out,
                                              int64_t* raw_out = nullptr) {
    const int64_t slot = load_i(a.slots, a.slots64, b);
    const int64_t raw = load_i(a.ctx, a.ctx64, b);
    const int64_t cap = a.bt_width * a.block_size;
    int64_t len = raw < 0 ? 0 : (raw > cap ? cap : raw);
    if (slot < 0 || slot >= a.bt_rows) len = 0;
    *slot_out = slot;
    if (raw_out) *raw_out = raw;
    return len;
}

// Fused append + decode: whether sequence b's new token, at position
// context_lengths[b] - 1, is one the decode attends: its slot is a table row and
// 1 <= context_lengths[b] <= bt_width * block_size. Only such a token is written.
__device__ __forceinline__ bool new_token_attended(const DecodeArgs& a, int64_t slot, int64_t raw_len) {
    return slot >= 0 && slot < a.bt_rows && raw_len >= 1 && raw_len <= a.bt_width * a.block_size;
}

__device__ __forceinline__ int32_t seq_chunks(int64_t len, int32_t chunk_tokens) {
    return (int32_t)((len + chunk_tokens - 1) / chunk_tokens);
}

// Exclusive prefix sum of per-sequence chunk counts into LDS:
// prefix[b] = sum_{i<b} chunks_i, prefix[batch] = total. Called by the whole block.
template <int THREADS>
__device__ void build_chunk_prefix(const DecodeArgs& a, int32_t* prefix) {
    __shared__ int32_t partial[THREADS];
    const int per = (a.batch + THREADS - 1) / THREADS;
    const int begin = threadIdx.x * per;
    int32_t local = 0;
    for (int i = 0; i < per; ++i) {
        const int b = begin + i;
        if (b < a.batch) {
            int64_t slot;
            const int32_t c = seq_chunks(seq_tokens(a, b, &slot), a.chunk_tokens);
            prefix[b] = local;
            local += c;
        }
    }
    partial[threadIdx.x] = local;
    __syncthreads();
    // Hillis-Steele inclusive scan of the per-thread totals.
    for (int off = 1; off < THREADS; off <<= 1) {
        const int32_t add = threadIdx.x >= off ? partial[threadIdx.x - off] : 0;
        __syncthreads();
        partial[threadIdx.x] += add;
        __syncthreads();
    }
    const int32_t base = threadIdx.x > 0 ? partial[threadIdx.x - 1] : 0;
    for (int i = 0; i < per; ++i) {
        const int b = begin + i;
        if (b < a.batch) prefix[b] += base;
    }
    if (threadIdx.x == THREADS - 1) prefix[a.batch] = partial[THREADS - 1];
    __syncthreads();
}

// Sequence owning flat chunk index `chunk`: the last b with prefix[b] <= chunk.
__device__ __forceinline__ int find_seq(const int32_t* prefix, int batch, int32_t chunk) {
    int lo = 0, hi = batch - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (prefix[mid] <= chunk) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__device__ __forceinline__ int64_t part_index(const DecodeArgs& a, int b, int c, int hq) {
    return ((int64_t)b * a.max_chunks + c) * a.num_q_heads + hq;
}

template <int QT>
__device__ __forceinline__ float load_q(const DecodeArgs& a, int b, int hq, int d) {
    using T = typename Elem<QT>::T;
    return Elem<QT>::load(reinterpret_cast<const T*>(a.q)[b * a.q_stride_b + hq * a.q_stride_h + d]);
}

template <int QT>
__device__ __forceinline__ void store_out(const DecodeArgs& a, int b, int hq, int d, float x) {
    using T = typename Elem<QT>::T;
    reinterpret_cast<T*>(a.out)[((int64_t)b * a.num_q_heads + hq) * a.head_dim + d] = Elem<QT>::store(x);
}

// Start/stop events of the next timed decode-kernel launch; both null unless a
// benchmark armed kvfp8_timing_enable. The events ride on the dispatch itself
// (hipExtLaunchKernel), so they time the kernel and not the queue around it.
struct KernelTiming {
    hipEvent_t start;
    hipEvent_t stop;
};
KernelTiming next_kernel_timing();

template <typename Kernel, typename... Args>
hipError_t launch_timed(Kernel kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                        const KernelTiming& timing, Args... args) {
    if (timing.start != nullptr)
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, timing.start, timing.stop, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    return hipGetLastError();
}

}  // namespace kvfp8
