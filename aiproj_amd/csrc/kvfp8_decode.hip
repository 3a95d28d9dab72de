// Paged decode attention over the (FP8 or plain) paged KV cache, gfx950.
//
// Replaces `decode_attention_wrapper` and the Triton split / reduction kernels of
// reference src/torch_llm/kernals/decode_attention.py:39-550.
//
// Launch structure (two kernels, one stream, no host synchronization):
//   1. a split kernel. Every workgroup first scans context_lengths into an LDS
//      prefix of per-sequence chunk counts (a chunk is `chunk_tokens` tokens of
//      one sequence), then its waves grid-stride over the flat work list
//      (sequence, chunk, head unit). A sequence that fits one chunk is finished
//      in place; otherwise each chunk leaves a partial softmax state (m, l, acc)
//      in the workspace.
//   2. a combine kernel, one wave per (sequence, q head), that merges the
//      partials of multi-chunk sequences (the reference's reduction kernel,
//      decode_attention.py:437-550) and writes zeros for empty sequences.
// Scores are kept in the base-2 domain (q * sm_scale * log2 e, then exp2).
//
// The split kernels here run on the vector ALU, for every cache dtype:
//   * decode_split_grouped: one wave per (sequence, chunk, KV head, group of up to
//     4 q heads), for 4-byte aligned caches and head sizes D = parts x P with
//     parts in {4, 8, 16} and P in {4, 8, 16, 20};
//   * decode_split_generic: one wave per (sequence, chunk, q head), any head size
//     up to 512 and any alignment.
// The FP8 MFMA kernel in kvfp8_decode_mfma.hip is dispatched when its shape
// conditions hold.
#include "kvfp8_decode_common.h"
#include "kvfp8_decode_mfma.h"

#include <mutex>
#include <vector>

namespace kvfp8 {

constexpr int kDecodeThreads = 256;
constexpr int kWavesPerBlock = kDecodeThreads / 64;
constexpr int kMaxBatch = 8191;          // LDS prefix of (batch + 1) int32 <= 32 KiB
constexpr int kGenericChunkTokens = 256;
constexpr int kMaxGrid = 2048;

// Cache elements as float32, exactly: KvRow<KVT>::unpack converts the kPerDword
// elements of one dword, KvRow<KVT>::one reads and converts element i.
template <int KVT> struct KvRow;
template <> struct KvRow<KVFP8_E4M3FN> {
    static constexpr int kPerDword = 4;
    static __device__ __forceinline__ void unpack(uint32_t w, float* x) {
        // Exact OCP e4m3fn -> float32 conversion, two codes at a time.
        const auto lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
        const auto hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, true);
        x[0] = lo[0];
        x[1] = lo[1];
        x[2] = hi[0];
        x[3] = hi[1];
    }
    static __device__ __forceinline__ float one(const void* p, int64_t i) {
        return decode_e4m3fn(reinterpret_cast<const uint8_t*>(p)[i]);
    }
};
template <> struct KvRow<KVFP8_BF16> {
    static constexpr int kPerDword = 2;
    static __device__ __forceinline__ void unpack(uint32_t w, float* x) {
        x[0] = __builtin_bit_cast(float, w << 16);
        x[1] = __builtin_bit_cast(float, w & 0xFFFF0000u);
    }
    static __device__ __forceinline__ float one(const void* p, int64_t i) {
        return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    }
};
template <> struct KvRow<KVFP8_F16> {
    static constexpr int kPerDword = 2;
    static __device__ __forceinline__ void unpack(uint32_t w, float* x) {
        x[0] = f16_to_f32((uint16_t)(w & 0xFFFFu));
        x[1] = f16_to_f32((uint16_t)(w >> 16));
    }
    static __device__ __forceinline__ float one(const void* p, int64_t i) {
        return f16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    }
};
template <> struct KvRow<KVFP8_F32> {
    static constexpr int kPerDword = 1;
    static __device__ __forceinline__ void unpack(uint32_t w, float* x) { x[0] = __builtin_bit_cast(float, w); }
    static __device__ __forceinline__ float one(const void* p, int64_t i) {
        return reinterpret_cast<const float*>(p)[i];
    }
};

template <int KVT, int DQ>
__device__ __forceinline__ void load_slice(const void* cache, int64_t e, int n, float (&x)[DQ]) {
#pragma unroll
    for (int i = 0; i < DQ; ++i) x[i] = i < n ? KvRow<KVT>::one(cache, e + i) : 0.0f;
}

// A lane's slice of one K or V row as raw dwords (n elements from element e; the
// slice starts on a 4-byte boundary and spans whole dwords), converted at use.
template <int KVT, int DQ>
struct RawSlice {
    static constexpr int kPer = KvRow<KVT>::kPerDword;
    static constexpr int kW = (DQ + kPer - 1) / kPer;
    uint32_t w[kW];
    __device__ __forceinline__ void load(const void* cache, int64_t e, int n) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(cache) + e * (4 / kPer));
#pragma unroll
        for (int i = 0; i < kW; ++i) w[i] = kPer * i < n ? p[i] : 0u;
    }
    __device__ __forceinline__ void clear() {
#pragma unroll
        for (int i = 0; i < kW; ++i) w[i] = 0u;
    }
    // Element i (a compile-time index after unrolling).
    template <int I>
    __device__ __forceinline__ float at() const {
        float y[kPer];
        KvRow<KVT>::unpack(w[I / kPer], y);
        return y[I % kPer];
    }
};

template <int KVT, int DQ, int I = 0>
__device__ __forceinline__ float dot_raw(const RawSlice<KVT, DQ>& r, const float (&q)[DQ]) {
    if constexpr (I == DQ) return 0.0f;
    else return q[I] * r.template at<I>() + dot_raw<KVT, DQ, I + 1>(r, q);
}

template <int KVT, int DQ, int I = 0>
__device__ __forceinline__ void accumulate_raw(const RawSlice<KVT, DQ>& r, float alpha, float pv, float (&acc)[DQ]) {
    if constexpr (I < DQ) {
        acc[I] = acc[I] * alpha + pv * r.template at<I>();
        accumulate_raw<KVT, DQ, I + 1>(r, alpha, pv, acc);
    }
}

// One wave per (sequence, chunk, q head). Lane = (token tok in 0..15, part in
// 0..3); part p covers the P = ceil(D / 4) contiguous head dims [p P, p P + P)
// (so D <= 4 DQ). When the rows and the slices are whole dwords
// (DecodeArgs::kv_dwords) each slice is read with 4-byte loads, and the page-table
// entry and the K and V slices of the next 16 tokens are loaded while the current
// ones are used; otherwise element by element.
template <int KVT, int QT, int DQ>
__global__ void __launch_bounds__(kDecodeThreads)
decode_split_generic(DecodeArgs a) {
    extern __shared__ int32_t prefix[];
    build_chunk_prefix<kDecodeThreads>(a, prefix);

    const int U = a.num_q_heads;
    const int64_t total = (int64_t)prefix[a.batch] * U;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int tok = lane >> 2, part = lane & 3;
    const int G = a.num_q_heads / a.num_kv_heads;
    const int D = a.head_dim;
    const int P = (D + 3) >> 2;
    const int d0 = part * P;
    const int nd = max(0, min(P, D - d0));      // dims of this lane
    const bool dwords = a.kv_dwords != 0;
    const int64_t bs_mask = a.block_size - 1;
    constexpr bool kQuant = KVT == KVFP8_E4M3FN;

    for (int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wave; w < total;
         w += (int64_t)gridDim.x * kWavesPerBlock) {
        const int32_t chunk = (int32_t)(w / U);
        const int hq = (int)(w - (int64_t)chunk * U);
        const int b = find_seq(prefix, a.batch, chunk);
        const int c = chunk - prefix[b];
        const int nchunks = prefix[b + 1] - prefix[b];
        int64_t slot;
        const int64_t len = seq_tokens(a, b, &slot);
        const int h = hq / G;
        const int64_t t0 = (int64_t)c * a.chunk_tokens;
        const int64_t t1 = min(t0 + (int64_t)a.chunk_tokens, len);
        const int32_t* table_row = a.block_table + slot * a.bt_width;

        float qv[DQ], acc[DQ];
#pragma unroll
        for (int i = 0; i < DQ; ++i) {
            qv[i] = i < nd ? load_q<QT>(a, b, hq, d0 + i) * a.score_scale : 0.0f;
            acc[i] = 0.0f;
        }
        float m = kNegInf, l = 0.0f;

        // Cache row of this lane's token in the 16 tokens starting at `base`; valid
        // false past the chunk or on a page outside the pool.
        auto row_of = [&](int64_t base, bool& valid) -> int64_t {
            const int64_t t = base + tok;
            valid = t < t1;
            int64_t row = 0;
            if (valid) {
                const int64_t phys = table_row[t >> a.bs_shift];
                valid = phys >= 0 && phys < a.num_blocks;
                row = ((phys << a.bs_shift) + (t & bs_mask)) * a.num_kv_heads + h;
            }
            return valid ? row : 0;
        };
        // Online softmax per token slot: the four lanes of slot `tok` (tokens tok,
        // tok + 16, ... of the chunk) keep their own max, sum and accumulators, and
        // the 16 slots are merged once, after the chunk.
        auto update = [&](float s, bool valid, float vs, auto&& accumulate) {
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            if (!valid) return;
            const float m_new = fmaxf(m, s);
            const float m_use = m_new == kNegInf ? 0.0f : m_new;
            const float alpha = exp2f(m - m_use);       // 0 while m is -inf
            const float p = exp2f(s - m_use);
            l = l * alpha + p;
            accumulate(alpha, p * vs);
            m = m_new;
        };

        if (dwords) {
            RawSlice<KVT, DQ> kr, vr;
            bool valid;
            int64_t row = row_of(t0, valid);
            float ks = 1.0f, vs = 1.0f;
            if (valid) {
                kr.load(a.k_cache, row * D + d0, nd);
                vr.load(a.v_cache, row * D + d0, nd);
                if (kQuant) {
                    ks = a.k_scales[row];
                    vs = a.v_scales[row];
                }
            } else {
                kr.clear();
                vr.clear();
            }
            for (int64_t base = t0; base < t1; base += 16) {
                // The next 16 tokens' loads go out before this group is used.
                bool nvalid;
                const int64_t nrow = row_of(base + 16, nvalid);
                RawSlice<KVT, DQ> nk, nv;
                float nks = 1.0f, nvs = 1.0f;
                if (nvalid) {
                    nk.load(a.k_cache, nrow * D + d0, nd);
                    nv.load(a.v_cache, nrow * D + d0, nd);
                    if (kQuant) {
                        nks = a.k_scales[nrow];
                        nvs = a.v_scales[nrow];
                    }
                } else {
                    nk.clear();
                    nv.clear();
                }
                const float s = valid ? dot_raw<KVT, DQ>(kr, qv) * ks : 0.0f;
                update(s, valid, vs, [&](float alpha, float pv) { accumulate_raw<KVT, DQ>(vr, alpha, pv, acc); });
                kr = nk;
                vr = nv;
                ks = nks;
                vs = nvs;
                valid = nvalid;
            }
        } else {
            for (int64_t base = t0; base < t1; base += 16) {
                bool valid;
                const int64_t row = row_of(base, valid);
                float s = 0.0f, ks = 1.0f, vs = 1.0f;
                if (valid) {
                    float kx[DQ];
                    load_slice<KVT, DQ>(a.k_cache, row * D + d0, nd, kx);
#pragma unroll
                    for (int i = 0; i < DQ; ++i) s += qv[i] * kx[i];
                    if (kQuant) {
                        ks = a.k_scales[row];
                        vs = a.v_scales[row];
                    }
                }
                update(s * ks, valid, vs, [&](float alpha, float pv) {
                    float vx[DQ];
                    load_slice<KVT, DQ>(a.v_cache, row * D + d0, nd, vx);
#pragma unroll
                    for (int i = 0; i < DQ; ++i) acc[i] = acc[i] * alpha + pv * vx[i];
                });
            }
        }

        // Merge the 16 token slots (lanes l and l ^ off, off = 4 .. 32, hold the same
        // dims of different slots).
#pragma unroll
        for (int off = 4; off < 64; off <<= 1) {
            const float mo = __shfl_xor(m, off);
            const float lo = __shfl_xor(l, off);
            const float mn = fmaxf(m, mo);
            const float mu = mn == kNegInf ? 0.0f : mn;
            const float sa = exp2f(m - mu), sb = exp2f(mo - mu);
            l = l * sa + lo * sb;
#pragma unroll
            for (int i = 0; i < DQ; ++i) acc[i] = acc[i] * sa + __shfl_xor(acc[i], off) * sb;
            m = mn;
        }

        if (nchunks == 1) {
            if (tok == 0) {
                const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
                for (int i = 0; i < DQ; ++i)
                    if (i < nd) store_out<QT>(a, b, hq, d0 + i, l > 0.0f ? acc[i] * inv : 0.0f);
            }
        } else {
            const int64_t pi = part_index(a, b, c, hq);
            if (lane == 0) {
                a.part_m[pi] = m;
                a.part_l[pi] = l;
            }
            if (tok == 0) {
#pragma unroll
                for (int i = 0; i < DQ; ++i)
                    if (i < nd) a.part_acc[pi * D + d0 + i] = acc[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Grouped VALU kernel: one wave per (sequence, chunk, KV head, group of q heads),
// so each K/V row is read once for every q head of its group.
// ---------------------------------------------------------------------------

// DPP lane permutations within rows of 16 lanes.
constexpr int kDppXor1 = 0xB1;          // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;   // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;       // lane i <-> 15 - i within each row
constexpr int kDppRor4 = 0x124;         // rotate each row by 4 lanes
constexpr int kDppRor8 = 0x128;         // rotate each row by 8 lanes

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over lanes l, l ^ 16, l ^ 32 and l ^ 48, through ds_bpermute. (A
// v_permlane16/32_swap of a value with itself would do it without the LDS
// crossbar, but this compiler's optimizer folds an operation on the two results
// of such a swap into an operation on the first result twice.)
__device__ __forceinline__ float sum_rows4(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

// Sum over the `parts` consecutive lanes of one token (parts = 4, 8 or 16); every
// one of them receives the same value (each step adds a commuted pair).
__device__ __forceinline__ float sum_parts(float x, int parts) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    if (parts >= 8) x += dpp<kDppHalfMirror>(x);
    if (parts >= 16) x += dpp<kDppMirror>(x);
    return x;
}

// Sum over the lanes holding the same part of different tokens (lane = token x
// parts + part); every lane receives its part's total.
__device__ __forceinline__ float sum_tokens(float x, int parts) {
    if (parts == 4) x += dpp<kDppRor4>(x);
    if (parts <= 8) x += dpp<kDppRor8>(x);
    return sum_rows4(x);
}

// Maximum over the wave: each row's maximum in all its lanes, then the four rows'
// values read into scalar registers.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<kDppXor1>(x));
    x = fmaxf(x, dpp<kDppXor2>(x));
    x = fmaxf(x, dpp<kDppHalfMirror>(x));
    x = fmaxf(x, dpp<kDppMirror>(x));
    const int u = __builtin_bit_cast(int, x);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// q rows hq0 + g (g < KG; rows past nh repeat row nh - 1), elements d0 .. d0 + P,
// times `scale`. One branch on the q dtype around all the loads, so that they are
// in flight together.
template <int KG, int P>
__device__ __forceinline__ void load_q_group(const DecodeArgs& a, int b, int hq0, int nh, int d0, float scale,
                                             float (&x)[KG][P]) {
    int64_t row[KG];
#pragma unroll
    for (int g = 0; g < KG; ++g)
        row[g] = (int64_t)b * a.q_stride_b + (int64_t)(hq0 + min(g, nh - 1)) * a.q_stride_h + d0;
    if (a.q_dtype == KVFP8_F32) {
        const float* q = reinterpret_cast<const float*>(a.q);
#pragma unroll
        for (int g = 0; g < KG; ++g)
#pragma unroll
            for (int e = 0; e < P; ++e) x[g][e] = q[row[g] + e] * scale;
    } else {
        const uint16_t* q = reinterpret_cast<const uint16_t*>(a.q);
        uint16_t h[KG][P];
#pragma unroll
        for (int g = 0; g < KG; ++g)
#pragma unroll
            for (int e = 0; e < P; ++e) h[g][e] = q[row[g] + e];
        const bool f16 = a.q_dtype == KVFP8_F16;
#pragma unroll
        for (int g = 0; g < KG; ++g)
#pragma unroll
            for (int e = 0; e < P; ++e) x[g][e] = (f16 ? f16_to_f32(h[g][e]) : bf16_to_f32(h[g][e])) * scale;
    }
}

// out[b, hq, d0 .. d0 + P) = x, converted to the q dtype (one branch).
template <int P>
__device__ __forceinline__ void store_out_row(const DecodeArgs& a, int b, int hq, int d0, const float (&x)[P]) {
    const int64_t i0 = ((int64_t)b * a.num_q_heads + hq) * a.head_dim + d0;
    if (a.q_dtype == KVFP8_F32) {
#pragma unroll
        for (int e = 0; e < P; ++e) reinterpret_cast<float*>(a.out)[i0 + e] = x[e];
    } else if (a.q_dtype == KVFP8_F16) {
#pragma unroll
        for (int e = 0; e < P; ++e) reinterpret_cast<uint16_t*>(a.out)[i0 + e] = f32_to_f16(x[e]);
    } else {
#pragma unroll
        for (int e = 0; e < P; ++e) reinterpret_cast<uint16_t*>(a.out)[i0 + e] = f32_to_bf16(x[e]);
    }
}

// A lane's P elements of one K or V row, read with unconditional 4-byte-aligned
// loads (which the compiler merges into 16-byte loads).
template <int KVT, int P>
struct RowSlice {
    static constexpr int kPer = KvRow<KVT>::kPerDword;
    static constexpr int kW = P / kPer;
    static_assert(P % kPer == 0, "a slice spans whole dwords");
    uint32_t w[kW];
    __device__ __forceinline__ void load(const void* cache, int64_t e) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(cache) + e * (4 / kPer));
#pragma unroll
        for (int i = 0; i < kW; ++i) w[i] = p[i];
    }
    __device__ __forceinline__ void unpack(float (&x)[P]) const {
#pragma unroll
        for (int i = 0; i < kW; ++i) KvRow<KVT>::unpack(w[i], x + i * kPer);
    }
};

// Register plan of the grouped kernel: q and the accumulators take 2 x heads x P
// registers, each stage of K/V slices and scales 2 P / (elements per dword) + 3.
// Both stay within 190 of the 256 registers of two waves per SIMD (a budget
// measured on the compiled kernels: the rest hold addresses, unpacked slices and
// softmax state). Heads come first (up to 4: each K/V row is then read once for
// four q heads), then three stages (loads two steps ahead) where they fit, else two.
template <int KVT, int P>
struct GroupedPlan {
    static constexpr int kStage = 2 * P / KvRow<KVT>::kPerDword + 3;
    static constexpr int heads() {
        for (int h = 4; h > 1; --h)
            if (2 * h * P + 2 * kStage <= 190) return h;
        return 1;
    }
    static constexpr int kHeads = heads();
    static constexpr int kStages = 2 * kHeads * P + 3 * kStage <= 190 ? 3 : 2;
};

template <int KVT, int P>
constexpr int grouped_heads() {
    return GroupedPlan<KVT, P>::kHeads;
}

constexpr int kGroupPages = 256;   // page-list entries per wave: one chunk at page size 1
static_assert(kGenericChunkTokens <= kGroupPages, "a chunk's page list fits the wave's LDS region");
constexpr float kRescaleLog2 = 8.0f;  // the reference max moves when a score exceeds it by 2^8

// One wave per (sequence, chunk, KV head, group of `group_heads` q heads).
// Lane = (token tok, part): parts = D / P lanes share a token, part p holding the
// contiguous dims [p P, p P + P) of its K and V rows for every q head of the
// group; a step covers 64 / parts tokens. The page-table entries of the chunk are
// staged once into the wave's LDS region; the next step's K/V slices load while
// the current ones are used.
// Softmax: a wave-uniform reference max per head that moves only when some score
// exceeds it by 2^8 (then the accumulators are rescaled); each token's probability
// is exp2(s - max) <= 256. The token slots are summed once, after the chunk.
template <int KVT, int P>
__global__ void __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(2)))
decode_split_grouped(DecodeArgs a) {
    extern __shared__ int32_t prefix[];
    build_chunk_prefix<kDecodeThreads>(a, prefix);
    constexpr int kGH = grouped_heads<KVT, P>();
    constexpr bool kQuant = KVT == KVFP8_E4M3FN;
    using Slice = RowSlice<KVT, P>;

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int32_t* pages = prefix + ((a.batch + 4) & ~3) + wave * kGroupPages;
    const int D = a.head_dim;
    const int parts = D / P;                                   // 4, 8 or 16
    const int pshift = parts == 4 ? 2 : (parts == 8 ? 3 : 4);
    const int tok = lane >> pshift, part = lane & (parts - 1);
    const int step = 64 >> pshift;
    const int d0 = part * P;
    const int G = a.num_q_heads / a.num_kv_heads;
    const int gh = a.group_heads;
    const int ngroups = (G + gh - 1) / gh;
    const int U = a.num_kv_heads * ngroups;
    const int64_t total = (int64_t)prefix[a.batch] * U;
    const int64_t bs_mask = a.block_size - 1;

    for (int64_t w = (int64_t)blockIdx.x * kWavesPerBlock + wave; w < total;
         w += (int64_t)gridDim.x * kWavesPerBlock) {
        const int32_t chunk = (int32_t)(w / U);
        const int r = (int)(w - (int64_t)chunk * U);
        const int h = r / ngroups, grp = r - h * ngroups;
        const int hq0 = h * G + grp * gh;
        const int nh = min(gh, G - grp * gh);
        const int b = find_seq(prefix, a.batch, chunk);
        const int c = chunk - prefix[b];
        const int nchunks = prefix[b + 1] - prefix[b];
        int64_t slot;
        const int64_t len = seq_tokens(a, b, &slot);
        const int64_t t0 = (int64_t)c * a.chunk_tokens;
        const int64_t t1 = min(t0 + (int64_t)a.chunk_tokens, len);
        const int32_t* table_row = a.block_table + slot * a.bt_width;
        const int64_t first_page = t0 >> a.bs_shift;
        const int npages = (int)(((t1 - 1) >> a.bs_shift) - first_page + 1);
        // LDS accesses of one wave complete in order: the reads below see these
        // writes, and the previous unit's reads are done before they land.
        for (int i = lane; i < npages; i += 64) pages[i] = table_row[first_page + i];

        float qv[kGH][P], acc[kGH][P], m[kGH], l[kGH];
        load_q_group<kGH, P>(a, b, hq0, nh, d0, a.score_scale, qv);
#pragma unroll
        for (int g = 0; g < kGH; ++g) {
#pragma unroll
            for (int e = 0; e < P; ++e) acc[g][e] = 0.0f;
            m[g] = kNegInf;
            l[g] = 0.0f;
        }

        // One step's K/V slices and scales in registers.
        struct Stage {
            Slice k, v;
            float ks, vs;
            bool valid;
        };
        // Loads of the step at `base` for this lane's token. The loads are
        // unconditional, so that the compiler counts them exactly and waits for each
        // stage alone: a lane whose token lies past the chunk or on a page outside
        // the pool reads row 0 of the pool instead and is marked invalid; `use`
        // ignores its K and zeroes its V and V scale.
        auto fetch = [&](int64_t base, Stage& st) __attribute__((always_inline)) {
            const int64_t t = base + tok;
            bool valid = t < t1;
            int64_t row = 0;
            if (valid) {
                const int64_t phys = pages[(int)((t >> a.bs_shift) - first_page)];
                valid = phys >= 0 && phys < a.num_blocks;
                row = valid ? ((phys << a.bs_shift) + (t & bs_mask)) * a.num_kv_heads + h : 0;
            }
            st.k.load(a.k_cache, row * D + d0);
            st.v.load(a.v_cache, row * D + d0);
            if (kQuant) {
                st.ks = a.k_scales[row];
                st.vs = a.v_scales[row];
            } else {
                st.ks = 1.0f;
                st.vs = 1.0f;
            }
            st.valid = valid;
        };
        // Scores, softmax update and PV product of one step.
        auto use = [&](Stage& st) __attribute__((always_inline)) {
            const bool valid = st.valid;
            float kx[P];
            st.k.unpack(kx);
            float s[kGH];
            bool need = false;
#pragma unroll
            for (int g = 0; g < kGH; ++g) {
                s[g] = kNegInf;
                if (g >= nh) continue;
                float x = 0.0f;
#pragma unroll
                for (int e = 0; e < P; ++e) x += qv[g][e] * kx[e];
                s[g] = valid ? sum_parts(x, parts) * st.ks : kNegInf;
                need |= valid && s[g] > m[g] + kRescaleLog2;
            }
            if (__any(need)) {
#pragma unroll
                for (int g = 0; g < kGH; ++g) {
                    if (g >= nh) break;
                    const float mn = fmaxf(m[g], wave_max(s[g]));
                    const float alpha = m[g] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m[g] - mn);
                    l[g] *= alpha;
#pragma unroll
                    for (int e = 0; e < P; ++e) acc[g][e] *= alpha;
                    m[g] = mn;
                }
            }
#pragma unroll
            for (int i = 0; i < Slice::kW; ++i) st.v.w[i] = valid ? st.v.w[i] : 0u;
            const float vs = valid ? st.vs : 0.0f;
            float vx[P];
            st.v.unpack(vx);
#pragma unroll
            for (int g = 0; g < kGH; ++g) {
                if (g >= nh) break;
                const float p = valid ? __builtin_amdgcn_exp2f(s[g] - m[g]) : 0.0f;
                l[g] += p;
                const float pv = p * vs;
#pragma unroll
                for (int e = 0; e < P; ++e) acc[g][e] += pv * vx[e];
            }
        };

        // kStages stages in a ring, loads kStages - 1 steps ahead of use; the loop is
        // unrolled by kStages so that no stage is copied (a copy would wait for its
        // loads).
        if constexpr (GroupedPlan<KVT, P>::kStages == 3) {
            Stage s0, s1, s2;
            fetch(t0, s0);
            fetch(t0 + step, s1);
            for (int64_t base = t0;; base += 3 * step) {
                fetch(base + 2 * step, s2);
                use(s0);
                if (base + step >= t1) break;
                fetch(base + 3 * step, s0);
                use(s1);
                if (base + 2 * step >= t1) break;
                fetch(base + 4 * step, s1);
                use(s2);
                if (base + 3 * step >= t1) break;
            }
        } else {
            Stage s0, s1;
            fetch(t0, s0);
            for (int64_t base = t0;; base += 2 * step) {
                fetch(base + step, s1);
                use(s0);
                if (base + step >= t1) break;
                fetch(base + 2 * step, s0);
                use(s1);
                if (base + 2 * step >= t1) break;
            }
        }

        // Sum the token slots; lanes tok == 0 write their part's dims.
#pragma unroll
        for (int g = 0; g < kGH; ++g) {
            l[g] = sum_tokens(l[g], parts);
#pragma unroll
            for (int e = 0; e < P; ++e) acc[g][e] = sum_tokens(acc[g][e], parts);
        }
        if (nchunks == 1) {
            if (tok == 0) {
#pragma unroll
                for (int g = 0; g < kGH; ++g) {
                    if (g >= nh) break;
                    const float inv = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
                    float o[P];
#pragma unroll
                    for (int e = 0; e < P; ++e) o[e] = l[g] > 0.0f ? acc[g][e] * inv : 0.0f;
                    store_out_row<P>(a, b, hq0 + g, d0, o);
                }
            }
        } else {
#pragma unroll
            for (int g = 0; g < kGH; ++g) {
                if (g >= nh) break;
                const int64_t pi = part_index(a, b, c, hq0 + g);
                if (lane == 0) {
                    a.part_m[pi] = m[g];
                    a.part_l[pi] = l[g];
                }
                if (tok == 0) {
#pragma unroll
                    for (int e = 0; e < P; ++e) a.part_acc[pi * D + d0 + e] = acc[g][e];
                }
            }
        }
    }
}

// Merge of split-K partials, reference decode_attention.py:437-550:
//   M = max_c m_c; den = sum_c 2^(m_c - M) l_c; num = sum_c 2^(m_c - M) acc_c
//   out = den > 0 ? num / den : 0
// One wave per (sequence, q head); sequences with one chunk were written by the
// split kernel, sequences with none get zeros here. The chunks' (m, l) are read one
// per lane, 64 chunks at a time, and each lane keeps its chunk's weight; the
// accumulator rows (lane = dims d, d + 64, ...; ND = ceil(D / 64)) are read four
// chunks at a time with unconditional loads, so that they are in flight together,
// each weighted by its chunk's weight read from that chunk's lane.
template <int QT, int ND>
__global__ void __launch_bounds__(kDecodeThreads)
decode_combine(DecodeArgs a) {
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int64_t pair = (int64_t)blockIdx.x * kWavesPerBlock + wave;
    if (pair >= (int64_t)a.batch * a.num_q_heads) return;
    const int b = (int)(pair / a.num_q_heads);
    const int hq = (int)(pair - (int64_t)b * a.num_q_heads);
    int64_t slot;
    const int n = seq_chunks(seq_tokens(a, b, &slot), a.chunk_tokens);
    if (n == 1) return;
    const int D = a.head_dim;
    if (n == 0) {
        for (int d = lane; d < D; d += 64) store_out<QT>(a, b, hq, d, 0.0f);
        return;
    }
    // Consecutive chunks of one (sequence, q head) are num_q_heads states apart.
    const int64_t p0 = part_index(a, b, 0, hq);
    const int64_t cs = a.num_q_heads;
    float M = kNegInf;
    for (int c0 = 0; c0 < n; c0 += 64) {
        const int c = c0 + lane;
        M = fmaxf(M, wave_max(c < n ? a.part_m[p0 + (int64_t)c * cs] : kNegInf));
    }
    int dd[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) dd[i] = min(lane + 64 * i, D - 1);
    float num[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) num[i] = 0.0f;
    float den = 0.0f;
    for (int c0 = 0; c0 < n; c0 += 64) {
        const int c = c0 + lane;
        float w = 0.0f;
        if (c < n && M != kNegInf) {
            const int64_t pi = p0 + (int64_t)c * cs;
            w = exp2f(a.part_m[pi] - M);
            den += w * a.part_l[pi];
        }
        const int cn = min(64, n - c0);
        int j = 0;
        for (; j + 4 <= cn; j += 4) {
            float x[4][ND];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float* row = a.part_acc + (p0 + (int64_t)(c0 + j + u) * cs) * D;
#pragma unroll
                for (int i = 0; i < ND; ++i) x[u][i] = row[dd[i]];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), j + u));
#pragma unroll
                for (int i = 0; i < ND; ++i) num[i] += wj * x[u][i];
            }
        }
        for (; j < cn; ++j) {
            const float* row = a.part_acc + (p0 + (int64_t)(c0 + j) * cs) * D;
            const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), j));
#pragma unroll
            for (int i = 0; i < ND; ++i) num[i] += wj * row[dd[i]];
        }
    }
    den += dpp<kDppXor1>(den);
    den += dpp<kDppXor2>(den);
    den += dpp<kDppHalfMirror>(den);
    den += dpp<kDppMirror>(den);
    den = sum_rows4(den);
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const int d = lane + 64 * i;
        if (d < D) store_out<QT>(a, b, hq, d, den > 0.0f ? num[i] / den : 0.0f);
    }
}

}  // namespace kvfp8

using namespace kvfp8;

namespace {

// New tokens of a fused append + decode call (kvfp8_append_paged_decode).
struct NewTokens {
    const void* k;
    const void* v;
    int dtype;
    int32_t k_sb, v_sb;
    const void* blocks;
    const void* offsets;
    int blocks64, offsets64;
    int32_t* refused;
};

struct Plan {
    bool mfma;
    int32_t chunk_tokens;   // generic kernel
    int32_t max_chunks;
};

Plan make_plan(int32_t batch, int32_t hq, int32_t hkv, int32_t d, int64_t bt_width, int32_t bs, int kv_dtype) {
    Plan p;
    p.mfma = mfma_decode_supported(batch, hq, hkv, d, bt_width, bs, kv_dtype);
    p.chunk_tokens = kGenericChunkTokens;
    const int64_t cap = bt_width * bs;
    p.max_chunks = (int32_t)((cap + p.chunk_tokens - 1) / p.chunk_tokens);
    return p;
}

bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int ilog2(int64_t x) {
    int s = 0;
    while ((int64_t)1 << s < x) ++s;
    return s;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int64_t generic_workspace(const Plan& p, int32_t batch, int32_t hq, int32_t d) {
    const int64_t states = (int64_t)batch * p.max_chunks * hq;
    return (int64_t)(2 * align256(states * sizeof(float)) + align256(states * d * sizeof(float)));
}

// The MFMA path falls back to the vector-ALU kernels (grouped or generic, which
// share this workspace layout) when a pointer is not 16-byte aligned, so the size
// quoted from shapes alone covers every kernel the call may take.
int64_t workspace_for(const Plan& p, int32_t batch, int32_t hq, int32_t hkv, int32_t d) {
    int64_t need = generic_workspace(p, batch, hq, d);
    if (p.mfma) {
        int64_t off[4];
        const int64_t m = mfma_workspace_layout(batch, hq, hkv, d, off);
        need = need > m ? need : m;
    }
    return need;
}

// What the kernel a call actually takes needs (its pointers decide MFMA or generic).
int64_t workspace_taken(const Plan& p, bool mfma, int32_t batch, int32_t hq, int32_t hkv, int32_t d) {
    if (!mfma) return generic_workspace(p, batch, hq, d);
    int64_t off[4];
    return mfma_workspace_layout(batch, hq, hkv, d, off);
}

// Workspace of kvfp8_paged_decode_noalloc: one static array per device, in place
// of a caller's allocation. Host code never uses the symbol itself (its host-side
// name is a stand-in, not a device address): the address comes from
// hipGetSymbolAddress, fetched once per device with that device current and kept
// in scratch_ptr. Nothing in it needs clearing: the decode kernels write every
// byte they read back (tile plan, then partial states) within one call.
constexpr int64_t kScratchBytes = KVFP8_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
void* scratch_ptr[kMaxDevices] = {};
std::mutex scratch_mutex;

// The current device's scratch address, looked up on the first call per device.
int device_scratch(void** out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return (int)err;
    if (dev < 0 || dev >= kMaxDevices) return KVFP8_ELIMIT;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return (int)err;
        if (p == nullptr) return (int)hipErrorInvalidSymbol;
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return KVFP8_OK;
}

template <int KVT, int QT>
hipError_t launch_generic(const DecodeArgs& a, int64_t units_total, hipStream_t s) {
    const size_t lds = (size_t)(a.batch + 1) * sizeof(int32_t);
    int64_t blocks = (units_total + kWavesPerBlock - 1) / kWavesPerBlock;
    blocks = blocks < 1 ? 1 : (blocks > kMaxGrid ? kMaxGrid : blocks);
    const dim3 grid((unsigned)blocks), block(kDecodeThreads);
    const KernelTiming timing = next_kernel_timing();
    if (a.head_dim <= 128) return launch_timed(decode_split_generic<KVT, QT, 32>, grid, block, lds, s, timing, a);
    if (a.head_dim <= 256) return launch_timed(decode_split_generic<KVT, QT, 64>, grid, block, lds, s, timing, a);
    return launch_timed(decode_split_generic<KVT, QT, 128>, grid, block, lds, s, timing, a);
}

// Slice width P of the grouped kernel for head size d, or 0 when it does not take
// the shape: d = parts x P with parts in {4, 8, 16} and P in {4, 8, 16, 20}.
int grouped_slice(int d) {
    for (int parts = 4; parts <= 16; parts *= 2) {
        if (d % parts != 0) continue;
        const int p = d / parts;
        if (p == 4 || p == 8 || p == 16 || p == 20) return p;
    }
    return 0;
}

template <int KVT, int P>
hipError_t launch_grouped_p(DecodeArgs a, const Plan& p, hipStream_t s) {
    constexpr int kGH = grouped_heads<KVT, P>();
    const int G = a.num_q_heads / a.num_kv_heads;
    const int ngroups = (G + kGH - 1) / kGH;
    a.group_heads = (G + ngroups - 1) / ngroups;          // balanced groups of at most kGH heads
    const int64_t units = (int64_t)a.batch * p.max_chunks * a.num_kv_heads * ngroups;
    const size_t lds = (size_t)((a.batch + 4) & ~3) * sizeof(int32_t) +
                       (size_t)kWavesPerBlock * kGroupPages * sizeof(int32_t);
    int64_t blocks = (units + kWavesPerBlock - 1) / kWavesPerBlock;
    blocks = blocks < 1 ? 1 : (blocks > kMaxGrid ? kMaxGrid : blocks);
    return launch_timed(decode_split_grouped<KVT, P>, dim3((unsigned)blocks), dim3(kDecodeThreads), lds, s,
                        next_kernel_timing(), a);
}

template <int KVT>
hipError_t launch_grouped(const DecodeArgs& a, int slice, const Plan& p, hipStream_t s) {
    switch (slice) {
        case 4: return launch_grouped_p<KVT, 4>(a, p, s);
        case 8: return launch_grouped_p<KVT, 8>(a, p, s);
        case 16: return launch_grouped_p<KVT, 16>(a, p, s);
        default: return launch_grouped_p<KVT, 20>(a, p, s);
    }
}

template <int QT>
hipError_t launch_combine(const DecodeArgs& a, hipStream_t s) {
    const int64_t pairs = (int64_t)a.batch * a.num_q_heads;
    const dim3 grid((unsigned)((pairs + kWavesPerBlock - 1) / kWavesPerBlock)), block(kDecodeThreads);
    if (a.head_dim <= 64) hipLaunchKernelGGL((decode_combine<QT, 1>), grid, block, 0, s, a);
    else if (a.head_dim <= 128) hipLaunchKernelGGL((decode_combine<QT, 2>), grid, block, 0, s, a);
    else if (a.head_dim <= 256) hipLaunchKernelGGL((decode_combine<QT, 4>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((decode_combine<QT, 8>), grid, block, 0, s, a);
    return hipGetLastError();
}

// Event pairs of timed decode-kernel launches, armed by kvfp8_timing_enable.
struct DecodeTiming {
    std::vector<hipEvent_t> start, stop;
    int32_t armed = 0;
    int32_t used = 0;
};
DecodeTiming g_timing;

}  // namespace

KernelTiming kvfp8::next_kernel_timing() {
    if (g_timing.used >= g_timing.armed) return KernelTiming{nullptr, nullptr};
    const int32_t i = g_timing.used++;
    return KernelTiming{g_timing.start[i], g_timing.stop[i]};
}

namespace {

// Whether a call runs on the MFMA kernel: the plan allows it, the caches are
// 16-byte aligned, an f16 cache comes with f16 q, and slot * 32 + count fits the
// kernel's int32 per sequence.
bool takes_mfma(const Plan& p, const void* k_cache, const void* v_cache, int64_t bt_rows, int q_dtype,
                int kv_dtype) {
    const bool aligned = (((uintptr_t)k_cache | (uintptr_t)v_cache) & 15) == 0;
    // An f16 cache runs on f16 products, which take f16 q exactly and nothing else.
    const bool operands = kv_dtype != KVFP8_F16 || q_dtype == KVFP8_F16;
    return p.mfma && aligned && operands && bt_rows < ((int64_t)1 << 26);
}

template <int QT>
hipError_t dispatch_kv(const DecodeArgs& a, int kv_dtype, const Plan& p, void* workspace, hipStream_t s,
                       int phases) {
    if (takes_mfma(p, a.k_cache, a.v_cache, a.bt_rows, a.q_dtype, kv_dtype))
        return launch_mfma_decode<QT>(a, kv_dtype, workspace, s, phases);
    if (phases & kPhaseSplit) {
        const int64_t units_total = (int64_t)a.batch * p.max_chunks * a.num_q_heads;
        // The grouped kernel reads whole dwords: 4-byte aligned caches, and a head
        // size it splits into slices.
        const bool aligned4 = (((uintptr_t)a.k_cache | (uintptr_t)a.v_cache) & 3) == 0;
        const int slice = aligned4 ? grouped_slice(a.head_dim) : 0;
        hipError_t err;
        if (slice != 0) {
            switch (kv_dtype) {
                case KVFP8_E4M3FN: err = launch_grouped<KVFP8_E4M3FN>(a, slice, p, s); break;
                case KVFP8_BF16: err = launch_grouped<KVFP8_BF16>(a, slice, p, s); break;
                case KVFP8_F16: err = launch_grouped<KVFP8_F16>(a, slice, p, s); break;
                default: err = launch_grouped<KVFP8_F32>(a, slice, p, s); break;
            }
        } else switch (kv_dtype) {
            case KVFP8_E4M3FN: err = launch_generic<KVFP8_E4M3FN, QT>(a, units_total, s); break;
            case KVFP8_BF16: err = launch_generic<KVFP8_BF16, QT>(a, units_total, s); break;
            case KVFP8_F16: err = launch_generic<KVFP8_F16, QT>(a, units_total, s); break;
            default: err = launch_generic<KVFP8_F32, QT>(a, units_total, s); break;
        }
        if (err != hipSuccess) return err;
    }
    if (!(phases & kPhaseReduce)) return hipSuccess;
    return launch_combine<QT>(a, s);
}

int paged_decode(const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h, int32_t batch,
                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, const void* k_cache,
                 const void* v_cache, int kv_dtype, const float* k_scales, const float* v_scales,
                 int64_t num_blocks, int32_t block_size, const int32_t* block_table, int64_t bt_rows,
                 int64_t bt_width, const void* slots, int slots_dtype, const void* context_lengths, int ctx_dtype,
                 float sm_scale, void* out, void* workspace, int64_t workspace_bytes, void* stream, int phases,
                 const NewTokens* fresh, bool use_scratch = false);

}  // namespace

extern "C" int64_t kvfp8_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                                int32_t head_dim, int64_t bt_width, int32_t block_size,
                                                int kv_dtype) {
    if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || bt_width <= 0 ||
        block_size <= 0)
        return 0;
    const Plan p = make_plan(batch, num_q_heads, num_kv_heads, head_dim, bt_width, block_size, kv_dtype);
    return workspace_for(p, batch, num_q_heads, num_kv_heads, head_dim);
}

// The three decode entry points share one argument list; they differ in which
// of the two launches they enqueue.
#define KVFP8_DECODE_PARAMS                                                                                  \
    const void *q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h, int32_t batch, int32_t num_q_heads,  \
        int32_t num_kv_heads, int32_t head_dim, const void *k_cache, const void *v_cache, int kv_dtype,      \
        const float *k_scales, const float *v_scales, int64_t num_blocks, int32_t block_size,                \
        const int32_t *block_table, int64_t bt_rows, int64_t bt_width, const void *slots, int slots_dtype,   \
        const void *context_lengths, int ctx_dtype, float sm_scale, void *out, void *workspace,              \
        int64_t workspace_bytes, void *stream
#define KVFP8_DECODE_ARGS                                                                                    \
    q, q_dtype, q_stride_b, q_stride_h, batch, num_q_heads, num_kv_heads, head_dim, k_cache, v_cache,        \
        kv_dtype, k_scales, v_scales, num_blocks, block_size, block_table, bt_rows, bt_width, slots,         \
        slots_dtype, context_lengths, ctx_dtype, sm_scale, out, workspace, workspace_bytes, stream

extern "C" int kvfp8_paged_decode(KVFP8_DECODE_PARAMS) {
    return paged_decode(KVFP8_DECODE_ARGS, kPhaseSplit | kPhaseReduce, nullptr);
}

extern "C" int kvfp8_paged_decode_split(KVFP8_DECODE_PARAMS) {
    return paged_decode(KVFP8_DECODE_ARGS, kPhaseSplit, nullptr);
}

extern "C" int kvfp8_paged_decode_reduce(KVFP8_DECODE_PARAMS) {
    return paged_decode(KVFP8_DECODE_ARGS, kPhaseReduce, nullptr);
}

// kvfp8_paged_decode with the library's per-device static scratch array as its
// workspace: no allocation, and sizes whose workspace would not fit are refused.
extern "C" int kvfp8_paged_decode_noalloc(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h, int32_t batch, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, const void* k_cache, const void* v_cache, int kv_dtype,
    const float* k_scales, const float* v_scales, int64_t num_blocks, int32_t block_size,
    const int32_t* block_table, int64_t bt_rows, int64_t bt_width, const void* slots, int slots_dtype,
    const void* context_lengths, int ctx_dtype, float sm_scale, void* out, void* stream) {
    return paged_decode(q, q_dtype, q_stride_b, q_stride_h, batch, num_q_heads, num_kv_heads, head_dim, k_cache,
                        v_cache, kv_dtype, k_scales, v_scales, num_blocks, block_size, block_table, bt_rows,
                        bt_width, slots, slots_dtype, context_lengths, ctx_dtype, sm_scale, out, nullptr, 0, stream,
                        kPhaseSplit | kPhaseReduce, nullptr, true);
}

extern "C" int kvfp8_append_decode_supported(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                             int32_t head_dim, int64_t bt_rows, int64_t bt_width,
                                             int32_t block_size, int kv_dtype) {
    if (kv_dtype != KVFP8_E4M3FN || batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || bt_rows <= 0 ||
        bt_width <= 0 || !pow2(block_size) || num_q_heads % num_kv_heads != 0)
        return 0;
    const Plan p = make_plan(batch, num_q_heads, num_kv_heads, head_dim, bt_width, block_size, kv_dtype);
    return p.mfma && bt_rows < ((int64_t)1 << 26) ? 1 : 0;
}

extern "C" int kvfp8_append_paged_decode(KVFP8_DECODE_PARAMS, const void* k_new, const void* v_new, int new_dtype,
                                         int64_t k_new_stride_b, int64_t k_new_stride_h, int64_t v_new_stride_b,
                                         int64_t v_new_stride_h, const void* new_blocks, int new_blocks_dtype,
                                         const void* new_offsets, int new_offsets_dtype, int32_t* refused) {
    if (new_dtype != KVFP8_F32 && new_dtype != KVFP8_F16 && new_dtype != KVFP8_BF16) return KVFP8_EDTYPE;
    if ((new_blocks_dtype != KVFP8_I32 && new_blocks_dtype != KVFP8_I64) ||
        (new_offsets_dtype != KVFP8_I32 && new_offsets_dtype != KVFP8_I64))
        return KVFP8_EDTYPE;
    if (batch > 0 && (!k_new || !v_new || !new_blocks || !new_offsets)) return KVFP8_ENULL;
    // Heads are contiguous within a row; row strides are int32 element counts.
    if (k_new_stride_h != head_dim || v_new_stride_h != head_dim || k_new_stride_b < 0 || v_new_stride_b < 0 ||
        k_new_stride_b > INT32_MAX || v_new_stride_b > INT32_MAX)
        return KVFP8_ESTRIDE;
    const NewTokens fresh{k_new,
                          v_new,
                          new_dtype,
                          (int32_t)k_new_stride_b,
                          (int32_t)v_new_stride_b,
                          new_blocks,
                          new_offsets,
                          new_blocks_dtype == KVFP8_I64,
                          new_offsets_dtype == KVFP8_I64,
                          refused};
    return paged_decode(KVFP8_DECODE_ARGS, kPhaseSplit | kPhaseReduce, &fresh);
}

namespace {

int paged_decode(const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h, int32_t batch,
                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, const void* k_cache,
                 const void* v_cache, int kv_dtype, const float* k_scales, const float* v_scales,
                 int64_t num_blocks, int32_t block_size, const int32_t* block_table, int64_t bt_rows,
                 int64_t bt_width, const void* slots, int slots_dtype, const void* context_lengths, int ctx_dtype,
                 float sm_scale, void* out, void* workspace, int64_t workspace_bytes, void* stream, int phases,
                 const NewTokens* fresh, bool use_scratch) {
    if (q_dtype != KVFP8_F32 && q_dtype != KVFP8_F16 && q_dtype != KVFP8_BF16) return KVFP8_EDTYPE;
    if (kv_dtype != KVFP8_E4M3FN && kv_dtype != KVFP8_BF16 && kv_dtype != KVFP8_F16 && kv_dtype != KVFP8_F32)
        return KVFP8_EDTYPE;
    if ((slots_dtype != KVFP8_I32 && slots_dtype != KVFP8_I64) || (ctx_dtype != KVFP8_I32 && ctx_dtype != KVFP8_I64))
        return KVFP8_EDTYPE;
    if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0 ||
        bt_rows <= 0 || bt_width <= 0 || num_q_heads % num_kv_heads != 0 || !pow2(block_size))
        return KVFP8_ESHAPE;
    if (batch == 0) return KVFP8_OK;
    if (batch > kMaxBatch || head_dim > 512) return KVFP8_ELIMIT;
    if (!q || !k_cache || !v_cache || !block_table || !slots || !context_lengths || !out) return KVFP8_ENULL;
    if (kv_dtype == KVFP8_E4M3FN && (!k_scales || !v_scales)) return KVFP8_ENULL;

    const Plan p = make_plan(batch, num_q_heads, num_kv_heads, head_dim, bt_width, block_size, kv_dtype);
    const bool mfma = takes_mfma(p, k_cache, v_cache, bt_rows, q_dtype, kv_dtype);
    const int64_t need = workspace_taken(p, mfma, batch, num_q_heads, num_kv_heads, head_dim);
    if (use_scratch) {
        if (need > kScratchBytes) return KVFP8_ELIMIT;
        const int rc = device_scratch(&workspace);
        if (rc != KVFP8_OK) return rc;
        workspace_bytes = kScratchBytes;
    }
    if (!workspace || workspace_bytes < need) return KVFP8_EWORKSPACE;
    // The fused append runs inside the MFMA kernel over an e4m3fn cache only.
    if (fresh && (kv_dtype != KVFP8_E4M3FN || !mfma)) return KVFP8_ESHAPE;

    const int64_t states = (int64_t)batch * p.max_chunks * num_q_heads;
    char* ws = reinterpret_cast<char*>(workspace);
    DecodeArgs a;
    a.q = q;
    a.q_stride_b = q_stride_b;
    a.q_stride_h = q_stride_h;
    a.batch = batch;
    a.num_q_heads = num_q_heads;
    a.num_kv_heads = num_kv_heads;
    a.head_dim = head_dim;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_scales = k_scales;
    a.v_scales = v_scales;
    a.num_blocks = num_blocks;
    a.block_size = block_size;
    a.bs_shift = ilog2(block_size);
    a.block_table = block_table;
    a.bt_rows = bt_rows;
    a.bt_width = bt_width;
    a.slots = slots;
    a.ctx = context_lengths;
    a.slots64 = slots_dtype == KVFP8_I64;
    a.ctx64 = ctx_dtype == KVFP8_I64;
    a.score_scale = sm_scale * kLog2e;
    a.out = out;
    a.part_m = reinterpret_cast<float*>(ws);
    a.part_l = reinterpret_cast<float*>(ws + align256(states * sizeof(float)));
    a.part_acc = reinterpret_cast<float*>(ws + 2 * align256(states * sizeof(float)));
    a.chunk_tokens = p.chunk_tokens;
    a.max_chunks = p.max_chunks;
    {
        // Dword slices: each lane's P = D / 4 dims are whole dwords (D a multiple of
        // 4 elements per dword x 4 parts) and the caches are 4-byte aligned.
        const int esize = kv_dtype == KVFP8_E4M3FN ? 1 : kv_dtype == KVFP8_F32 ? 4 : 2;
        const int per_dword = 4 / esize;
        const bool aligned = (((uintptr_t)k_cache | (uintptr_t)v_cache) & 3) == 0;
        a.kv_dwords = aligned && head_dim % (4 * per_dword) == 0 ? 1 : 0;
    }
    a.q_dtype = q_dtype;
    a.group_heads = 1;
    a.new_k = fresh ? fresh->k : nullptr;
    a.new_v = fresh ? fresh->v : nullptr;
    a.new_dtype = fresh ? fresh->dtype : KVFP8_BF16;
    a.new_k_sb = fresh ? fresh->k_sb : 0;
    a.new_v_sb = fresh ? fresh->v_sb : 0;
    a.new_blocks = fresh ? fresh->blocks : nullptr;
    a.new_offsets = fresh ? fresh->offsets : nullptr;
    a.new_blocks64 = fresh ? fresh->blocks64 : 0;
    a.new_offsets64 = fresh ? fresh->offsets64 : 0;
    a.new_refused = fresh ? fresh->refused : nullptr;

    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t err;
    switch (q_dtype) {
        case KVFP8_F32: err = dispatch_kv<KVFP8_F32>(a, kv_dtype, p, workspace, s, phases); break;
        case KVFP8_F16: err = dispatch_kv<KVFP8_F16>(a, kv_dtype, p, workspace, s, phases); break;
        default: err = dispatch_kv<KVFP8_BF16>(a, kv_dtype, p, workspace, s, phases); break;
    }
    return (int)err;
}

}  // namespace

extern "C" const char* kvfp8_strerror(int code) {
    switch (code) {
        case KVFP8_OK: return "ok";
        case KVFP8_EDTYPE: return "unsupported dtype";
        case KVFP8_ESHAPE: return "inconsistent or non-positive sizes";
        case KVFP8_ESTRIDE: return "unsupported stride or alignment";
        case KVFP8_ENULL: return "required pointer is NULL";
        case KVFP8_EWORKSPACE: return "workspace too small";
        case KVFP8_ELIMIT: return "size beyond what the kernels support";
        default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
    }
}

extern "C" int kvfp8_timing_enable(int32_t max_launches) {
    g_timing.armed = 0;
    g_timing.used = 0;
    if (max_launches <= 0) return KVFP8_OK;
    while ((int32_t)g_timing.start.size() < max_launches) {
        hipEvent_t a, b;
        hipError_t err = hipEventCreate(&a);
        if (err != hipSuccess) return (int)err;
        err = hipEventCreate(&b);
        if (err != hipSuccess) return (int)err;
        g_timing.start.push_back(a);
        g_timing.stop.push_back(b);
    }
    g_timing.armed = max_launches;
    return KVFP8_OK;
}

extern "C" int kvfp8_timing_read(double* total_ms, int64_t* launches) {
    double sum = 0.0;
    for (int32_t i = 0; i < g_timing.used; ++i) {
        hipError_t err = hipEventSynchronize(g_timing.stop[i]);
        if (err != hipSuccess) return (int)err;
        float ms = 0.0f;
        err = hipEventElapsedTime(&ms, g_timing.start[i], g_timing.stop[i]);
        if (err != hipSuccess) return (int)err;
        sum += ms;
    }
    if (total_ms) *total_ms = sum;
    if (launches) *launches = g_timing.used;
    g_timing.armed = 0;
    g_timing.used = 0;
    return KVFP8_OK;
}

extern "C" const char* kvfp8_version(void) { return "kvfp8 1 gfx950"; }
