// Varlen causal prefill attention on the gfx950 matrix cores.
//
// Replaces the Triton forward of reference
// src/torch_llm/kernals/flash_attention.py:51-211: packed sequences q [T, Hq, D],
// k, v [T, Hkv, D] delimited by cu_seqlens [B + 1]; query row i of a sequence
// attends keys 0..i of the same sequence (GQA: q head h reads KV head h / G);
// out [T, Hq, D] in q's dtype and lse [T, Hq] float32 = max + log(sum) of the
// scaled scores in natural-log units. Rows outside every sequence are not written,
// and sequences longer than max_seq_len are covered only up to it, as in the
// reference (its grid is sized from batch_max_seq_len; there whole 64-row blocks
// past it may still be written, here exactly the rows below it are).
//
// Work split. A workgroup (4 waves) takes one (sequence, KV head, query block)
// for gw q heads of that KV head: gw = 4, 2 or 1 (the largest dividing G), and
// 32 query rows per wave, so the block has 32 * 4 / gw rows. Its K/V blocks of
// 64 keys are staged once in LDS (double-buffered, loaded a block ahead through
// registers) and read by all four waves. Query blocks are dispatched last-first:
// the longest causal ranges start first.
//
// Per wave and KV block (MFMA 16x16x32, layouts as in the decode kernel:
// A[row = l % 16][k = 8 (l/16) + i], B[k = 8 (l/16) + i][col = l % 16],
// D[row = 4 (l/16) + j][col = l % 16]):
//   S^T[key, row] = K Q^T   A = K rows from LDS (16-byte runs, padded rows),
//                           B = Q^T from registers (loaded once)
//   softmax       online, base 2, fp32; lane (row, l / 16) holds 16 of the 64 keys
//   O^T[d, row]  += V^T P^T  B = P^T straight from the score registers; A = V^T
//                           from a 16-bit v_perm transpose of eight V rows
// bf16 inputs run bf16 products, f16 inputs f16 products, float32 inputs a bf16
// hi + lo split of every operand (three products each, about 16 mantissa bits).
#include "kvfp8_common.h"

#include <type_traits>

namespace kvfp8 {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kPThreads = 256;     // 4 waves
constexpr int kKeys = 64;          // keys per KV block
constexpr int kWaveRows = 32;      // query rows per wave
constexpr float kLn2 = 0.693147180559945309f;
constexpr float kNegInf = -__builtin_huge_valf();

struct PrefillArgs {
    const uint8_t* q;
    const uint8_t* k;
    const uint8_t* v;
    uint8_t* out;
    float* lse;
    const void* cu;
    int32_t cu64;
    int32_t batch, hq, hkv, d;
    int32_t heads_per_block;   // gw
    int32_t blocks_per_kv;     // G / gw
    int32_t rows;              // query rows per workgroup, 32 * 4 / gw
    int32_t qblocks;           // ceil(max_seq_len / rows)
    int32_t max_len;           // max_seq_len
    int64_t total_tokens;
    float scale_log2;          // scale * log2(e)
};

// One 8-element MFMA operand: 16-bit values in four dwords; float32 inputs keep
// a bf16 hi and lo part.
template <bool kSplit>
struct Opnd {
    u32x4_t h;
    u32x4_t l;
};

template <bool kF16>
__device__ __forceinline__ f32x4_t mma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    if constexpr (kF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                     c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                      __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// c += a b, with the split inputs' hi hi + hi lo + lo hi terms.
template <bool kF16, bool kSplit>
__device__ __forceinline__ f32x4_t mma(const Opnd<kSplit>& a, const Opnd<kSplit>& b, f32x4_t c) {
    c = mma16<kF16>(a.h, b.h, c);
    if constexpr (kSplit) {
        c = mma16<kF16>(a.h, b.l, c);
        c = mma16<kF16>(a.l, b.h, c);
    }
    return c;
}

// The element is passed by value: clang's __builtin_bit_cast applied directly to an
// element of an ext_vector_type reads element 0.
__device__ __forceinline__ float as_float(uint32_t u) { return __builtin_bit_cast(float, u); }

__device__ __forceinline__ uint32_t bf16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
}
__device__ __forceinline__ uint32_t f16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// Eight floats -> operand (bf16, or f16 for f16 inputs; split for float32).
template <bool kF16, bool kSplit>
__device__ __forceinline__ Opnd<kSplit> pack8(const float (&x)[8]) {
    Opnd<kSplit> o;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if constexpr (kF16) {
            o.h[w] = f16_bits(x[2 * w]) | (f16_bits(x[2 * w + 1]) << 16);
        } else {
            const __bf16 h0 = (__bf16)x[2 * w], h1 = (__bf16)x[2 * w + 1];
            o.h[w] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            if constexpr (kSplit)
                o.l[w] = bf16_bits(x[2 * w] - (float)h0) | (bf16_bits(x[2 * w + 1] - (float)h1) << 16);
        }
    }
    return o;
}

// Eight consecutive input elements at byte address p (16-byte aligned) as an
// operand: 16-bit inputs pass through, float32 inputs are split.
template <int IT>
__device__ __forceinline__ Opnd<IT == KVFP8_F32> load8(const uint8_t* p, bool valid) {
    constexpr bool kSplit = IT == KVFP8_F32;
    Opnd<kSplit> o;
    if constexpr (kSplit) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(p);
        const u32x4_t b = *reinterpret_cast<const u32x4_t*>(p + 16);
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = valid ? as_float(a[i]) : 0.0f;
            x[4 + i] = valid ? as_float(b[i]) : 0.0f;
        }
        o = pack8<false, true>(x);
    } else {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) o.h[i] = valid ? a[i] : 0u;
    }
    return o;
}

template <int C, int IT>
__global__ void __launch_bounds__(kPThreads)
prefill_attention_kernel(PrefillArgs a) {
    constexpr int kD = 64 * C;
    constexpr bool kSplit = IT == KVFP8_F32;
    constexpr bool kF16 = IT == KVFP8_F16;
    constexpr int ES = kSplit ? 4 : 2;
    constexpr int KROW = kD * ES + 16;               // padded: 16 lanes reading one column hit 16 bank groups
    constexpr int VROW = kD * ES;
    constexpr int CPR = kD * ES / 16;                // 16-byte chunks per row
    constexpr int CPT = kKeys * CPR / kPThreads;     // chunks per thread per tensor and block
    constexpr int NB = 4 * C;                        // head dims per lane in the PV product
    constexpr int KS = 2 * C;                        // 32-dim steps of the QK product
    __shared__ __attribute__((aligned(16))) uint8_t lds_k[2][kKeys * KROW];
    __shared__ __attribute__((aligned(16))) uint8_t lds_v[2][kKeys * VROW];

    // Work item: query block (longest first), sequence, KV head, head block.
    const int64_t per_qb = (int64_t)a.batch * a.hkv * a.blocks_per_kv;
    const int64_t idx = blockIdx.x;
    const int qb = a.qblocks - 1 - (int)(idx / per_qb);
    int64_t rest = idx - (int64_t)(a.qblocks - 1 - qb) * per_qb;
    const int b = (int)(rest / ((int64_t)a.hkv * a.blocks_per_kv));
    rest -= (int64_t)b * a.hkv * a.blocks_per_kv;
    const int hk = (int)(rest / a.blocks_per_kv);
    const int hb = (int)(rest - (int64_t)hk * a.blocks_per_kv);

    int64_t s0, s1;
    if (a.cu64) {
        s0 = reinterpret_cast<const int64_t*>(a.cu)[b];
        s1 = reinterpret_cast<const int64_t*>(a.cu)[b + 1];
    } else {
        s0 = reinterpret_cast<const int32_t*>(a.cu)[b];
        s1 = reinterpret_cast<const int32_t*>(a.cu)[b + 1];
    }
    s0 = s0 < 0 ? 0 : s0;
    s1 = s1 > a.total_tokens ? a.total_tokens : s1;
    // Rows past max_seq_len are not computed; causal rows below it never read keys past it.
    int64_t len64 = s1 > s0 ? s1 - s0 : 0;
    len64 = len64 < a.max_len ? len64 : a.max_len;
    const int L = (int)len64;
    const int r0 = qb * a.rows;
    if (r0 >= L) return;                                  // whole workgroup

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m16 = lane & 15, j = lane >> 4;
    const int G = a.hq / a.hkv;
    const int gw = a.heads_per_block;
    const int hq = hk * G + hb * gw + wave % gw;
    const int qa = r0 + kWaveRows * (wave / gw);          // first query row of this wave
    const bool active = qa < L;
    const int kv_end = min(L, r0 + a.rows);               // keys the workgroup needs
    const int n_kv = (kv_end + kKeys - 1) / kKeys;
    const int wave_nkv = active ? (min(L, qa + kWaveRows) + kKeys - 1) / kKeys : 0;
    const int64_t q_row = (int64_t)a.hq * a.d * ES;       // bytes between tokens
    const int64_t kv_row = (int64_t)a.hkv * a.d * ES;

    // Q^T operands: lane (row 16 qt + l % 16, l / 16) holds dims 32 s + 8 (l / 16) .. + 7.
    Opnd<kSplit> qop[2][KS];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int row = qa + 16 * qt + m16;
        const bool rv = active && row < L;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int d0 = 32 * s + 8 * j;
            const bool valid = rv && d0 < a.d;
            const uint8_t* p = valid ? a.q + (s0 + row) * q_row + ((int64_t)hq * a.d + d0) * ES : a.q;
            qop[qt][s] = load8<IT>(p, valid);
        }
    }

    // K/V staging: chunk c = tid + 256 i of a block is row c / CPR, 16-byte piece c % CPR.
    u32x4_t kr[CPT], vr[CPT];
    auto load_block = [&](int kb) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = threadIdx.x + kPThreads * i;
            const int key = kb * kKeys + c / CPR, piece = c % CPR;
            const bool valid = key < L && piece * (16 / ES) < a.d;
            const int64_t off = valid ? (s0 + key) * kv_row + (int64_t)hk * a.d * ES + 16 * piece : 0;
            const u32x4_t x = *reinterpret_cast<const u32x4_t*>(a.k + off);
            const u32x4_t y = *reinterpret_cast<const u32x4_t*>(a.v + off);
            kr[i] = valid ? x : u32x4_t{0u, 0u, 0u, 0u};
            vr[i] = valid ? y : u32x4_t{0u, 0u, 0u, 0u};
        }
    };
    auto store_block = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = threadIdx.x + kPThreads * i;
            const int key = c / CPR, piece = c % CPR;
            *reinterpret_cast<u32x4_t*>(&lds_k[buf][key * KROW + 16 * piece]) = kr[i];
            *reinterpret_cast<u32x4_t*>(&lds_v[buf][key * VROW + 16 * piece]) = vr[i];
        }
    };

    f32x4_t o[2][NB];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) o[qt][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m[2] = {kNegInf, kNegInf}, l[2] = {0.0f, 0.0f};

    auto compute_block = [&](int kb, int buf) {
        const uint8_t* kl = lds_k[buf];
        const uint8_t* vl = lds_v[buf];
        // Scores of 4 key tiles x 2 row tiles.
        f32x4_t sacc[4][2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) sacc[kt][qt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const Opnd<kSplit> kop = load8<IT>(kl + (16 * kt + m16) * KROW + (32 * s + 8 * j) * ES, true);
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) sacc[kt][qt] = mma<kF16, kSplit>(kop, qop[qt][s], sacc[kt][qt]);
            }
        }
        const bool full = kb * kKeys + kKeys - 1 <= qa && kb * kKeys + kKeys <= L;   // wave-uniform
        Opnd<kSplit> pop[2][2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            float sc[16];
            const int row = qa + 16 * qt + m16;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int key = kb * kKeys + 16 * kt + 4 * j + jj;
                    const float x = sacc[kt][qt][jj] * a.scale_log2;
                    sc[4 * kt + jj] = (full || (key <= row && key < L)) ? x : kNegInf;
                }
            }
            float mx = sc[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sc[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m[qt], mx);
            const float m_use = m_new == kNegInf ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m[qt] - m_use);
            l[qt] *= alpha;
            if (__ballot(alpha != 1.0f)) {
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) o[qt][nb] *= alpha;
            }
            m[qt] = m_new;
            float p[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                p[i] = __builtin_amdgcn_exp2f(sc[i] - m_use);
                l[qt] += p[i];
            }
            // P^T operand pp holds keys 16 (2 pp + i / 4) + 4 j + i % 4, i = 0..7.
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                float x[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = p[8 * pp + i];
                pop[qt][pp] = pack8<kF16, kSplit>(x);
            }
        }
        // O^T += V^T P^T: lane reads NB dims at NB (l % 16) of the eight V rows of its
        // keys, and row pairs are transposed into one operand per dim.
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            if constexpr (kSplit) {
                float vrow[8][NB];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int key = 16 * (2 * pp + (i >> 2)) + 4 * j + (i & 3);
                    const uint8_t* p = vl + key * VROW + NB * m16 * ES;
#pragma unroll
                    for (int w = 0; w < NB / 4; ++w) {
                        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(p + 16 * w);
#pragma unroll
                        for (int e = 0; e < 4; ++e) vrow[i][4 * w + e] = as_float(x[e]);
                    }
                }
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) x[i] = vrow[i][nb];
                    const Opnd<kSplit> av = pack8<false, true>(x);
#pragma unroll
                    for (int qt = 0; qt < 2; ++qt) o[qt][nb] = mma<kF16, kSplit>(av, pop[qt][pp], o[qt][nb]);
                }
            } else {
                constexpr int VW = NB / 2;       // dwords per row and lane
                uint32_t rowv[8][VW];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int key = 16 * (2 * pp + (i >> 2)) + 4 * j + (i & 3);
                    const uint8_t* p = vl + key * VROW + NB * m16 * ES;
                    if constexpr (VW == 4) {
                        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
                        for (int w = 0; w < 4; ++w) rowv[i][w] = x[w];
                    } else {
                        const uint2 x = *reinterpret_cast<const uint2*>(p);
                        rowv[i][0] = x.x;
                        rowv[i][1] = x.y;
                    }
                }
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
                    Opnd<kSplit> av;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        av.h[q] = __builtin_amdgcn_perm(rowv[2 * q + 1][nb >> 1], rowv[2 * q][nb >> 1], sel);
#pragma unroll
                    for (int qt = 0; qt < 2; ++qt) o[qt][nb] = mma<kF16, kSplit>(av, pop[qt][pp], o[qt][nb]);
                }
            }
        }
    };

    load_block(0);
    store_block(0);
    __syncthreads();
    for (int kb = 0; kb < n_kv; ++kb) {
        const bool more = kb + 1 < n_kv;
        if (more) load_block(kb + 1);
        if (kb < wave_nkv) compute_block(kb, kb & 1);
        if (more) store_block((kb + 1) & 1);
        __syncthreads();
    }
    if (!active) return;

    // Normalize and store: lane (row, j) holds dims NB (4 j + jj) + nb of its row.
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int row = qa + 16 * qt + m16;
        float lt = l[qt] + __shfl_xor(l[qt], 16);
        lt += __shfl_xor(lt, 32);
        if (row >= L) continue;
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int64_t tok = s0 + row;
        uint8_t* orow = a.out + tok * q_row + (int64_t)hq * a.d * ES;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int d0 = NB * (4 * j + jj);
            if (d0 >= a.d) continue;
            float y[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) y[nb] = o[qt][nb][jj] * inv;
            if constexpr (kSplit) {
#pragma unroll
                for (int w = 0; w < NB / 4; ++w) {
                    if (d0 + 4 * w < a.d)
                        *reinterpret_cast<float4*>(orow + (d0 + 4 * w) * 4) =
                            make_float4(y[4 * w], y[4 * w + 1], y[4 * w + 2], y[4 * w + 3]);
                }
            } else {
                uint32_t wv[NB / 2];
#pragma unroll
                for (int w = 0; w < NB / 2; ++w)
                    wv[w] = kF16 ? (f16_bits(y[2 * w]) | (f16_bits(y[2 * w + 1]) << 16))
                                 : (bf16_bits(y[2 * w]) | (bf16_bits(y[2 * w + 1]) << 16));
                if constexpr (NB == 8) {
                    *reinterpret_cast<u32x4_t*>(orow + d0 * 2) = u32x4_t{wv[0], wv[1], wv[2], wv[3]};
                } else {
                    *reinterpret_cast<uint2*>(orow + d0 * 2) = make_uint2(wv[0], wv[1]);
                }
            }
        }
        if (j == 0) a.lse[tok * a.hq + hq] = (m[qt] + __builtin_log2f(lt)) * kLn2;
    }
}

// ---------------------------------------------------------------------------
// Eight-wave kernel for 16-bit inputs with D in {64, 128}.
//
// A workgroup of eight waves takes one (sequence, KV head, query block): its
// waves are `gw` q heads x (8 / gw) groups of 32 query rows, and its K/V blocks of
// 64 keys are staged once in LDS for all of them. Every wave keeps its whole state
// (Q^T operands, accumulators, scores) within 256 registers, so two waves share
// each SIMD and one wave's softmax runs while the other's MFMAs do.
// Work items run (sequence, KV head) by (sequence, KV head), longest query block
// first, and each XCD takes one contiguous run of items, so the query blocks of
// one sequence and head meet its K/V in the same L2.
// ---------------------------------------------------------------------------
constexpr int kFaRows = 32;        // query rows per wave
constexpr int kFaTiles = kFaRows / 16;
constexpr int kFaWaves = 8;
constexpr int kFaThreads = 64 * kFaWaves;
constexpr int kXcds = 8;           // workgroups are dispatched round-robin over the XCDs
constexpr int kFaBufs = 3;         // K/V block buffers in LDS

template <int C, bool kF16>
__global__ void __launch_bounds__(kFaThreads)
prefill_fa_kernel(PrefillArgs a, int64_t items, int64_t per_xcd) {
    constexpr int kD = 64 * C;
    constexpr int ROW = kD * 2;                      // bytes per K/V row
    constexpr int CPR = kD * 2 / 16;                 // 16-byte chunks per row
    constexpr int CPT = kKeys * CPR / kFaThreads;    // chunks per thread per tensor and block
    // s_waitcnt immediate for "vmcnt <= the 2 CPT loads of one block" (expcnt and
    // lgkmcnt left at their maxima): older loads done, the newest block's in flight.
    constexpr int kKeep = 2 * CPT;
    constexpr int kVmcntKeep = (kKeep & 15) | (7 << 4) | (0 << 8) | (((kKeep >> 4) & 3) << 14);
    // Workgroup barrier that does not drain the K/V prefetch: __syncthreads() would
    // wait for every outstanding load. This wave's LDS reads and its loads older
    // than the newest block are complete (s_waitcnt above); the compiler-level fences
    // keep every LDS access on its side of the barrier.
    auto barrier = [&]() {
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
    };
    constexpr int NB = 4 * C;                        // head dims per lane in the PV product
    constexpr int KS = 2 * C;                        // 32-dim steps of the QK product
    // K/V blocks go from global memory straight into LDS (global_load_lds_dwordx4:
    // lane t of an instruction writes the t-th 16 bytes after the wave's base), so
    // the layout is the load order: chunk slot c holds row c / CPR, chunk
    // (c % CPR) ^ (row % CPR). The xor spreads the 16 rows that one operand read
    // touches at one column over 16 different chunk positions (bank groups).
    __shared__ __attribute__((aligned(16))) uint8_t lds_k[kFaBufs][kKeys * ROW];
    __shared__ __attribute__((aligned(16))) uint8_t lds_v[kFaBufs][kKeys * ROW];
    typedef __attribute__((address_space(3))) void* lds_ptr;

    // Item of this workgroup: XCD x = blockIdx % 8 takes items [x per_xcd, (x + 1) per_xcd).
    const int64_t item = (int64_t)(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (item >= items) return;
    // Items: (sequence, KV head, head block) major, query block descending.
    const int64_t unit = item / a.qblocks;
    const int qb = a.qblocks - 1 - (int)(item - unit * a.qblocks);
    const int b = (int)(unit / ((int64_t)a.hkv * a.blocks_per_kv));
    const int64_t rest = unit - (int64_t)b * a.hkv * a.blocks_per_kv;
    const int hk = (int)(rest / a.blocks_per_kv);
    const int hb = (int)(rest - (int64_t)hk * a.blocks_per_kv);

    int64_t s0, s1;
    if (a.cu64) {
        s0 = reinterpret_cast<const int64_t*>(a.cu)[b];
        s1 = reinterpret_cast<const int64_t*>(a.cu)[b + 1];
    } else {
        s0 = reinterpret_cast<const int32_t*>(a.cu)[b];
        s1 = reinterpret_cast<const int32_t*>(a.cu)[b + 1];
    }
    s0 = s0 < 0 ? 0 : s0;
    s1 = s1 > a.total_tokens ? a.total_tokens : s1;
    int64_t len64 = s1 > s0 ? s1 - s0 : 0;
    len64 = len64 < a.max_len ? len64 : a.max_len;
    const int L = (int)len64;
    const int r0 = qb * a.rows;
    if (r0 >= L) return;                                  // whole workgroup

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m16 = lane & 15, j = lane >> 4;
    const int G = a.hq / a.hkv;
    const int gw = a.heads_per_block;
    const int hq = hk * G + hb * gw + wave % gw;
    const int qa = r0 + kFaRows * (wave / gw);            // first query row of this wave
    const bool active = qa < L;
    const int kv_end = min(L, r0 + a.rows);               // keys the workgroup needs
    const int n_kv = (kv_end + kKeys - 1) / kKeys;
    const int wave_nkv = active ? (min(L, qa + kFaRows) + kKeys - 1) / kKeys : 0;
    const int64_t q_row = (int64_t)a.hq * kD * 2;         // bytes between tokens
    const int64_t kv_row = (int64_t)a.hkv * kD * 2;

    // Q^T operands: lane (row 16 qt + l % 16, l / 16) holds dims 32 s + 8 (l / 16) .. + 7.
    u32x4_t qop[kFaTiles][KS];
#pragma unroll
    for (int qt = 0; qt < kFaTiles; ++qt) {
        const int row = qa + 16 * qt + m16;
        const bool rv = active && row < L;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const uint8_t* p = rv ? a.q + (s0 + row) * q_row + ((int64_t)hq * kD + 32 * s + 8 * j) * 2 : a.q;
            const u32x4_t x = *reinterpret_cast<const u32x4_t*>(p);
            qop[qt][s] = rv ? x : u32x4_t{0u, 0u, 0u, 0u};
        }
    }

    // Asynchronous K/V block load into LDS buffer `buf`. Keys past the sequence read
    // its last key (finite data, masked out of the scores).
    //
    // The loads are issued as inline assembly: the compiler's wait insertion would
    // otherwise assume that any LDS read may alias an LDS write in flight and wait
    // for every outstanding load before it (defeating the prefetch). The kernel
    // waits for them itself: the s_waitcnt before each block's closing barrier.
    auto load_block = [&](int kb, int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = threadIdx.x + kFaThreads * i;         // slot written by this lane
            const int row = c / CPR;
            const int chunk = (c % CPR) ^ (row % CPR);
            const int key = min(kb * kKeys + row, L - 1);
            const int64_t off = (s0 + key) * kv_row + (int64_t)hk * kD * 2 + 16 * chunk;
            const int wave_slot = kFaThreads * i + 64 * wave;   // first slot of this wave's instruction
            const uint32_t k_lds = (uint32_t)(uintptr_t)(lds_ptr)(&lds_k[buf][16 * wave_slot]);
            const uint32_t v_lds = (uint32_t)(uintptr_t)(lds_ptr)(&lds_v[buf][16 * wave_slot]);
            const uint8_t* kg = a.k + off;
            const uint8_t* vg = a.v + off;
            __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                             :: "s"(__builtin_amdgcn_readfirstlane(k_lds)), "v"(kg) : "memory");
            __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                             :: "s"(__builtin_amdgcn_readfirstlane(v_lds)), "v"(vg) : "memory");
        }
    };
    // Per-lane byte offsets of the operand reads (key tile bases are multiples of 16
    // rows, which the swizzle ignores: (16 t + r) % CPR = r % CPR):
    //   K operand, 32-dim step s: row m16, chunk 4 s + j;
    //   V rows of key 16 t + 4 j + e (e < 4): the NB dims at NB m16.
    int k_off[KS], v_off[4];
#pragma unroll
    for (int s = 0; s < KS; ++s) k_off[s] = m16 * ROW + 16 * ((4 * s + j) ^ (m16 % CPR));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int r = 4 * j + e;
        v_off[e] = r * ROW + 16 * (((NB * m16) >> 3) ^ (r % CPR)) + ((NB * m16 * 2) & 15);
    }

    f32x4_t o[kFaTiles][NB];
#pragma unroll
    for (int qt = 0; qt < kFaTiles; ++qt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) o[qt][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m[kFaTiles], l[kFaTiles];
#pragma unroll
    for (int qt = 0; qt < kFaTiles; ++qt) {
        m[qt] = kNegInf;
        l[qt] = 0.0f;
    }

    // The buffer index is a compile-time constant in every call (the block loop is
    // unrolled by kFaBufs), so all LDS operand addresses are a per-lane offset plus
    // an immediate.
    auto compute_block = [&](int kb, auto buf_c) {
        constexpr int buf = decltype(buf_c)::value;
        const uint8_t* kl = lds_k[buf];
        const uint8_t* vl = lds_v[buf];
        // S^T tiles: 4 key tiles x 2 row tiles; each K operand feeds both row tiles.
        f32x4_t sacc[4][kFaTiles];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const u32x4_t kop = *reinterpret_cast<const u32x4_t*>(kl + 16 * kt * ROW + k_off[s]);
#pragma unroll
                for (int qt = 0; qt < kFaTiles; ++qt)
                    sacc[kt][qt] = mma16<kF16>(kop, qop[qt][s], s == 0 ? f32x4_t{0.0f, 0.0f, 0.0f, 0.0f} : sacc[kt][qt]);
            }
        }
        const bool full = kb * kKeys + kKeys - 1 <= qa && kb * kKeys + kKeys <= L;   // wave-uniform
        // Online softmax per row tile; P^T operand pp holds keys 16 (2 pp + i / 4) + 4 j + i % 4.
        u32x4_t pop[kFaTiles][2];
#pragma unroll
        for (int qt = 0; qt < kFaTiles; ++qt) {
            // Raw scores (the scale is applied inside the exponent below).
            float sc[16];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) sc[4 * kt + jj] = sacc[kt][qt][jj];
            if (!full) {
                const int row = qa + 16 * qt + m16;
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int key = kb * kKeys + 16 * kt + 4 * j + jj;
                        const bool keep = (key <= row) & (key < L);
                        sc[4 * kt + jj] = keep ? sc[4 * kt + jj] : kNegInf;
                    }
                }
            }
            float mx = sc[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sc[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            mx *= a.scale_log2;                       // base-2 units (scale > 0 keeps the order)
            // Lazy rescale: the accumulators keep a reference max m that is only moved
            // when some row's max grows by more than 2^8 (p <= 256 meanwhile, far
            // inside float32 and bf16 range), so the accumulators are rarely scaled.
            if (__ballot(mx > m[qt] + 8.0f)) {
                const float m_new = fmaxf(m[qt], mx);
                const float m_use = m_new == kNegInf ? 0.0f : m_new;
                const float alpha = __builtin_amdgcn_exp2f(m[qt] - m_use);
                l[qt] *= alpha;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) o[qt][nb] *= alpha;
                m[qt] = m_new;
            }
            const float neg_m = m[qt] == kNegInf ? 0.0f : -m[qt];
            float pr[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], a.scale_log2, neg_m));
                l[qt] += pr[i];
            }
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                float x[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = pr[8 * pp + i];
                pop[qt][pp] = pack8<kF16, false>(x).h;
            }
        }
        // O^T += V^T P^T: the lane reads NB dims at NB (l % 16) of the eight V rows of
        // its keys; row pairs are transposed into one operand per dim, which feeds
        // both row tiles.
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            constexpr int VW = NB / 2;       // dwords per row and lane
            uint32_t rowv[8][VW];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                // Key 16 (2 pp + i / 4) + 4 j + i % 4.
                const uint8_t* p = vl + 16 * (2 * pp + (i >> 2)) * ROW + v_off[i & 3];
                if constexpr (VW == 4) {
                    const u32x4_t x = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
                    for (int w = 0; w < 4; ++w) rowv[i][w] = x[w];
                } else {
                    const uint2 x = *reinterpret_cast<const uint2*>(p);
                    rowv[i][0] = x.x;
                    rowv[i][1] = x.y;
                }
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
                u32x4_t av;
#pragma unroll
                for (int q = 0; q < 4; ++q) av[q] = __builtin_amdgcn_perm(rowv[2 * q + 1][nb >> 1], rowv[2 * q][nb >> 1], sel);
#pragma unroll
                for (int qt = 0; qt < kFaTiles; ++qt) o[qt][nb] = mma16<kF16>(av, pop[qt][pp], o[qt][nb]);
            }
        }
    };

    // Three LDS buffers: block kb + 2 streams in while block kb is computed. Before
    // the barrier that ends block kb every wave waits for its loads of block kb + 1
    // (issued a block earlier); the barrier then publishes them, and it also ends
    // the last reads of the buffer that block kb + 3 will overwrite.
    auto step = [&](int kb, auto buf_c) {
        constexpr int buf = decltype(buf_c)::value;
        if (kb + 2 < n_kv) load_block(kb + 2, (buf + 2) % kFaBufs);
        if (kb < wave_nkv) compute_block(kb, buf_c);
        if (kb + 2 < n_kv) __builtin_amdgcn_s_waitcnt(kVmcntKeep);   // loads of kb + 2 stay in flight
        else __builtin_amdgcn_s_waitcnt(0);
        barrier();
    };
    load_block(0, 0);
    if (n_kv > 1) load_block(1, 1);
    if (n_kv > 1) __builtin_amdgcn_s_waitcnt(kVmcntKeep);
    else __builtin_amdgcn_s_waitcnt(0);
    barrier();
    for (int kb = 0; kb < n_kv; kb += kFaBufs) {
        step(kb, std::integral_constant<int, 0>{});
        if (kb + 1 < n_kv) step(kb + 1, std::integral_constant<int, 1>{});
        if (kb + 2 < n_kv) step(kb + 2, std::integral_constant<int, 2>{});
    }
    if (!active) return;

    // Normalize and store: lane (row, j) holds dims NB (4 j + jj) + nb of its row.
#pragma unroll
    for (int qt = 0; qt < kFaTiles; ++qt) {
        const int row = qa + 16 * qt + m16;
        float lt = l[qt] + __shfl_xor(l[qt], 16);
        lt += __shfl_xor(lt, 32);
        if (row >= L) continue;
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int64_t tok = s0 + row;
        uint8_t* orow = a.out + tok * q_row + (int64_t)hq * kD * 2;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int d0 = NB * (4 * j + jj);
            uint32_t wv[NB / 2];
#pragma unroll
            for (int w = 0; w < NB / 2; ++w) {
                const float y0 = o[qt][2 * w][jj] * inv, y1 = o[qt][2 * w + 1][jj] * inv;
                wv[w] = kF16 ? (f16_bits(y0) | (f16_bits(y1) << 16)) : (bf16_bits(y0) | (bf16_bits(y1) << 16));
            }
            if constexpr (NB == 8) {
                *reinterpret_cast<u32x4_t*>(orow + d0 * 2) = u32x4_t{wv[0], wv[1], wv[2], wv[3]};
            } else {
                *reinterpret_cast<uint2*>(orow + d0 * 2) = make_uint2(wv[0], wv[1]);
            }
        }
        if (j == 0) a.lse[tok * a.hq + hq] = (m[qt] + __builtin_log2f(lt)) * kLn2;
    }
}

template <int IT>
hipError_t launch_prefill(const PrefillArgs& a, int64_t blocks, hipStream_t s) {
    if (a.d <= 64)
        hipLaunchKernelGGL((prefill_attention_kernel<1, IT>), dim3((unsigned)blocks), dim3(kPThreads), 0, s, a);
    else
        hipLaunchKernelGGL((prefill_attention_kernel<2, IT>), dim3((unsigned)blocks), dim3(kPThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace

}  // namespace kvfp8

using namespace kvfp8;

extern "C" int kvfp8_prefill_attention(const void* q, const void* k, const void* v, int dtype, int64_t total_tokens,
                                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                       const void* cu_seqlens, int cu_dtype, int32_t batch, int32_t max_seq_len,
                                       float scale, void* out, float* lse, void* stream) {
    if (dtype != KVFP8_F32 && dtype != KVFP8_F16 && dtype != KVFP8_BF16) return KVFP8_EDTYPE;
    if (cu_dtype != KVFP8_I32 && cu_dtype != KVFP8_I64) return KVFP8_EDTYPE;
    if (total_tokens < 0 || batch < 0 || max_seq_len < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
        num_q_heads % num_kv_heads != 0)
        return KVFP8_ESHAPE;
    // Head sizes: multiples of 8 up to 128 (8-element operand runs).
    if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 128) return KVFP8_ESHAPE;
    if (total_tokens == 0 || batch == 0 || max_seq_len == 0) return KVFP8_OK;
    if (!q || !k || !v || !out || !lse || !cu_seqlens) return KVFP8_ENULL;
    if ((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15) != 0) return KVFP8_ESTRIDE;
    PrefillArgs a;
    a.q = reinterpret_cast<const uint8_t*>(q);
    a.k = reinterpret_cast<const uint8_t*>(k);
    a.v = reinterpret_cast<const uint8_t*>(v);
    a.out = reinterpret_cast<uint8_t*>(out);
    a.lse = lse;
    a.cu = cu_seqlens;
    a.cu64 = cu_dtype == KVFP8_I64;
    a.batch = batch;
    a.hq = num_q_heads;
    a.hkv = num_kv_heads;
    a.d = head_dim;
    const int G = num_q_heads / num_kv_heads;
    a.heads_per_block = G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1);
    a.blocks_per_kv = G / a.heads_per_block;
    a.max_len = max_seq_len;
    a.total_tokens = total_tokens;
    a.scale_log2 = scale * 1.44269504088896340736f;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // 16-bit inputs with D 64 or 128: the wide-tile kernel.
    if ((dtype == KVFP8_BF16 || dtype == KVFP8_F16) && (head_dim == 64 || head_dim == 128)) {
        a.rows = kFaRows * kFaWaves / a.heads_per_block;
        a.qblocks = (max_seq_len + a.rows - 1) / a.rows;
        const int64_t items = (int64_t)a.qblocks * batch * num_kv_heads * a.blocks_per_kv;
        const int64_t per_xcd = (items + kXcds - 1) / kXcds;
        if (per_xcd * kXcds >= ((int64_t)1 << 31)) return KVFP8_ESHAPE;
        const dim3 grid((unsigned)(per_xcd * kXcds)), block(kFaThreads);
        if (dtype == KVFP8_BF16) {
            if (head_dim == 64) hipLaunchKernelGGL((prefill_fa_kernel<1, false>), grid, block, 0, s, a, items, per_xcd);
            else hipLaunchKernelGGL((prefill_fa_kernel<2, false>), grid, block, 0, s, a, items, per_xcd);
        } else {
            if (head_dim == 64) hipLaunchKernelGGL((prefill_fa_kernel<1, true>), grid, block, 0, s, a, items, per_xcd);
            else hipLaunchKernelGGL((prefill_fa_kernel<2, true>), grid, block, 0, s, a, items, per_xcd);
        }
        return (int)hipGetLastError();
    }
    a.rows = kWaveRows * 4 / a.heads_per_block;
    a.qblocks = (max_seq_len + a.rows - 1) / a.rows;
    const int64_t blocks = (int64_t)a.qblocks * batch * num_kv_heads * a.blocks_per_kv;
    if (blocks >= ((int64_t)1 << 31)) return KVFP8_ESHAPE;
    hipError_t err;
    switch (dtype) {
        case KVFP8_F32: err = launch_prefill<KVFP8_F32>(a, blocks, s); break;
        case KVFP8_F16: err = launch_prefill<KVFP8_F16>(a, blocks, s); break;
        default: err = launch_prefill<KVFP8_BF16>(a, blocks, s); break;
    }
    return (int)err;
}
