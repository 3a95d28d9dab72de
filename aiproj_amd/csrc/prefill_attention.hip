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

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> one dword of two 16-bit values, rounded to nearest even (one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
template <bool kF16>
__device__ __forceinline__ uint32_t pack2(float x0, float x1) {
    const f32x2_t v = {x0, x1};
    if constexpr (kF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Maximum over lanes l, l ^ 16, l ^ 32 and l ^ 48. Each permlane swap leaves the
// values of a lane pair (l, l ^ 16), then (l, l ^ 32), in the two results, so
// their maximum is the pair's in every lane; no LDS round trip.
__device__ __forceinline__ float max_across_rows(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float y = fmaxf(as_float(a[0]), as_float(a[1]));
    const uint32_t v = __builtin_bit_cast(uint32_t, y);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return fmaxf(as_float(b[0]), as_float(b[1]));
}

// Sum over the same four lanes (equal in all four: float addition commutes).
__device__ __forceinline__ float sum_across_rows(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float y = as_float(a[0]) + as_float(a[1]);
    const uint32_t v = __builtin_bit_cast(uint32_t, y);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return as_float(b[0]) + as_float(b[1]);
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
// An item is one (sequence, KV head, query block): the eight waves are `gw` q heads
// x (8 / gw) groups of 32 query rows, and its K/V blocks of 64 keys are staged once
// in LDS for all of them. Every wave keeps its whole state (Q^T operands,
// accumulators, scores) within 256 registers, so two waves share each SIMD.
// Workgroups are persistent, one per CU, and walk a list of items with the K/V
// and Q loads of the next item issued during the current one. Each XCD takes one
// contiguous run of (sequence, KV head) units, so the query blocks of one sequence
// and head meet its K/V in the same L2; it orders them in groups of kGroupUnits
// units, longest query block first across the group.
// ---------------------------------------------------------------------------
constexpr int kFaRows = 32;        // query rows per wave
constexpr int kFaTiles = kFaRows / 16;
constexpr int kFaWaves = 8;
constexpr int kFaThreads = 64 * kFaWaves;
constexpr int kXcds = 8;           // workgroups are dispatched round-robin over the XCDs
constexpr int kGroupUnits = 8;     // units per longest-first group (their K/V: 8 x 512 KB at L 1024, D 128)
constexpr int kFaBufs = 3;         // K/V block buffers in LDS

// Wave-uniform loads through the scalar data cache: a pointer into the constant
// address space (read-only for the kernel's lifetime) lets the compiler use
// s_load. A plain load of this memory would be a vector load here (the kernel also
// stores to global memory), and the compiler would then wait for every
// vector-memory operation in flight, K/V prefetches included.
typedef __attribute__((address_space(4))) const int64_t* const_i64_ptr;
typedef __attribute__((address_space(4))) const int32_t* const_i32_ptr;

// One work item: query block qb of a unit (sequence b, KV head hk, head block hb).
struct FaItem {
    int32_t s0;        // first token of the sequence
    int32_t L;         // its length, capped at max_seq_len
    int32_t qb;
    int32_t hk, hb;
    int32_t n_kv;      // K/V blocks of 64 keys the query block reads
};

// The items of one workgroup. XCD x = blockIdx % 8 owns units [x upx, (x + 1) upx),
// ordered in groups of kGroupUnits units, longest query block first across each
// group: item t is query block qblocks - 1 - (t % span) / gsize of unit
// g kGroupUnits + (t % span) % gsize, g = t / span. The XCD's P workgroups take
// these items in snake order: in round k, workgroup c takes item k P + c (k even)
// or k P + P - 1 - c (k odd), so long and short query blocks pair up.
struct FaSchedule {
    int32_t u_lo;      // first unit of the XCD
    int32_t nu;        // its units
    int32_t T;         // its items, nu * qblocks
    int32_t P;         // workgroups per XCD
    int32_t c;         // this workgroup's index within the XCD
};

// The first item at or after round k that has query rows (query blocks past the
// end of a shorter sequence are skipped); k is left at its round. False when the
// workgroup has no more items. (The host keeps items and tokens below 2^31.)
__device__ __forceinline__ bool fa_item(const PrefillArgs& a, const FaSchedule& sc, int32_t& k, FaItem& it) {
    const int32_t span = kGroupUnits * a.qblocks;
    for (;; ++k) {
        const int32_t t = k * sc.P + ((k & 1) ? sc.P - 1 - sc.c : sc.c);
        if (t >= sc.T) return false;
        const int32_t g = t / span, r = t - g * span;
        const int32_t gsize = min(kGroupUnits, sc.nu - g * kGroupUnits);
        const int32_t qbi = r / gsize;
        const int32_t unit = sc.u_lo + g * kGroupUnits + (r - qbi * gsize);
        const int32_t b = unit / (a.hkv * a.blocks_per_kv);
        const int32_t rest = unit - b * a.hkv * a.blocks_per_kv;
        int64_t s0, s1;
        if (a.cu64) {
            const const_i64_ptr cu = (const_i64_ptr)a.cu;
            s0 = cu[b];
            s1 = cu[b + 1];
        } else {
            const const_i32_ptr cu = (const_i32_ptr)a.cu;
            s0 = cu[b];
            s1 = cu[b + 1];
        }
        s0 = s0 < 0 ? 0 : s0;
        s1 = s1 > a.total_tokens ? a.total_tokens : s1;
        int64_t len64 = s1 > s0 ? s1 - s0 : 0;
        len64 = len64 < a.max_len ? len64 : a.max_len;
        const int L = (int)len64;
        const int qb = a.qblocks - 1 - qbi;
        const int r0 = qb * a.rows;
        if (r0 >= L) continue;
        it.s0 = (int32_t)s0;
        it.L = L;
        it.qb = qb;
        it.hk = rest / a.blocks_per_kv;
        it.hb = rest - it.hk * a.blocks_per_kv;
        it.n_kv = (min(L, r0 + a.rows) + kKeys - 1) / kKeys;
        return true;
    }
}

template <int C, bool kF16>
__global__ void __launch_bounds__(kFaThreads)
prefill_fa_kernel(PrefillArgs a, int32_t units, int32_t upx, int32_t per_xcd) {
    constexpr int kD = 64 * C;
    constexpr int ROW = kD * 2;                      // bytes per K/V row
    constexpr int CPR = kD * 2 / 16;                 // 16-byte chunks per row
    constexpr int CPT = kKeys * CPR / kFaThreads;    // chunks per thread per tensor and block
    constexpr int NB = 4 * C;                        // head dims per lane in the PV product
    constexpr int KS = 2 * C;                        // 32-dim steps of the QK product
    // Vector-memory instructions a wave issues: kBlockLoads per K/V block, kQLoads
    // for its Q operands of one item.
    constexpr int kBlockLoads = 2 * CPT;
    constexpr int kQLoads = kFaTiles * KS;
    // Every lambda below is forced inline: a call would keep its captures (the
    // accumulator arrays among them) in scratch memory.
    //
    // Workgroup barrier that does not drain the K/V prefetch: __syncthreads() would
    // wait for every outstanding load. Before it the wave waits (s_waitcnt) for its
    // LDS reads and for its loads older than the ones it keeps in flight; the
    // compiler-level fences keep every LDS access on its side of the barrier.
    auto barrier = [&]() __attribute__((always_inline)) {
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
    };
    // K/V blocks go from global memory straight into LDS (global_load_lds_dwordx4:
    // lane t of an instruction writes the t-th 16 bytes after the wave's base), so
    // the layout is the load order: chunk slot c holds row c / CPR, chunk
    // (c % CPR) ^ (row % CPR). The xor spreads the 16 rows that one operand read
    // touches at one column over 16 different chunk positions (bank groups).
    // V buffers first, then K buffers (96 KiB at D 128): every V^T operand address is
    // a per-lane offset plus an immediate below 64 KiB; the K reads take a per-lane
    // base register that includes the K region's start.
    __shared__ __attribute__((aligned(16))) uint8_t lds_kv[2 * kFaBufs][kKeys * ROW];
    typedef __attribute__((address_space(3))) void* lds_ptr;

    // LDS byte addresses of the K and V buffers (the DMA loads take them in m0).
    const uint32_t k_lds0 = (uint32_t)(uintptr_t)(lds_ptr)(&lds_kv[kFaBufs][0]);
    const uint32_t v_lds0 = (uint32_t)(uintptr_t)(lds_ptr)(&lds_kv[0][0]);

    FaSchedule sc;
    sc.P = per_xcd;
    sc.c = (int32_t)(blockIdx.x / kXcds);
    sc.u_lo = (int32_t)(blockIdx.x % kXcds) * upx;
    sc.nu = max(min(units, sc.u_lo + upx) - sc.u_lo, 0);
    sc.T = sc.nu * a.qblocks;

    // Two cursors walk the workgroup's items block by block: the load cursor
    // (lk, li, lkb) two K/V blocks ahead of the compute cursor (ck, ci, ckb).
    int32_t lk = 0;
    FaItem li;
    bool lhas = fa_item(a, sc, lk, li);
    if (!lhas) return;                                   // whole workgroup: no items
    int lkb = 0;
    int32_t ck = lk;
    FaItem ci = li;
    int ckb = 0;

    // The wave index as a wave-uniform (scalar) value, so that branches on it and on
    // what derives from it are scalar branches.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int m16 = lane & 15, j = lane >> 4;
    const int G = a.hq / a.hkv;
    const int gw = a.heads_per_block;
    const int64_t q_row = (int64_t)a.hq * kD * 2;         // bytes between tokens
    const int64_t kv_row = (int64_t)a.hkv * kD * 2;
    // This lane's byte offset in a full K/V block: chunk slot c = lane + kFaThreads i
    // holds row c / CPR, chunk (c % CPR) ^ (row % CPR) (below 64 kv_row < 2^32).
    uint32_t chunk_off[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = threadIdx.x + kFaThreads * i;
        const int row = c / CPR;
        chunk_off[i] = (uint32_t)(row * kv_row + 16 * ((c % CPR) ^ (row % CPR)));
    }

    // Asynchronous load of block kb of item it into LDS buffer `buf`. Keys past the
    // sequence read its last key (finite data, masked out of the scores).
    //
    // The loads are issued as inline assembly: the compiler's wait insertion would
    // otherwise assume that any LDS read may alias an LDS write in flight and wait
    // for every outstanding load before it (defeating the prefetch). The kernel
    // waits for them itself: the s_waitcnt before each block's closing barrier.
    // They set m0 (the LDS destination) themselves. The compiler reserves m0 and
    // writes it right before each instruction of its own that reads it, so it
    // holds no value across these statements (and a clobber list may not name it).
    //
    // A block whose 64 keys all lie inside the sequence is addressed as a wave-uniform
    // base (scalar registers) plus this lane's fixed 32-bit offset (`chunk_off`, the
    // same for every full block), so it costs no vector instructions. The sequence's
    // last, partial block clamps each key to the sequence (per-lane 64-bit addresses).
    auto load_block = [&](const FaItem& it, int kb, int buf) __attribute__((always_inline)) {
        if ((kb + 1) * kKeys <= it.L) {
            const int64_t base = (int64_t)(it.s0 + kb * kKeys) * kv_row + (int64_t)it.hk * kD * 2;
            const uint8_t* kb_base = a.k + base;
            const uint8_t* vb_base = a.v + base;
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                const uint32_t slot = (uint32_t)buf * (kKeys * ROW) + 16u * (uint32_t)(kFaThreads * i + 64 * wave);
                __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                                 :: "s"(__builtin_amdgcn_readfirstlane(k_lds0 + slot)), "v"(chunk_off[i]),
                                    "s"(kb_base) : "memory");
                __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                                 :: "s"(__builtin_amdgcn_readfirstlane(v_lds0 + slot)), "v"(chunk_off[i]),
                                    "s"(vb_base) : "memory");
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = threadIdx.x + kFaThreads * i;         // slot written by this lane
            const int row = c / CPR;
            const int chunk = (c % CPR) ^ (row % CPR);
            const int key = min(kb * kKeys + row, it.L - 1);
            const int64_t off = (int64_t)(it.s0 + key) * kv_row + (int64_t)it.hk * kD * 2 + 16 * chunk;
            // First slot of this wave's instruction (wave-uniform).
            const uint32_t slot = (uint32_t)buf * (kKeys * ROW) + 16u * (uint32_t)(kFaThreads * i + 64 * wave);
            const uint8_t* kg = a.k + off;
            const uint8_t* vg = a.v + off;
            __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                             :: "s"(__builtin_amdgcn_readfirstlane(k_lds0 + slot)), "v"(kg) : "memory");
            __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                             :: "s"(__builtin_amdgcn_readfirstlane(v_lds0 + slot)), "v"(vg) : "memory");
        }
    };
    // Load the load cursor's block into `buf` and advance the cursor; false when
    // every block has been loaded. Every wave issues the same loads.
    auto load_next = [&](int buf) __attribute__((always_inline)) -> bool {
        if (!lhas) return false;
        load_block(li, lkb, buf);
        if (++lkb == li.n_kv) {
            ++lk;
            lhas = fa_item(a, sc, lk, li);
            lkb = 0;
        }
        return true;
    };

    // This wave's rows of an item: q head hq, query rows qa .. qa + 31.
    auto wave_head = [&](const FaItem& it) __attribute__((always_inline)) { return it.hk * G + it.hb * gw + wave % gw; };
    auto wave_row = [&](const FaItem& it) __attribute__((always_inline)) { return it.qb * a.rows + kFaRows * (wave / gw); };

    // Q^T operands: lane (row 16 qt + l % 16, l / 16) holds dims 32 s + 8 (l / 16) .. + 7.
    // Rows past the sequence load its last row: their results are never stored, and
    // every row's softmax is its own, so they need no zeroing (which would have to
    // wait for the loads where they are issued).
    u32x4_t qop[kFaTiles][KS];
    auto load_q = [&](const FaItem& it) __attribute__((always_inline)) {
        const int hq_n = wave_head(it), qa_n = wave_row(it);
#pragma unroll
        for (int qt = 0; qt < kFaTiles; ++qt) {
            const int row = min(qa_n + 16 * qt + m16, it.L - 1);
#pragma unroll
            for (int s = 0; s < KS; ++s)
                qop[qt][s] = *reinterpret_cast<const u32x4_t*>(a.q + (int64_t)(it.s0 + row) * q_row +
                                                               ((int64_t)hq_n * kD + 32 * s + 8 * j) * 2);
        }
    };

    // Per-lane byte offsets of the operand reads (key tile bases are multiples of 16
    // rows, which the swizzle ignores: (16 t + r) % CPR = r % CPR):
    //   K operand, 32-dim step s: row m16, chunk 4 s + j;
    //   V^T operand, dims 16 nb .. + 15: the transposing LDS read (ds_read_b64_tr_b16)
    //   gives lane i of each 16-lane group element i % 4 of the 8 bytes read by lane
    //   4 r + i / 4 (r = 0..3). Lane (j, m16) therefore reads dims 16 nb + 4 (m16 % 4)
    //   .. + 3 of key row 4 j + m16 / 4 of a 16-key tile and receives
    //   V[4 j + r][16 nb + m16]: four keys of its dim, in the P^T operand's key order.
    // The K offsets are LDS addresses that include the K region's start, computed in
    // assembly so that the compiler keeps them as base registers: folded into a
    // constant, the start plus a buffer's offset exceeds the 16-bit immediate of the
    // LDS instructions, and every read would take its own address addition.
    uint32_t k_addr[KS];
    int vt_off[NB];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const uint32_t off = (uint32_t)(m16 * ROW + 16 * ((4 * s + j) ^ (m16 % CPR)));
        __asm__("v_add_u32 %0, %1, %2" : "=v"(k_addr[s]) : "s"(k_lds0), "v"(off));
    }
    {
        const int vrow = 4 * j + (m16 >> 2);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            vt_off[nb] = vrow * ROW + 16 * ((2 * nb + ((m16 >> 1) & 1)) ^ (vrow % CPR)) + 8 * (m16 & 1);
    }
    typedef __attribute__((address_space(3))) const uint8_t lds_u8;
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
    typedef __attribute__((address_space(3))) const u32x4_t lds_u32x4;
    lds_u8* const v_lds = (lds_u8*)(&lds_kv[0][0]);

    // Compute state of the current item: accumulators o[qt][nb] for the head dims;
    // l[qt] holds a lane's part (16 of every 64 keys) of its row's float32
    // probability sum.
    f32x4_t o[kFaTiles][NB];
    float m[kFaTiles], neg_m[kFaTiles], l[kFaTiles];
    int hq = 0, qa = 0, wave_nkv = 0;
    bool active = false;
    auto enter = [&](const FaItem& it) __attribute__((always_inline)) {
        hq = wave_head(it);
        qa = wave_row(it);
        active = qa < it.L;
        wave_nkv = active ? (min(it.L, qa + kFaRows) + kKeys - 1) / kKeys : 0;
#pragma unroll
        for (int qt = 0; qt < kFaTiles; ++qt) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) o[qt][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            m[qt] = kNegInf;
            neg_m[qt] = 0.0f;
            l[qt] = 0.0f;
        }
    };

    // A block's work is qk (S^T = K Q^T, matrix cores), then softmax_pv: the softmax
    // (vector ALU) and pv (O^T += V^T P^T, matrix cores), overlapped over the two key
    // halves. The buffer index is a compile-time constant in every call (the block
    // loop is unrolled by kFaBufs), so all LDS operand addresses are a per-lane
    // register plus an immediate.
    f32x4_t sacc[4][kFaTiles];
    u32x4_t pop[kFaTiles][2];           // P^T operands; pp holds keys 16 (2 pp + i / 4) + 4 j + i % 4
    auto qk = [&](auto buf_c) __attribute__((always_inline)) {
        constexpr int buf = decltype(buf_c)::value;
        // 4 key tiles x 2 row tiles; each K operand feeds both row tiles.
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            lds_u8* const kl = (lds_u8*)(uintptr_t)k_addr[s] + buf * (kKeys * ROW);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const u32x4_t kop = *(lds_u32x4*)(kl + 16 * kt * ROW);
#pragma unroll
                for (int qt = 0; qt < kFaTiles; ++qt)
                    sacc[kt][qt] = mma16<kF16>(kop, qop[qt][s], s == 0 ? f32x4_t{0.0f, 0.0f, 0.0f, 0.0f} : sacc[kt][qt]);
            }
        }
    };
    // Softmax and PV of one block, in three parts. (1) Per row tile: the mask, the
    // max test and the rare rescale (the only branches). (2) The probabilities of
    // keys 0..31, packed into the P^T operands of the first key half. (3) The PV
    // products of that half, with the probabilities of keys 32..63 computed between
    // them (one score per row tile and product pair: straight-line code, so the vector
    // ALU works while the matrix core runs), then the PV products of the second half.
    // V^T operands come straight from the transposing reads: half h of pair pp covers
    // the keys of tile 2 pp + h; each operand feeds both row tiles.
    auto softmax_pv = [&](int kb, int L, auto buf_c) __attribute__((always_inline)) {
        constexpr int buf = decltype(buf_c)::value;
        const bool full = kb * kKeys + kKeys - 1 <= qa && kb * kKeys + kKeys <= L;   // wave-uniform
#pragma unroll
        for (int qt = 0; qt < kFaTiles; ++qt) {
            // Raw scores (the scale is applied inside the exponent below), masked in
            // place so that blocks without a mask keep them in their registers.
            if (!full) {
                // Keep key kb * 64 + 16 kt + 4 j + jj when it is <= min(row, L - 1).
                const int lim = min(qa + 16 * qt + m16, L - 1) - (kb * kKeys + 4 * j);
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj)
                        sacc[kt][qt][jj] = 16 * kt + jj <= lim ? sacc[kt][qt][jj] : kNegInf;
            }
            float mx = sacc[0][qt][0];
#pragma unroll
            for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sacc[i / 4][qt][i % 4]);
            mx *= a.scale_log2;                        // base-2 units (scale > 0 keeps the order)
            // Lazy rescale: the accumulators keep a reference max m that is only moved
            // when some row's max grows by more than 2^8 (p <= 256 meanwhile, far
            // inside float32 and bf16 range), so the accumulators are rarely scaled.
            // Each lane tests its own 16 keys; only a rescale needs the row's max over
            // its four lanes.
            if (__ballot(mx > m[qt] + 8.0f)) {
                const float m_new = fmaxf(m[qt], max_across_rows(mx));
                const float m_use = m_new == kNegInf ? 0.0f : m_new;
                // An item's first block finds the accumulators at zero: nothing to scale.
                if (kb != 0) {
                    const float alpha = __builtin_amdgcn_exp2f(m[qt] - m_use);
                    l[qt] *= alpha;
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) o[qt][nb] *= alpha;
                }
                m[qt] = m_new;
                neg_m[qt] = -m_use;
            }
        }
        float pr[kFaTiles][16];
        auto prob = [&](int qt, int i) __attribute__((always_inline)) {
            pr[qt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[i / 4][qt][i % 4], a.scale_log2, neg_m[qt]));
            l[qt] += pr[qt][i];
        };
        auto pack_half = [&](int pp) __attribute__((always_inline)) {
#pragma unroll
            for (int qt = 0; qt < kFaTiles; ++qt)
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    pop[qt][pp][w] = pack2<kF16>(pr[qt][8 * pp + 2 * w], pr[qt][8 * pp + 2 * w + 1]);
        };
        auto pv_pair = [&](int pp, int nb) __attribute__((always_inline)) {
            u32x4_t av;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const s16x4_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(v_lds + buf * (kKeys * ROW) + 16 * (2 * pp + h) * ROW + vt_off[nb]));
                const uint2 w = __builtin_bit_cast(uint2, x);
                av[2 * h] = w.x;
                av[2 * h + 1] = w.y;
            }
#pragma unroll
            for (int qt = 0; qt < kFaTiles; ++qt) o[qt][nb] = mma16<kF16>(av, pop[qt][pp], o[qt][nb]);
        };
#pragma unroll
        for (int qt = 0; qt < kFaTiles; ++qt)
#pragma unroll
            for (int i = 0; i < 8; ++i) prob(qt, i);
        pack_half(0);
        constexpr int kPerPair = 8 / NB;     // second-half scores per row tile and product pair
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            pv_pair(0, nb);
#pragma unroll
            for (int qt = 0; qt < kFaTiles; ++qt)
#pragma unroll
                for (int u = 0; u < kPerPair; ++u) prob(qt, 8 + kPerPair * nb + u);
        }
        pack_half(1);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) pv_pair(1, nb);
    };
    // Normalize and store the current item's rows: lane (row, j) holds dims
    // 16 nb + 4 j + jj of its row (tile nb of the V^T operand covers dims 16 nb ..).
    auto finish = [&](const FaItem& it) __attribute__((always_inline)) {
        if (!active) return;
#pragma unroll
        for (int qt = 0; qt < kFaTiles; ++qt) {
            const int row = qa + 16 * qt + m16;
            const float lt = sum_across_rows(l[qt]);
            if (row >= it.L) continue;
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            const int64_t tok = (int64_t)it.s0 + row;
            uint8_t* orow = a.out + tok * q_row + (int64_t)hq * kD * 2;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int d0 = 16 * nb + 4 * j;
                *reinterpret_cast<uint2*>(orow + d0 * 2) =
                    make_uint2(pack2<kF16>(o[qt][nb][0] * inv, o[qt][nb][1] * inv),
                               pack2<kF16>(o[qt][nb][2] * inv, o[qt][nb][3] * inv));
            }
            if (j == 0) a.lse[tok * a.hq + hq] = (m[qt] + __builtin_log2f(lt)) * kLn2;
        }
    };

    // Block stream. The blocks of the workgroup's items form one sequence; block g
    // uses LDS buffer g % 3. Step g: the QK product of block g, the loads of block
    // g + 2 (the load cursor; into the buffer of block g - 1, free since the last
    // barrier), the rest of block g, then a wait for this wave's loads of block g + 1
    // and the barrier, which publishes block g + 1 and ends every read of buffer
    // g % 3 before step g + 1 loads block g + 3 into it. At an item's last block the
    // wave issues the Q loads of its next item after the QK product (the last use of
    // the current Q operands), so they arrive while the block finishes and the item
    // is stored. The block loads come after the QK product because the compiler waits
    // for all older vector-memory operations before the first use of new Q operands.
    //
    // s_waitcnt immediates (vmcnt = n, expcnt at its maximum, lgkmcnt 0).
    constexpr int kW0 = (7 << 4);
    constexpr int kWBlock = (kBlockLoads & 15) | (7 << 4) | (((kBlockLoads >> 4) & 3) << 14);
    constexpr int kWQ = (kQLoads & 15) | (7 << 4) | (((kQLoads >> 4) & 3) << 14);
    constexpr int kWBoth = ((kBlockLoads + kQLoads) & 15) | (7 << 4) | ((((kBlockLoads + kQLoads) >> 4) & 3) << 14);
    auto step = [&](auto buf_c) __attribute__((always_inline)) -> bool {
        constexpr int buf = decltype(buf_c)::value;
        const bool last = ckb + 1 == ci.n_kv;
        int32_t nk = ck + 1;
        FaItem ni = ci;
        const bool next = last && fa_item(a, sc, nk, ni);
        const bool compute = ckb < wave_nkv;
        if (compute) qk(buf_c);
        const bool loaded = load_next((buf + 2) % kFaBufs);
        if (next) load_q(ni);
        if (compute) softmax_pv(ckb, ci.L, buf_c);
        if (loaded) {
            if (next) __builtin_amdgcn_s_waitcnt(kWBoth);
            else __builtin_amdgcn_s_waitcnt(kWBlock);
        } else {
            if (next) __builtin_amdgcn_s_waitcnt(kWQ);
            else __builtin_amdgcn_s_waitcnt(kW0);
        }
        barrier();
        if (!last) {
            ++ckb;
            return true;
        }
        finish(ci);
        if (!next) return false;
        ck = nk;
        ci = ni;
        ckb = 0;
        enter(ci);
        return true;
    };

    // Prologue: blocks 0 and 1 and the first item's Q, all complete before block 0.
    const bool loaded1 = load_next(0) && load_next(1);
    (void)loaded1;
    load_q(ci);
    enter(ci);
    __builtin_amdgcn_s_waitcnt(kW0);
    barrier();
    for (;;) {
        if (!step(std::integral_constant<int, 0>{})) break;
        if (!step(std::integral_constant<int, 1>{})) break;
        if (!step(std::integral_constant<int, 2>{})) break;
    }
}

// Compute units of the current device (cached per device id).
int fa_device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// ---------------------------------------------------------------------------
// Vector-ALU kernel for the head sizes the matrix-core kernels do not take (not a
// multiple of 8, or above 128; up to kGenMaxD), as the reference's Triton kernel
// takes any head size (reference kernals/flash_attention.py:72 pads it to a power
// of two). One wave per (sequence, q head, query row): the row's q is staged in the
// wave's LDS slot as float32; each lane scores one key of a 64-key block (a float32
// dot product over D), the block enters the online softmax (base 2), and each lane
// accumulates D / 64 output dims (rounded up: ND per lane) from the block's V rows,
// the probabilities broadcast from their lanes. Element loads only: no alignment
// beyond the element's. Rows past max_seq_len are not computed.
constexpr int kGenMaxD = 512;
constexpr int kGenWaves = 4;

template <int IT, int ND>
__global__ void __launch_bounds__(64 * kGenWaves)
prefill_generic_kernel(PrefillArgs a) {
    using T = typename Elem<IT>::T;
    __shared__ float q_lds[kGenWaves][kGenMaxD];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // Unit (sequence b, q head hq, row r): consecutive rows of one head share a workgroup.
    const int64_t unit = (int64_t)blockIdx.x * kGenWaves + wave;
    const int64_t per_b = (int64_t)a.hq * a.max_len;
    const int b = (int)(unit / per_b);
    if (b >= a.batch) return;
    const int64_t rest = unit - (int64_t)b * per_b;
    const int hq = (int)(rest / a.max_len);
    const int r = (int)(rest - (int64_t)hq * a.max_len);
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
    const int64_t len = s1 > s0 ? s1 - s0 : 0;
    if (r >= len) return;                  // r < max_seq_len by construction

    const int D = a.d;
    const int hk = hq / (a.hq / a.hkv);
    const int64_t tok = s0 + r;
    const int64_t kv_stride = (int64_t)a.hkv * D;
    const T* qrow = reinterpret_cast<const T*>(a.q) + (tok * a.hq + hq) * D;
    const T* kbase = reinterpret_cast<const T*>(a.k) + s0 * kv_stride + (int64_t)hk * D;
    const T* vbase = reinterpret_cast<const T*>(a.v) + s0 * kv_stride + (int64_t)hk * D;
    float* qs = q_lds[wave];
    for (int d = lane; d < D; d += 64) qs[d] = Elem<IT>::load(qrow[d]);
    __builtin_amdgcn_wave_barrier();      // one wave's LDS operations complete in order

    float m = kNegInf, l = 0.0f;
    float acc[ND];
#pragma unroll
    for (int e = 0; e < ND; ++e) acc[e] = 0.0f;
    for (int k0 = 0; k0 <= r; k0 += 64) {
        const int key = k0 + lane;
        const bool valid = key <= r;     // causal, and r < len
        float s = kNegInf;
        if (valid) {
            const T* krow = kbase + key * kv_stride;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += qs[d] * Elem<IT>::load(krow[d]);
            s = dot * a.scale_log2;
        }
        float mb = s;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) mb = fmaxf(mb, __shfl_xor(mb, o));
        const float m_new = fmaxf(m, mb);              // finite: key k0 <= r is valid
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        const float p = valid ? __builtin_amdgcn_exp2f(s - m_new) : 0.0f;
        float ps = p;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) ps += __shfl_xor(ps, o);
        l = l * alpha + ps;
#pragma unroll
        for (int e = 0; e < ND; ++e) acc[e] *= alpha;
        const int nkeys = min(64, r - k0 + 1);
        for (int jj = 0; jj < nkeys; ++jj) {
            const float pj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), jj));
            const T* vrow = vbase + (int64_t)(k0 + jj) * kv_stride;
#pragma unroll
            for (int e = 0; e < ND; ++e) {
                const int d = lane + 64 * e;
                if (d < D) acc[e] += pj * Elem<IT>::load(vrow[d]);
            }
        }
        m = m_new;
    }
    T* orow = reinterpret_cast<T*>(a.out) + (tok * a.hq + hq) * D;
    const float inv = 1.0f / l;                      // l >= 1: the row's largest score enters as 1
#pragma unroll
    for (int e = 0; e < ND; ++e) {
        const int d = lane + 64 * e;
        if (d < D) orow[d] = Elem<IT>::store(acc[e] * inv);
    }
    if (lane == 0) a.lse[tok * a.hq + hq] = (m + __builtin_log2f(l)) * kLn2;
}

template <int IT>
hipError_t launch_generic_prefill(const PrefillArgs& a, int64_t blocks, hipStream_t s) {
    const dim3 grid((unsigned)blocks), block(64 * kGenWaves);
    if (a.d <= 64) hipLaunchKernelGGL((prefill_generic_kernel<IT, 1>), grid, block, 0, s, a);
    else if (a.d <= 128) hipLaunchKernelGGL((prefill_generic_kernel<IT, 2>), grid, block, 0, s, a);
    else if (a.d <= 256) hipLaunchKernelGGL((prefill_generic_kernel<IT, 4>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((prefill_generic_kernel<IT, 8>), grid, block, 0, s, a);
    return hipGetLastError();
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
    // Head sizes: multiples of 8 up to 128 on the matrix cores (8-element operand
    // runs), every other size up to kGenMaxD on the vector-ALU kernel.
    if (head_dim <= 0 || head_dim > kGenMaxD) return KVFP8_ESHAPE;
    const bool matrix = head_dim % 8 == 0 && head_dim <= 128;
    if (total_tokens == 0 || batch == 0 || max_seq_len == 0) return KVFP8_OK;
    if (!q || !k || !v || !out || !lse || !cu_seqlens) return KVFP8_ENULL;
    const uintptr_t align = matrix ? 15 : (dtype == KVFP8_F32 ? 3 : 1);
    if ((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & align) != 0) return KVFP8_ESTRIDE;
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
    if (!matrix) {
        const int64_t units = (int64_t)batch * num_q_heads * max_seq_len;
        const int64_t blocks = (units + kGenWaves - 1) / kGenWaves;
        if (blocks >= ((int64_t)1 << 31)) return KVFP8_ELIMIT;
        switch (dtype) {
            case KVFP8_F32: return (int)launch_generic_prefill<KVFP8_F32>(a, blocks, s);
            case KVFP8_F16: return (int)launch_generic_prefill<KVFP8_F16>(a, blocks, s);
            default: return (int)launch_generic_prefill<KVFP8_BF16>(a, blocks, s);
        }
    }
    // 16-bit inputs with D 64 or 128: the wide-tile kernel, whose item and token
    // indices are int32 (larger inputs take the general kernel below).
    const int fa_rows = kFaRows * kFaWaves / a.heads_per_block;
    const int64_t fa_units = (int64_t)batch * num_kv_heads * a.blocks_per_kv;
    const int64_t fa_upx = (fa_units + kXcds - 1) / kXcds;
    const bool fa_fits = total_tokens < ((int64_t)1 << 31) &&
                         fa_upx * kXcds * (((int64_t)max_seq_len + fa_rows - 1) / fa_rows) < ((int64_t)1 << 31);
    if ((dtype == KVFP8_BF16 || dtype == KVFP8_F16) && (head_dim == 64 || head_dim == 128) && fa_fits) {
        a.rows = fa_rows;
        a.qblocks = (max_seq_len + a.rows - 1) / a.rows;
        // One persistent workgroup per CU (its LDS holds one), per_xcd of them on
        // each XCD, each walking its share of the XCD's items.
        const int64_t units = fa_units;
        const int64_t upx = fa_upx;
        const int64_t items_per_xcd = upx * (int64_t)a.qblocks;
        int64_t per_xcd = fa_device_cus() / kXcds;
        per_xcd = per_xcd < 1 ? 1 : per_xcd;
        per_xcd = per_xcd < items_per_xcd ? per_xcd : items_per_xcd;
        const dim3 grid((unsigned)(kXcds * per_xcd)), block(kFaThreads);
        if (dtype == KVFP8_BF16) {
            if (head_dim == 64) hipLaunchKernelGGL((prefill_fa_kernel<1, false>), grid, block, 0, s, a, (int32_t)units, (int32_t)upx, (int32_t)per_xcd);
            else hipLaunchKernelGGL((prefill_fa_kernel<2, false>), grid, block, 0, s, a, (int32_t)units, (int32_t)upx, (int32_t)per_xcd);
        } else {
            if (head_dim == 64) hipLaunchKernelGGL((prefill_fa_kernel<1, true>), grid, block, 0, s, a, (int32_t)units, (int32_t)upx, (int32_t)per_xcd);
            else hipLaunchKernelGGL((prefill_fa_kernel<2, true>), grid, block, 0, s, a, (int32_t)units, (int32_t)upx, (int32_t)per_xcd);
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
