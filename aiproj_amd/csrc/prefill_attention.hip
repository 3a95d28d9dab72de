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
    a.rows = kWaveRows * 4 / a.heads_per_block;
    a.qblocks = (max_seq_len + a.rows - 1) / a.rows;
    a.max_len = max_seq_len;
    a.total_tokens = total_tokens;
    a.scale_log2 = scale * 1.44269504088896340736f;
    const int64_t blocks = (int64_t)a.qblocks * batch * num_kv_heads * a.blocks_per_kv;
    if (blocks >= ((int64_t)1 << 31)) return KVFP8_ESHAPE;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t err;
    switch (dtype) {
        case KVFP8_F32: err = launch_prefill<KVFP8_F32>(a, blocks, s); break;
        case KVFP8_F16: err = launch_prefill<KVFP8_F16>(a, blocks, s); break;
        default: err = launch_prefill<KVFP8_BF16>(a, blocks, s); break;
    }
    return (int)err;
}
