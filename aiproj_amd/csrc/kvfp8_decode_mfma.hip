// FP8 paged decode attention on the gfx950 matrix cores.
//
// Replaces the Triton split and reduction kernels of reference
// src/torch_llm/kernals/decode_attention.py:194-550 for e4m3fn and bf16 caches
// (and f16 caches read with f16 q) with D in {64, 128} and pages of 16k tokens.
//
// Work split. The attended tokens of the batch form one list of 16-token tiles
// (sequence by sequence, tile prefix built in LDS from context_lengths, no host
// synchronization). Workgroup w of `groups` takes the contiguous tile range
// [w W / groups, (w+1) W / groups), so every workgroup reads the same number of
// bytes whatever the length distribution. A sequence that lies inside one range
// is finished in place; a sequence cut by range boundaries leaves one partial
// softmax state per piece (at most two per workgroup: its first and last
// segment) and the combine kernel merges them.
//
// Inside a workgroup wave i serves KV head i (and i + waves, ...), so the
// workgroup reads whole pages: 16 tokens x Hkv x D contiguous bytes of K and V.
// The two waves that share a SIMD keep pace through an LDS step counter and the
// wave issue priority (the arbiter would otherwise favour the older one).
// One step of a wave covers two tiles (32 tokens) of its head:
//
//   scores   S^T[t, g] = K[t, :] . Q[g, :]      MFMA 16x16x32 bf16, A = K codes
//            converted fp8 -> bf16 (exact), B = Q^T (bf16; f32/f16 q as hi + lo)
//            then x k_scale[t] x sm_scale x log2(e)   (fp32)
//   softmax  online, base 2, state per lane = per q head column g
//   output   O^T[d, g] += V^T[d, t] . P'^T[t, g]    MFMA 16x16x32 bf16,
//            P' = p x v_scale[t]; V^T from an in-register byte transpose
//
// MFMA 16x16x32 bf16 operand layout (lane l, element i, output element j):
//   A[row = l % 16][k = 8 (l / 16) + i], B[k = 8 (l / 16) + i][col = l % 16],
//   D[row = 4 (l / 16) + j][col = l % 16].
// The reduction index of each product may be permuted freely as long as both
// operands use the same permutation; the kernel picks the permutations that let
// every lane load long contiguous runs:
//   * QK, e4m3fn with D = 128 (whole-row K): an MFMA row is (token t of an
//     8-token sub-tile, half h of D) = 2t + h and a column is (q head g, half
//     h') = g + 8h', so lane 2t + h + 16j reads the 16 bytes at 64h + 16j of
//     token t and one load instruction covers eight whole 128-byte rows. The
//     score of (t, g) is the sum of the two diagonal blocks h = h', which sit 8
//     lanes apart (one DPP row rotate). q heads 8..15 use a second set of
//     products.
//   * QK otherwise: lane l reads 16-byte runs of token (l % 16) at byte 64 c +
//     16 (l / 16); bytes 8h..8h+7 of run c feed MFMA 2c + h.
//   * PV: lane l reads 4C contiguous bytes at column 4C (l % 16) of eight token
//     rows: tokens step_token(i, l / 16) of tile A (i < 4) and of tile B
//     (i >= 4), the same tokens its scores belong to. v_perm_b32 pairs rows (2p, 2p+1)
//     of one column and v_cvt_scalef32_pk_bf16_fp8 widens the pair.
#include "kvfp8_decode_mfma.h"

#include <type_traits>

namespace kvfp8 {

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kMaxWaves = 8;            // KV heads served by one workgroup at a time
constexpr int kMaxThreads = 64 * kMaxWaves;
constexpr int kMinTilesPerGroup = 2;    // a group gets at least 32 tokens per head
// Waves per CU the grid is sized for (caps the grid and sizes the workspace): with fewer
// KV heads than 8 and no replicas the workgroups are narrower, and fewer, longer ones (one
// 4-wave group per CU at 4 KV heads) measured faster than filling each CU: 16q/4kv over
// 64 x 1040 tokens 19.9 -> 19.0 us, 16q/2kv over 32 x 4096 21.7 -> 20.7 us (same-box A/B);
// 8 KV heads are unaffected.
constexpr int kWavesPerCu = 4;
constexpr int kMfmaMaxBatch = 8191;     // LDS: tile prefix (batch + 1) and sequence metadata (batch) int32

struct MfmaArgs {
    DecodeArgs d;
    int32_t tps_shift;   // log2(block_size / 16): 16-token tiles per page
    int32_t* plan;       // [batch + 1] tile prefix, then the workgroup count used
    float* part_m;       // [2 * max_groups, Hq]
    float* part_l;       // [2 * max_groups, Hq]
    float* part_acc;     // [2 * max_groups, Hq, D]
    int32_t q_vec;       // q rows start 16-byte aligned: 8 elements per vector load
};

__device__ __forceinline__ int32_t uniform(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// floor(n / d) for 0 <= n < 2^53 and d >= 1 through one IEEE double division, in
// place of the long instruction sequence of a 64-bit integer division. Exact: n and d
// convert exactly, the quotient q = n / d rounds to within q 2^-53 < 1 / d of itself,
// and when q is not an integer the next integer above it is at least 1 / d away (an
// integer q is exact), so the truncation lands on floor(q).
__device__ __forceinline__ int32_t floor_div(int64_t n, int64_t d) {
    return (int32_t)((double)n / (double)d);
}

__device__ __forceinline__ int64_t uniform64(int64_t x) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)x);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)((uint64_t)x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ bf16x8_t cat8(bf16x2_t a, bf16x2_t b, bf16x2_t c, bf16x2_t d) {
    const bf16x4_t ab = __builtin_shufflevector(a, b, 0, 1, 2, 3);
    const bf16x4_t cd = __builtin_shufflevector(c, d, 0, 1, 2, 3);
    return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Two e4m3fn codes (bytes 0-1 or 2-3 of x) -> two bf16, exact.
__device__ __forceinline__ bf16x2_t fp8x2_lo(uint32_t x) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, false);
}
__device__ __forceinline__ bf16x2_t fp8x2_hi(uint32_t x) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, true);
}

// Eight codes (x0 bytes 0..3, then x1) -> bf16x8 in byte order.
__device__ __forceinline__ bf16x8_t fp8x8(uint32_t x0, uint32_t x1) {
    return cat8(fp8x2_lo(x0), fp8x2_hi(x0), fp8x2_lo(x1), fp8x2_hi(x1));
}

__device__ __forceinline__ f32x4_t mma(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mma(f16x8_t a, f16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Operand type of the products: bf16 (e4m3fn codes widen to it exactly, bf16 caches
// are it), or f16 for an f16 cache read with f16 q (both exact in f16).
template <bool kF16> using OpT = std::conditional_t<kF16, f16x8_t, bf16x8_t>;
template <bool kF16> using OpE = std::conditional_t<kF16, _Float16, __bf16>;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value of lane (l ^ 8) (DPP row_ror:8 inside each row of 16 lanes).
__device__ __forceinline__ float row_ror8(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xF, 0xF, false));
}

// The e4m3fn D = 128 kernel reads K in whole 128-byte rows (see load_step).
template <int C, int ES>
constexpr bool kWholeRowK = ES == 1 && C == 2;

// Token (within its 16-token tile, tile i / 4) of score i and V row i of lane group j.
template <bool kWL>
__device__ __forceinline__ int step_token(int i, int j) {
    if constexpr (kWL) return 8 * ((i >> 1) & 1) + 2 * j + (i & 1);
    else return 4 * j + (i & 3);
}

// Tile prefix over the batch in LDS: prefix[b] = sum_{i<b} ceil(len_i / 16),
// and meta[b] = slot_b * 32 + (tokens in the last tile of b) for sequences with
// tokens (slots are below 2^26, checked by the host). Per-thread runs, a shuffle
// scan inside each wave, then the wave totals. kMark (fused append + decode): bit
// 31 of meta[b] marks a sequence whose new token, at position len_b - 1, is one
// the decode attends (new_token_attended).
template <bool kMark>
__device__ void build_tile_prefix(const DecodeArgs& a, int32_t* prefix, int32_t* meta, int32_t* wave_total) {
    const int threads = blockDim.x, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int per = (a.batch + threads - 1) / threads;
    const int begin = tid * per;
    int32_t local = 0;
    for (int i = 0; i < per; ++i) {
        const int b = begin + i;
        if (b < a.batch) {
            int64_t slot, raw;
            const int64_t len = seq_tokens(a, b, &slot, &raw);
            const int32_t tiles = (int32_t)((len + 15) >> 4);
            const int32_t mark = kMark && new_token_attended(a, slot, raw) ? INT32_MIN : 0;
            prefix[b] = local;
            meta[b] = tiles > 0 ? (int32_t)(slot << 5) | (int32_t)(len - 16 * (int64_t)(tiles - 1)) | mark : 0;
            local += tiles;
        }
    }
    int32_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int32_t y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
    }
    if (lane == 63) wave_total[wave] = incl;
    __syncthreads();
    int32_t base = incl - local;
    for (int w = 0; w < wave; ++w) base += wave_total[w];
    for (int i = 0; i < per; ++i) {
        const int b = begin + i;
        if (b < a.batch) prefix[b] += base;
    }
    if (tid == threads - 1) prefix[a.batch] = base + local;
    __syncthreads();
}

// Global row (page * block_size + token base) of a 16-token tile; 0 when the
// page entry is outside the pool (the tile's tokens are then masked).
struct TileRef {
    int64_t row0;
    int32_t valid;
};

typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;

__device__ __forceinline__ TileRef tile_ref(const MfmaArgs& a, const int32_t* table_row, int32_t tile) {
    // The block table is read-only during the kernel and the address is
    // wave-uniform: read it with a scalar load, whose wait (lgkmcnt) does not
    // also wait for the K/V loads in flight the way a vector load's would.
    const int32_t page = tile >> a.tps_shift;
    const int64_t addr = uniform64((int64_t)(uintptr_t)(table_row + page));
    const int64_t phys = *(const_i32_ptr)(uintptr_t)addr;
    const bool ok = phys >= 0 && phys < a.d.num_blocks;
    const int32_t base = (tile & ((1 << a.tps_shift) - 1)) << 4;
    TileRef r;
    r.row0 = ok ? phys * a.d.block_size + base : 0;
    r.valid = ok;
    return r;
}

// Loads of one 32-token step of one KV head. ES is the byte size of a cache
// element: 1 for e4m3fn codes, 2 for bf16 values.
template <int C, int ES>
struct StepData {
    u32x4_t ka[C * ES];      // tile A: token (l % 16), 16-byte runs at bytes 64 r + 16 (l / 16)
                             // (whole-row K: run r holds token 8r + (l % 16) / 2 at byte 64 (l % 2) + 16 (l / 16))
    u32x4_t kb[C * ES];      // tile B, same runs
    uint32_t v[8][C * ES];   // rows i: token step_token(i, l / 16) of tile (i < 4 ? A : B), 4C elements at element 4C (l % 16)
    float sc;                // e4m3fn: lane l holds the [k|v][tile A|B][token l % 16] scale
};

template <int C, int ES>
__device__ __forceinline__ void load_step(StepData<C, ES>& s, const MfmaArgs& a, int h, const TileRef& ta,
                                          const TileRef& tb, int lane) {
    constexpr int D = 64 * C;
    constexpr int NB = 4 * C;
    constexpr int KR = C * ES;
    constexpr int VW = C * ES;
    const int m16 = lane & 15, j = lane >> 4;
    const int32_t hkv = a.d.num_kv_heads;
    const int32_t row_stride = hkv * D * ES;                 // bytes between tokens
    const int64_t ea = (ta.row0 * hkv + h) * D * ES;
    const int64_t eb = (tb.row0 * hkv + h) * D * ES;
    const uint8_t* kc = reinterpret_cast<const uint8_t*>(a.d.k_cache);
    const uint8_t* vc = reinterpret_cast<const uint8_t*>(a.d.v_cache);
    constexpr bool kWL = kWholeRowK<C, ES>;
    if constexpr (kWL) {
        // Lane 2t + h + 16 j reads bytes 64 h + 16 j .. + 15 of token t (8 tokens
        // per instruction): every instruction reads eight whole 128-byte rows,
        // streamed with nontemporal loads.
        const uint32_t koff = (uint32_t)((m16 >> 1) * row_stride + 64 * (m16 & 1) + 16 * j);
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            s.ka[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kc + ea + koff + 8 * r * row_stride));
            s.kb[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kc + eb + koff + 8 * r * row_stride));
        }
    } else {
        // Token (l % 16), 16-byte runs at 64 r + 16 (l / 16). With D = 64 codes a
        // run set is the whole row (nontemporal); wider rows are read as pieces
        // by separate instructions, and normal loads keep the line in L2 between them.
        const uint32_t koff = (uint32_t)(m16 * row_stride + 16 * j);
#pragma unroll
        for (int r = 0; r < KR; ++r) {
            if constexpr (KR == 1) {
                s.ka[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kc + ea + koff + 64 * r));
                s.kb[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kc + eb + koff + 64 * r));
            } else {
                s.ka[r] = *reinterpret_cast<const u32x4_t*>(kc + ea + koff + 64 * r);
                s.kb[r] = *reinterpret_cast<const u32x4_t*>(kc + eb + koff + 64 * r);
            }
        }
    }
    // Every V instruction reads whole rows (nontemporal).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint8_t* p = vc + (i < 4 ? ea : eb) + (uint32_t)(step_token<kWL>(i, j) * row_stride + NB * ES * m16);
        if constexpr (VW == 1) {
            s.v[i][0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
        } else if constexpr (VW == 2) {
            const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
            s.v[i][0] = x.x;
            s.v[i][1] = x.y;
        } else {
            const u32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
            s.v[i][0] = x.x;
            s.v[i][1] = x.y;
            s.v[i][2] = x.z;
            s.v[i][3] = x.w;
        }
    }
    if constexpr (ES == 1) {
        const int kv = lane >> 5, which = (lane >> 4) & 1;
        const int64_t r = (which ? tb.row0 : ta.row0) + m16;
        s.sc = (kv ? a.d.v_scales : a.d.k_scales)[r * hkv + h];
    }
}

// Online-softmax state of one wave (one KV head, its G q heads in columns g).
template <int C>
struct WaveState {
    f32x4_t o[4 * C];     // O^T[d = 4C (4 (l/16) + j) + nb][g = l % 16] in o[nb][j]
    float m;              // running max (base-2 scores) of column g
    float l;              // this lane's share of the softmax denominator
};

// Q head column and dimension feeding element i of Q^T operand kb in lane
// (c = l % 16, j = l / 16): the same permutation of the head dimension as the K
// runs of load_step. Whole-row K: operand kb = 2 set + m holds column (g, h') =
// c, head g = c % 8 + 8 set, dims of half h' = c / 8.
template <int C, int ES>
__device__ __forceinline__ int qk_head(int kb, int c) {
    if constexpr (kWholeRowK<C, ES>) return (c & 7) + 8 * (kb >> 1);
    else return c;
}
template <int C, int ES>
__device__ __forceinline__ int qk_dim(int kb, int c, int j, int i) {
    if constexpr (kWholeRowK<C, ES>) return 64 * (c >> 3) + 16 * j + 8 * (kb & 1) + i;
    else if constexpr (ES == 1) return 64 * (kb >> 1) + 16 * j + 8 * (kb & 1) + i;   // 16 codes per run, 2 MFMAs
    else return 32 * kb + 8 * j + i;                                                  // 8 values per run, 1 MFMA
}

// kSets = 2: whole-row K with G > 8 (a second set of QK products for heads 8..15).
// Raw q elements of the Q^T operands of lane (c = l % 16, j = l / 16) for the G
// q heads of KV head h of sequence b: operand kb holds q[b, h G + g, d .. d + 7]
// with g = qk_head(kb, c), d = qk_dim(kb, c, j, 0) (16 or 32 bytes). Operands
// whose heads are all >= G are not loaded (kOps of them are). Loads are 16 bytes
// wide when q allows them (MfmaArgs::q_vec), else element loads.
template <int C, int QT>
struct QRaw {
    static constexpr int kWords = QT == KVFP8_F32 ? 8 : 4;
    uint32_t w[2 * C][kWords];
};

template <int C, int ES, int QT, int kOps>
__device__ __forceinline__ void load_q_raw(const MfmaArgs& a, int b, int h, int G, int lane, QRaw<C, QT>& r) {
    using T = typename Elem<QT>::T;
    constexpr int kWords = QRaw<C, QT>::kWords;
    const int c = lane & 15, j = lane >> 4;
    const T* base = reinterpret_cast<const T*>(a.d.q) + (int64_t)b * a.d.q_stride_b;
    const T* p[kOps];
#pragma unroll
    for (int kb = 0; kb < kOps; ++kb) {
        const int g = min(qk_head<C, ES>(kb, c), G - 1);
        p[kb] = base + (int64_t)(h * G + g) * a.d.q_stride_h + qk_dim<C, ES>(kb, c, j, 0);
    }
    if (a.q_vec) {
#pragma unroll
        for (int kb = 0; kb < kOps; ++kb) {
#pragma unroll
            for (int v = 0; v < kWords / 4; ++v) {
                const u32x4_t u = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint8_t*>(p[kb]) + 16 * v);
                r.w[kb][4 * v] = u.x;
                r.w[kb][4 * v + 1] = u.y;
                r.w[kb][4 * v + 2] = u.z;
                r.w[kb][4 * v + 3] = u.w;
            }
        }
    } else {
#pragma unroll
        for (int kb = 0; kb < kOps; ++kb) {
            if constexpr (QT == KVFP8_F32) {
#pragma unroll
                for (int i = 0; i < 8; ++i) r.w[kb][i] = __builtin_bit_cast(uint32_t, p[kb][i]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) r.w[kb][i] = (uint32_t)p[kb][2 * i] | ((uint32_t)p[kb][2 * i + 1] << 16);
            }
        }
    }
}

// Q^T operands from the raw elements: bf16 (f32 and f16 q as hi + lo parts) or f16
// (f16 q, exact), zero for heads g >= G and for operands not loaded.
template <int C, int ES, int QT, int kOps, bool kHiLo, bool kF16>
__device__ __forceinline__ void q_operands(const QRaw<C, QT>& r, int G, int lane, OpT<kF16>* qh, OpT<kF16>* ql) {
    using E = OpE<kF16>;
    using T = typename Elem<QT>::T;
    const int c = lane & 15;
#pragma unroll
    for (int kb = 0; kb < 2 * C; ++kb) {
        const bool live = kb < kOps && qk_head<C, ES>(kb, c) < G;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float x = 0.0f;
            if (kb < kOps) {
                if constexpr (QT == KVFP8_F32) x = __builtin_bit_cast(float, r.w[kb][i]);
                else x = Elem<QT>::load((T)((r.w[kb][i >> 1] >> (16 * (i & 1))) & 0xFFFFu));
            }
            x = live ? x : 0.0f;
            const E hi = (E)x;
            qh[kb][i] = hi;
            if constexpr (kHiLo) ql[kb][i] = (E)(x - (float)hi);
        }
    }
}

template <int C, int ES, bool kHiLo, int kSets, bool kF16>
__device__ __forceinline__ void compute_step(WaveState<C>& st, const StepData<C, ES>& s, const OpT<kF16>* qh,
                                             const OpT<kF16>* ql, float4* stage, int lane, int lim_a,
                                             int lim_b, float score_scale) {
    static_assert(!kF16 || ES == 2, "f16 operands come from an f16 cache");
    using Op = OpT<kF16>;
    using E = OpE<kF16>;
    constexpr int VW = C * ES;
    const int j = lane >> 4;
    const bool full = lim_a == 16 && lim_b == 16;   // wave-uniform

    constexpr bool kWL = kWholeRowK<C, ES>;
    // Per-token scales of score i (k, with sm_scale * log2(e)) and V row i (v).
    float ks[8], vs[8];
    if constexpr (ES == 1) {
        // Through this wave's LDS slot: lane l holds the scale of [k|v] (l / 32),
        // step token l % 32, stored so that each lane reads its 8 tokens as two
        // float4 runs.
        float* stage_f = reinterpret_cast<float*>(stage);
        int widx = lane;
        if constexpr (kWL) {
            const int p = lane & 31;    // step token 8 x + 2 j' + s -> slot 8 j' + 2 x + s
            widx = (lane & 32) + 8 * ((p >> 1) & 3) + 2 * (p >> 3) + (p & 1);
        }
        stage_f[widx] = lane < 32 ? s.sc * score_scale : s.sc;
        __builtin_amdgcn_wave_barrier();
        float4 k0, k1, v0, v1;
        if constexpr (kWL) {
            k0 = stage[2 * j];
            k1 = stage[2 * j + 1];
            v0 = stage[8 + 2 * j];
            v1 = stage[9 + 2 * j];
        } else {
            k0 = stage[j];
            k1 = stage[4 + j];
            v0 = stage[8 + j];
            v1 = stage[12 + j];
        }
        __builtin_amdgcn_wave_barrier();
        ks[0] = k0.x; ks[1] = k0.y; ks[2] = k0.z; ks[3] = k0.w;
        ks[4] = k1.x; ks[5] = k1.y; ks[6] = k1.z; ks[7] = k1.w;
        vs[0] = v0.x; vs[1] = v0.y; vs[2] = v0.z; vs[3] = v0.w;
        vs[4] = v1.x; vs[5] = v1.y; vs[6] = v1.z; vs[7] = v1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ks[i] = score_scale;
            vs[i] = 1.0f;
        }
    }

    // Scores of the 32 tokens, 8 per lane: score i is token step_token(i, j) of
    // tile i / 4.
    float sc[8];
    if constexpr (kWL) {
        // Sub-tile x (tokens 8x .. 8x + 7 of the step): MFMA rows are (token t,
        // half h of D) = 2t + h, columns (q head g, half h') = g + 8h' for the q
        // heads g < 8 (set 0) and, with G > 8, 8 + g (set 1). D[(t, h)][(g, h')]
        // is the dot product over half h of K with half h' of Q, so the score of
        // (t, g) is D[(t,0)][(g,0)] + D[(t,1)][(g,1)]: register 2s of lane c and
        // register 2s + 1 of lane c + 8 (c < 8, token t = 2 j + s). Lane c keeps
        // its half and takes its partner's through a row rotate by 8; lanes
        // c >= 8 end with the scores of column c (set 1) or a copy of column c - 8.
        const bool upper = (lane & 8) != 0;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            const u32x4_t kr = x < 2 ? s.ka[x] : s.kb[x - 2];
            const bf16x8_t k0 = fp8x8(kr[0], kr[1]), k1 = fp8x8(kr[2], kr[3]);
            f32x4_t d0 = {0.0f, 0.0f, 0.0f, 0.0f};
            d0 = mma(k0, qh[0], d0);
            d0 = mma(k1, qh[1], d0);
            if constexpr (kHiLo) {
                d0 = mma(k0, ql[0], d0);
                d0 = mma(k1, ql[1], d0);
            }
            f32x4_t d1 = d0;
            if constexpr (kSets == 2) {
                d1 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                d1 = mma(k0, qh[2], d1);
                d1 = mma(k1, qh[3], d1);
                if constexpr (kHiLo) {
                    d1 = mma(k0, ql[2], d1);
                    d1 = mma(k1, ql[3], d1);
                }
            }
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float own = upper ? d1[2 * e + 1] : d0[2 * e];
                const float send = upper ? d0[2 * e + 1] : d1[2 * e];
                sc[2 * x + e] = (own + row_ror8(send)) * ks[2 * x + e];
            }
        }
    } else {
        f32x4_t sa = {0.0f, 0.0f, 0.0f, 0.0f}, sb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 2 * C; ++kb) {
            Op ka, kbv;
            if constexpr (ES == 1) {
                const int c = kb >> 1, half = kb & 1;
                ka = fp8x8(s.ka[c][2 * half], s.ka[c][2 * half + 1]);
                kbv = fp8x8(s.kb[c][2 * half], s.kb[c][2 * half + 1]);
            } else {
                ka = __builtin_bit_cast(Op, s.ka[kb]);
                kbv = __builtin_bit_cast(Op, s.kb[kb]);
            }
            sa = mma(ka, qh[kb], sa);
            sb = mma(kbv, qh[kb], sb);
            if constexpr (kHiLo) {
                sa = mma(ka, ql[kb], sa);
                sb = mma(kbv, ql[kb], sb);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = sa[i] * ks[i];
            sc[4 + i] = sb[i] * ks[4 + i];
        }
    }
    bool live[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) live[i] = full || step_token<kWL>(i, j) < (i < 4 ? lim_a : lim_b);
    if (!full) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!live[i]) sc[i] = kNegInf;
    }

    // Online softmax over the 32 tokens (8 per lane, 4 lane groups per column).
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sc[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(st.m, mx);
    const float m_use = m_new == kNegInf ? 0.0f : m_new;
    const float alpha = fast_exp2(st.m - m_use);
    st.l *= alpha;
    if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (int nb = 0; nb < 4 * C; ++nb) st.o[nb] *= alpha;
    }
    st.m = m_new;
    float pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float p = fast_exp2(sc[i] - m_use);
        st.l += p;
        pv[i] = p * vs[i];
    }
    if (!full) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!live[i]) pv[i] = 0.0f;
    }
    Op ph, pl;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        ph[i] = (E)pv[i];
        if constexpr (kHiLo) pl[i] = (E)(pv[i] - (float)ph[i]);
    }

    // V rows: zero the rows of masked tokens (stale pages may hold NaN).
    uint32_t vr[8][VW];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int c = 0; c < VW; ++c) vr[i][c] = live[i] ? s.v[i][c] : 0u;
    }
    if constexpr (ES == 1) {
        // Byte transpose: pair the codes of rows (2p, 2p + 1) at one column, widen.
#pragma unroll
        for (int c = 0; c < C; ++c) {
            bf16x2_t e[4][4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t x = __builtin_amdgcn_perm(vr[2 * p + 1][c], vr[2 * p][c], 0x05010400u);
                const uint32_t y = __builtin_amdgcn_perm(vr[2 * p + 1][c], vr[2 * p][c], 0x07030602u);
                e[0][p] = fp8x2_lo(x);
                e[1][p] = fp8x2_hi(x);
                e[2][p] = fp8x2_lo(y);
                e[3][p] = fp8x2_hi(y);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const bf16x8_t av = cat8(e[q][0], e[q][1], e[q][2], e[q][3]);
                st.o[4 * c + q] = mma(av, ph, st.o[4 * c + q]);
                if constexpr (kHiLo) st.o[4 * c + q] = mma(av, pl, st.o[4 * c + q]);
            }
        }
    } else {
        // 16-bit transpose: element nb of rows (2p, 2p + 1) into one dword.
#pragma unroll
        for (int nb = 0; nb < 4 * C; ++nb) {
            const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
            u32x4_t w;
#pragma unroll
            for (int p = 0; p < 4; ++p) w[p] = __builtin_amdgcn_perm(vr[2 * p + 1][nb >> 1], vr[2 * p][nb >> 1], sel);
            const Op av = __builtin_bit_cast(Op, w);
            st.o[nb] = mma(av, ph, st.o[nb]);
            if constexpr (kHiLo) st.o[nb] = mma(av, pl, st.o[nb]);
        }
    }
}

// Fused append of one sequence's new token for KV head h, by the wave that serves
// h in the workgroup attending over the sequence's last tile: the same rule and
// arithmetic as quantize_append_kernel (amax as an integer max of |x| bits, which
// propagates NaN; scale = amax / 448 by IEEE division, 1 when amax is 0 or NaN;
// codes from the corrected reciprocal on finite rows, else clamp and encode).
// The row goes where the caller's write location (new_blocks[b], new_offsets[b])
// points, and nowhere when that lies outside the pool, as in the append kernel,
// provided that location is the sequence's last attended position: page
// block_table[slot, (len - 1) / block_size] (the entry fetch() reads) at offset
// (len - 1) % block_size, with the new token attended (meta bit 31). It then lies in
// the tile this wave reads last, and no other wave reads it. Any other location
// (or a new token the decode does not attend) is refused: nothing is stored, 1 goes
// to *new_refused, and the wave attends the row the cache holds, as the decode of the
// unchanged cache would. The write therefore never races with a read.
// Lane l holds elements C l .. C l + C - 1. fetch() issues the loads and put()
// quantizes and stores; the wave's own loads of that page row come after put()
// in its instruction order, which the memory pipeline keeps for one wave, so
// they read the new codes and scales.
// fetch() issues every load at once, with no branch and no wait in front of them:
// the kernel-argument fields are read together, the write location as two dword
// scalar loads per index (the low word, then the high word of an int64 entry or
// the low word again of an int32 one), and each element as two 16-bit loads (the
// two halves of a float32, or the 16-bit value twice), all at element alignment.
// The range check and the conversion to float wait for put(), which runs after
// the wave has issued its first K/V loads.
template <int C>
struct NewRow {
    uint32_t k_lo[C], k_hi[C], v_lo[C], v_hi[C];   // the two 16-bit loads of each element
    uint32_t page_lo, page_hi, off_lo, off_hi;
    uint32_t last_page;    // block-table entry of the last attended position
    int32_t last_off;      // its offset in the page, or -1 when the new token is not attended
    int32_t idx64;         // bit 0: new_blocks is int64; bit 1: new_offsets is int64
    int32_t dtype;
    int32_t h;             // KV head
};

typedef const __attribute__((address_space(4))) uint32_t* const_u32_ptr;
typedef const __attribute__((address_space(1))) uint16_t* const_g_u16_ptr;   // global memory

// table_row, len, attended: the sequence's block-table row, its attended length
// (at least 1) and whether its new token is attended (meta bit 31).
template <int C>
__device__ __forceinline__ void fetch_new_token(const MfmaArgs& a, int b, int h, int lane, NewRow<C>& r,
                                                const int32_t* table_row, int64_t len, bool attended) {
    constexpr int D = 64 * C;
    // The new-row fields are read from the kernel-argument segment here, where they
    // are used: the empty asm keeps the compiler from hoisting these loads to the
    // kernel's entry and holding them in scalar registers through the step loop.
    uint64_t kargs = (uint64_t)(uintptr_t)__builtin_amdgcn_kernarg_segment_ptr();
    __asm__ volatile("" : "+s"(kargs));
    typedef const __attribute__((address_space(4))) DecodeArgs* const_args_ptr;
    const_args_ptr na = (const_args_ptr)(uintptr_t)(kargs + offsetof(MfmaArgs, d));
    const uint64_t pb = (uint64_t)(uintptr_t)na->new_blocks, po = (uint64_t)(uintptr_t)na->new_offsets;
    const int32_t b64 = na->new_blocks64, o64 = na->new_offsets64;
    const int32_t dtype = na->new_dtype;
    const int64_t k_sb = na->new_k_sb, v_sb = na->new_v_sb;
    const uint64_t src_k = (uint64_t)(uintptr_t)na->new_k, src_v = (uint64_t)(uintptr_t)na->new_v;
    // Write location: scalar loads (their wait does not cover the vector loads in
    // flight). The index arrays are read-only for the whole kernel.
    const uint64_t pb_at = pb + (uint64_t)b * (b64 ? 8 : 4), po_at = po + (uint64_t)b * (o64 ? 8 : 4);
    r.page_lo = *(const_u32_ptr)pb_at;
    r.page_hi = *(const_u32_ptr)(pb_at + (b64 ? 4 : 0));
    r.off_lo = *(const_u32_ptr)po_at;
    r.off_hi = *(const_u32_ptr)(po_at + (o64 ? 4 : 0));
    const int32_t bs_shift = na->bs_shift;
    r.last_page = *(const_u32_ptr)(uintptr_t)(table_row + ((len - 1) >> bs_shift));
    r.last_off = attended ? (int32_t)((len - 1) & ((1 << bs_shift) - 1)) : -1;
    r.idx64 = (b64 ? 1 : 0) | (o64 ? 2 : 0);
    r.dtype = dtype;
    r.h = h;
    const uint64_t esz = dtype == KVFP8_F32 ? 4 : 2;
    const uint64_t hi_step = dtype == KVFP8_F32 ? 2 : 0;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
        const uint64_t row = (kv ? src_v : src_k) + ((uint64_t)b * (uint64_t)(kv ? v_sb : k_sb) + (uint64_t)h * D) * esz;
        uint32_t* lo = kv ? r.v_lo : r.k_lo;
        uint32_t* hi = kv ? r.v_hi : r.k_hi;
#pragma unroll
        for (int e = 0; e < C; ++e) {
            const uint64_t at = row + (uint64_t)(C * lane + e) * esz;
            lo[e] = *(const_g_u16_ptr)(uintptr_t)at;
            hi[e] = *(const_g_u16_ptr)(uintptr_t)(at + hi_step);
        }
    }
}

template <int C>
__device__ __forceinline__ void put_new_token(const MfmaArgs& a, const NewRow<C>& r, int lane) {
    constexpr int D = 64 * C;
    // The fetched values enter here: the empty asm (a memory clobber, the values as
    // operands) keeps the compiler from computing on them earlier, so their wait
    // comes after the loads the caller issued before this call rather than before
    // them (which would hold those loads back by one memory round trip).
    uint32_t rk[C], rv[C];
#pragma unroll
    for (int e = 0; e < C; ++e) {
        uint32_t kl = r.k_lo[e], kh = r.k_hi[e], vl = r.v_lo[e], vh = r.v_hi[e];
        __asm__ volatile("" : "+v"(kl), "+v"(kh), "+v"(vl), "+v"(vh) : : "memory");
        rk[e] = kl | (kh << 16);     // float32 bits, or the 16-bit value in the low half
        rv[e] = vl | (vh << 16);
    }
    const int64_t page = (r.idx64 & 1) ? (int64_t)(((uint64_t)r.page_hi << 32) | r.page_lo) : (int64_t)(int32_t)r.page_lo;
    const int64_t off = (r.idx64 & 2) ? (int64_t)(((uint64_t)r.off_hi << 32) | r.off_lo) : (int64_t)(int32_t)r.off_lo;
    if (r.last_off < 0 || page != (int64_t)(int32_t)r.last_page || off != r.last_off) {
        // The flag's address is read here, where it is used (see fetch_new_token).
        uint64_t kargs = (uint64_t)(uintptr_t)__builtin_amdgcn_kernarg_segment_ptr();
        __asm__ volatile("" : "+s"(kargs));
        typedef const __attribute__((address_space(4))) DecodeArgs* const_args_ptr;
        int32_t* flag = ((const_args_ptr)(uintptr_t)(kargs + offsetof(MfmaArgs, d)))->new_refused;
        if (lane == 0 && flag != nullptr) *flag = 1;
        return;
    }
    if (page < 0 || page >= a.d.num_blocks || off < 0 || off >= a.d.block_size) return;
    const int64_t row = (page * a.d.block_size + off) * a.d.num_kv_heads + r.h;
    float xk[C], xv[C];
#pragma unroll
    for (int e = 0; e < C; ++e) {
        xk[e] = r.dtype == KVFP8_F32 ? __uint_as_float(rk[e])
              : r.dtype == KVFP8_F16 ? f16_to_f32((uint16_t)rk[e]) : bf16_to_f32((uint16_t)rk[e]);
        xv[e] = r.dtype == KVFP8_F32 ? __uint_as_float(rv[e])
              : r.dtype == KVFP8_F16 ? f16_to_f32((uint16_t)rv[e]) : bf16_to_f32((uint16_t)rv[e]);
    }
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
        const float* x = kv ? xv : xk;
        uint32_t amax = abs_bits(x[0]);
#pragma unroll
        for (int e = 1; e < C; ++e) amax = max(amax, abs_bits(x[e]));
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, s));
        const float scale = row_scale(amax);
        const RowDivider div(scale);
        uint32_t codes;
        if (div.fast && amax < 0x7F800000u) {
            codes = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(div.corrected(x[0]), C > 1 ? div.corrected(x[C - 1]) : 0.0f,
                                                              0, false);
        } else {
            codes = clamp_encode(x[0] / scale);
            if constexpr (C > 1) codes |= (uint32_t)clamp_encode(x[C - 1] / scale) << 8;
        }
        uint8_t* dst = reinterpret_cast<uint8_t*>(const_cast<void*>(kv ? a.d.v_cache : a.d.k_cache)) + row * D + C * lane;
        if constexpr (C == 2) *reinterpret_cast<uint16_t*>(dst) = (uint16_t)codes;
        else *dst = (uint8_t)codes;
        if (lane == 0) const_cast<float*>(kv ? a.d.v_scales : a.d.k_scales)[row] = scale;
    }
}

template <int C, int QT, int ES, int kSets, bool kAppend, bool kF16, bool kRep>
__global__ void __launch_bounds__(kMaxThreads)
decode_mfma_kernel(MfmaArgs a) {
    constexpr int D = 64 * C;
    constexpr int NB = 4 * C;
    // q as bf16 hi + lo unless it is the operand type already (bf16 q on bf16
    // operands, f16 q on f16 operands).
    constexpr bool kHiLo = kF16 ? QT != KVFP8_F16 : QT != KVFP8_BF16;
    extern __shared__ int32_t prefix[];                // [batch + 1], then meta [batch]
    __shared__ int32_t wave_total[kMaxWaves];
    __shared__ float4 stage_all[kMaxWaves][16];
    __shared__ int32_t progress[kMaxWaves];     // steps computed by each wave
    if (threadIdx.x < kMaxWaves) progress[threadIdx.x] = 0;   // visible after the plan's barriers

    int32_t* meta = prefix + a.d.batch + 1;
    build_tile_prefix<kAppend>(a.d, prefix, meta, wave_total);
    const int32_t total = prefix[a.d.batch];
    const int32_t want = (total + kMinTilesPerGroup - 1) / kMinTilesPerGroup;
    const int32_t groups = min((int32_t)gridDim.x, max(want, 1));
    if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i <= a.d.batch; i += blockDim.x) a.plan[i] = prefix[i];
        if (threadIdx.x == 0) a.plan[a.d.batch + 1] = groups;
    }
    const int w = blockIdx.x;
    if (w >= groups) return;
    // w * total < 2^11 * 2^31 (groups <= the grid, tiles < 2^31 on the host).
    const int32_t start = uniform(floor_div((int64_t)w * total, groups));
    const int32_t end = uniform(floor_div((int64_t)(w + 1) * total, groups));

    const int waves = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int m16 = lane & 15, j = lane >> 4;
    const int G = a.d.num_q_heads / a.d.num_kv_heads;
    float4* stage = stage_all[wave];

    if constexpr (kAppend) {
        // Sequences with no attended tile (no context, or a slot outside the table)
        // attend no new token: their rows are refused (workgroup b % groups says so).
        if (threadIdx.x == 0 && a.d.new_refused != nullptr) {
            for (int b = w; b < a.d.batch; b += groups)
                if (prefix[b + 1] == prefix[b]) *a.d.new_refused = 1;
        }
    }

    // Waves w and w + 4 share a SIMD, whose arbiter favours the older wave: left
    // alone, waves 0-3 finish their (equal) work about 10% before waves 4-7 and the
    // CU streams with half its waves for the rest of the range. After every step a
    // wave publishes its step count and raises its issue priority while it is
    // behind its partner, so both finish together.
    const int partner = (wave ^ 4) < waves ? (wave ^ 4) : wave;
    int32_t steps_done = 0;
    // The counters are relaxed workgroup-scope atomics on the LDS array (ds_write /
    // ds_read); a volatile access through a generic pointer would compile to flat
    // system-coherent memory operations followed by a full vmcnt/lgkmcnt wait.
    auto keep_pace = [&]() {
        ++steps_done;
        if (lane == 0) __hip_atomic_store(&progress[wave], steps_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int32_t other =
            uniform(__hip_atomic_load(&progress[partner], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (steps_done < other) __builtin_amdgcn_s_setprio(2);
        else __builtin_amdgcn_s_setprio(0);
    };

    // Fewer than 8 KV heads (a divisor of 8; kRep): the workgroup still has 8 waves,
    // R = 8 / Hkv replicas per head. Replica r of a head takes steps r, r + R, r + 2R,
    // ... of every segment, and at the segment's end the replicas merge their
    // softmax states through LDS into replica 0, which stores. A CU then streams
    // with two waves per SIMD instead of one.
    const int hw = kRep ? a.d.num_kv_heads : waves;        // heads served at a time
    const int rep_r = kRep ? wave / hw : 0;                   // this wave's replica
    const int reps = kRep ? waves / hw : 1;
    const int dT = 2 * reps;                                  // tiles between this wave's steps
    for (int h = kRep ? wave - rep_r * hw : wave; h < a.d.num_kv_heads; h += hw) {
        int32_t tile = start;
        int b = uniform(find_seq(prefix, a.d.batch, tile));
        while (tile < end) {
            while (prefix[b + 1] <= tile) ++b;
            b = uniform(b);
            const int32_t seq0 = uniform(prefix[b]);
            const int32_t seq1 = uniform(prefix[b + 1]);
            const int32_t seg1 = min(end, seq1);
            const int32_t t0 = tile - seq0, t1 = seg1 - seq0;
            const bool whole = tile == seq0 && seg1 == seq1;
            const int slot_index = 2 * w + (start >= seq0 ? 0 : 1);
            // Slot and length from the LDS metadata (the segment has tiles).
            const int32_t mt = uniform(meta[b]);
            const int64_t slot = (mt >> 5) & ((1 << 26) - 1);
            const int64_t len = 16 * (int64_t)(seq1 - seq0 - 1) + (mt & 31);
            const int32_t* table_row = a.d.block_table + slot * a.d.bt_width;
            // This workgroup attends over the sequence's last tile: it writes the
            // sequence's new token. Its loads go out first; the quantized row is
            // stored before the loads of the tile that holds it (after the first
            // issued steps when that tile is not among them).
            // With replicas, the one whose steps include the last tile writes.
            const bool append = kAppend && seg1 == seq1 && (!kRep || ((t1 - 1 - t0) >> 1) % reps == rep_r);
            NewRow<C> fresh;
            if constexpr (kAppend) {
                if (append) fetch_new_token<C>(a, b, h, lane, fresh, table_row, len, mt < 0);
            }
            const int32_t T0 = t0 + 2 * rep_r;     // this wave's first step
            const bool put_early = t1 - 1 < T0 + (ES == 1 ? 2 * dT : 2);
            if constexpr (kAppend) {
                if (append && put_early) put_new_token<C>(a, fresh, lane);
            }

            WaveState<C> st;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) st.o[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            st.m = kNegInf;
            st.l = 0.0f;

            // Load pipeline: e4m3fn issues the loads of step T + 4 right after step T
            // is computed, into the buffer step T - 2 used (three buffers), so step
            // T + 2 is in flight while T is computed and two steps while the wave
            // waits; bf16 steps are twice the bytes and keep one step in flight (two
            // buffers).
            // Q^T operands of this head's G query heads: loads issued before the
            // first K/V loads, converted after them, so that the first step waits
            // for nothing else.
            constexpr int kQOps = kWholeRowK<C, ES> ? 2 * kSets : 2 * C;
            QRaw<C, QT> qraw;
            load_q_raw<C, ES, QT, kQOps>(a, b, h, G, lane, qraw);
            const int hq = h * G + m16;     // output column of this lane
            const bool qlive = m16 < G;

            StepData<C, ES> buf0, buf1, buf2;
            TileRef r0a, r0b, r1a, r1b, r2a, r2b;
            auto issue = [&](StepData<C, ES>& dst, int32_t tile0, TileRef& ra, TileRef& rb) {
                ra = tile_ref(a, table_row, tile0);
                rb = tile0 + 1 < t1 ? tile_ref(a, table_row, tile0 + 1) : TileRef{0, 0};
                load_step<C, ES>(dst, a, h, ra, rb, lane);
            };
            int32_t T = T0;
            if (!kRep || T < t1) issue(buf0, T, r0a, r0b);
            if constexpr (ES == 1) {
                if (T + dT < t1) issue(buf1, T + dT, r1a, r1b);
            }
            if constexpr (kAppend) {
                if (append && !put_early) put_new_token<C>(a, fresh, lane);
            }
            OpT<kF16> qh[2 * C], ql[2 * C];
            q_operands<C, ES, QT, kQOps, kHiLo, kF16>(qraw, G, lane, qh, ql);


            auto compute = [&](const StepData<C, ES>& cur, int32_t tile0, const TileRef& ra, const TileRef& rb) {
                const int64_t pos = (int64_t)tile0 * 16;
                const int lim_a = ra.valid ? (int)max((int64_t)0, min((int64_t)16, len - pos)) : 0;
                const int lim_b = rb.valid ? (int)max((int64_t)0, min((int64_t)16, len - pos - 16)) : 0;
                compute_step<C, ES, kHiLo, kSets, kF16>(st, cur, qh, ql, stage, lane, lim_a, lim_b, a.d.score_scale);
            };
            if constexpr (ES == 1) {
                while (!kRep || T < t1) {
                    compute(buf0, T, r0a, r0b);
                    if (T + 2 * dT < t1) issue(buf2, T + 2 * dT, r2a, r2b);
                    keep_pace();
                    T += dT;
                    if (T >= t1) break;
                    compute(buf1, T, r1a, r1b);
                    if (T + 2 * dT < t1) issue(buf0, T + 2 * dT, r0a, r0b);
                    keep_pace();
                    T += dT;
                    if (T >= t1) break;
                    compute(buf2, T, r2a, r2b);
                    if (T + 2 * dT < t1) issue(buf1, T + 2 * dT, r1a, r1b);
                    keep_pace();
                    T += dT;
                    if (T >= t1) break;
                }
            } else {
                while (!kRep || T < t1) {
                    if (T + dT < t1) issue(buf1, T + dT, r1a, r1b);
                    compute(buf0, T, r0a, r0b);
                    keep_pace();
                    T += dT;
                    if (T >= t1) break;
                    if (T + dT < t1) issue(buf0, T + dT, r0a, r0b);
                    compute(buf1, T, r1a, r1b);
                    keep_pace();
                    T += dT;
                    if (T >= t1) break;
                }
            }
            if constexpr (kRep) {
                // Tree merge of the replicas' softmax states into replica 0: in each
                // round replicas [half, 2 half) publish (structure of arrays, one float
                // per lane and value: conflict-free) and replica r < half merges that
                // of r + half. The second barrier keeps the next publications behind
                // the merge. At most 4 states are published at a time.
                constexpr int kVals = 4 * NB + 2;
                float* merge = reinterpret_cast<float*>(meta + a.d.batch);   // after the metadata
                for (int half = reps >> 1; half > 0; half >>= 1) {
                    if (rep_r >= half && rep_r < 2 * half) {
                        float* mine = merge + ((rep_r - half) * hw + h) * (kVals * 64);
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                            for (int jj = 0; jj < 4; ++jj) mine[(4 * nb + jj) * 64 + lane] = st.o[nb][jj];
                        mine[(4 * NB) * 64 + lane] = st.m;
                        mine[(4 * NB + 1) * 64 + lane] = st.l;
                    }
                    __syncthreads();
                    if (rep_r < half) {
                        const float* other = merge + (rep_r * hw + h) * (kVals * 64);
                        const float mo = other[(4 * NB) * 64 + lane];
                        const float lo = other[(4 * NB + 1) * 64 + lane];
                        const float mn = fmaxf(st.m, mo);
                        const float mu = mn == kNegInf ? 0.0f : mn;
                        const float sa = fast_exp2(st.m - mu), sb = fast_exp2(mo - mu);
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                            for (int jj = 0; jj < 4; ++jj)
                                st.o[nb][jj] = st.o[nb][jj] * sa + other[(4 * nb + jj) * 64 + lane] * sb;
                        st.l = st.l * sa + lo * sb;
                        st.m = mn;
                    }
                    __syncthreads();
                }
            }

            // Denominator: sum the four lane groups of each column.
            float lt = st.l + __shfl_xor(st.l, 16);
            lt += __shfl_xor(lt, 32);
            if (qlive && rep_r == 0) {
                if (whole) {
                    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb)
                            store_out<QT>(a.d, b, hq, NB * (4 * j + jj) + nb, lt > 0.0f ? st.o[nb][jj] * inv : 0.0f);
                    }
                } else {
                    const int64_t pi = (int64_t)slot_index * a.d.num_q_heads + hq;
                    float* acc = a.part_acc + pi * D;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) acc[NB * (4 * j + jj) + nb] = st.o[nb][jj];
                    }
                    if (j == 0) {
                        a.part_m[pi] = st.m;
                        a.part_l[pi] = lt;
                    }
                }
            }
            tile = seg1;
        }
    }
}

// Four consecutive output elements d0 .. d0 + 3 (d0 a multiple of 4) as one store.
template <int QT>
__device__ __forceinline__ void store_out4(const DecodeArgs& a, int b, int hq, int d0, float x0, float x1, float x2,
                                           float x3) {
    using T = typename Elem<QT>::T;
    T* dst = reinterpret_cast<T*>(a.out) + ((int64_t)b * a.num_q_heads + hq) * a.head_dim + d0;
    if constexpr (QT == KVFP8_F32) {
        *reinterpret_cast<float4*>(dst) = make_float4(x0, x1, x2, x3);
    } else {
        const uint32_t lo = (uint32_t)Elem<QT>::store(x0) | ((uint32_t)Elem<QT>::store(x1) << 16);
        const uint32_t hi = (uint32_t)Elem<QT>::store(x2) | ((uint32_t)Elem<QT>::store(x3) << 16);
        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
    }
}

// Workgroup whose tile range holds tile x: the largest w with w W / groups <= x.
__device__ __forceinline__ int32_t group_of(int64_t x, int64_t total, int64_t groups) {
    return floor_div((x + 1) * groups - 1, total);     // < 2^42
}

// Merge of the pieces of every cut sequence (reference decode_attention.py:437-550):
//   M = max m_i; den = sum 2^(m_i - M) l_i; num = sum 2^(m_i - M) acc_i;
//   out = den > 0 ? num / den : 0. Empty sequences get zeros.
// One wave per (sequence, q head). Piece states are read lane-parallel (m and l
// one piece per lane, acc as float4 runs with D/4 lanes per piece), so the merge
// costs a couple of memory latencies whatever the number of pieces.
template <int C, int QT>
__global__ void __launch_bounds__(256)
combine_mfma_kernel(MfmaArgs a) {
    constexpr int D = 64 * C;
    constexpr int kLanesPerPiece = D / 4;
    constexpr int kPiecesPerPass = 64 / kLanesPerPiece;
    // The wave index as a scalar, so that the per-sequence plan entries below are
    // scalar loads.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t pair = (int64_t)blockIdx.x * 4 + wave;
    if (pair >= (int64_t)a.d.batch * a.d.num_q_heads) return;
    const int b = uniform(floor_div(pair, a.d.num_q_heads));
    const int hq = (int)(pair - (int64_t)b * a.d.num_q_heads);
    const int32_t t0 = a.plan[b], t1 = a.plan[b + 1];
    const int d4 = lane % kLanesPerPiece, po = lane / kLanesPerPiece;
    if (t1 == t0) {
        if (po == 0) store_out4<QT>(a.d, b, hq, 4 * d4, 0.0f, 0.0f, 0.0f, 0.0f);
        return;
    }
    const int64_t total = a.plan[a.d.batch];
    const int64_t groups = a.plan[a.d.batch + 1];
    const int32_t w0 = uniform(group_of(t0, total, groups)), w1 = uniform(group_of(t1 - 1, total, groups));
    if (w0 == w1) return;    // finished by the decode kernel
    const int32_t pieces = w1 - w0 + 1;
    const int64_t hq_count = a.d.num_q_heads;
    // Piece i is in workgroup w0 + i. The workgroups after w0 start inside the
    // sequence, so it is their first segment (state 2 w); w0 holds it as its first
    // segment only when its range starts at t0, else as its last (state 2 w + 1).
    // One division per wave instead of one per piece.
    const int32_t cut0 = floor_div((int64_t)w0 * total, groups) < t0 ? 1 : 0;
    auto state_index = [&](int32_t i) -> int64_t {
        const int64_t w = w0 + i;
        return (2 * w + (i == 0 ? cut0 : 0)) * hq_count + hq;
    };

    // Each lane merges its pieces online (all loads independent, issued
    // together), then the lane groups merge pairwise through shuffles.
    float mr = kNegInf, den = 0.0f;
    float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
    for (int32_t i = po; i < pieces; i += kPiecesPerPass) {
        const int64_t si = state_index(i);
        const float mi = a.part_m[si];
        const float li = a.part_l[si];
        const float4 x = reinterpret_cast<const float4*>(a.part_acc + si * D)[d4];
        const float mn = fmaxf(mr, mi);
        const float mu = mn == kNegInf ? 0.0f : mn;
        const float sa = fast_exp2(mr - mu), sb = fast_exp2(mi - mu);
        num.x = num.x * sa + x.x * sb;
        num.y = num.y * sa + x.y * sb;
        num.z = num.z * sa + x.z * sb;
        num.w = num.w * sa + x.w * sb;
        den = den * sa + li * sb;
        mr = mn;
    }
#pragma unroll
    for (int off = kLanesPerPiece; off < 64; off <<= 1) {
        const float mo = __shfl_xor(mr, off);
        const float mn = fmaxf(mr, mo);
        const float mu = mn == kNegInf ? 0.0f : mn;
        const float sa = fast_exp2(mr - mu), sb = fast_exp2(mo - mu);
        num.x = num.x * sa + __shfl_xor(num.x, off) * sb;
        num.y = num.y * sa + __shfl_xor(num.y, off) * sb;
        num.z = num.z * sa + __shfl_xor(num.z, off) * sb;
        num.w = num.w * sa + __shfl_xor(num.w, off) * sb;
        den = den * sa + __shfl_xor(den, off) * sb;
        mr = mn;
    }
    if (po == 0) {
        const bool ok = den > 0.0f;
        store_out4<QT>(a.d, b, hq, 4 * d4, ok ? num.x / den : 0.0f, ok ? num.y / den : 0.0f,
                       ok ? num.z / den : 0.0f, ok ? num.w / den : 0.0f);
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int ilog2(int64_t x) {
    int s = 0;
    while ((int64_t)1 << s < x) ++s;
    return s;
}

// Waves that serve distinct KV heads: one per head, up to kMaxWaves.
int waves_for(int32_t num_kv_heads) { return num_kv_heads < kMaxWaves ? num_kv_heads : kMaxWaves; }

// Compute units of the current device (cached per device id).
int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Fewer KV heads than kMaxWaves, dividing it: the plain decode runs kMaxWaves waves per
// workgroup, R = kMaxWaves / heads replicas of each head (kRep), when
//   - the replicas' merge buffer fits in LDS beside the batch-sized tables, and
//   - the batch can give every replica steps: its tile capacity (batch x table width)
//     is at least 2 R tiles per CU. Below that most replicas idle and the 8-wave
//     workgroups measured slower (cfg1: 8.5 against 6.5 us).
// The fused append + decode kernel keeps one wave per head: with the replicas' merge
// it spills registers and measured 1.3-2.7 us slower.
constexpr size_t kMaxGroupLds = 64 * 1024;
template <int C>
constexpr size_t replica_merge_bytes() { return (size_t)(kMaxWaves / 2) * (4 * (4 * C) + 2) * 64 * sizeof(float); }
template <int C>
bool replicated(const DecodeArgs& d, size_t table_lds) {
    if (d.num_kv_heads >= kMaxWaves || kMaxWaves % d.num_kv_heads != 0) return false;
    if (table_lds + replica_merge_bytes<C>() > kMaxGroupLds) return false;
    const int64_t tiles = (int64_t)d.batch * d.bt_width * (d.block_size / 16);
    return tiles >= (int64_t)device_cus() * 2 * (kMaxWaves / d.num_kv_heads);
}

int64_t max_groups(int32_t num_kv_heads) {
    const int per_cu = kWavesPerCu / waves_for(num_kv_heads);
    return (int64_t)device_cus() * (per_cu > 0 ? per_cu : 1);
}

template <int C, int QT, int ES, int kSets, bool kAppend, bool kF16, bool kRep>
hipError_t launch_w(const MfmaArgs& a, int64_t cap, hipStream_t s, int phases) {
    const int threads = 64 * (kRep ? kMaxWaves : waves_for(a.d.num_kv_heads));
    const size_t lds = (size_t)(2 * a.d.batch + 1) * sizeof(int32_t) + (kRep ? replica_merge_bytes<C>() : 0);
    // Resident workgroups per CU: the register limit, queried once per (device,
    // workgroup size) without dynamic LDS, capped by what the dynamic LDS (batch-sized
    // tables, replica merge buffer; up to 64 KiB) leaves room for. Only a sizing
    // choice: the work split is correct for any grid.
    static int resident[64][kMaxWaves + 1] = {};     // per template instance
    static int lds_per_cu[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int& per_cu = resident[dev][threads / 64];
    if (per_cu == 0) {
        const void* fn = reinterpret_cast<const void*>(&decode_mfma_kernel<C, QT, ES, kSets, kAppend, kF16, kRep>);
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, 0) != hipSuccess || n <= 0) n = 1;
        per_cu = n;
    }
    if (lds_per_cu[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess || n <= 0)
            n = 64 * 1024;
        lds_per_cu[dev] = n;
    }
    const int64_t by_lds = (int64_t)lds_per_cu[dev] / (int64_t)(lds + 4096);   // + static LDS
    const int64_t fit = by_lds < per_cu ? by_lds : per_cu;
    int64_t groups = (int64_t)device_cus() * (fit > 0 ? fit : 1);
    groups = groups < cap ? groups : cap;
    if (phases & kPhaseSplit) {
        const hipError_t err =
            launch_timed(decode_mfma_kernel<C, QT, ES, kSets, kAppend, kF16, kRep>, dim3((unsigned)groups),
                         dim3(threads), lds, s, next_kernel_timing(), a);
        if (err != hipSuccess) return err;
    }
    if (!(phases & kPhaseReduce)) return hipSuccess;
    const int64_t pairs = (int64_t)a.d.batch * a.d.num_q_heads;
    hipLaunchKernelGGL((combine_mfma_kernel<C, QT>), dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int C, int QT, int ES, int kSets, bool kAppend = false, bool kF16 = false>
hipError_t launch_c(const MfmaArgs& a, int64_t cap, hipStream_t s, int phases) {
    if constexpr (!kAppend) {
        if (replicated<C>(a.d, (size_t)(2 * a.d.batch + 1) * sizeof(int32_t)))
            return launch_w<C, QT, ES, kSets, kAppend, kF16, true>(a, cap, s, phases);
    }
    return launch_w<C, QT, ES, kSets, kAppend, kF16, false>(a, cap, s, phases);
}

}  // namespace

bool mfma_decode_supported(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int64_t bt_width, int32_t block_size, int kv_dtype) {
    if (kv_dtype != KVFP8_E4M3FN && kv_dtype != KVFP8_BF16 && kv_dtype != KVFP8_F16) return false;
    if (head_dim != 64 && head_dim != 128) return false;
    if (block_size < 16 || block_size % 16 != 0) return false;
    if (num_q_heads % num_kv_heads != 0 || num_q_heads / num_kv_heads > 16) return false;
    if (num_kv_heads > kMaxWaves && num_kv_heads % kMaxWaves != 0) return false;
    if (batch <= 0 || batch > kMfmaMaxBatch) return false;
    // Tile indices are int32.
    if ((int64_t)batch * bt_width * (block_size / 16) >= ((int64_t)1 << 31)) return false;
    return true;
}

}  // namespace kvfp8

namespace kvfp8 {

// Workspace layout of the MFMA path: plan [batch + 2] int32, part_m, part_l
// [2 G_max Hq] float, part_acc [2 G_max Hq D] float (each 256-byte aligned).
int64_t mfma_workspace_layout(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                              int64_t offsets[4]) {
    const int64_t states = 2 * max_groups(num_kv_heads) * num_q_heads;
    int64_t off = 0;
    offsets[0] = off;
    off += (int64_t)align256((size_t)(batch + 2) * sizeof(int32_t));
    offsets[1] = off;
    off += (int64_t)align256((size_t)states * sizeof(float));
    offsets[2] = off;
    off += (int64_t)align256((size_t)states * sizeof(float));
    offsets[3] = off;
    off += (int64_t)align256((size_t)states * head_dim * sizeof(float));
    return off;
}

template <int QT>
hipError_t launch_mfma_decode(const DecodeArgs& d, int kv_dtype, void* workspace, hipStream_t stream, int phases) {
    int64_t off[4];
    mfma_workspace_layout(d.batch, d.num_q_heads, d.num_kv_heads, d.head_dim, off);
    char* ws = reinterpret_cast<char*>(workspace);
    MfmaArgs a;
    a.d = d;
    a.tps_shift = ilog2(d.block_size / 16);
    a.plan = reinterpret_cast<int32_t*>(ws + off[0]);
    a.part_m = reinterpret_cast<float*>(ws + off[1]);
    a.part_l = reinterpret_cast<float*>(ws + off[2]);
    a.part_acc = reinterpret_cast<float*>(ws + off[3]);
    const int64_t qsize = QT == KVFP8_F32 ? 4 : 2;
    a.q_vec = ((uintptr_t)d.q % 16 == 0 && (d.q_stride_b * qsize) % 16 == 0 && (d.q_stride_h * qsize) % 16 == 0) ? 1 : 0;
    const int64_t cap = max_groups(d.num_kv_heads);
    if (kv_dtype == KVFP8_BF16)
        return d.head_dim == 64 ? launch_c<1, QT, 2, 1>(a, cap, stream, phases)
                                : launch_c<2, QT, 2, 1>(a, cap, stream, phases);
    if (kv_dtype == KVFP8_F16) {
        // f16 cache with f16 q (the caller checked): f16 operands.
        if constexpr (QT == KVFP8_F16)
            return d.head_dim == 64 ? launch_c<1, QT, 2, 1, false, true>(a, cap, stream, phases)
                                    : launch_c<2, QT, 2, 1, false, true>(a, cap, stream, phases);
        else return hipErrorInvalidValue;
    }
    if (d.new_k != nullptr) {
        // Fused append + decode (e4m3fn only; the caller checked the shape).
        if (d.head_dim == 64) return launch_c<1, QT, 1, 1, true>(a, cap, stream, phases);
        return d.num_q_heads / d.num_kv_heads > 8 ? launch_c<2, QT, 1, 2, true>(a, cap, stream, phases)
                                                   : launch_c<2, QT, 1, 1, true>(a, cap, stream, phases);
    }
    if (d.head_dim == 64) return launch_c<1, QT, 1, 1>(a, cap, stream, phases);
    // Whole-row K layout: q heads 8..15 of a group need the second QK set.
    return d.num_q_heads / d.num_kv_heads > 8 ? launch_c<2, QT, 1, 2>(a, cap, stream, phases)
                                               : launch_c<2, QT, 1, 1>(a, cap, stream, phases);
}

template hipError_t launch_mfma_decode<KVFP8_F32>(const DecodeArgs&, int, void*, hipStream_t, int);
template hipError_t launch_mfma_decode<KVFP8_F16>(const DecodeArgs&, int, void*, hipStream_t, int);
template hipError_t launch_mfma_decode<KVFP8_BF16>(const DecodeArgs&, int, void*, hipStream_t, int);

}  // namespace kvfp8
