// Drafter attention over the compressed mirror.
// Reference: the read + einsum + softmax + note_attention of the model
// forwards against CompressedKVCache (draftkv/compress.py:135-151,
// draftkv/llama.py:202-218, gpt2.py:197-206, model.py:117-127).
//
// One query position per sequence; the G query heads of a KV head share its
// rows. A split of `rps` rows (a multiple of the 32-row page) is one unit of
// work; a combine kernel merges the splits' (max, sum, output) partials.
// With want_mass the scaled logits are spilled and a third kernel turns them
// into each row's probability mass summed over query heads, added to the
// row's score.
//
// Fast path (4/8-bit codes, D = 64 or 128, groups a multiple of 16,
// G * groups <= 16): v_mfma_f32_16x16x32_f16 on the raw codes.
//   Codes enter the MFMA as f16 subnormals: the bits (word & 0x000F000F)
//   read as an f16 pair are exactly (code * 2^-24, code' * 2^-24), and the
//   MFMA keeps subnormal inputs, so one AND (plus a shift) turns two codes
//   into an exact operand. The 2^24 is folded into the softmax scale (QK) and
//   into the output (PV).
//   QK: S'[16 rows][16 cols] = code . Qg^T, where column j = (group g, head
//       h) holds q_h restricted to group g (zero elsewhere), split into f16
//       hi + lo parts. Folding scale and zero in fp32 per (row, group) and
//       summing the group columns of a head gives its logit:
//         s_h = sum_g scale_g * S'[g,h] + lo_g * sum_{d in g} q_h[d]
//   PV: O'[16 d][16 cols] = code_V^T . B with B[row][(g,h)] =
//       f16(p_h[row] * scaleV_g[row]); then
//         o_h[d] = O'[d][(g(d),h)] + sum_rows p_h * loV_g
// The accumulator lanes of the QK product already hold the 8 rows of one
// column that the PV B operand needs, so probabilities never move between
// lanes; the V page layout (mirror_layout.h) is the PV A operand.
#include <hip/hip_ext.h>

#include <atomic>
#include <type_traits>

#include "mirror_layout.h"

namespace dkv {

constexpr int DQB = 16;     // max query heads per KV head (generic path)
constexpr int DMAXD = 128;  // LDS tiles stay under 64 KB

__host__ __device__ inline int rows_per_split(const dkv_drafter_t& m, int G) {
    // enough splits to fill the chip at small batch, few partials at large
    // batch; at most 2048 (row, query head) logits per split (8 KB of LDS
    // staging per wave in the MFMA kernel)
    const int base = (m.batch * m.n_kv_heads >= 128) ? 512 : 128;
    return std::max(PAGE, std::min(base, (2048 / std::max(G, 1)) / PAGE * PAGE));
}

// ---------------------------------------------------------------- generic path
__global__ void __launch_bounds__(256) draft_attn_kernel(dkv_drafter_t m, int layer, dkv_qcfg_t cfg,
                                                         const float* __restrict__ q, int Hq, float scale, int rps,
                                                         int n_splits, float* __restrict__ part,
                                                         float* __restrict__ logits) {
    const int split = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
    const int D = m.head_dim, G = Hq / m.n_kv_heads;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int r_begin = split * rps;
    const int r_end = min(r_begin + rps, n);
    const int tid = threadIdx.x;
    const PageFmt f = page_fmt(cfg, D);

    extern __shared__ float smem[];
    float* sQ = smem;                   // [DQB][D]
    float* sK = sQ + DQB * D;           // [PAGE][D+1]
    float* sV = sK + PAGE * (D + 1);    // [PAGE][D]
    float* sS = sV + PAGE * D;          // [DQB][PAGE]
    float* sM = sS + DQB * PAGE;
    float* sL = sM + DQB;
    float* sA = sL + DQB;

    for (int i = tid; i < DQB * D; i += blockDim.x) {
        const int r = i / D, d = i % D;
        sQ[i] = r < G ? q[((int64_t)s * Hq + h * G + r) * D + d] : 0.0f;
    }
    if (tid < DQB) {
        sM[tid] = -INFINITY;
        sL[tid] = 0.0f;
    }
    constexpr int MAXACC = DQB * DMAXD / 256;
    float acc[MAXACC];
#pragma unroll
    for (int j = 0; j < MAXACC; ++j) acc[j] = 0.0f;
    const int n_out = DQB * D;

    for (int rt = r_begin; rt < r_end; rt += PAGE) {
        __syncthreads();
        const uint8_t* pg = page_ptr(m, s, layer, h, rt / PAGE);
        for (int x = tid; x < PAGE * D; x += blockDim.x) {
            const int i = x / D, d = x % D;
            float kv = 0.0f, vv = 0.0f;
            if (rt + i < r_end) {
                if (f.cb == 32) {
                    kv = reinterpret_cast<const float*>(pg + f.kc)[(int64_t)i * D + d];
                    vv = reinterpret_cast<const float*>(pg + f.vc)[(int64_t)i * D + d];
                } else {
                    const int g = d / f.group;
                    int64_t w;
                    int sh;
                    k_code_loc(f, i, d, &w, &sh);
                    kv = dequant(read_code(pg + f.kc, w, sh, f.cb), read_meta(pg + k_meta_off(f, i, g), f.meta_f16));
                    v_code_loc(f, i, d, &w, &sh);
                    vv = dequant(read_code(pg + f.vc, w, sh, f.cb), read_meta(pg + v_meta_off(f, i, g), f.meta_f16));
                }
            }
            sK[i * (D + 1) + d] = kv;
            sV[i * D + d] = vv;
        }
        __syncthreads();
        for (int x = tid; x < DQB * PAGE; x += blockDim.x) {
            const int r = x / PAGE, j = x % PAGE;
            float sc = -INFINITY;
            if (r < G && rt + j < r_end) {
                float dot = 0.0f;
                for (int d = 0; d < D; ++d) dot = fmaf(sQ[r * D + d], sK[j * (D + 1) + d], dot);
                sc = dot * scale;
                if (logits) logits[((int64_t)s * Hq + h * G + r) * m.cap + rt + j] = sc;
            }
            sS[x] = sc;
        }
        __syncthreads();
        {
            const int r = tid / 16, l16 = tid % 16;
            float mx = -INFINITY;
            for (int j = l16; j < PAGE; j += 16) mx = fmaxf(mx, sS[r * PAGE + j]);
            for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
            const float m_old = sM[r];
            const float m_new = fmaxf(m_old, mx);
            float sum = 0.0f;
            for (int j = l16; j < PAGE; j += 16) {
                const float sc = sS[r * PAGE + j];
                const float p = (sc == -INFINITY) ? 0.0f : __expf(sc - m_new);
                sS[r * PAGE + j] = p;
                sum += p;
            }
            for (int o = 8; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 16);
            __syncthreads();
            if (l16 == 0) {
                const float a = (m_old == -INFINITY) ? 0.0f : __expf(m_old - m_new);
                sA[r] = a;
                sL[r] = sL[r] * a + sum;
                sM[r] = m_new;
            }
        }
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < MAXACC; ++jj) {
            const int o = tid + 256 * jj;
            if (o < n_out) {
                const int r = o / D, d = o % D;
                float a = acc[jj] * sA[r];
                for (int j = 0; j < PAGE; ++j) a = fmaf(sS[r * PAGE + j], sV[j * D + d], a);
                acc[jj] = a;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < MAXACC; ++jj) {
        const int o = tid + 256 * jj;
        if (o < n_out) {
            const int r = o / D, d = o % D;
            if (r < G) {
                float* p = part + (((int64_t)s * Hq + h * G + r) * n_splits + split) * (D + 2);
                p[d] = acc[jj];
                if (d == 0) {
                    p[D] = sM[r];
                    p[D + 1] = sL[r];
                }
            }
        }
    }
}

// ---------------------------------------------------------------- MFMA path
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kTwo24 = 16777216.0f;            // 2^24
constexpr float kTwoM24 = 1.0f / 16777216.0f;    // 2^-24

#ifndef DKV_X16
#define DKV_X16 1
#endif
// element e of a 4-bit operand carries 16x its code when DKV_X16 and e & 2
__host__ __device__ constexpr bool x16_elem(int CB, int e) { return DKV_X16 && CB == 4 && (e & 2); }

// 8 codes of one word (cb 4) or two words (cb 8) -> 8 f16 subnormals
// code * 2^-24 (the interleaved word order of mirror_layout.h puts two codes
// in the low bits of the two halves)
template <int CB>
__device__ __forceinline__ f16x8_t codes_to_f16(const uint32_t* w) {
    uint4 r;
    if (CB == 4) {
        const uint32_t x = w[0];
#if DKV_X16
        // codes at bits 4-7 of a half are subnormals too, 16x the value:
        // elements e = 2, 3, 6, 7 come out scaled by 16 (the other operand
        // carries 1/16 there), one AND per pair instead of a shift and an AND
        const uint32_t y = x >> 8;
        r.x = x & 0x000F000Fu;
        r.y = x & 0x00F000F0u;
        r.z = y & 0x000F000Fu;
        r.w = y & 0x00F000F0u;
#else
        r.x = x & 0x000F000Fu;
        r.y = (x >> 4) & 0x000F000Fu;
        r.z = (x >> 8) & 0x000F000Fu;
        r.w = (x >> 12) & 0x000F000Fu;
#endif
    } else {
        // bytes 0 and 2 by an AND; bytes 1 and 3 moved down by one byte
        // permute (selector 0x0c: a zero byte) instead of a shift and an AND
        r.x = w[0] & 0x00FF00FFu;
        r.y = __builtin_amdgcn_perm(w[0], 0u, 0x0c070c05u);
        r.z = w[1] & 0x00FF00FFu;
        r.w = __builtin_amdgcn_perm(w[1], 0u, 0x0c070c05u);
    }
    return __builtin_bit_cast(f16x8_t, r);
}

// Raw registers of one page as a lane needs them; loaded one page ahead so the
// memory latency of page p+1 overlaps the products of page p.
template <int D, int CB, int MF>
struct PageRegs {
    static constexpr int WPL = D / 4 * CB / 32;   // K code words per lane per 16-row tile
    static constexpr int NV = D / 16 * CB / 4;    // V code words per lane
    static constexpr int MW = MF ? 1 : 2;         // words per (scale, lo) pair
    uint32_t k[2][WPL];
    uint32_t km[2][4 * MW];
    uint32_t v[NV];
    uint32_t vm[8 * MW];
};

template <int N>
__device__ __forceinline__ void load_words(uint32_t (&dst)[N], const uint8_t* src) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int x = 0; x < N / 4; ++x) {
            const uint4 w = reinterpret_cast<const uint4*>(src)[x];
            dst[4 * x] = w.x;
            dst[4 * x + 1] = w.y;
            dst[4 * x + 2] = w.z;
            dst[4 * x + 3] = w.w;
        }
    } else {
#pragma unroll
        for (int x = 0; x < N; ++x) dst[x] = reinterpret_cast<const uint32_t*>(src)[x];
    }
}

// byte offsets of a lane's operands inside a page (the same for every page)
struct LaneOffsets {
    uint32_t k[2], km[2], v, vm;
};

// N words as N/4 pieces of 16 bytes, piece x at src + 1024 x, non-temporal
// (a page is read once per call; each load instruction of the wave reads 1 KB
// of contiguous bytes, so no 64-byte segment is split between instructions,
// which under this policy would be fetched twice)
typedef uint32_t pu32x4_t __attribute__((ext_vector_type(4)));
template <int N>
__device__ __forceinline__ void load_pieces_nt(uint32_t (&dst)[N], const uint8_t* src) {
    static_assert(N % 4 == 0, "whole 16-byte pieces");
#pragma unroll
    for (int x = 0; x < N / 4; ++x) {
        const pu32x4_t w = __builtin_nontemporal_load(reinterpret_cast<const pu32x4_t*>(src + 1024 * x));
        dst[4 * x] = w[0];
        dst[4 * x + 1] = w[1];
        dst[4 * x + 2] = w[2];
        dst[4 * x + 3] = w[3];
    }
}

template <int D, int CB, int MF>
__device__ __forceinline__ void load_page(PageRegs<D, CB, MF>& r, const uint8_t* pg, const LaneOffsets& o) {
    if constexpr (CB == 8) {   // K and V codes in lane load order (D % 64 == 0)
        static_assert(D % 64 == 0, "8-bit pages in lane load order");
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            load_pieces_nt(r.k[a], pg + o.k[a]);
            load_words(r.km[a], pg + o.km[a]);
        }
        load_pieces_nt(r.v, pg + o.v);
        load_words(r.vm, pg + o.vm);
        return;
    }
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        load_words(r.k[a], pg + o.k[a]);
        load_words(r.km[a], pg + o.km[a]);
    }
    load_words(r.v, pg + o.v);
    load_words(r.vm, pg + o.vm);
}

// (scale, lo) pair k of a lane's meta words
template <int MF>
__device__ __forceinline__ float meta_scale(const uint32_t* w, int k) {
    if (MF) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] & 0xffffu));
    return __uint_as_float(w[2 * k]);
}
template <int MF>
__device__ __forceinline__ float meta_lo(const uint32_t* w, int k) {
    if (MF) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] >> 16));
    return __uint_as_float(w[2 * k + 1]);
}

// an optional callback left out
struct NoHook {
    template <class... A>
    __device__ __forceinline__ void operator()(A&&...) const {}
};

// Column offset of group g within a 16-lane row (see the kernel): the
// subgroup of lane XORs generated by 15, 7 and 3, in butterfly order
// {0, 15, 7, 8, 3, 12, 4, 11}. A function, so that an unrolled loop folds it
// to immediates instead of loading a table.
__device__ __forceinline__ constexpr int col_xor(int g) {
    return (g & 1 ? 15 : 0) ^ (g & 2 ? 7 : 0) ^ (g & 4 ? 3 : 0);
}

template <bool B>
using bool_c = std::integral_constant<bool, B>;

// v[x] = v[lane (l ^ m) of the 16-lane row] + v[x] for the 8 values, one
// fused v_add_f32_dpp each (the compiler keeps DPP moves and adds apart). The
// s_nop covers the two wait states a DPP read needs after a VALU write; the
// later adds read registers written at least two instructions earlier.
#define DKV_DPP_ADD8(CTRL, v)                                                                        \
    asm volatile("s_nop 1\n\t"                                                                        \
                 "v_add_f32_dpp %0, %0, %0 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                  \
                 "v_add_f32_dpp %1, %1, %1 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                  \
                 "v_add_f32_dpp %2, %2, %2 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                  \
                 "v_add_f32_dpp %3, %3, %3 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                  \
                 "v_add_f32_dpp %4, %4, %4 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                  \
                 "v_add_f32_dpp %5, %5, %5 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                  \
                 "v_add_f32_dpp %6, %6, %6 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                  \
                 "v_add_f32_dpp %7, %7, %7 " CTRL " row_mask:0xf bank_mask:0xf"                        \
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), \
                   "+v"(v[7]))

// Max / sum over the 4 lane groups of a column (lanes l, l^16, l^32, l^48)
// with the VALU lane swaps of gfx950 instead of LDS permutes: after the swap
// of 32-lane halves and then of 16-lane rows, every lane holds the bitwise
// same result.
__device__ __forceinline__ float lanegroup_max(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float lanegroup_sum(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// One wave's split: its (group, head) column, the Q operands, and the online
// softmax state over the split's pages. Both MFMA kernels drive it; they
// differ only in how a page reaches registers and where the logits go.
template <int D, int CB, int MF>
struct SplitCore {
    static constexpr int NSTEP = D / 32;   // k-steps of the QK product
    static constexpr int NDT = D / 16;     // d-tiles of the PV product
    static constexpr int DL = D / 4;       // channels per lane group in QK
    using Regs = PageRegs<D, CB, MF>;

    int col, jj, group, NG, gcol, hcol, gmeta;
    bool cvalid;
    f16x8_t qhi[NSTEP], qlo[NSTEP];
    float qsum_s, scale_s;
    f32x4_t acc[NDT];
    float m_run, l_run, zsum;

    __device__ __forceinline__ void init(const float* __restrict__ q, int s, int h, int Hq, int G, int grp, int lane,
                                         float scale) {
        init_at(q + ((int64_t)s * Hq + h * G) * D, G, grp, lane, scale);
    }

    // qh: the KV head's G query heads, [G][D] floats (global memory or LDS)
    __device__ __forceinline__ void init_at(const float* __restrict__ qh, int G, int grp, int lane, float scale) {
        init_lanes(G, grp, lane);
        init_q(qh, scale);
    }

    // the lane's place: column, lane group, and the (group, head) its column holds
    __device__ __forceinline__ void init_lanes(int G, int grp, int lane) {
        col = lane % 16;
        jj = lane / 16;
        group = grp;
        NG = D / grp;
        // column col = hcol ^ col_xor(gcol): the NG columns of a head form an
        // orbit of the lane involutions row_mirror (^15), row_half_mirror (^7)
        // and quad reverse (^3), so their sum is a butterfly of DPP adds that
        // leaves the bitwise-same total in every column of the head
        gcol = 0;
        hcol = 0;
        cvalid = false;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int hh = col ^ col_xor(g);
            if (g < NG && hh < G) {
                gcol = g;
                hcol = hh;
                cvalid = true;
            }
        }
        gmeta = min(gcol, NG - 1);
    }

    // Q^T of the lane's column in f16 hi + lo, and the column's q sum
    __device__ __forceinline__ void init_q(const float* __restrict__ qh, float scale) {
        // Q^T columns (group, head) in f16 hi + lo, and the column's q sum: the
        // lane's DL channels as DL/4 vector loads, all in flight at once (hq is a
        // valid head for every lane); the group mask is a bit mask, so the loads
        // stay unconditional
        const float4* qr = reinterpret_cast<const float4*>(qh + hcol * D + DL * jj);
        const int d_lo = cvalid ? gcol * group : D, d_hi = d_lo + group;   // the column's group of channels
        float4 qv[DL / 4];
#pragma unroll
        for (int x = 0; x < DL / 4; ++x) qv[x] = qr[x];
        float qsum = 0.0f;
#pragma unroll
        for (int st = 0; st < NSTEP; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = DL * jj + 8 * st + e;
                const float4 w4 = qv[(8 * st + e) / 4];
                const float raw = (e % 4 == 0) ? w4.x : (e % 4 == 1) ? w4.y : (e % 4 == 2) ? w4.z : w4.w;
                const uint32_t keep = (d >= d_lo && d < d_hi) ? 0xFFFFFFFFu : 0u;
                float v = __uint_as_float(__float_as_uint(raw) & keep);
                if (x16_elem(CB, e)) v *= 0.0625f;   // exact: the code operand carries the 16
                const _Float16 hi = (_Float16)v;
                const _Float16 lo = (_Float16)(v - (float)hi);
                qhi[st][e] = hi;
                qlo[st][e] = lo;
                qsum += x16_elem(CB, e) ? ((float)hi + (float)lo) * 16.0f : (float)hi + (float)lo;
            }
        qsum += __shfl_xor(qsum, 16);
        qsum += __shfl_xor(qsum, 32);
        // the QK product runs on code * 2^-24: fold the 2^24 into the zero
        // term and the softmax scale (powers of two, exact)
        qsum_s = qsum * kTwoM24;
        scale_s = scale * kTwo24;
    }

    // fresh softmax state for the next split
    __device__ __forceinline__ void reset() {
#pragma unroll
        for (int t = 0; t < NDT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        m_run = -INFINITY;
        l_run = 0.0f;
        zsum = 0.0f;
    }

    // One page on operands already in registers. TAIL pages hold rows at or
    // past r_end (masked to exact zeros, their stale meta zeroed). sink(pv, p0)
    // receives the page's scaled logits (rows 4jj+x, 16+4jj+x-4 of column col).
    template <bool TAIL, class Sink>
    __device__ __forceinline__ void page(const Regs& cur, int p0, int r_end, Sink&& sink) {
        float sv[8];
        qk(cur, sv);
        rest<TAIL>(cur, sv, p0, r_end, sink);
    }

    // The page's scores (unscaled): sv[x] for rows 4jj+x (x < 4) and
    // 16+4jj+x-4 of column col's head, summed over the head's groups.
    __device__ __forceinline__ void qk(const Regs& cur, float (&sv)[8]) {
        f32x4_t sa[2];
        qk_mfma(cur, sa);
        qk_fold(cur, sa, sv);
    }

    // QK over the page's two 16-row tiles (the two tiles' MFMA chains
    // interleaved, so each hides the other's latency)
    __device__ __forceinline__ void qk_mfma(const Regs& cur, f32x4_t (&sa)[2]) {
        sa[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        sa[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < NSTEP; ++st) {
            const f16x8_t kv0 = codes_to_f16<CB>(cur.k[0] + st * (CB / 4));
            const f16x8_t kv1 = codes_to_f16<CB>(cur.k[1] + st * (CB / 4));
            sa[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv0, qhi[st], sa[0], 0, 0, 0);
            sa[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv1, qhi[st], sa[1], 0, 0, 0);
            sa[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv0, qlo[st], sa[0], 0, 0, 0);
            sa[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv1, qlo[st], sa[1], 0, 0, 0);
        }
    }

    // the products folded per (row, group) with the K meta, then summed over
    // the head's group columns
    __device__ __forceinline__ void qk_fold(const Regs& cur, const f32x4_t (&sa)[2], float (&sv)[8]) {
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                sv[4 * a + r] = fmaf(meta_scale<MF>(cur.km[a], r), sa[a][r],
                                     fmaf(meta_lo<MF>(cur.km[a], r), qsum_s, 0.0f));
        // sum the group columns of each head: a pairwise butterfly over the
        // orbit, as many steps as the group count needs (uniform branches)
        if (NG >= 2) DKV_DPP_ADD8("row_mirror", sv);            // col ^ 15
        if (NG >= 4) DKV_DPP_ADD8("row_half_mirror", sv);       // col ^ 7
        if (NG >= 8) DKV_DPP_ADD8("quad_perm:[3,2,1,0]", sv);   // col ^ 3
    }

    // The rest of a page on its scores: scale, mask, hand over the logits,
    // online softmax, PV. The optional hooks: resc(alpha, p0) when the
    // reference max moves (alpha = exp(old - new) per lane, before page p0's
    // probabilities), post(pv, p0) with the page's probabilities exp(logit -
    // reference).
    template <bool TAIL, class Sink, class Resc = NoHook, class Post = NoHook>
    __device__ __forceinline__ void rest(const Regs& cur, const float (&sv)[8], int p0, int r_end, Sink&& sink,
                                         Resc&& resc = Resc{}, Post&& post = Post{}) {
        float pv[8];
        rest_head<TAIL>(sv, p0, r_end, sink, pv, resc);
        rest_tail<TAIL>(cur, pv, p0, r_end, post);
    }

    // scale, mask the tail, hand over the logits, the column max and the lazy
    // rescale; pv gets the scaled logits
    template <bool TAIL, class Sink, class Resc = NoHook>
    __device__ __forceinline__ void rest_head(const float (&sv)[8], int p0, int r_end, Sink&& sink, float (&pv)[8],
                                              Resc&& resc = Resc{}) {
        float mx = -INFINITY;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            float v = sv[x] * scale_s;
            if (TAIL) v = (p0 + 16 * (x / 4) + 4 * jj + (x % 4) < r_end) ? v : -INFINITY;
            pv[x] = v;
            mx = fmaxf(mx, v);
        }
        sink(pv, p0);
        mx = lanegroup_max(mx);
        // Lazy rescale: the reference max only moves when a column's max grows
        // by more than 6 (so p <= e^6); o, l and the zero term share the
        // reference, and the combine merges partials on any reference.
        const bool grow = mx > m_run + 6.0f;
        if (__any(grow)) {
            const float m_new = grow ? mx : m_run;
            const float alpha = (m_run == -INFINITY) ? 0.0f : __expf(m_run - m_new);
            l_run *= alpha;
            zsum *= alpha;
#pragma unroll
            for (int t = 0; t < NDT; ++t) acc[t] *= alpha;
            resc(alpha, p0);
            m_run = m_new;
        }
    }

    // probabilities, row sums and the PV product of the page
    template <bool TAIL, class Post = NoHook>
    __device__ __forceinline__ void rest_tail(const Regs& cur, float (&pv)[8], int p0, int r_end,
                                              Post&& post = Post{}) {
        // m_run is finite from the first page on (every split starts with a
        // live row), so masked rows give exp(-inf) = 0 with no test
#pragma unroll
        for (int x = 0; x < 8; ++x) pv[x] = __expf(pv[x] - m_run);
        post(pv, p0);
        float sum = pv[0];
#pragma unroll
        for (int x = 1; x < 8; ++x) sum += pv[x];
        l_run += lanegroup_sum(sum);
        // ---- PV: B[row (jj, e)][col] = p * scaleV as an f16 pair hi + lo,
        // rows e<4: 4jj+e, e>=4: 16+4jj+e-4. One f16 alone would carry an
        // error of 2^-12 |v - zero| per row, which a peaked softmax over a
        // wide-range (outlier) channel does not average away; the pair
        // carries ~22 bits, and the codes (A) are exact.
        f16x8_t bhi, blo;
        float zs = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float sc = meta_scale<MF>(cur.vm, e), lo = meta_lo<MF>(cur.vm, e);
            if (TAIL) {
                // rows past the live count may hold stale meta: zero it (p is 0 there)
                const bool ok = p0 + (e < 4 ? 4 * jj + e : 16 + 4 * jj + e - 4) < r_end;
                sc = ok ? sc : 0.0f;
                lo = ok ? lo : 0.0f;
            }
            const float x = pv[e] * (x16_elem(CB, e) ? sc * 0.0625f : sc);   // p, sc >= 0
            bhi[e] = (_Float16)x;
            blo[e] = (_Float16)(x - (float)bhi[e]);   // exact difference, rounded once
            zs = fmaf(pv[e], lo, zs);
        }
        zsum += zs;
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
            const f16x8_t av = codes_to_f16<CB>(cur.v + t * (CB / 4));
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bhi, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, blo, acc[t], 0, 0, 0);
        }
    }

    // the split's partial: o = 2^24 * O' + zero term per d of the column's
    // group, then (m, l)
    __device__ __forceinline__ void finish(float* __restrict__ part, int s, int h, int Hq, int G, int n_splits,
                                           int split) {
        // total of the zero-point term over the 4 lane groups
        zsum += __shfl_xor(zsum, 16);
        zsum += __shfl_xor(zsum, 32);
        if (!cvalid) return;
        float* pp = part + (((int64_t)s * Hq + h * G + hcol) * n_splits + split) * (D + 2);
        const int t_lo = gcol * (group / 16), t_hi = t_lo + group / 16;   // the tiles of the column's group
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
            if (t < t_lo || t >= t_hi) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) pp[16 * t + 4 * jj + r] = acc[t][r] * kTwo24 + zsum;
        }
        if (gcol == 0 && jj == 0) {
            pp[D] = m_run;
            pp[D + 1] = l_run;
        }
    }
};

// byte offsets of a lane's operands inside a page (the same for every page)
template <int D, int CB, int MF>
__device__ __forceinline__ LaneOffsets lane_offsets(const PageFmt& f, int col, int jj, int gmeta) {
    using Regs = PageRegs<D, CB, MF>;
    LaneOffsets off;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        off.k[a] = (uint32_t)(f.kc + (16 * a + col) * (D * CB / 8) + Regs::WPL * 4 * jj);
        off.km[a] = (uint32_t)k_meta_off(f, 16 * a + 4 * jj, gmeta);
    }
    off.v = (uint32_t)(f.vc + (col * 4 + jj) * Regs::NV * 4);
    off.vm = (uint32_t)(f.vm + ((int64_t)gmeta * PAGE + jj * 8) * f.metaB);
    if constexpr (CB == 8) {   // lane load order: the lane's first 16-byte piece
#pragma unroll
        for (int a = 0; a < 2; ++a) off.k[a] = (uint32_t)(f.kc + a * 16 * D + 16 * (col + 16 * jj));
        off.v = (uint32_t)(f.vc + 16 * (col * 4 + jj));
    }
    return off;
}

// ---- register-staged kernel (8-bit codes): pages loaded straight into
// registers one page ahead; logits staged in LDS and written after the split.
// MERGE: one block of 8 waves per (sequence, KV head) segment (batches whose
// segments alone fill the chip): the waves' partials meet in LDS and the
// block writes the segment's output (and its rows' (max, sum)), so no
// combine kernel runs; the partials are merged as the combine merges them
// (the max over the waves first, then the weighted sums, waves in order).
constexpr int MERGE_WAVES = 8;
template <int D, int CB, int MF, bool MERGE = false>
__global__ void __launch_bounds__(MERGE ? 64 * MERGE_WAVES : 256, MERGE ? 1 : 2)
draft_attn_mfma_kernel(dkv_drafter_t m, int layer, dkv_qcfg_t cfg, const float* __restrict__ q, int Hq, float scale,
                       int rps, int n_splits, float* __restrict__ part, float* __restrict__ logits,
                       float* __restrict__ out, float* __restrict__ stats) {
    using Core = SplitCore<D, CB, MF>;
    using Regs = typename Core::Regs;
    constexpr int NWB = MERGE ? MERGE_WAVES : 4;   // waves per block
    constexpr int PD = D + 2;
    // the wave index through readfirstlane: the compiler then knows it (and
    // the split, row range and page addresses) to be wave-uniform, keeps them
    // in scalar registers and runs the page loop as a scalar loop
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int h = blockIdx.y, s = blockIdx.z;
    const int G = Hq / m.n_kv_heads;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    extern __shared__ float dyn_smem[];
    float* mp = dyn_smem + NWB * (G * rps + 8 * WAVE);   // MERGE: partials [G][NWB][D + 2]
    // the grid covers the splits of a few resident rounds; each wave walks
    // splits blockIdx.x*NWB + wave, + NWB*gridDim.x, ... while they hold rows
    const bool idle = (int)(blockIdx.x * NWB + wave) * rps >= n;
    if (!MERGE && idle) return;
    if (idle) {   // a neutral partial (no rows): max -inf, sum 0, output 0
        for (int i = lane; i < G * PD; i += WAVE)
            mp[((i / PD) * NWB + wave) * PD + i % PD] = (i % PD == D) ? -INFINITY : 0.0f;
    } else {
    const PageFmt f = page_fmt(cfg, D);
    Core c;
    c.init(q, s, h, Hq, G, cfg.group, lane, scale);
    const LaneOffsets off = lane_offsets<D, CB, MF>(f, c.col, c.jj, c.gmeta);
    float* slog = dyn_smem + wave * (G * rps + 8 * WAVE);
    const bool writer = c.cvalid && c.gcol == 0;
    const int slog_base = writer ? c.hcol * rps + 4 * c.jj : G * rps + 8 * lane;
    const int slog_step = writer ? 1 : 0, slog_second = writer ? 16 : 4;
    // one softmax state across all of the wave's splits: the wave writes a
    // single partial, in slot blockIdx.x*NWB + wave
    c.reset();
    const int part_slot = blockIdx.x * NWB + wave;
    for (int split = part_slot; split < n_splits && split * rps < n; split += NWB * gridDim.x) {
    const int r_begin = split * rps;
    const int r_end = min(r_begin + rps, n);

    // Logits for note_attention are staged in this wave's LDS region
    // [head][row - r_begin]; lanes that hold a head's logits (group column
    // 0) write two 16-byte runs of rows per page, the others write a dummy
    // slot of their own, so the loop issues no global stores and no branch.
    auto stage = [&](const float (&pv)[8], int p0) {
        float* dst = slog + slog_base + slog_step * (p0 - r_begin);
        *reinterpret_cast<float4*>(dst) = make_float4(pv[0], pv[1], pv[2], pv[3]);
        *reinterpret_cast<float4*>(dst + slog_second) = make_float4(pv[4], pv[5], pv[6], pv[7]);
    };

    const int np = (r_end - r_begin + PAGE - 1) / PAGE;
    const int nfull = (r_end - r_begin) / PAGE;   // pages whose 32 rows are all live
    const int pg0 = r_begin / PAGE;
    auto fetch = [&](Regs& b, int k) { load_page(b, page_ptr(m, s, layer, h, pg0 + k), off); };
    // Full pages: page k+1 is in flight while page k is computed (two
    // buffers, unrolled by 2). The scheduling barriers keep each fetch ahead
    // of the page's products: left alone, the scheduler sinks the loads into
    // the QK MFMAs, so the next page's latency hides behind half a page
    // instead of a whole one.
    Regs b0, b1;
    if (nfull > 0) {
        fetch(b0, 0);
        for (int k = 0; k < nfull; k += 2) {
            // (wave-uniform tests: no fetch past the split's last page, which
            // a split of whole pages would otherwise load twice)
            if (k + 1 < np) fetch(b1, k + 1);
            __builtin_amdgcn_sched_barrier(0);
            c.template page<false>(b0, r_begin + k * PAGE, r_end, stage);
            if (k + 1 >= nfull) break;
            if (k + 2 < np) fetch(b0, k + 2);
            __builtin_amdgcn_sched_barrier(0);
            c.template page<false>(b1, r_begin + (k + 1) * PAGE, r_end, stage);
        }
    }
    // the split's last page when it is partly live (the mirror's tail):
    // outside the loop, so the masking code adds no registers to it
    if (nfull < np) {
        fetch(b0, nfull);
        c.template page<true>(b0, r_begin + nfull * PAGE, r_end, stage);
    }
    // staged logits of the split's rows, one coalesced pass per query head
    if (logits) {
        // the wave reads back only its own LDS region, in program order
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int nr = r_end - r_begin;
        for (int i = lane; i < G * nr; i += WAVE) {
            const int g = i / nr, r = i % nr;
            logits[((int64_t)s * Hq + h * G + g) * m.cap + r_begin + r] = slog[g * rps + r];
        }
    }
    }
    if constexpr (MERGE) c.finish(mp, 0, 0, G, G, NWB, wave);
    else c.finish(part, s, h, Hq, G, n_splits, part_slot);
    }
    if constexpr (MERGE) {
        __syncthreads();
        for (int i = threadIdx.x; i < G * D; i += 64 * NWB) {
            const int hq = i / D, d = i % D;
            const float* ph = mp + hq * NWB * PD;
            float mm = -INFINITY;
#pragma unroll
            for (int w = 0; w < NWB; ++w) mm = fmaxf(mm, ph[w * PD + D]);
            float l = 0.0f, o = 0.0f;
#pragma unroll
            for (int w = 0; w < NWB; ++w) {
                const float mc = ph[w * PD + D];
                const float wt = (mc == -INFINITY) ? 0.0f : __expf(mc - mm);
                l = fmaf(ph[w * PD + D + 1], wt, l);
                o = fmaf(ph[w * PD + d], wt, o);
            }
            const int64_t row = (int64_t)s * Hq + h * G + hq;
            out[row * D + d] = (l > 0.0f) ? o / l : 0.0f;
            if (d == 0 && stats) {
                stats[row * 2] = mm;
                stats[row * 2 + 1] = l;
            }
        }
    }
}

// ---- LDS-staged kernel (4-bit codes). Each wave streams its pages through a
// ring of S page slots in LDS with direct-to-LDS loads (global_load_lds), S-1
// pages ahead of the products, without holding them in registers. A slot is
// LPP 1 KB loads, each 16 B per lane:
//   2: K codes, linear (row r at r * D/2 bytes)
//   D/64: V codes, gathered into lane order (load x: lane l's words 4x..4x+3)
//   the rest: K meta then V meta, linear
// The logits go straight from registers to the workspace (two 16-byte stores
// per writer lane per page). The loads are issued from inline asm and waited
// for by count (s_waitcnt vmcnt): the compiler's own tracking of LDS DMA would
// wait for every load in flight before any LDS read. Stores count in vmcnt
// too, so the count covers both.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from base + voff to LDS byte address lds + 16 * lane,
// non-temporal: the pages are read once per call, so they should not push
// other data out of the caches (measured 3% faster than the default policy)
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt vmcnt(n) for a wave-uniform n (the count is an immediate)
__device__ __forceinline__ void vm_wait(int n) {
    switch (n) {
#define DKV_VMW(k) \
    case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        DKV_VMW(0) DKV_VMW(1) DKV_VMW(2) DKV_VMW(3) DKV_VMW(4) DKV_VMW(5) DKV_VMW(6) DKV_VMW(7)
        DKV_VMW(8) DKV_VMW(9) DKV_VMW(10) DKV_VMW(11) DKV_VMW(12) DKV_VMW(13) DKV_VMW(14) DKV_VMW(15)
        DKV_VMW(16) DKV_VMW(17) DKV_VMW(18) DKV_VMW(19) DKV_VMW(20) DKV_VMW(21) DKV_VMW(22) DKV_VMW(23)
        DKV_VMW(24) DKV_VMW(25) DKV_VMW(26) DKV_VMW(27) DKV_VMW(28) DKV_VMW(29) DKV_VMW(30) DKV_VMW(31)
#undef DKV_VMW
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;   // never more in flight
    }
}

// 1 KB loads per page slot: 2 for K codes, D/64 for V codes, the rest for
// the K and V meta (f16 pairs of up to 4 groups fit one load, 8 groups or f32
// pairs need 2, f32 pairs of 8 groups 4)
__host__ __device__ inline int dma_lpp(const PageFmt& f, int D) {
    return 2 + D / 64 + (int)((2 * (f.vc - f.km) + 1023) / 1024);
}
// ring depth: 4 slots of 5 KB (80 KB per 4-wave block, 2 blocks per CU), 3 of larger
__host__ __device__ constexpr int dma_stages(int lpp) { return lpp <= 5 ? 4 : 3; }

template <int D, int MF, bool STORE, int LPP>
__global__ void __launch_bounds__(256, 2) draft_attn_dma_kernel(dkv_drafter_t m, int layer, dkv_qcfg_t cfg,
                                                                const float* __restrict__ q, int Hq, float scale,
                                                                int rps, int n_splits, float* __restrict__ part,
                                                                float* __restrict__ logits) {
    constexpr int CB = 4;
    using Core = SplitCore<D, CB, MF>;
    using Regs = typename Core::Regs;
    constexpr int NVL = D / 64;                 // V code loads per slot
    constexpr int SPP = STORE ? 2 : 0;          // logit stores per page
    constexpr int S = dma_stages(LPP);          // ring slots
    constexpr int SLOT = LPP * 1024;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int h = blockIdx.y, s = blockIdx.z;
    const int G = Hq / m.n_kv_heads;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    // The segment's live pages are dealt in contiguous, balanced runs to its
    // A = min(waves, pages) active waves: wave w streams pages
    // [w*np/A, (w+1)*np/A) as one run g = 0..T-1 and writes partial slot w.
    // Only the segment's last page can be partial, and it is the last wave's last.
    const int wid = blockIdx.x * 4 + wave;
    const int np = (n + PAGE - 1) / PAGE;
    const int A = min(min(4 * (int)gridDim.x, n_splits), np);
    if (wid >= A) return;
    const int pg0 = (int)(((int64_t)wid * np) / A);
    const int T = (int)(((int64_t)(wid + 1) * np) / A) - pg0;
    const bool tail = wid == A - 1 && n % PAGE != 0;   // the stream's last page is partial
    const PageFmt f = page_fmt(cfg, D);
    const uint32_t kmb = (uint32_t)(f.vc - f.km);   // K meta bytes (= V meta bytes)

    extern __shared__ __align__(16) char dma_smem[];
    char* ring = dma_smem + (size_t)wave * S * SLOT;
    int slot_in = 0, slot_out = 0;   // byte offsets of the next slot to fill / to read
    auto page_of = [&](int g) { return pg0 + g; };
    // source offset of each 1 KB load (the same for every page); the V code
    // loads gather into lane order and need the lane's column
    const int col = lane % 16, jj = lane / 16;
    uint32_t src[LPP];
    {
#pragma unroll
        for (int i = 0; i < LPP; ++i) {
            uint32_t o;
            if (i < 2) {
                o = (uint32_t)f.kc + i * 1024 + lane * 16;
            } else if (i < 2 + NVL) {
                o = (uint32_t)f.vc + (col * 4 + jj) * Regs::NV * 4 + (i - 2) * 16;
            } else {
                const uint32_t mo = (i - 2 - NVL) * 1024 + lane * 16;
                o = mo < kmb ? (uint32_t)f.km + mo : (mo < 2 * kmb ? (uint32_t)f.vm + (mo - kmb) : (uint32_t)f.km);
            }
            src[i] = o;
        }
    }
    auto issue = [&](int g) {
        const uint8_t* pg = page_ptr(m, s, layer, h, page_of(g));
        const uint32_t dst = lds_addr(ring + slot_in);
#pragma unroll
        for (int i = 0; i < LPP; ++i) dma16(pg, src[i], dst + i * 1024);
        slot_in = slot_in + SLOT == S * SLOT ? 0 : slot_in + SLOT;
    };
    // the first pages go out before the query loads, so their latency overlaps
    for (int j = 0; j < S - 1; ++j)
        if (j < T) issue(j);

    // one softmax state across the wave's whole run: a single partial, in
    // slot wid
    Core c;
    c.init(q, s, h, Hq, G, cfg.group, lane, scale);
    c.reset();
    // LDS offsets of the lane's operands inside a slot
    constexpr uint32_t mbase = (2 + NVL) * 1024;
    const uint32_t o_k = (c.col * 4 + c.jj) * 16;   // + a * 1024
    const uint32_t o_v = 2 * 1024 + lane * 16;      // + x * 1024
    const uint32_t o_km = mbase + (c.gmeta * PAGE + 4 * c.jj) * f.metaB;   // + 16 a * metaB
    const uint32_t o_vm = mbase + kmb + (c.gmeta * PAGE + 8 * c.jj) * f.metaB;
    auto operands = [&](Regs& r) {
        const char* sl = ring + slot_out;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            load_words(r.k[a], reinterpret_cast<const uint8_t*>(sl + a * 1024 + o_k));
            load_words(r.km[a], reinterpret_cast<const uint8_t*>(sl + o_km + 16 * a * f.metaB));
        }
#pragma unroll
        for (int x = 0; x < NVL; ++x) {
            const uint4 w = *reinterpret_cast<const uint4*>(sl + x * 1024 + o_v);
            r.v[4 * x] = w.x;
            r.v[4 * x + 1] = w.y;
            r.v[4 * x + 2] = w.z;
            r.v[4 * x + 3] = w.w;
        }
        load_words(r.vm, reinterpret_cast<const uint8_t*>(sl + o_vm));
        slot_out = slot_out + SLOT == S * SLOT ? 0 : slot_out + SLOT;
    };
    // logits of a page straight to the workspace: lanes of group column 0
    // hold rows 4jj..4jj+3 and 16+4jj..16+4jj+3 of head hcol
    const bool writer = c.cvalid && c.gcol == 0;
    float* lrow = STORE ? logits + ((int64_t)s * Hq + h * G + c.hcol) * m.cap + 4 * c.jj : nullptr;
    auto store = [&](const float (&pv)[8], int p0) {
        if (STORE && writer) {
            *reinterpret_cast<float4*>(lrow + p0) = make_float4(pv[0], pv[1], pv[2], pv[3]);
            *reinterpret_cast<float4*>(lrow + p0 + 16) = make_float4(pv[4], pv[5], pv[6], pv[7]);
        }
    };

    // Software-pipelined by one page: page g+1's operands are read from LDS
    // while page g's scores are scaled, stored and reduced to the column max;
    // then the QK MFMAs of page g+1 are issued, the matrix pipe works through
    // them while page g's probabilities and PV run, and their fold into
    // scores follows. Pages still enter the softmax in order, so the
    // arithmetic is that of one page at a time.
    // Waits: when page g+1 is awaited (iteration g, before issuing page
    // g+S-1), the loads in flight after its own are those of pages
    // g+2 .. g+S-2 and the logit stores of the pages computed since it was
    // issued (iterations g-S+2 .. g-1, or all so far for the first pages).
    Regs ra, rb;
    float sa_[8], sb_[8];
    vm_wait(LPP * min(S - 2, T - 1));   // page 0 landed
    operands(ra);
    c.qk(ra, sa_);
    // a page that has a successor (g + 1 < T; never the partial tail page)
    auto step = [&](int g, Regs& cur, float (&scur)[8], Regs& nxt, float (&snxt)[8]) {
        vm_wait(LPP * max(0, min(S - 3, T - 2 - g)) + SPP * min(g, S - 2));
        if (g + S - 1 < T) issue(g + S - 1);
        operands(nxt);
        float pv[8];
        c.template rest_head<false>(scur, (pg0 + g) * PAGE, n, store, pv);
        f32x4_t acc_next[2];
        c.qk_mfma(nxt, acc_next);
        c.template rest_tail<false>(cur, pv, (pg0 + g) * PAGE, n);
        c.qk_fold(nxt, acc_next, snxt);
    };
    // the stream's last page (g = T - 1)
    auto last = [&](int g, const Regs& cur, const float (&scur)[8]) {
        if (tail) c.template rest<true>(cur, scur, (pg0 + g) * PAGE, n, store);
        else c.template rest<false>(cur, scur, (pg0 + g) * PAGE, n, store);
    };
    int g = 0;
    for (; g + 2 < T; g += 2) {
        step(g, ra, sa_, rb, sb_);
        step(g + 1, rb, sb_, ra, sa_);
    }
    if (g + 1 < T) {   // two pages left
        step(g, ra, sa_, rb, sb_);
        last(g + 1, rb, sb_);
    } else {           // one page left
        last(g, ra, sa_);
    }
    c.finish(part, s, h, Hq, G, n_splits, wid);
}

// ---- segment kernel (4-bit codes, D = 128, 4 query heads x 4 groups per KV
// head): one block of 8 waves per (sequence, KV head) segment, used when the
// segments alone fill the chip (batch x KV heads >= 256). The waves stream
// their pages as the LDS-staged kernel does, but keep each page's
// probabilities in registers instead of writing logits to the workspace
// (33.5 MB of scattered writes at b=32 ctx 32k cost the split-K pass a
// quarter of its time, mixed into the read stream). After a block barrier
// the 8 partials meet in LDS -- the combine kernel's merge, in its order --
// and each lane scales its kept probabilities to the final max and sum and
// sums them over the KV head's 4 query heads across a lane quad: one float
// per row and KV head goes out, and draft_mass_sum_kernel adds the KV heads'
// sums to the row scores.
//
// The kept values: lane (gcol, hcol, jj) keeps rows 4jj+gcol and
// 16+4jj+gcol of head hcol (the 4 group columns of a head hold the same 8
// rows and share them out), two floats per page, exp(logit - the wave's
// running reference), rescaled with the accumulator when the reference
// moves. They sit in VGPRs above the compiler's allocation (amdgpu_num_vgpr
// caps it at SEG_VGPRS; the clobber of v255 sizes the wave's allocation to
// 256), written and read with s_set_gpr_idx at a wave-uniform index. Pages
// past SEG_TMAX spill to the workspace.
constexpr int SEG_WAVES = 8;
constexpr int SEG_VGPRS = 176;                  // the compiler's registers
constexpr int SEG_TMAX = (256 - SEG_VGPRS) / 2;  // pages per wave kept in registers
#ifndef SEG_OLD
#define SEG_OLD 10
#endif

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// buffer registers v176 + i2, v177 + i2 <- (a, b)
__device__ __forceinline__ void seg_put(int i2, float a, float b) {
    asm volatile("s_set_gpr_idx_on %0, gpr_idx(DST)\n\t"
                 "v_mov_b32 v176, %1\n\t"
                 "v_mov_b32 v177, %2\n\t"
                 "s_set_gpr_idx_off" ::"s"(i2),
                 "v"(a), "v"(b)
                 : "m0", "v255");
}
// (a, b) <- buffer registers v176 + i2, v177 + i2
__device__ __forceinline__ void seg_get(int i2, float& a, float& b) {
    asm volatile("s_set_gpr_idx_on %2, gpr_idx(SRC0)\n\t"
                 "v_mov_b32 %0, v176\n\t"
                 "v_mov_b32 %1, v177\n\t"
                 "s_set_gpr_idx_off"
                 : "=v"(a), "=v"(b)
                 : "s"(i2)
                 : "m0");
}
// 8 pages scaled: (a[k], b[k]) <- f * buffer registers v176 + i2 + 2k,
// v177 + i2 + 2k (the index applies to the products' first operand only;
// the outputs are early-clobber, as f is read after the first is written)
__device__ __forceinline__ void seg_get8_mul(int i2, float f, float (&a)[8], float (&b)[8]) {
    asm volatile("s_set_gpr_idx_on %16, gpr_idx(SRC0)\n\t"
                 "v_mul_f32 %0, v176, %17\n\tv_mul_f32 %1, v177, %17\n\tv_mul_f32 %2, v178, %17\n\t"
                 "v_mul_f32 %3, v179, %17\n\tv_mul_f32 %4, v180, %17\n\tv_mul_f32 %5, v181, %17\n\t"
                 "v_mul_f32 %6, v182, %17\n\tv_mul_f32 %7, v183, %17\n\tv_mul_f32 %8, v184, %17\n\t"
                 "v_mul_f32 %9, v185, %17\n\tv_mul_f32 %10, v186, %17\n\tv_mul_f32 %11, v187, %17\n\t"
                 "v_mul_f32 %12, v188, %17\n\tv_mul_f32 %13, v189, %17\n\tv_mul_f32 %14, v190, %17\n\t"
                 "v_mul_f32 %15, v191, %17\n\t"
                 "s_set_gpr_idx_off"
                 : "=&v"(a[0]), "=&v"(b[0]), "=&v"(a[1]), "=&v"(b[1]), "=&v"(a[2]), "=&v"(b[2]), "=&v"(a[3]),
                   "=&v"(b[3]), "=&v"(a[4]), "=&v"(b[4]), "=&v"(a[5]), "=&v"(b[5]), "=&v"(a[6]), "=&v"(b[6]),
                   "=&v"(a[7]), "=&v"(b[7])
                 : "s"(i2), "v"(f)
                 : "m0");
}

// lane-quad sums (lanes 4k..4k+3) of 16 values, the bitwise-same total in
// each lane: one fused v_add_f32_dpp per value and step (quad_perm [1,0,3,2]
// then [2,3,0,1]); the s_nop covers the two wait states a DPP read needs
// after a VALU write, and every later add reads a register written at least
// two instructions before it.
#define DKV_QADD16(CTRL)                                                                                         \
    "v_add_f32_dpp %0, %0, %0 " CTRL " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %1, %1, %1 " CTRL           \
    " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %2, %2, %2 " CTRL " row_mask:0xf bank_mask:0xf\n\t"            \
    "v_add_f32_dpp %3, %3, %3 " CTRL " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %4, %4, %4 " CTRL           \
    " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %5, %5, %5 " CTRL " row_mask:0xf bank_mask:0xf\n\t"            \
    "v_add_f32_dpp %6, %6, %6 " CTRL " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %7, %7, %7 " CTRL           \
    " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %8, %8, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"            \
    "v_add_f32_dpp %9, %9, %9 " CTRL " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %10, %10, %10 " CTRL        \
    " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %11, %11, %11 " CTRL " row_mask:0xf bank_mask:0xf\n\t"         \
    "v_add_f32_dpp %12, %12, %12 " CTRL " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %13, %13, %13 " CTRL     \
    " row_mask:0xf bank_mask:0xf\n\tv_add_f32_dpp %14, %14, %14 " CTRL " row_mask:0xf bank_mask:0xf\n\t"         \
    "v_add_f32_dpp %15, %15, %15 " CTRL " row_mask:0xf bank_mask:0xf\n\t"
__device__ __forceinline__ void quad_sum16(float (&a)[8], float (&b)[8]) {
    asm volatile("s_nop 1\n\t" DKV_QADD16("quad_perm:[1,0,3,2]") DKV_QADD16("quad_perm:[2,3,0,1]")
                 : "+v"(a[0]), "+v"(b[0]), "+v"(a[1]), "+v"(b[1]), "+v"(a[2]), "+v"(b[2]), "+v"(a[3]), "+v"(b[3]),
                   "+v"(a[4]), "+v"(b[4]), "+v"(a[5]), "+v"(b[5]), "+v"(a[6]), "+v"(b[6]), "+v"(a[7]), "+v"(b[7]));
}
#undef DKV_QADD16
#pragma clang diagnostic pop

// t where the lane's bit of mask is set, else f (one v_cndmask_b32; written out
// so that a select between registers does not become an indexed stack load)
__device__ __forceinline__ float lane_select(float f, float t, uint64_t mask) {
    float r;
    asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(r) : "v"(f), "v"(t), "s"(mask));
    return r;
}
// the same on operands that may come straight from a transcendental (v_exp):
// a VALU read of its result needs one wait state, which the compiler inserts
// before its own instructions but not before inline asm
__device__ __forceinline__ float lane_select_tr(float f, float t, uint64_t mask) {
    float r;
    asm("s_nop 0\n\tv_cndmask_b32 %0, %1, %2, %3" : "=v"(r) : "v"(f), "v"(t), "s"(mask));
    return r;
}

// SPLIT: a segment is cut into nb blocks of whole pages (gridDim.x = nb;
// for batches whose segments alone do not fill the chip). A block then
// leaves its merged partial (o, max, sum) per query head in part
// [b][Hkv][nb][G][D+2], and instead of the per-KV-head mass the kept
// probabilities against its merged max, per query head, in pmass
// [b][Hkv][cap][G] (pmass may be the spill buffer: a page's 512 bytes there
// are read, then written, by the one wave that owns it);
// draft_seg_merge_kernel merges the blocks and adds the mass.
template <int MF, int LPP, bool SPLIT>
__global__ void __launch_bounds__(64 * SEG_WAVES, 1) __attribute__((amdgpu_num_vgpr(SEG_VGPRS)))
draft_attn_seg_kernel(dkv_drafter_t m, int layer, dkv_qcfg_t cfg, const float* __restrict__ q, int Hq, float scale,
                      float* __restrict__ out, float* __restrict__ spill, float* __restrict__ pmass, int nb,
                      float* __restrict__ part) {
    constexpr int D = 128, CB = 4, G = 4;
    using Core = SplitCore<D, CB, MF>;
    using Regs = typename Core::Regs;
    constexpr int NVL = D / 64;
    constexpr int S = dma_stages(LPP);
    constexpr int SLOT = LPP * 1024;
    constexpr int PD = D + 2;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int h = blockIdx.y, s = blockIdx.z;
    const int Hkv = m.n_kv_heads;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int np_seg = (n + PAGE - 1) / PAGE;
    // the block's pages [b0, b0 + np): the whole segment, or (SPLIT) its
    // share of ceil(np_seg / nb) pages
    int b0 = 0, np = np_seg;
    if constexpr (SPLIT) {
        const int ppb = (np_seg + nb - 1) / nb;
        b0 = blockIdx.x * ppb;
        np = min(np_seg - b0, ppb);
        if (np <= 0) return;   // a block past the segment's end (its partial is never read)
    }
    // contiguous page runs; with at least 64 pages, waves 0-3 (the older
    // wave of each SIMD, which wins issue by age) take SEG_OLD/16 of them
    // (every wave keeps at least 4 pages for SEG_OLD <= 12)
    const int A = min(SEG_WAVES, np);
    const bool active = wave < A;
    auto cut = [&](int w) -> int {
        if (SPLIT || A < SEG_WAVES || np < 64) return (int)(((int64_t)w * np) / A);   // every wave >= 1 page
        const int c = w <= 4 ? w * SEG_OLD : 4 * SEG_OLD + (w - 4) * (16 - SEG_OLD);   // in 64ths
        return (int)(((int64_t)c * np) / 64);
    };
    const int pg0 = active ? b0 + cut(wave) : 0;
    const int T = active ? b0 + cut(wave + 1) - pg0 : 0;
    const bool tail = wave == A - 1 && b0 + np == np_seg && n % PAGE != 0;
    const bool keep = pmass != nullptr;
    extern __shared__ __align__(16) char dma_smem[];
    Core c;
    if (active) {
        const PageFmt f = page_fmt(cfg, D);
        const uint32_t kmb = (uint32_t)(f.vc - f.km);
        char* ring = dma_smem + (size_t)wave * S * SLOT;
        int slot_in = 0, slot_out = 0;
        const int col = lane % 16, jj = lane / 16;
        uint32_t src[LPP];
#pragma unroll
        for (int i = 0; i < LPP; ++i) {
            uint32_t o;
            if (i < 2) {
                o = (uint32_t)f.kc + i * 1024 + lane * 16;
            } else if (i < 2 + NVL) {
                o = (uint32_t)f.vc + (col * 4 + jj) * Regs::NV * 4 + (i - 2) * 16;
            } else {
                const uint32_t mo = (i - 2 - NVL) * 1024 + lane * 16;
                o = mo < kmb ? (uint32_t)f.km + mo : (mo < 2 * kmb ? (uint32_t)f.vm + (mo - kmb) : (uint32_t)f.km);
            }
            src[i] = o;
        }
        auto issue = [&](int g) {
            const uint8_t* pg = page_ptr(m, s, layer, h, pg0 + g);
            const uint32_t dst = lds_addr(ring + slot_in);
#pragma unroll
            for (int i = 0; i < LPP; ++i) dma16(pg, src[i], dst + i * 1024);
            slot_in = slot_in + SLOT == S * SLOT ? 0 : slot_in + SLOT;
        };
        // the KV head's G x D floats of q (2 KB) go into the ring's last slot,
        // which no page uses before the first step, ahead of the pages: the
        // wait for q then leaves the pages in flight
        char* qs = ring + (S - 1) * SLOT;
        const float* qg = q + ((int64_t)s * Hq + h * G) * D;
        static_assert(G * D * 4 == 2048 && S >= 2, "q takes two 1 KB loads into a free slot");
        dma16(qg, lane * 16, lds_addr(qs));
        dma16(qg, 1024 + lane * 16, lds_addr(qs) + 1024);
        for (int j = 0; j < S - 1; ++j)
            if (j < T) issue(j);
        c.init_lanes(G, cfg.group, lane);
        vm_wait(LPP * min(S - 1, T));
        c.init_q(reinterpret_cast<const float*>(qs), scale);
        c.reset();
        constexpr uint32_t mbase = (2 + NVL) * 1024;
        const uint32_t o_k = (c.col * 4 + c.jj) * 16;
        const uint32_t o_v = 2 * 1024 + lane * 16;
        const uint32_t o_km = mbase + (c.gmeta * PAGE + 4 * c.jj) * f.metaB;
        const uint32_t o_vm = mbase + kmb + (c.gmeta * PAGE + 8 * c.jj) * f.metaB;
        auto operands = [&](Regs& r) {
            const char* sl = ring + slot_out;
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                load_words(r.k[a], reinterpret_cast<const uint8_t*>(sl + a * 1024 + o_k));
                load_words(r.km[a], reinterpret_cast<const uint8_t*>(sl + o_km + 16 * a * f.metaB));
            }
#pragma unroll
            for (int x = 0; x < NVL; ++x) {
                const uint4 w = *reinterpret_cast<const uint4*>(sl + x * 1024 + o_v);
                r.v[4 * x] = w.x;
                r.v[4 * x + 1] = w.y;
                r.v[4 * x + 2] = w.z;
                r.v[4 * x + 3] = w.w;
            }
            load_words(r.vm, reinterpret_cast<const uint8_t*>(sl + o_vm));
            slot_out = slot_out + SLOT == S * SLOT ? 0 : slot_out + SLOT;
        };
        // a page's probabilities exp(logit - reference): the lane's two rows
        // (x = gcol and gcol + 4 of its 8)
        const uint64_t g1 = __ballot((c.gcol & 1) != 0), g2 = __ballot((c.gcol & 2) != 0);
        float* spill_w = spill + ((int64_t)(s * Hkv + h) * (m.cap / PAGE) + pg0) * (2 * WAVE) + 2 * lane;
        auto stash = [&](const float (&pv)[8], int p0) {
            if (!keep) return;
            const float a = lane_select(lane_select_tr(pv[0], pv[1], g1), lane_select_tr(pv[2], pv[3], g1), g2);
            const float b = lane_select(lane_select_tr(pv[4], pv[5], g1), lane_select_tr(pv[6], pv[7], g1), g2);
            const int g = __builtin_amdgcn_readfirstlane(p0 / PAGE - pg0);
            if (g < SEG_TMAX) seg_put(2 * g, a, b);
            else *reinterpret_cast<float2*>(spill_w + (int64_t)g * (2 * WAVE)) = make_float2(a, b);
        };
        // the reference moved before page p0 (rare: a column's max grew by
        // more than 6): the pages kept so far take the factor too
        auto restash = [&](float alpha, int p0) {
            if (!keep) return;
            const int gc = __builtin_amdgcn_readfirstlane(p0 / PAGE - pg0);
            for (int k = 0; k < min(gc, SEG_TMAX); ++k) {
                float a, b;
                seg_get(2 * k, a, b);
                seg_put(2 * k, a * alpha, b * alpha);
            }
            for (int k = SEG_TMAX; k < gc; ++k) {
                float2* pk = reinterpret_cast<float2*>(spill_w + (int64_t)k * (2 * WAVE));
                const float2 v = *pk;
                *pk = make_float2(v.x * alpha, v.y * alpha);
            }
        };
        // the LDS-staged kernel's page pipeline, with the probabilities kept
        // instead of logits stored: the waits count loads only (spilled pages
        // wait as if they were not there; a spill store or a rescale's
        // read-modify-write only makes a wait longer)
        Regs ra, rb;
        float sa_[8], sb_[8];
        vm_wait(LPP * min(S - 2, T - 1));
        operands(ra);
        c.qk(ra, sa_);
        auto step = [&](int g, Regs& cur, float (&scur)[8], Regs& nxt, float (&snxt)[8]) {
            vm_wait(LPP * max(0, min(S - 3, T - 2 - g)));
            if (g + S - 1 < T) issue(g + S - 1);
            operands(nxt);
            float pv[8];
            c.template rest_head<false>(scur, (pg0 + g) * PAGE, n, NoHook{}, pv, restash);
            f32x4_t acc_next[2];
            c.qk_mfma(nxt, acc_next);
            c.template rest_tail<false>(cur, pv, (pg0 + g) * PAGE, n, stash);
            c.qk_fold(nxt, acc_next, snxt);
        };
        auto last = [&](int g, const Regs& cur, const float (&scur)[8]) {
            if (tail) c.template rest<true>(cur, scur, (pg0 + g) * PAGE, n, NoHook{}, restash, stash);
            else c.template rest<false>(cur, scur, (pg0 + g) * PAGE, n, NoHook{}, restash, stash);
        };
        int g = 0;
        for (; g + 2 < T; g += 2) {
            step(g, ra, sa_, rb, sb_);
            step(g + 1, rb, sb_, ra, sa_);
        }
        if (g + 1 < T) {
            step(g, ra, sa_, rb, sb_);
            last(g + 1, rb, sb_);
        } else {
            last(g, ra, sa_);
        }
    }
    // ---- merge: the partials [head][wave][D+2] and the heads' (max, 1/sum)
    // in the LDS the ring held (every page has landed and been read)
    __syncthreads();
    float* sp = reinterpret_cast<float*>(dma_smem);
    float* sst = sp + G * SEG_WAVES * PD;
    if (active) {
        c.finish(sp, 0, 0, G, G, SEG_WAVES, wave);
    } else {
        // a wave without pages (segments under 8 pages): a neutral partial
        // (max -inf, sum 0, zeros), so the merge runs over every wave
        for (int i = lane; i < G * PD; i += WAVE)
            sp[((i / PD) * SEG_WAVES + wave) * PD + i % PD] = (i % PD == D) ? -INFINITY : 0.0f;
    }
    __syncthreads();
    {
        // all the waves' loads at once (the loops unroll), then the sums in
        // wave order
        const int hl = threadIdx.x / D, d = threadIdx.x % D;   // 512 threads = G x D outputs
        const float* ph = sp + hl * SEG_WAVES * PD;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < SEG_WAVES; ++w) mm = fmaxf(mm, ph[w * PD + D]);
        float l = 0.0f, o = 0.0f;
#pragma unroll
        for (int w = 0; w < SEG_WAVES; ++w) {
            const float mc = ph[w * PD + D], lc = ph[w * PD + D + 1];
            const float wt = (mc == -INFINITY) ? 0.0f : __expf(mc - mm);
            l = fmaf(lc, wt, l);
            o = fmaf(ph[w * PD + d], wt, o);
        }
        if constexpr (SPLIT) {
            float* pp = part + ((((int64_t)s * Hkv + h) * nb + blockIdx.x) * G + hl) * PD;
            pp[d] = o;
            if (d == 0) {
                pp[D] = mm;
                pp[D + 1] = l;
                sst[2 * hl] = mm;
                sst[2 * hl + 1] = 1.0f;   // kept values against the block's max, unnormalised
            }
        } else {
            __builtin_nontemporal_store((l > 0.0f) ? o / l : 0.0f, &out[((int64_t)s * Hq + h * G + hl) * D + d]);
            if (d == 0) {
                sst[2 * hl] = mm;
                sst[2 * hl + 1] = l > 0.0f ? 1.0f / l : 0.0f;
            }
        }
    }
    if (!keep) return;
    __syncthreads();
    if (!active) return;
    // ---- mass: p = exp(logit - max) / sum per kept value, summed over the
    // quad of the KV head's 4 query heads (lanes hcol 0..3 of a group column);
    // the kept values are exp(logit - the wave's reference), so p is a kept
    // value times exp(reference - max) / sum
    if constexpr (SPLIT) {
        // every kept value against the block's max, per query head: lane
        // (gcol, hcol, jj) holds rows 4jj + gcol and 16 + 4jj + gcol of each
        // page for head hcol, stored at [row][hcol] (a quad's four heads of a
        // row are 16 contiguous bytes)
        const float fac = __expf(c.m_run - sst[2 * c.hcol]);
        float* pr = pmass + ((int64_t)(s * Hkv + h) * m.cap + (int64_t)pg0 * PAGE + 4 * c.jj + c.gcol) * G + c.hcol;
        const float* spill_w = spill + ((int64_t)(s * Hkv + h) * (m.cap / PAGE) + pg0) * (2 * WAVE) + 2 * lane;
        for (int g = 0; g < T; ++g) {
            float a, b;
            if (g < SEG_TMAX) {
                seg_get(2 * g, a, b);
            } else {
                const float2 v = *reinterpret_cast<const float2*>(spill_w + (int64_t)g * (2 * WAVE));
                a = v.x;
                b = v.y;
            }
            pr[(int64_t)g * PAGE * G] = a * fac;
            pr[((int64_t)g * PAGE + 16) * G] = b * fac;
        }
        return;
    }
    {
        const float fac = __expf(c.m_run - sst[2 * c.hcol]) * sst[2 * c.hcol + 1];
        const uint64_t hb0 = __ballot((c.hcol & 1) != 0), hb1 = __ballot((c.hcol & 2) != 0);
        const int row2 = (c.hcol >> 1) * PAGE + (c.hcol & 1) * 16 + 4 * c.jj + c.gcol;   // row in the page pair
        float* pm = pmass + (int64_t)(s * Hkv + h) * m.cap + pg0 * PAGE + row2;
        const float* spill_w = spill + ((int64_t)(s * Hkv + h) * (m.cap / PAGE) + pg0) * (2 * WAVE) + 2 * lane;
        const int r_end = (pg0 + T) * PAGE <= n ? T * PAGE : n - pg0 * PAGE;   // the wave's live rows
        // 8 pages at a time, so the reads, products and quad sums of different
        // pages overlap. Every lane of a quad ends with both sums of its rows:
        // lane hcol writes page g0 + k + (hcol >> 1), half (hcol & 1), so one
        // store covers two pages (64 rows, 256 contiguous bytes); non-temporal,
        // as the output's (written once, read once by the mass sum: measured
        // 1 us faster per call at b=32 ctx 32k)
        constexpr int U = 8;
        // WHOLE (a compile-time flag): every row of the chunk is live, so the
        // stores need no row test
        auto emit = [&](int g0, float (&a)[U], float (&b)[U], auto whole) {
            quad_sum16(a, b);
#pragma unroll
            for (int k = 0; k < U; k += 2) {
                const float lo = lane_select(a[k], b[k], hb0), hi = lane_select(a[k + 1], b[k + 1], hb0);
                const float v = lane_select(lo, hi, hb1);
                if (decltype(whole)::value || (g0 + k) * PAGE + row2 < r_end)
                    __builtin_nontemporal_store(v, &pm[(g0 + k) * PAGE]);
            }
        };
        // chunks in registers: 16 products with indexed operands
        const int Tr = min(T, SEG_TMAX);
        int g0 = 0;
        for (; g0 + U <= Tr; g0 += U) {
            float a[U], b[U];
            seg_get8_mul(2 * g0, fac, a, b);
            if ((g0 + U) * PAGE <= r_end) emit(g0, a, b, bool_c<true>{});
            else emit(g0, a, b, bool_c<false>{});
        }
        for (; g0 < T; g0 += U) {
            float a[U], b[U];
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const int g = g0 + k;
                if (g < T && g < SEG_TMAX) {
                    seg_get(2 * g, a[k], b[k]);
                } else if (g < T) {
                    const float2 v = *reinterpret_cast<const float2*>(spill_w + (int64_t)g * (2 * WAVE));
                    a[k] = v.x;
                    b[k] = v.y;
                } else {
                    a[k] = b[k] = 0.0f;
                }
                a[k] *= fac;
                b[k] *= fac;
            }
            emit(g0, a, b, bool_c<false>{});
        }
    }
}

// score[row] += sum over KV heads of the per-KV-head masses of the segment
// kernel (KV heads in order), 4 rows per thread: float4 reads of the masses,
// double2 read-modify-writes of the scores
constexpr int MSUM_ROWS = 4;
__global__ void __launch_bounds__(256) draft_mass_sum_kernel(dkv_drafter_t m, int layer,
                                                             const float* __restrict__ pmass) {
    const int s = blockIdx.y;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int r = (blockIdx.x * blockDim.x + threadIdx.x) * MSUM_ROWS;
    if (r >= n) return;
    const float* p = pmass + (int64_t)s * m.n_kv_heads * m.cap + r;
    double* sc = m.score + row_index(m, s, layer) + r;
    // (cap and r are multiples of 4, so p and sc are 16-byte aligned when
    // the workspace and the scores are)
    if (r + MSUM_ROWS <= n && ((reinterpret_cast<uintptr_t>(sc) | reinterpret_cast<uintptr_t>(p)) & 15) == 0) {
        float4 t = *reinterpret_cast<const float4*>(p);
        for (int hk = 1; hk < m.n_kv_heads; ++hk) {
            const float4 v = *reinterpret_cast<const float4*>(p + (int64_t)hk * m.cap);
            t.x += v.x;
            t.y += v.y;
            t.z += v.z;
            t.w += v.w;
        }
        double2* d2 = reinterpret_cast<double2*>(sc);
        double2 a = d2[0], b = d2[1];
        a.x += static_cast<double>(t.x);
        a.y += static_cast<double>(t.y);
        b.x += static_cast<double>(t.z);
        b.y += static_cast<double>(t.w);
        d2[0] = a;
        d2[1] = b;
        return;
    }
    for (int k = 0; k < MSUM_ROWS && r + k < n; ++k) {
        float t = p[k];
        for (int hk = 1; hk < m.n_kv_heads; ++hk) t += p[(int64_t)hk * m.cap + k];
        sc[k] += static_cast<double>(t);
    }
}

// The segment kernel's SPLIT mode, second half. Grid (Hkv + row blocks,
// batch), 256 threads. Every block first turns the segment blocks' (max,
// sum) into factors c = exp(max_b - M) / L per (KV head, block, query head)
// in LDS (M, L: the merged max and sum). Blocks x < Hkv then write KV head
// x's outputs, sum_b o_b * c_b over the segment blocks in order; the others
// take SMERGE_ROWS rows each and add to each row's score the sum over KV heads (in
// order) of that head's mass, the kept values times their block's factors
// summed over the query heads pairwise.
constexpr int SMERGE_ROWS = 256;    // rows per block of the mass part (one per thread)
constexpr int SMERGE_MAX_NB = 64;    // segment blocks
constexpr int SMERGE_MAX_HKV = 16;   // KV heads
constexpr int SMERGE_PRE = 32;       // partial outputs per merge thread loaded with the statistics
constexpr int SMERGE_PER = 4;        // statistics loads per thread
__global__ void __launch_bounds__(256) draft_seg_merge_kernel(dkv_drafter_t m, int layer, int nb,
                                                              const float* __restrict__ part,
                                                              const float* __restrict__ pk, float* __restrict__ out,
                                                              int want_mass) {
    constexpr int D = 128, G = 4, PD = D + 2;
    const int s = blockIdx.y, Hkv = m.n_kv_heads, Hq = Hkv * G;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int np = (n + PAGE - 1) / PAGE;
    const int ppb = (np + nb - 1) / nb;
    const int nbl = np > 0 ? (np + ppb - 1) / ppb : 0;   // blocks that hold pages
    const bool merge = (int)blockIdx.x < Hkv;
    if (!merge && (!want_mass || ((int)blockIdx.x - Hkv) * SMERGE_ROWS >= n)) return;
    __shared__ float sm[SMERGE_MAX_HKV * SMERGE_MAX_NB * G], sl[SMERGE_MAX_HKV * SMERGE_MAX_NB * G];
    const int h_lo = merge ? blockIdx.x : 0, h_hi = merge ? blockIdx.x + 1 : Hkv;
    const int nh = h_hi - h_lo, cnt = nh * nbl * G;   // (head, block, query head) entries
    // The loads go out together before the first wait: what the sums need
    // besides the factors (a merge block's partial outputs of the first
    // SMERGE_PRE blocks, a mass block's kept values and old score) does not
    // depend on the blocks' statistics, and the statistics are SMERGE_PER
    // independent loads per thread (cnt <= 1024: the host keeps nb * Hkv <=
    // 256). Clamped indices keep the loads unconditional; what they read past
    // nbl is never used.
    float xo[2][SMERGE_PRE];   // merge: partial outputs i = tid, tid + 256
    float4 p[SMERGE_MAX_HKV];  // mass: kept values of row r, every KV head
    double old = 0.0;
    const int r = ((int)blockIdx.x - Hkv) * SMERGE_ROWS + threadIdx.x;
    double* score = merge ? nullptr : m.score + row_index(m, s, layer) + r;
    if (merge) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = threadIdx.x + 256 * k, hq = i / D, d = i % D;
            const float* pp = part + (((int64_t)s * Hkv + h_lo) * nb * G + hq) * PD + d;
#pragma unroll
            for (int b = 0; b < SMERGE_PRE; ++b) xo[k][b] = pp[(int64_t)min(b, max(nbl - 1, 0)) * G * PD];
        }
    } else if (r < n) {
        old = *score;
#pragma unroll
        for (int hh = 0; hh < SMERGE_MAX_HKV; ++hh)
            if (hh < Hkv) p[hh] = *reinterpret_cast<const float4*>(pk + (((int64_t)s * Hkv + hh) * m.cap + r) * G);
    }
    const int nb1 = max(nbl, 1);   // (no page: the merge blocks still read one in-bounds partial)
    auto stat_ptr = [&](int i) {
        const int hq = i % G, b = (i / G) % nb1, hh = i / (G * nb1);
        // (max, sum) of one partial: PD * 4 and D * 4 are multiples of 8
        return reinterpret_cast<const float2*>(part + ((((int64_t)s * Hkv + h_lo + hh) * nb + b) * G + hq) * PD + D);
    };
    {
        float2 st[SMERGE_PER];
#pragma unroll
        for (int k = 0; k < SMERGE_PER; ++k) st[k] = *stat_ptr(min((int)threadIdx.x + 256 * k, max(cnt - 1, 0)));
#pragma unroll
        for (int k = 0; k < SMERGE_PER; ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < cnt) {
                sm[i] = st[k].x;
                sl[i] = st[k].y;
            }
        }
        for (int i = threadIdx.x + 256 * SMERGE_PER; i < cnt; i += 256) {   // not reached while nb * Hkv <= 256
            const float2 v = *stat_ptr(i);
            sm[i] = v.x;
            sl[i] = v.y;
        }
    }
    __syncthreads();
    // the merged (max, 1/sum) of each (head, query head): 4 lanes per pair
    // (up to 64 pairs), each over every 4th block, then two xor shuffles
    // (the same values and order in every block of the grid)
    __shared__ float sM[SMERGE_MAX_HKV * G], siL[SMERGE_MAX_HKV * G];
    {
        const int pr = threadIdx.x / 4, sub = threadIdx.x % 4;
        const bool live = pr < nh * G;
        const int hh = live ? pr / G : 0, hq = pr % G;
        float M = -INFINITY;
        if (live)
            for (int b = sub; b < nbl; b += 4) M = fmaxf(M, sm[(hh * nbl + b) * G + hq]);
        M = fmaxf(M, __shfl_xor(M, 1));
        M = fmaxf(M, __shfl_xor(M, 2));
        float L = 0.0f;
        if (live)
            for (int b = sub; b < nbl; b += 4) {
                const float mb = sm[(hh * nbl + b) * G + hq];
                L = fmaf(sl[(hh * nbl + b) * G + hq], mb == -INFINITY ? 0.0f : __expf(mb - M), L);
            }
        L += __shfl_xor(L, 1);
        L += __shfl_xor(L, 2);
        if (live && sub == 0) {
            sM[pr] = M;
            siL[pr] = L > 0.0f ? 1.0f / L : 0.0f;
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < cnt; i += blockDim.x) {
        const int hq = i % G, hh = i / (G * nbl);
        const float mb = sm[i];
        sm[i] = mb == -INFINITY ? 0.0f : __expf(mb - sM[hh * G + hq]) * siL[hh * G + hq];
    }
    __syncthreads();
    if (merge) {
        // outputs (query head hq, channel d) of KV head h_lo, two per thread:
        // the blocks' terms in block order
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = threadIdx.x + 256 * k, hq = i / D, d = i % D;
            float o = 0.0f;
#pragma unroll
            for (int b = 0; b < SMERGE_PRE; ++b)
                if (b < nbl) o = fmaf(xo[k][b], sm[b * G + hq], o);
            const float* pp = part + (((int64_t)s * Hkv + h_lo) * nb * G + hq) * PD + d;
            for (int b = SMERGE_PRE; b < nbl; ++b) o = fmaf(pp[(int64_t)b * G * PD], sm[b * G + hq], o);
            out[((int64_t)s * Hq + h_lo * G + hq) * D + d] = o;
        }
        return;
    }
    if (r >= n) return;
    const int b = (r / PAGE) / ppb;
    // the sums over KV heads in order
    float t = 0.0f;
#pragma unroll
    for (int hh = 0; hh < SMERGE_MAX_HKV; ++hh)
        if (hh < Hkv) {
            const float* c = sm + (hh * nbl + b) * G;
            t += (p[hh].x * c[0] + p[hh].y * c[1]) + (p[hh].z * c[2] + p[hh].w * c[3]);
        }
    *score = old + static_cast<double>(t);
}

// ---------------------------------------------------------------- combine + mass
// Merge the partials of (seq, query head) and record the final (max, sum).
// Partial slots [0, min(live units, n_splits, n_parts)) hold data, a unit
// being a split (register-staged and generic kernels) or a page (the
// LDS-staged kernel, whose waves take contiguous runs of pages). The global max
// comes first, so the weighted sums over the partials are independent terms:
// wave w of the block takes partials w, w + nw, ... (lane: channels lane and
// lane + 64), 8 of them in flight, and the waves' sums meet in LDS in a
// fixed order.
constexpr int COMB_WAVES = 16;
__global__ void __launch_bounds__(64 * COMB_WAVES) draft_combine_kernel(dkv_drafter_t m, int layer,
                                                                        const float* __restrict__ part, int Hq,
                                                                        int unit, int n_splits, int n_parts,
                                                                        float* __restrict__ out,
                                                                        float* __restrict__ stats) {
    const int hq = blockIdx.x, s = blockIdx.y;
    const int D = m.head_dim, PD = D + 2;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int ns = min(min((n + unit - 1) / unit, n_splits), n_parts);
    const float* p = part + ((int64_t)s * Hq + hq) * n_splits * PD;
    const int nw = blockDim.x / WAVE, w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    __shared__ float smax[COMB_WAVES], sl[COMB_WAVES];
    __shared__ float so[COMB_WAVES][2 * WAVE];
    float mm = -INFINITY;
    for (int c = threadIdx.x; c < ns; c += blockDim.x) mm = fmaxf(mm, p[(int64_t)c * PD + D]);
    for (int o = WAVE / 2; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
    if (lane == 0) smax[w] = mm;
    __syncthreads();
    mm = smax[0];
    for (int i = 1; i < nw; ++i) mm = fmaxf(mm, smax[i]);
    const bool a0 = lane < D, a1 = lane + WAVE < D;
    float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll 8
    for (int c = w; c < ns; c += nw) {
        const float* pc = p + (int64_t)c * PD;
        const float mc = pc[D], lc = pc[D + 1];
        const float x0 = a0 ? pc[lane] : 0.0f, x1 = a1 ? pc[lane + WAVE] : 0.0f;
        const float wt = (mc == -INFINITY) ? 0.0f : __expf(mc - mm);
        l = fmaf(lc, wt, l);
        o0 = fmaf(x0, wt, o0);
        o1 = fmaf(x1, wt, o1);
    }
    so[w][lane] = o0;
    so[w][lane + WAVE] = o1;
    if (lane == 0) sl[w] = l;
    __syncthreads();
    // every channel, whatever the block width (one wave covers 64 per pass)
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float lt = 0.0f, ot = 0.0f;
        for (int i = 0; i < nw; ++i) {
            lt += sl[i];
            ot += so[i][d];
        }
        out[((int64_t)s * Hq + hq) * D + d] = (lt > 0.0f) ? ot / lt : 0.0f;
        if (d == 0 && stats) {
            stats[((int64_t)s * Hq + hq) * 2] = mm;
            stats[((int64_t)s * Hq + hq) * 2 + 1] = lt;
        }
    }
}

// score[row] += sum over query heads of exp(logit - max) / sum. A thread
// takes 4 consecutive rows (16-byte loads of each head's logits), 8 heads'
// loads in flight at a time; the heads' (max, 1/sum) sit in LDS.
constexpr int MASS_ROWS = 4;
constexpr int MASS_HEADS = 8;
__global__ void __launch_bounds__(256) draft_mass_kernel(dkv_drafter_t m, int layer, int Hq,
                                                         const float* __restrict__ logits,
                                                         const float* __restrict__ stats) {
    extern __shared__ float st[];   // [Hq][2]: max, 1 / sum
    const int s = blockIdx.y;
    for (int i = threadIdx.x; i < Hq; i += blockDim.x) {
        const float l = stats[((int64_t)s * Hq + i) * 2 + 1];
        st[2 * i] = stats[((int64_t)s * Hq + i) * 2];
        st[2 * i + 1] = l > 0.0f ? 1.0f / l : 0.0f;
    }
    __syncthreads();
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int r0 = (blockIdx.x * blockDim.x + threadIdx.x) * MASS_ROWS;
    if (r0 >= n) return;
    float mass[MASS_ROWS] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* lg = logits + (int64_t)s * Hq * m.cap + r0;
    for (int h0 = 0; h0 < Hq; h0 += MASS_HEADS) {
        float4 x[MASS_HEADS];
#pragma unroll
        for (int j = 0; j < MASS_HEADS; ++j)
            x[j] = (h0 + j < Hq) ? *reinterpret_cast<const float4*>(lg + (int64_t)(h0 + j) * m.cap)
                                 : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
#pragma unroll
        for (int j = 0; j < MASS_HEADS; ++j) {
            const int hq = min(h0 + j, Hq - 1);
            const float mm = st[2 * hq], il = (h0 + j < Hq) ? st[2 * hq + 1] : 0.0f;
            mass[0] = fmaf(__expf(x[j].x - mm), il, mass[0]);
            mass[1] = fmaf(__expf(x[j].y - mm), il, mass[1]);
            mass[2] = fmaf(__expf(x[j].z - mm), il, mass[2]);
            mass[3] = fmaf(__expf(x[j].w - mm), il, mass[3]);
        }
    }
    double* sc = m.score + row_index(m, s, layer) + r0;
#pragma unroll
    for (int j = 0; j < MASS_ROWS; ++j)
        if (r0 + j < n) sc[j] += static_cast<double>(mass[j]);
}

static size_t smem_bytes(int D) {
    return sizeof(float) * (DQB * D + PAGE * (D + 1) + PAGE * D + DQB * PAGE + 3 * DQB);
}

static bool fast_path(const dkv_drafter_t& m, const dkv_qcfg_t& c, int Hq) {
    const int D = m.head_dim;
    if (c.bits >= 16 || (D != 64 && D != 128) || c.group <= 0 || c.group % 16 != 0 || D % c.group != 0) return false;
    return (Hq / m.n_kv_heads) * (D / c.group) <= 16;
}

}  // namespace dkv

using namespace dkv;

// Workgroups of `fn` (`threads` threads, `lds` bytes of dynamic LDS) the
// device holds at once; kept per kernel (recomputed if the LDS size changes)
struct Resident {
    std::atomic<size_t> lds{0};
    std::atomic<int> blocks{0};
};
static int resident_blocks(const void* fn, int threads, size_t lds, Resident& r) {
    const int b = r.blocks.load(std::memory_order_relaxed);
    if (b > 0 && r.lds.load(std::memory_order_relaxed) == lds) return b;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess || cus <= 0 ||
        per_cu <= 0)
        cus = 256, per_cu = 2;
    r.blocks.store(0, std::memory_order_relaxed);
    r.lds.store(lds, std::memory_order_relaxed);
    r.blocks.store(cus * per_cu, std::memory_order_relaxed);
    return cus * per_cu;
}

static int n_splits_of(const dkv_drafter_t* m, int n_q_heads) {
    const int rps = rows_per_split(*m, n_q_heads / std::max(m->n_kv_heads, 1));
    return (m->cap + rps - 1) / rps;
}

// workspace sections, each starting on a 256-byte boundary: partials
// [b][Hq][splits][D+2], stats [b][Hq][2], logits [b][Hq][cap] and the segment
// kernel's per-KV-head masses [b][Hkv][cap] (with mass)
static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
struct DraftWork {
    size_t stats_off, logits_off, pmass_off, bytes;
};
static DraftWork draft_work(const dkv_drafter_t& m, int n_q_heads, int want_mass) {
    const size_t b = m.batch, D = m.head_dim;
    DraftWork w;
    w.stats_off = align256(sizeof(float) * b * n_q_heads * n_splits_of(&m, n_q_heads) * (D + 2));
    w.logits_off = align256(w.stats_off + sizeof(float) * b * n_q_heads * 2);
    w.pmass_off = align256(w.logits_off + sizeof(float) * b * n_q_heads * (size_t)m.cap);
    w.bytes = want_mass ? w.pmass_off + sizeof(float) * b * m.n_kv_heads * (size_t)m.cap : w.logits_off;
    return w;
}

// Measurement hook: when on, dkv_drafter_attention records a pair of HIP
// events around its split-K kernel on the launch stream, into the next of
// TIMING_PAIRS slots (the last slot is reused once they run out). The events
// skip the system-scope fence: they only order device work on the stream,
// and the fence alone adds ~1.7 us to every timed launch (and slows the
// launches around it).
constexpr int TIMING_PAIRS = 1024;
static bool g_time_splitk = false;
static int g_timed = 0;   // pairs recorded since timing was switched on
static hipEvent_t g_splitk_ev[2][TIMING_PAIRS] = {};

static int timing_slot() { return g_timed < TIMING_PAIRS ? g_timed : TIMING_PAIRS - 1; }

// Launch the split-K kernel, timed when the hook is on: the events ride on
// the kernel's own dispatch (hipExtLaunchKernel), so they bracket its
// execution without marker packets of their own around it.
template <typename... KArgs, typename... Args>
static void launch_splitk(void (*kfn)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
    if (g_time_splitk) {
        const int i = timing_slot();
        hipExtLaunchKernelGGL(kfn, grid, block, (uint32_t)lds, st, g_splitk_ev[0][i], g_splitk_ev[1][i], 0, args...);
        if (g_timed < TIMING_PAIRS) ++g_timed;
    } else {
        hipLaunchKernelGGL(kfn, grid, block, lds, st, args...);
    }
}

extern "C" int dkv_drafter_kernel_timing(int32_t on) {
    if (on && !g_splitk_ev[0][0]) {
        for (int i = 0; i < TIMING_PAIRS; ++i)
            if (hipEventCreateWithFlags(&g_splitk_ev[0][i], hipEventDisableSystemFence) != hipSuccess ||
                hipEventCreateWithFlags(&g_splitk_ev[1][i], hipEventDisableSystemFence) != hipSuccess)
                return fail(DKV_ELAUNCH, "dkv_drafter_kernel_timing: cannot create events");
    }
    if (on) g_timed = 0;
    g_time_splitk = on != 0;
    return DKV_OK;
}

extern "C" float dkv_drafter_kernel_last_ms(void) {
    float ms = -1.0f;
    if (g_timed == 0) return -1.0f;
    const int i = min(g_timed, TIMING_PAIRS) - 1;
    if (hipEventSynchronize(g_splitk_ev[1][i]) != hipSuccess ||
        hipEventElapsedTime(&ms, g_splitk_ev[0][i], g_splitk_ev[1][i]) != hipSuccess)
        return -1.0f;
    return ms;
}

extern "C" float dkv_drafter_kernel_total_ms(int32_t* n_pairs) {
    const int n = min(g_timed, TIMING_PAIRS);
    if (n_pairs) *n_pairs = n;
    if (n == 0) return 0.0f;
    if (hipEventSynchronize(g_splitk_ev[1][n - 1]) != hipSuccess) return -1.0f;
    double total = 0.0;
    for (int i = 0; i < n; ++i) {
        float ms;
        if (hipEventElapsedTime(&ms, g_splitk_ev[0][i], g_splitk_ev[1][i]) != hipSuccess) return -1.0f;
        total += ms;
    }
    return static_cast<float>(total);
}

extern "C" size_t dkv_drafter_attention_workspace(const dkv_drafter_t* mirror, int32_t n_q_heads,
                                                  int32_t want_mass) {
    if (!mirror || n_q_heads <= 0) return 0;
    return draft_work(*mirror, n_q_heads, want_mass).bytes;
}

extern "C" int dkv_drafter_attention(const dkv_drafter_t* mirror, int32_t layer, dkv_qcfg_t cfg, const float* q,
                                     int32_t n_q_heads, int32_t want_mass, float* out, void* work,
                                     size_t work_bytes, dkv_stream_t stream) {
    DKV_REQUIRE(mirror && q && out, "dkv_drafter_attention: NULL argument");
    const dkv_drafter_t m = *mirror;
    DKV_REQUIRE(m.pages && m.n_rows && m.cap > 0 && m.cap % PAGE == 0, "dkv_drafter_attention: bad mirror");
    DKV_REQUIRE(layer >= 0 && layer < m.n_layers, "dkv_drafter_attention: layer out of range");
    DKV_REQUIRE(m.head_dim > 0 && m.head_dim <= DMAXD, "dkv_drafter_attention: head_dim must be 1..128");
    DKV_REQUIRE(n_q_heads > 0 && n_q_heads % m.n_kv_heads == 0 && n_q_heads / m.n_kv_heads <= DQB,
                "dkv_drafter_attention: query heads must be 1..16 per KV head");
    DKV_REQUIRE(cfg.bits >= 16 || cfg.group > 0, "dkv_drafter_attention: bad group");
    DKV_REQUIRE(page_fmt(cfg, m.head_dim).bytes <= m.page_stride,
                "dkv_drafter_attention: arm needs more bytes per page than the mirror reserves");
    const size_t need = dkv_drafter_attention_workspace(mirror, n_q_heads, want_mass);
    if (!work || work_bytes < need)
        return fail(DKV_EWORKSPACE, "dkv_drafter_attention: workspace too small (need " + std::to_string(need) + ")");
    const int G = n_q_heads / m.n_kv_heads;
    const int ns = n_splits_of(mirror, n_q_heads), rps = rows_per_split(m, G);
    const DraftWork wl = draft_work(m, n_q_heads, want_mass);
    float* part = static_cast<float*>(work);
    float* stats = reinterpret_cast<float*>(static_cast<char*>(work) + wl.stats_off);
    float* logits = want_mass ? reinterpret_cast<float*>(static_cast<char*>(work) + wl.logits_off) : nullptr;
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(m.head_dim)));
    hipStream_t st = as_stream(stream);
    bool merged = false;   // the attention kernel merged its partials itself
    int n_parts = ns;   // partial slots written (one per split in the generic kernel)
    int unit = rps;     // rows per unit of work that owns a partial slot
    // One block of 8 waves per (sequence, KV head) segment when the segments
    // alone fill the chip: split-K, merge and the per-KV-head mass in one
    // kernel (4-bit codes, D = 128, 4 query heads and 4 groups per KV head,
    // fp16 meta)
    const bool seg_shape = fast_path(m, cfg, n_q_heads) && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                           cfg.bits <= 4 && m.head_dim == 128 && G == 4 && m.head_dim / cfg.group == 4 &&
                           cfg.meta_f16 && dma_lpp(page_fmt(cfg, 128), 128) == 5;
    const size_t seg_lds = (size_t)SEG_WAVES * dma_stages(5) * 5 * 1024;
    if (seg_shape && m.batch * m.n_kv_heads >= 256) {
        auto kfn = draft_attn_seg_kernel<1, 5, false>;
        static size_t lds_done[16] = {};
        if (!reserve_lds(reinterpret_cast<const void*>(kfn), seg_lds, lds_done))
            return fail(DKV_ELAUNCH, "dkv_drafter_attention: cannot reserve " + std::to_string(seg_lds) + " B of LDS");
        float* pmass = want_mass ? reinterpret_cast<float*>(static_cast<char*>(work) + wl.pmass_off) : nullptr;
        launch_splitk(kfn, dim3(1, m.n_kv_heads, m.batch), dim3(64 * SEG_WAVES), seg_lds, st, m, (int)layer, cfg, q,
                      (int)n_q_heads, scale, out, logits, pmass, 1, static_cast<float*>(nullptr));
        int rc = check_launch("dkv_drafter_attention(segment)");
        if (rc || !want_mass) return rc;
        hipLaunchKernelGGL(draft_mass_sum_kernel, dim3((m.cap + 256 * MSUM_ROWS - 1) / (256 * MSUM_ROWS), m.batch),
                           dim3(256), 0, st, m, layer, pmass);
        return check_launch("dkv_drafter_attention(mass)");
    }
    // Segments too few to fill the chip (small batch, long context): each
    // one cut into nb blocks, at most 256 in all (one block per CU: a second
    // round of blocks would double the time); the blocks' partials and kept
    // values (in the partial and logit sections) are merged, and the mass
    // added, by draft_seg_merge_kernel.
    // (nb is also bounded by the merge kernel's table and by the partial
    // section, which holds ns partials per query head)
    const int nb = std::max(1, std::min(std::min(SMERGE_MAX_NB, ns), 256 / (m.batch * m.n_kv_heads)));
    if (seg_shape && m.n_kv_heads <= SMERGE_MAX_HKV) {
        auto kfn = draft_attn_seg_kernel<1, 5, true>;
        static size_t lds_done[16] = {};
        if (!reserve_lds(reinterpret_cast<const void*>(kfn), seg_lds, lds_done))
            return fail(DKV_ELAUNCH, "dkv_drafter_attention: cannot reserve " + std::to_string(seg_lds) + " B of LDS");
        launch_splitk(kfn, dim3(nb, m.n_kv_heads, m.batch), dim3(64 * SEG_WAVES), seg_lds, st, m, (int)layer, cfg,
                      q, (int)n_q_heads, scale, out, logits, want_mass ? logits : nullptr, nb, part);
        int rc = check_launch("dkv_drafter_attention(segment split)");
        if (rc) return rc;
        const int row_blocks = want_mass ? (m.cap + SMERGE_ROWS - 1) / SMERGE_ROWS : 0;
        hipLaunchKernelGGL(draft_seg_merge_kernel, dim3(m.n_kv_heads + row_blocks, m.batch), dim3(256), 0, st, m,
                           (int)layer, nb, part, logits, out, want_mass);
        return check_launch("dkv_drafter_attention(segment merge)");
    }
    // the fast path reads q rows with 16-byte vector loads
    if (fast_path(m, cfg, n_q_heads) && reinterpret_cast<uintptr_t>(q) % 16 == 0) {
        // blocks of 4 waves; each wave walks splits blockIdx.x*4 + wave, +
        // 4*gridDim.x, ..., so any row count up to cap is covered. Both
        // kernels run one resident round: 512 blocks of the LDS-staged one
        // (8 waves per CU), and for the register-staged one as many as the
        // device holds at once by its registers and LDS (two blocks per CU
        // above 128 VGPRs: 512 at b=32 ctx 32k int8, 359-363 against 365-372
        // us for two rounds of 1024; a round of waves that each take the same
        // number of splits measured 8-10% faster than 1536 blocks)
        const bool dma = cfg.bits <= 4 && m.head_dim == 128;
        const int key = (m.head_dim == 128 ? 4 : 0) | (cfg.bits == 8 ? 2 : 0) | (cfg.meta_f16 ? 1 : 0);
        const void* rk[8] = {reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 4, 0>),
                             reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 4, 1>),
                             reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 8, 0>),
                             reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 8, 1>),
                             nullptr,
                             nullptr,
                             reinterpret_cast<const void*>(draft_attn_mfma_kernel<128, 8, 0>),
                             reinterpret_cast<const void*>(draft_attn_mfma_kernel<128, 8, 1>)};
        const size_t rlds = sizeof(float) * 4 * ((size_t)G * rps + 8 * WAVE);
        static Resident resident[8];
        const int round = dma ? 512 : resident_blocks(rk[key] ? rk[key] : rk[7], 256, rlds, resident[key]);
        const int per_seg = std::max(1, round / std::max(1, m.n_kv_heads * m.batch));
        const dim3 grid(std::min((ns + 3) / 4, per_seg), m.n_kv_heads, m.batch);
        n_parts = 4 * (int)grid.x;   // one partial per wave
        if (dma) {
            n_parts = std::min(n_parts, ns);   // the waves past the partial slots stay idle
            unit = PAGE;
            // 4-bit codes: pages streamed through an LDS ring, S-1 ahead; the
            // kernel is instantiated per loads-per-page count, which fixes its
            // slot size and ring depth (and so the LDS it is given)
            const int LPP = dma_lpp(page_fmt(cfg, 128), 128);
#define DKV_DMA(MM, ST, LP)                                                                                       \
    do {                                                                                                          \
        auto kfn = draft_attn_dma_kernel<128, MM, ST, LP>;                                                        \
        const size_t lds = (size_t)4 * dma_stages(LP) * LP * 1024;                                                \
        static size_t lds_done[16] = {};                                                                         \
        if (!reserve_lds(reinterpret_cast<const void*>(kfn), lds, lds_done))                                      \
            return fail(DKV_ELAUNCH, "dkv_drafter_attention: cannot reserve " + std::to_string(lds) + " B of LDS"); \
        launch_splitk(kfn, grid, dim3(256), lds, st, m, (int)layer, cfg, q, (int)n_q_heads, scale, rps, ns, part, \
                      logits);                                                                                    \
    } while (0)
#define DKV_DMA2(MM, LP)              \
    do {                              \
        if (logits) DKV_DMA(MM, true, LP); \
        else DKV_DMA(MM, false, LP);  \
    } while (0)
            // (meta bytes per section: 32 rows x groups x 4 (f16 pair) or 8 (f32 pair))
            const int key = (cfg.meta_f16 ? 100 : 0) + LPP;
            switch (key) {
                case 105: DKV_DMA2(1, 5); break;   // f16, up to 4 groups
                case 106: DKV_DMA2(1, 6); break;   // f16, 8 groups
                case 5: DKV_DMA2(0, 5); break;     // f32, up to 2 groups
                case 6: DKV_DMA2(0, 6); break;     // f32, 4 groups
                case 8: DKV_DMA2(0, 8); break;     // f32, 8 groups
                default:
                    return fail(DKV_EINVAL, "dkv_drafter_attention: no 4-bit kernel for " + std::to_string(LPP) +
                                                " loads per page");
            }
#undef DKV_DMA2
#undef DKV_DMA
        } else {
            // when one block per (sequence, KV head) segment fills the device,
            // 8-wave blocks (the same waves per segment as two 4-wave blocks)
            // merge their partials in LDS and no combine kernel runs
            const size_t mlds = sizeof(float) * ((size_t)MERGE_WAVES * ((size_t)G * rps + 8 * WAVE) +
                                                 (size_t)G * MERGE_WAVES * (m.head_dim + 2));
            const void* mk[8] = {reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 4, 0, true>),
                                 reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 4, 1, true>),
                                 reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 8, 0, true>),
                                 reinterpret_cast<const void*>(draft_attn_mfma_kernel<64, 8, 1, true>),
                                 nullptr,
                                 nullptr,
                                 reinterpret_cast<const void*>(draft_attn_mfma_kernel<128, 8, 0, true>),
                                 reinterpret_cast<const void*>(draft_attn_mfma_kernel<128, 8, 1, true>)};
            const void* mfn = mk[key] ? mk[key] : mk[7];
            static size_t mlds_done[16] = {};
            static Resident mresident[8];
            merged = reserve_lds(mfn, mlds, mlds_done) &&
                     m.n_kv_heads * m.batch >= resident_blocks(mfn, 64 * MERGE_WAVES, mlds, mresident[key]);
#define DKV_LAUNCH(DD, CC, MM)                                                                                  \
    do {                                                                                                         \
        if (merged)                                                                                              \
            launch_splitk(draft_attn_mfma_kernel<DD, CC, MM, true>, dim3(1, m.n_kv_heads, m.batch),              \
                          dim3(64 * MERGE_WAVES), mlds, st, m, (int)layer, cfg, q, (int)n_q_heads, scale, rps, ns, \
                          part, logits, out, stats);                                                             \
        else                                                                                                     \
            launch_splitk(draft_attn_mfma_kernel<DD, CC, MM>, grid, dim3(256), rlds, st, m, (int)layer, cfg, q,  \
                          (int)n_q_heads, scale, rps, ns, part, logits, out, stats);                             \
    } while (0)
            switch (key) {
                case 0: DKV_LAUNCH(64, 4, 0); break;
                case 1: DKV_LAUNCH(64, 4, 1); break;
                case 2: DKV_LAUNCH(64, 8, 0); break;
                case 3: DKV_LAUNCH(64, 8, 1); break;
                case 6: DKV_LAUNCH(128, 8, 0); break;
                default: DKV_LAUNCH(128, 8, 1); break;
            }
#undef DKV_LAUNCH
        }
    } else {
        launch_splitk(draft_attn_kernel, dim3(ns, m.n_kv_heads, m.batch), dim3(256), smem_bytes(m.head_dim), st, m,
                      (int)layer, cfg, q, (int)n_q_heads, scale, rps, ns, part, logits);
    }
    int rc = check_launch("dkv_drafter_attention");
    if (rc) return rc;
    if (!merged) {
        // one wave of the combine per 8 partials, up to 16 waves
        const int comb_waves = std::min(COMB_WAVES, std::max(1, (std::min(n_parts, ns) + 7) / 8));
        hipLaunchKernelGGL(draft_combine_kernel, dim3(n_q_heads, m.batch), dim3(WAVE * comb_waves), 0, st, m, layer,
                           part, n_q_heads, unit, ns, n_parts, out, stats);
        if ((rc = check_launch("dkv_drafter_attention(combine)"))) return rc;
    }
    if (want_mass) {
        const int per_block = 256 * MASS_ROWS;
        hipLaunchKernelGGL(draft_mass_kernel, dim3((m.cap + per_block - 1) / per_block, m.batch), dim3(256),
                           sizeof(float) * 2 * n_q_heads, st, m, layer, n_q_heads, logits, stats);
        rc = check_launch("dkv_drafter_attention(mass)");
    }
    return rc;
}
