// (a5, a6) Drafter attention over the compressed mirror.
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
//   QK: S'[16 rows][16 cols] = code . Qg^T, where column j = (group g, head
//       h) holds q_h restricted to group g (zero elsewhere), split into f16
//       hi + lo parts. The magic-number conversion (code | 0x6400) gives the
//       exact f16 value 1024 + code in one and/or per two codes; a packed f16
//       subtract removes the 1024 exactly. Folding scale and zero in fp32 per
//       (row, group) and summing the group columns of a head gives its logit:
//         s_h = sum_g scale_g * S'[g,h] + lo_g * sum_{d in g} q_h[d]
//   PV: O'[16 d][16 cols] = (1024 + code_V)^T . B with B[row][(g,h)] =
//       f16(p_h[row] * scaleV_g[row]); then
//         o_h[d] = O'[d][(g(d),h)] - 1024 * sum_rows B + sum_rows p_h * loV_g
// The accumulator lanes of the QK product already hold the 8 rows of one
// column that the PV B operand needs, so probabilities never move between
// lanes; the V page layout (mirror_layout.h) is the PV A operand.
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

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// 8 codes of one word (cb 4) or two words (cb 8) -> f16 (1024 + code) x 8
template <int CB>
__device__ __forceinline__ f16x8_t codes_to_f16(const uint32_t* w, uint32_t magic);

// the same codes as exact f16 integers (one packed f16 subtract per pair):
// the QK fold multiplies by the group scale, so an uncancelled 1024 offset
// would cost precision when scales are large
template <int CB>
__device__ __forceinline__ f16x8_t codes_to_f16_exact(const uint32_t* w, uint32_t magic) {
    f16x8_t x = codes_to_f16<CB>(w, magic);
    const f16x2_t off = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f16x2_t p = {x[2 * i], x[2 * i + 1]};
        p = p - off;
        x[2 * i] = p[0];
        x[2 * i + 1] = p[1];
    }
    return x;
}

// (x & mask) | 0x64006400. Written as a bitfield insert of x into an opaque
// copy of the constant, so it becomes one v_bfi_b32 instead of an and + or
// (the constant would otherwise fold and the pattern be lost).
__device__ __forceinline__ uint32_t magic_f16x2() {
    uint32_t y;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(y));
    return y;
}
__device__ __forceinline__ uint32_t and_or_magic(uint32_t x, uint32_t mask, uint32_t magic) {
    return (x & mask) | (magic & ~mask);
}

template <int CB>
__device__ __forceinline__ f16x8_t codes_to_f16(const uint32_t* w, uint32_t magic) {
    uint4 r;
    if (CB == 4) {
        const uint32_t x = w[0];
        r.x = and_or_magic(x, 0x000F000Fu, magic);
        r.y = and_or_magic(x >> 4, 0x000F000Fu, magic);
        r.z = and_or_magic(x >> 8, 0x000F000Fu, magic);
        r.w = and_or_magic(x >> 12, 0x000F000Fu, magic);
    } else {
        r.x = and_or_magic(w[0], 0x00FF00FFu, magic);
        r.y = and_or_magic(w[0] >> 8, 0x00FF00FFu, magic);
        r.z = and_or_magic(w[1], 0x00FF00FFu, magic);
        r.w = and_or_magic(w[1] >> 8, 0x00FF00FFu, magic);
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
__device__ __forceinline__ void load_words(uint32_t (&dst)[N], const uint32_t* src) {
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
        for (int x = 0; x < N; ++x) dst[x] = src[x];
    }
}

template <int MF>
__device__ __forceinline__ GroupMeta pair_of(const uint32_t* w, int k) {
    if (MF) return {half_bits_to_f32(w[k] & 0xffffu), half_bits_to_f32(w[k] >> 16)};
    return {__uint_as_float(w[2 * k]), __uint_as_float(w[2 * k + 1])};
}

template <int D, int CB, int MF>
__device__ __forceinline__ void load_page(PageRegs<D, CB, MF>& r, const uint8_t* pg, const PageFmt& f, int col, int jj,
                                          int gmeta) {
    using R = PageRegs<D, CB, MF>;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        load_words(r.k[a], reinterpret_cast<const uint32_t*>(pg + f.kc + (int64_t)(16 * a + col) * (D * CB / 8)) +
                               R::WPL * jj);
        load_words(r.km[a], reinterpret_cast<const uint32_t*>(pg + k_meta_off(f, 16 * a + 4 * jj, gmeta)));
    }
    load_words(r.v, reinterpret_cast<const uint32_t*>(pg + f.vc) + (col * 4 + jj) * R::NV);
    load_words(r.vm, reinterpret_cast<const uint32_t*>(pg + f.vm + ((int64_t)gmeta * PAGE + jj * 8) * f.metaB));
}

// Column offsets of group g within a 16-lane row (see the kernel): the
// subgroup of lane XORs generated by 15, 7 and 3, in butterfly order.
__constant__ int kColXor[8] = {0, 15, 7, 8, 3, 12, 4, 11};

// value of lane (l ^ mask) of the same 16-lane row, through a DPP move
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int D, int CB, int MF>
__global__ void __launch_bounds__(256) draft_attn_mfma_kernel(dkv_drafter_t m, int layer, dkv_qcfg_t cfg,
                                                              const float* __restrict__ q, int Hq, float scale,
                                                              int rps, int n_splits, float* __restrict__ part,
                                                              float* __restrict__ logits) {
    constexpr int NSTEP = D / 32;     // k-steps of the QK product
    constexpr int NDT = D / 16;       // d-tiles of the PV product
    constexpr int DL = D / 4;         // channels per lane group in QK
    // the wave index through readfirstlane: the compiler then knows it (and
    // the split, row range and page addresses) to be wave-uniform, keeps them
    // in scalar registers and runs the page loop as a scalar loop
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int split = blockIdx.x * 4 + wave;
    if (split >= n_splits) return;
    const int h = blockIdx.y, s = blockIdx.z;
    const int G = Hq / m.n_kv_heads;
    const int group = cfg.group, NG = D / group, ncol = G * NG;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int r_begin = split * rps;
    if (r_begin >= n) return;
    const int r_end = min(r_begin + rps, n);
    const PageFmt f = page_fmt(cfg, D);
    const int col = lane % 16, jj = lane / 16;
    // column col = hcol ^ kColXor[gcol]: the NG columns of a head form an
    // orbit of the lane involutions row_mirror (^15), row_half_mirror (^7) and
    // quad reverse (^3), so their sum is a butterfly of DPP adds that leaves
    // the bitwise-same total in every column of the head
    int gcol = 0, hcol = 0;
    bool cvalid = false;
    for (int g = 0; g < NG; ++g) {
        const int hh = col ^ kColXor[g];
        if (hh < G) {
            gcol = g;
            hcol = hh;
            cvalid = true;
        }
    }
    (void)ncol;
    const int hq = h * G + hcol;
    const int gmeta = min(gcol, NG - 1);

    // Q^T columns (group, head) in f16 hi + lo, and the column's q sum
    f16x8_t qhi[NSTEP], qlo[NSTEP];
    float qsum = 0.0f;
    {
        // the lane's DL channels as DL/4 vector loads, all in flight at once
        // (hq is a valid head for every lane); the column's group mask is a
        // bit mask, so the loads stay unconditional
        const float4* qr = reinterpret_cast<const float4*>(q + ((int64_t)s * Hq + hq) * D + DL * jj);
        float4 qv[DL / 4];
#pragma unroll
        for (int x = 0; x < DL / 4; ++x) qv[x] = qr[x];
#pragma unroll
        for (int st = 0; st < NSTEP; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = DL * jj + 8 * st + e;
                const float4 w4 = qv[(8 * st + e) / 4];
                const float raw = (e % 4 == 0) ? w4.x : (e % 4 == 1) ? w4.y : (e % 4 == 2) ? w4.z : w4.w;
                const uint32_t keep = (cvalid && d / group == gcol) ? 0xFFFFFFFFu : 0u;
                const float v = __uint_as_float(__float_as_uint(raw) & keep);
                const _Float16 hi = (_Float16)v;
                const _Float16 lo = (_Float16)(v - (float)hi);
                qhi[st][e] = hi;
                qlo[st][e] = lo;
                qsum += (float)hi + (float)lo;
            }
        qsum += __shfl_xor(qsum, 16);
        qsum += __shfl_xor(qsum, 32);
    }
    f32x4_t acc[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f, bsum = 0.0f, zsum = 0.0f;

    const uint32_t magic = magic_f16x2();
    const uint32_t use2 = NG >= 2 ? 0xFFFFFFFFu : 0u, use4 = NG >= 4 ? 0xFFFFFFFFu : 0u,
                   use8 = NG >= 8 ? 0xFFFFFFFFu : 0u;
    // Logit spill through a buffer resource over this sequence's logits: lanes
    // with nothing to store get an offset past the end, which the hardware
    // drops, so the store needs no branch (a branch would split the loop body
    // and let the compiler sink the next page's loads to their use).
    // Logits for note_attention are staged in this wave's LDS region
    // [head][row - r_begin] (lanes with nothing to keep write a dummy slot),
    // so the loop issues no memory stores; they go out after the split.
    extern __shared__ float dyn_smem[];
    float* slog = dyn_smem + wave * (G * rps + WAVE);
    // one page of work on registers already loaded
    auto step = [&](const PageRegs<D, CB, MF>& cur, const int p0) {
        // ---- QK over the page's two 16-row tiles, folded per (row, group)
        float sv[8];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            f32x4_t sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < NSTEP; ++st) {
                const f16x8_t kv = codes_to_f16_exact<CB>(cur.k[a] + st * (CB / 4), magic);
                sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qhi[st], sa, 0, 0, 0);
                sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qlo[st], sa, 0, 0, 0);
            }
            // columns outside every (group, head) pair have q = 0 and stay
            // finite; rows past the live count are masked below
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const GroupMeta mt = pair_of<MF>(cur.km[a], r);
                sv[4 * a + r] = fmaf(mt.scale, sa[r], mt.lo * qsum);
            }
        }
        // sum the group columns of each head (pairwise butterfly over the
        // orbit); a step the group count does not use adds +0 (masked bits,
        // no branch)
        float sh[8];
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            float v = sv[x];
            v += __uint_as_float(__float_as_uint(dpp_f32<0x140>(v)) & use2);   // row_mirror: col ^ 15
            v += __uint_as_float(__float_as_uint(dpp_f32<0x141>(v)) & use4);   // row_half_mirror: col ^ 7
            v += __uint_as_float(__float_as_uint(dpp_f32<0x1B>(v)) & use8);    // quad [3,2,1,0]: col ^ 3
            sh[x] = v;
        }
        // mask, scale, optional spill, online softmax per column
        float pv[8];
        float mx = -INFINITY;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            const int row = p0 + 16 * (x / 4) + 4 * jj + (x % 4);
            const bool ok = row < r_end;
            const float v = ok ? sh[x] * scale : -INFINITY;
            slog[(ok && cvalid && gcol == 0) ? hcol * rps + (row - r_begin) : G * rps + lane] = v;
            pv[x] = v;
            mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // Lazy rescale: the reference max only moves when a column's max grows
        // by more than 6 (so p <= e^6); o, l and the corrections share the
        // reference, and the combine merges partials on any reference.
        const bool grow = mx > m_run + 6.0f;
        if (__any(grow)) {
            const float m_new = grow ? mx : m_run;
            const float alpha = (m_run == -INFINITY) ? 0.0f : __expf(m_run - m_new);
            l_run *= alpha;
            bsum *= alpha;
            zsum *= alpha;
#pragma unroll
            for (int t = 0; t < NDT; ++t) acc[t] *= alpha;
            m_run = m_new;
        }
        // m_run is finite from the first page on (every split starts with a
        // live row), so masked rows give exp(-inf) = 0 with no test
        float sum = 0.0f;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            pv[x] = __expf(pv[x] - m_run);
            sum += pv[x];
        }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        l_run += sum;
        // ---- PV: B[row (jj, e)][col] = f16(p * scaleV), rows e<4: 4jj+e, e>=4: 16+4jj+e-4
        f16x8_t bop;
        float bs = 0.0f, zs = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const GroupMeta mt = pair_of<MF>(cur.vm, e);
            const int row = p0 + (e < 4 ? 4 * jj + e : 16 + 4 * jj + e - 4);
            // rows past the live count may hold stale meta: zero it (p is 0 there)
            const bool ok = row < r_end;
            const float sc = ok ? mt.scale : 0.0f, lo = ok ? mt.lo : 0.0f;
            _Float16 b = (_Float16)(pv[e] * sc);
            // pin the rounded f16: the correction -1024 * sum(b) cancels the
            // MFMA's 1024 offset only if it adds exactly the operand's bits
            asm volatile("" : "+v"(b));
            bop[e] = b;
            bs += (float)b;
            zs += pv[e] * lo;
        }
        bsum += bs;
        zsum += zs;
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
            const f16x8_t av = codes_to_f16<CB>(cur.v + t * (CB / 4), magic);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bop, acc[t], 0, 0, 0);
        }
    };
    const int np = (r_end - r_begin + PAGE - 1) / PAGE;
    const int pg0 = r_begin / PAGE;
    auto fetch = [&](PageRegs<D, CB, MF>& b, int k) {
        // past the last page, reload the last one (no branch around the loads)
        load_page(b, page_ptr(m, s, layer, h, pg0 + min(k, np - 1)), f, col, jj, gmeta);
    };
    // page k+1 is in flight while page k is computed (two buffers, unrolled by 2)
    // The scheduling barriers keep each fetch ahead of the page's products:
    // left alone, the scheduler sinks the loads into the QK MFMAs, so the
    // next page's latency hides behind half a page instead of a whole one.
    PageRegs<D, CB, MF> b0, b1;
    fetch(b0, 0);
    for (int k = 0; k < np; k += 2) {
        fetch(b1, k + 1);
        __builtin_amdgcn_sched_barrier(0);
        step(b0, r_begin + k * PAGE);
        if (k + 1 >= np) break;
        fetch(b0, k + 2);
        __builtin_amdgcn_sched_barrier(0);
        step(b1, r_begin + (k + 1) * PAGE);
    }
    // staged logits of the split's rows, one coalesced pass per query head
    if (logits) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int nr = r_end - r_begin;
        for (int i = lane; i < G * nr; i += WAVE) {
            const int g = i / nr, r = i % nr;
            logits[((int64_t)s * Hq + h * G + g) * m.cap + r_begin + r] = slog[g * rps + r];
        }
    }
    // totals of the per-column corrections over the 4 lane groups
    bsum += __shfl_xor(bsum, 16);
    bsum += __shfl_xor(bsum, 32);
    zsum += __shfl_xor(zsum, 16);
    zsum += __shfl_xor(zsum, 32);
    if (!cvalid) return;
    float* pp = part + (((int64_t)s * Hq + hq) * n_splits + split) * (D + 2);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
        if ((16 * t) / group != gcol) continue;   // this column's group covers tile t
#pragma unroll
        for (int r = 0; r < 4; ++r) pp[16 * t + 4 * jj + r] = acc[t][r] - 1024.0f * bsum + zsum;
    }
    if (gcol == 0 && jj == 0) {
        pp[D] = m_run;
        pp[D + 1] = l_run;
    }
}

// ---------------------------------------------------------------- combine + mass
// merge splits per (seq, query head); also records the final (max, sum)
__global__ void __launch_bounds__(128) draft_combine_kernel(dkv_drafter_t m, int layer, const float* __restrict__ part,
                                                            int Hq, int rps, int n_splits, float* __restrict__ out,
                                                            float* __restrict__ stats) {
    const int hq = blockIdx.x, s = blockIdx.y;
    const int D = m.head_dim;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int ns = min((n + rps - 1) / rps, n_splits);
    const float* p = part + ((int64_t)s * Hq + hq) * n_splits * (D + 2);
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float mm = -INFINITY, l = 0.0f, o = 0.0f;
        for (int c = 0; c < ns; ++c) {
            const float* pc = p + (int64_t)c * (D + 2);
            const float mc = pc[D], lc = pc[D + 1];
            const float mn = fmaxf(mm, mc);
            const float a = (mm == -INFINITY) ? 0.0f : __expf(mm - mn);
            const float b = (mc == -INFINITY) ? 0.0f : __expf(mc - mn);
            l = l * a + lc * b;
            o = o * a + pc[d] * b;
            mm = mn;
        }
        out[((int64_t)s * Hq + hq) * D + d] = (l > 0.0f) ? o / l : 0.0f;
        if (d == 0 && stats) {
            stats[((int64_t)s * Hq + hq) * 2] = mm;
            stats[((int64_t)s * Hq + hq) * 2 + 1] = l;
        }
    }
}

// score[row] += sum over query heads of exp(logit - max) / sum. A thread
// takes 4 consecutive rows (16-byte loads of each head's logits); the heads'
// (max, sum) sit in LDS.
constexpr int MASS_ROWS = 4;
__global__ void __launch_bounds__(256) draft_mass_kernel(dkv_drafter_t m, int layer, int Hq,
                                                         const float* __restrict__ logits,
                                                         const float* __restrict__ stats) {
    extern __shared__ float st[];   // [Hq][2]
    const int s = blockIdx.y;
    for (int i = threadIdx.x; i < 2 * Hq; i += blockDim.x) st[i] = stats[(int64_t)s * Hq * 2 + i];
    __syncthreads();
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int r0 = (blockIdx.x * blockDim.x + threadIdx.x) * MASS_ROWS;
    if (r0 >= n) return;
    float mass[MASS_ROWS] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* lg = logits + (int64_t)s * Hq * m.cap + r0;
    for (int hq = 0; hq < Hq; ++hq) {
        const float mm = st[2 * hq], l = st[2 * hq + 1];
        const float4 x = *reinterpret_cast<const float4*>(lg + (int64_t)hq * m.cap);
        mass[0] += __expf(x.x - mm) / l;
        mass[1] += __expf(x.y - mm) / l;
        mass[2] += __expf(x.z - mm) / l;
        mass[3] += __expf(x.w - mm) / l;
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

static int n_splits_of(const dkv_drafter_t* m, int n_q_heads) {
    const int rps = rows_per_split(*m, n_q_heads / std::max(m->n_kv_heads, 1));
    return (m->cap + rps - 1) / rps;
}

// workspace sections, each starting on a 256-byte boundary: partials
// [b][Hq][splits][D+2], stats [b][Hq][2], logits [b][Hq][cap] (with mass)
static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
struct DraftWork {
    size_t stats_off, logits_off, bytes;
};
static DraftWork draft_work(const dkv_drafter_t& m, int n_q_heads, int want_mass) {
    const size_t b = m.batch, D = m.head_dim;
    DraftWork w;
    w.stats_off = align256(sizeof(float) * b * n_q_heads * n_splits_of(&m, n_q_heads) * (D + 2));
    w.logits_off = align256(w.stats_off + sizeof(float) * b * n_q_heads * 2);
    w.bytes = want_mass ? w.logits_off + sizeof(float) * b * n_q_heads * (size_t)m.cap : w.logits_off;
    return w;
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
    // the fast path reads q rows with 16-byte vector loads
    if (fast_path(m, cfg, n_q_heads) && reinterpret_cast<uintptr_t>(q) % 16 == 0) {
        const dim3 grid((ns + 3) / 4, m.n_kv_heads, m.batch);
        const int key = (m.head_dim == 128 ? 4 : 0) | (cfg.bits == 8 ? 2 : 0) | (cfg.meta_f16 ? 1 : 0);
        const size_t lds = sizeof(float) * 4 * ((size_t)G * rps + WAVE);
#define DKV_LAUNCH(DD, CC, MM)                                                                                      \
    hipLaunchKernelGGL((draft_attn_mfma_kernel<DD, CC, MM>), grid, dim3(256), lds, st, m, layer, cfg, q, n_q_heads, \
                       scale, rps, ns, part, logits)
        switch (key) {
            case 0: DKV_LAUNCH(64, 4, 0); break;
            case 1: DKV_LAUNCH(64, 4, 1); break;
            case 2: DKV_LAUNCH(64, 8, 0); break;
            case 3: DKV_LAUNCH(64, 8, 1); break;
            case 4: DKV_LAUNCH(128, 4, 0); break;
            case 5: DKV_LAUNCH(128, 4, 1); break;
            case 6: DKV_LAUNCH(128, 8, 0); break;
            default: DKV_LAUNCH(128, 8, 1); break;
        }
#undef DKV_LAUNCH
    } else {
        hipLaunchKernelGGL(draft_attn_kernel, dim3(ns, m.n_kv_heads, m.batch), dim3(256), smem_bytes(m.head_dim), st,
                           m, layer, cfg, q, n_q_heads, scale, rps, ns, part, logits);
    }
    int rc = check_launch("dkv_drafter_attention");
    if (rc) return rc;
    hipLaunchKernelGGL(draft_combine_kernel, dim3(n_q_heads, m.batch), dim3(128), 0, st, m, layer, part, n_q_heads,
                       rps, ns, out, stats);
    if ((rc = check_launch("dkv_drafter_attention(combine)"))) return rc;
    if (want_mass) {
        const int per_block = 256 * MASS_ROWS;
        hipLaunchKernelGGL(draft_mass_kernel, dim3((m.cap + per_block - 1) / per_block, m.batch), dim3(256),
                           sizeof(float) * 2 * n_q_heads, st, m, layer, n_q_heads, logits, stats);
        rc = check_launch("dkv_drafter_attention(mass)");
    }
    return rc;
}
