// Paged full-cache append and causal attention over it.
// Reference: draftkv/paged.py:76-176 (cache), draftkv/llama.py:202-218 and
// gpt2.py/model.py equivalents (read + masked softmax attention).
#include <algorithm>

#include "dkv_common.h"

namespace dkv {

// ---------------------------------------------------------------- append
__global__ void __launch_bounds__(256) paged_append_kernel(dkv_paged_t c, int layer, const void* __restrict__ k,
                                                           const void* __restrict__ v, int in_dtype, int T,
                                                           const int32_t* __restrict__ start,
                                                           const int32_t* __restrict__ count) {
    const int t = blockIdx.x, s = blockIdx.y;
    if (count && t >= count[s]) return;
    const int pos = start[s] + t;
    const int32_t blk = paged_block(c, s, layer, pos);
    const int off = pos % c.block_size;
    const int HD = c.n_kv_heads * c.head_dim;
    const int64_t src = ((int64_t)s * T + t) * HD;
    for (int i = threadIdx.x; i < HD; i += blockDim.x) {
        const int h = i / c.head_dim, d = i % c.head_dim;
        const float kv = load_elem(k, src + i, in_dtype);
        const float vv = load_elem(v, src + i, in_dtype);
        const int64_t ko = paged_k_off(c, blk, off, h, d), vo = paged_v_off(c, blk, off, h, d);
        if (c.dtype == DKV_BF16) {
            static_cast<uint16_t*>(c.pool)[ko] = f32_to_bf16_rne(kv);
            static_cast<uint16_t*>(c.pool)[vo] = f32_to_bf16_rne(vv);
        } else {
            static_cast<float*>(c.pool)[ko] = kv;
            static_cast<float*>(c.pool)[vo] = vv;
        }
    }
}

// ---------------------------------------------------------------- attention
// Grid: x = chunk * n_qtiles + qtile, y = kv head, z = sequence.
// A block owns QB query rows (query row r -> step t = r / G, head h*G + r%G)
// and the keys [chunk*CH, min((chunk+1)*CH, len)). Keys are walked in tiles
// of KT at fixed absolute offsets; per query row the arithmetic (dot order,
// tile max/sum order, rescale sequence) depends only on absolute key indices,
// never on T or on how many rows share the block, so a row's partial is
// bit-identical whether it is computed in a verify pass (T = gamma+1) or in a
// one-token decode step. Masked keys contribute exact zeros. The cache ends
// at start + count (count null: all T rows were appended); positions past it
// are never read as keys -- their pages may hold stale bytes, and 0 * NaN is
// NaN -- and a padding row (t >= count) attends over the whole cache.
constexpr int QB = 16;
constexpr int KT = 32;
constexpr int MAXD = 128;   // LDS tiles stay under 64 KB

__global__ void __launch_bounds__(256) paged_attn_kernel(dkv_paged_t c, int layer, const float* __restrict__ q,
                                                         int T, int Hq, const int32_t* __restrict__ start,
                                                         const int32_t* __restrict__ count, int CH, int n_chunks,
                                                         int n_qtiles, float scale, float* __restrict__ part) {
    const int chunk = blockIdx.x / n_qtiles, qtile = blockIdx.x % n_qtiles;
    const int h = blockIdx.y, s = blockIdx.z;
    const int D = c.head_dim, G = Hq / c.n_kv_heads;
    const int s0 = start[s];
    const int len = s0 + (count ? count[s] : T);  // cache holds positions 0..len-1
    const int k_begin = chunk * CH;
    if (k_begin >= len) return;
    const int k_end = min(k_begin + CH, len);
    const int n_rows = T * G;
    const int r0 = qtile * QB;
    if (r0 >= n_rows) return;
    const int nr = min(QB, n_rows - r0);
    // last key any of this block's rows may see
    const int max_qpos = s0 + (r0 + nr - 1) / G;
    if (k_begin > max_qpos) return;

    extern __shared__ float smem[];
    float* sQ = smem;                               // [QB][D]
    float* sK = sQ + QB * D;                        // [KT][D+1]
    float* sV = sK + KT * (D + 1);                  // [KT][D]
    float* sS = sV + KT * D;                        // [QB][KT]
    float* sM = sS + QB * KT;                       // [QB] running max
    float* sL = sM + QB;                            // [QB] running sum
    float* sA = sL + QB;                            // [QB] rescale factor of this tile

    const int tid = threadIdx.x;
    for (int i = tid; i < QB * D; i += blockDim.x) {
        const int r = i / D, d = i % D;
        float val = 0.0f;
        if (r < nr) {
            const int rr = r0 + r, t = rr / G, hq = h * G + rr % G;
            val = q[(((int64_t)s * T + t) * Hq + hq) * D + d];
        }
        sQ[i] = val;
    }
    if (tid < QB) {
        sM[tid] = -INFINITY;
        sL[tid] = 0.0f;
    }
    // accumulators: outputs o = tid + 256*j (row o / D, dim o % D)
    constexpr int MAXACC = QB * MAXD / 256;
    float acc[MAXACC];
#pragma unroll
    for (int j = 0; j < MAXACC; ++j) acc[j] = 0.0f;
    const int n_out = QB * D;

    const int kend_eff = min(k_end, max_qpos + 1);
    for (int kt = k_begin; kt < kend_eff; kt += KT) {
        __syncthreads();
        // load K and V tiles (keys kt .. kt+KT-1, zero past the cache)
        for (int i = tid; i < KT * D; i += blockDim.x) {
            const int j = i / D, d = i % D;
            const int pos = kt + j;
            float kv = 0.0f, vv = 0.0f;
            if (pos < len) {
                const int32_t blk = paged_block(c, s, layer, pos);
                const int off = pos % c.block_size;
                kv = load_elem(c.pool, paged_k_off(c, blk, off, h, d), c.dtype);
                vv = load_elem(c.pool, paged_v_off(c, blk, off, h, d), c.dtype);
            }
            sK[j * (D + 1) + d] = kv;
            sV[j * D + d] = vv;
        }
        __syncthreads();
        // scores
        for (int i = tid; i < QB * KT; i += blockDim.x) {
            const int r = i / KT, j = i % KT;
            const int pos = kt + j;
            float sc = -INFINITY;
            if (r < nr) {
                const int qpos = s0 + (r0 + r) / G;
                if (pos <= qpos && pos < len) {
                    float dot = 0.0f;
                    for (int d = 0; d < D; ++d) dot = fmaf(sQ[r * D + d], sK[j * (D + 1) + d], dot);
                    sc = dot * scale;
                }
            }
            sS[i] = sc;
        }
        __syncthreads();
        // online softmax per row: 16 lanes per row, fixed reduction tree
        {
            const int r = tid / 16, l16 = tid % 16;   // 256 threads = QB rows x 16
            float mx = -INFINITY;
            for (int j = l16; j < KT; j += 16) mx = fmaxf(mx, sS[r * KT + j]);
            for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
            const float m_old = sM[r];
            const float m_new = fmaxf(m_old, mx);
            float sum = 0.0f;
            for (int j = l16; j < KT; j += 16) {
                const float sc = sS[r * KT + j];
                const float p = (sc == -INFINITY) ? 0.0f : __expf(sc - m_new);
                sS[r * KT + j] = p;
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
        // PV
#pragma unroll
        for (int jj = 0; jj < MAXACC; ++jj) {
            const int o = tid + 256 * jj;
            if (o < n_out) {
                const int r = o / D, d = o % D;
                float a = acc[jj] * sA[r];
                for (int j = 0; j < KT; ++j) a = fmaf(sS[r * KT + j], sV[j * D + d], a);
                acc[jj] = a;
            }
        }
    }
    __syncthreads();
    // write partials: [((s*T + t)*Hq + hq) * n_chunks + chunk] * (D + 2)
#pragma unroll
    for (int jj = 0; jj < MAXACC; ++jj) {
        const int o = tid + 256 * jj;
        if (o < n_out) {
            const int r = o / D, d = o % D;
            if (r < nr) {
                const int rr = r0 + r, t = rr / G, hq = h * G + rr % G;
                float* p = part + ((((int64_t)s * T + t) * Hq + hq) * n_chunks + chunk) * (D + 2);
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
// bf16 cache with 16-token blocks, D = 64 or 128. A workgroup owns one
// (sequence, KV head, key chunk) and W q-tiles of 16 query rows, one wave per
// q-tile, and walks the chunk 32 keys (two blocks) per step:
//   S^T[16 keys][16 rows] = K[16 keys][D] . Q^T     (v_mfma_f32_16x16x32_bf16)
//   O^T[16 d][16 rows]   += V^T[16 d][32 keys] . P^T
// Q and P are split into bf16 hi + lo parts (two MFMAs each), which keeps the
// products at ~16 mantissa bits against the exact bf16 K/V. In the S^T
// accumulator a lane holds keys 4*(l/16)+r of one query row l%16; the PV
// B operand wants 8 keys of one row per lane, so the k-slots of the PV
// product are ordered {4j..4j+3, 16+4j..16+4j+3} (j = l/16) and the
// probabilities never leave their lane. In k-step st of the QK product lane
// group j holds d in [32 st + 8 j, +8), so a step's K load reads 64
// contiguous bytes of each key row.
//
// Staging. The K and V of a step go to LDS through direct-to-LDS loads
// (global_load_lds_dwordx4), VERIFY_STAGES steps deep, so HBM latency hides
// behind the products of earlier steps without holding registers, and the
// workgroup reads each byte of its chunk from HBM once whatever the number
// of q-tiles. K lands in the order of the QK A operand (slot (tile, k-step)
// = 1 KB, 16 B per lane), so an operand read is one conflict-free
// ds_read_b128; V keeps the block's V^T layout [d][16 keys]. The loads are
// issued from inline asm and waited for by hand (s_waitcnt vmcnt + s_barrier):
// the compiler's own tracking of LDS DMA would make every LDS read wait for
// all loads in flight, prefetches included.
//
// Every per-row operation depends only on absolute key positions (keys past a
// row's position add exact zeros, with the rescale factor exactly 1), and
// floating-point contraction is off, so a row's partial is bit-identical for
// any T and any W (batch invariance between verify and decode).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// round to nearest even in hardware (v_cvt_pk_bf16_f32); the split operands
// are finite, where this equals the integer rounding of f32_to_bf16_rne
__device__ __forceinline__ __bf16 to_bf16(float f) { return (__bf16)f; }
__device__ __forceinline__ float from_bf16(__bf16 h) { return (float)h; }

template <int D>
struct VerifyStage {
    static constexpr int NSTEP = D / 32;               // k-steps of the QK product
    static constexpr int K_BYTES = 2 * NSTEP * 1024;   // two 16-key tiles, operand order
    static constexpr int V_BLOCK = D * 16 * 2;         // one block's V^T of one head
    static constexpr int NVI = V_BLOCK / 1024;         // 1 KB loads per V block
    static constexpr int NI = 2 * NSTEP + 2 * NVI;     // 1 KB loads per step
    static constexpr int BYTES = K_BYTES + 2 * V_BLOCK;
};
constexpr int VERIFY_STAGES = 2;

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from g to LDS byte address lds + 16 * lane (m0 = base),
// non-temporal: the K/V stream is read once, and every load instruction
// reads whole 64-byte segments (a K load takes 64 contiguous bytes of each
// of 16 rows, a V load 1 KB), so no line is split between loads -- on split
// lines the non-temporal policy refetched them and ran ~15% slower; on whole
// ones it streams faster than the default (b=32 ctx 32k decode: 719 -> 672 us)
__device__ __forceinline__ void dma_b128(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// at most N of this wave's loads still in flight, its LDS reads done, then
// the workgroup barrier
template <int N>
__device__ __forceinline__ void wait_loads_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// keys at or past the cache end read as zero (their probability is 0, and
// 0 * garbage could be NaN): mask of the 4 bf16 keys starting nv before it
__device__ __forceinline__ uint64_t key_mask4(int nv) {
    return nv >= 4 ? ~0ull : nv <= 0 ? 0ull : (1ull << (16 * nv)) - 1ull;
}

template <int D, int W>
__global__ void __launch_bounds__(64 * W) paged_attn_mfma_kernel(dkv_paged_t c, int layer, const float* __restrict__ q,
                                                                 int T, int Hq, const int32_t* __restrict__ start,
                                                                 const int32_t* __restrict__ count, int CH,
                                                                 int n_qgroups, int n_chunks, int n_qtiles,
                                                                 float scale, float* __restrict__ part) {
#pragma clang fp contract(off)
    using St = VerifyStage<D>;
    constexpr int S = VERIFY_STAGES;
    constexpr int NSTEP = St::NSTEP;
    constexpr int NDT = D / 16;        // d-tiles of the PV product
    constexpr int LPW = St::NI / W;    // loads per wave per step
    static_assert(St::NI % W == 0, "a step's loads split evenly over the waves");
    // wave index through readfirstlane: the q-tile and everything derived
    // from it are then wave-uniform (scalar registers and branches)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    // grid (q-group, head x sequence, chunk): the chunk is the slowest index, so
    // the workgroups of the full chunks are dispatched first and the short
    // last chunk fills the tail instead of splitting a round
    const int qg = blockIdx.x, chunk = blockIdx.z;
    const int h = blockIdx.y % c.n_kv_heads, s = blockIdx.y / c.n_kv_heads;
    const int G = Hq / c.n_kv_heads;
    const int s0 = start[s];
    const int len = s0 + (count ? count[s] : T);
    const int k_begin = chunk * CH;
    const int n_rows = T * G;
    // the group's last row bounds the keys any of its rows may see
    const int last_row = min((qg + 1) * W * 16, n_rows) - 1;
    const int max_qpos = s0 + last_row / G;
    if (k_begin >= len || k_begin > max_qpos) return;   // uniform over the workgroup
    const int k_end = min(min(k_begin + CH, len), max_qpos + 1);
    const int nsteps = (k_end - k_begin + 31) / 32;
    const int qtile = qg * W + wave;
    const bool active = qtile < n_qtiles;               // wave-uniform
    const int col = lane % 16, jj = lane / 16;
    const int r = qtile * 16 + col;
    const bool rvalid = active && r < n_rows;
    const int t = rvalid ? r / G : 0;
    const int hq = h * G + (rvalid ? r % G : 0);
    const int qpos = s0 + t;

    extern __shared__ __align__(16) char lds[];
    // block ids of the keys [k_begin, min(k_begin + 32 * nsteps, len))
    int32_t* sblk = reinterpret_cast<int32_t*>(lds + S * St::BYTES);
    {
        const int32_t* btab = c.block_table + ((int64_t)s * c.n_layers + layer) * c.max_blocks + k_begin / 16;
        const int nblk = (min(k_begin + 32 * nsteps, len) - k_begin + 15) / 16;
        for (int i = threadIdx.x; i < nblk; i += 64 * W) sblk[i] = btab[i];
    }

    bf16x8_t qhi[NSTEP], qlo[NSTEP];
    {
        const float* qr = q + (((int64_t)s * T + t) * Hq + hq) * D + 8 * jj;
#pragma unroll
        for (int st = 0; st < NSTEP; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = rvalid ? qr[32 * st + e] : 0.0f;
                const __bf16 hi = to_bf16(v);
                qhi[st][e] = hi;
                qlo[st][e] = to_bf16(v - from_bf16(hi));
            }
    }
    __syncthreads();   // block ids visible (no staging load is in flight yet)

    const uint16_t* pool = static_cast<const uint16_t*>(c.pool);
    const int64_t bel = paged_block_elems(c);
    const int64_t vbase = (int64_t)c.n_kv_heads * 16 * D;
    // this wave's share of the loads of step j, into stage j % S
    auto issue = [&](int j) {
        const int kb = k_begin + 32 * j;
        const int32_t b0 = sblk[2 * j];
        const int32_t b1 = (kb + 16 < len) ? sblk[2 * j + 1] : b0;
        const uint32_t base = lds_offset(lds + (j % S) * St::BYTES);
#pragma unroll
        for (int x = 0; x < LPW; ++x) {
            const int i = wave * LPW + x;   // load index within the step (uniform)
            const uint16_t* g;
            if (i < 2 * NSTEP) {            // K tile a, k-step st: 16 B of row col
                const int a = i / NSTEP, st = i % NSTEP;
                g = pool + (int64_t)(a ? b1 : b0) * bel + ((int64_t)h * 16 + col) * D + 32 * st + 8 * jj;
            } else {                        // V^T of block a, 1 KB piece pc, linear
                const int v = i - 2 * NSTEP, a = v / St::NVI, pc = v % St::NVI;
                g = pool + (int64_t)(a ? b1 : b0) * bel + vbase + (int64_t)h * D * 16 + (pc * 64 + lane) * 8;
            }
            dma_b128(g, base + i * 1024);
        }
    };

    f32x4_t acc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;

    for (int j = 0; j < S - 1; ++j)
        if (j < nsteps) issue(j);
    for (int i = 0; i < nsteps; ++i) {
        // this wave's loads of step i are done once at most those of the
        // S-2 later steps remain; the barrier makes every wave's loads of
        // step i visible and frees stage (i-1) % S for step i+S-1
        if (i + S - 2 < nsteps) wait_loads_barrier<(S - 2) * LPW>();
        else wait_loads_barrier<0>();
        if (i + S - 1 < nsteps) issue(i + S - 1);
        if (!active) continue;
        const int kb = k_begin + 32 * i;
        const char* stage = lds + (i % S) * St::BYTES;
        // ---- S^T for the two 16-key tiles
        f32x4_t sacc[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            f32x4_t sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < NSTEP; ++st) {
                const bf16x8_t kv = *reinterpret_cast<const bf16x8_t*>(stage + (a * NSTEP + st) * 1024 + lane * 16);
                sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qhi[st], sa, 0, 0, 0);
                sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qlo[st], sa, 0, 0, 0);
            }
            sacc[a] = sa;
        }
        // ---- mask, scale, online softmax for this lane's row (keys 4jj+r, 16+4jj+r)
        float p[8];
        float mx = -INFINITY;
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int key = kb + 16 * a + 4 * jj + rr;
                const float sv = (rvalid && key <= qpos && key < len) ? sacc[a][rr] * scale : -INFINITY;
                p[4 * a + rr] = sv;
                mx = fmaxf(mx, sv);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            p[k] = (p[k] == -INFINITY) ? 0.0f : __expf(p[k] - m_new);
            sum += p[k];
        }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        // alpha is exactly 1 when the row's max did not move (exp(0) = 1, and
        // a row with no live key yet has o = 0 and l = 0 either way), so the
        // accumulators need rescaling only when some row of the wave moved
        const float alpha = (m_new == m_run) ? 1.0f : (m_run == -INFINITY) ? 0.0f : __expf(m_run - m_new);
        l_run = l_run * alpha + sum;
        m_run = m_new;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
        }
        bf16x8_t phi, plo;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const __bf16 hi = to_bf16(p[k]);
            phi[k] = hi;
            plo[k] = to_bf16(p[k] - from_bf16(hi));
        }
        // ---- O^T += V^T . P^T over the 32 keys
        const char* vs = stage + St::K_BYTES;
        const uint64_t m0 = key_mask4(len - (kb + 4 * jj)), m1 = key_mask4(len - (kb + 16 + 4 * jj));
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const int d = 16 * dt + col;
            const uint2 lo2 = *reinterpret_cast<const uint2*>(vs + (d * 16 + 4 * jj) * 2);
            const uint2 hi2 = *reinterpret_cast<const uint2*>(vs + St::V_BLOCK + (d * 16 + 4 * jj) * 2);
            const uint4 w = {lo2.x & (uint32_t)m0, lo2.y & (uint32_t)(m0 >> 32), hi2.x & (uint32_t)m1,
                             hi2.y & (uint32_t)(m1 >> 32)};
            const bf16x8_t vv = __builtin_bit_cast(bf16x8_t, w);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv, phi, acc[dt], 0, 0, 0);
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv, plo, acc[dt], 0, 0, 0);
        }
    }
    if (!rvalid) return;
    float* pp = part + ((((int64_t)s * T + t) * Hq + hq) * n_chunks + chunk) * (D + 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) pp[16 * dt + 4 * jj + rr] = acc[dt][rr];
    if (jj == 0) {
        pp[D] = m_run;
        pp[D + 1] = l_run;
    }
}

// Merge the chunk partials of each query row; chunks that start past the
// row's position were never computed for it and are skipped. The global max
// comes first, so the weighted sums are independent terms: wave w sums
// chunks w, w + 4, ... (lane: channels lane and lane + 64, 8 chunks' loads in
// flight) and the 4 waves' sums meet in LDS in wave order. The result depends
// only on the row's own chunks, never on the batch or the launch shape.
constexpr int PCOMB_WAVES = 4;
__global__ void __launch_bounds__(64 * PCOMB_WAVES) paged_combine_kernel(const float* __restrict__ part, int T,
                                                                         int Hq, int D,
                                                                         const int32_t* __restrict__ start,
                                                                         const int32_t* __restrict__ count, int CH,
                                                                         int n_chunks, float* __restrict__ out) {
    const int hq = blockIdx.x, t = blockIdx.y, s = blockIdx.z;
    // the last key the row saw: its own position, or the cache end for a
    // padding row (t >= count[s]), which attends over the whole cache
    const int len = start[s] + (count ? count[s] : T);
    const int last = min(start[s] + t, len - 1);
    if (last < 0) {   // an empty cache (count 0 at start 0): nothing to attend to
        for (int d = threadIdx.x; d < D; d += blockDim.x) out[(((int64_t)s * T + t) * Hq + hq) * D + d] = 0.0f;
        return;
    }
    const int nc = min(last / CH + 1, n_chunks);   // never past the workspace
    const int PD = D + 2;
    const float* p = part + (((int64_t)s * T + t) * Hq + hq) * n_chunks * PD;
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    __shared__ float smax[PCOMB_WAVES], sl[PCOMB_WAVES];
    __shared__ float so[PCOMB_WAVES][2 * WAVE];
    float mm = -INFINITY;
    for (int c = threadIdx.x; c < nc; c += blockDim.x) mm = fmaxf(mm, p[(int64_t)c * PD + D]);
    for (int o = WAVE / 2; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
    if (lane == 0) smax[w] = mm;
    __syncthreads();
    mm = smax[0];
#pragma unroll
    for (int i = 1; i < PCOMB_WAVES; ++i) mm = fmaxf(mm, smax[i]);
    const bool a0 = lane < D, a1 = lane + WAVE < D;
    float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll 8
    for (int c = w; c < nc; c += PCOMB_WAVES) {
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
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int i = 0; i < PCOMB_WAVES; ++i) {
            lt += sl[i];
            ot += so[i][d];
        }
        out[(((int64_t)s * T + t) * Hq + hq) * D + d] = ot / lt;
    }
}

static size_t attn_smem(int D) {
    return sizeof(float) * (QB * D + KT * (D + 1) + KT * D + QB * KT + 3 * QB);
}

}  // namespace dkv

extern "C" int dkv_paged_append(const dkv_paged_t* cache, int32_t layer, const void* k, const void* v,
                                int32_t in_dtype, int32_t T, const int32_t* start, const int32_t* count,
                                dkv_stream_t stream) {
    DKV_REQUIRE(cache && k && v && start, "dkv_paged_append: NULL argument");
    const dkv_paged_t c = *cache;
    DKV_REQUIRE(layer >= 0 && layer < c.n_layers, "dkv_paged_append: layer out of range");
    DKV_REQUIRE(c.dtype == DKV_F32 || c.dtype == DKV_BF16, "dkv_paged_append: bad cache dtype");
    DKV_REQUIRE(in_dtype == DKV_F32 || in_dtype == DKV_BF16, "dkv_paged_append: bad input dtype");
    DKV_REQUIRE(c.batch > 0 && c.block_size > 0 && c.max_blocks > 0, "dkv_paged_append: bad cache shape");
    if (T <= 0) return DKV_OK;
    hipLaunchKernelGGL(dkv::paged_append_kernel, dim3(T, c.batch), dim3(256), 0, dkv::as_stream(stream), c, layer,
                       k, v, in_dtype, T, start, count);
    return dkv::check_launch("dkv_paged_append");
}

static int n_chunks_for(int max_len, int chunk_keys) { return (max_len + chunk_keys - 1) / chunk_keys; }

extern "C" size_t dkv_paged_attention_workspace(const dkv_paged_t* cache, int32_t T, int32_t n_q_heads,
                                                int32_t max_len, int32_t chunk_keys) {
    if (!cache || T <= 0 || n_q_heads <= 0 || max_len <= 0 || chunk_keys <= 0) return 0;
    return sizeof(float) * (size_t)cache->batch * T * n_q_heads * n_chunks_for(max_len, chunk_keys) *
           (cache->head_dim + 2);
}

extern "C" int dkv_paged_attention(const dkv_paged_t* cache, int32_t layer, const float* q, int32_t T,
                                   int32_t n_q_heads, const int32_t* start, const int32_t* count, int32_t max_len,
                                   int32_t chunk_keys, float* out, void* work, size_t work_bytes,
                                   dkv_stream_t stream) {
    DKV_REQUIRE(cache && q && start && out, "dkv_paged_attention: NULL argument");
    const dkv_paged_t c = *cache;
    DKV_REQUIRE(layer >= 0 && layer < c.n_layers, "dkv_paged_attention: layer out of range");
    DKV_REQUIRE(c.head_dim > 0 && c.head_dim <= dkv::MAXD, "dkv_paged_attention: head_dim must be 1..128");
    DKV_REQUIRE(n_q_heads > 0 && n_q_heads % c.n_kv_heads == 0,
                "dkv_paged_attention: query heads must be a multiple of KV heads");
    DKV_REQUIRE(chunk_keys > 0 && chunk_keys % dkv::KT == 0, "dkv_paged_attention: chunk_keys must be a multiple of 32");
    DKV_REQUIRE(max_len > 0, "dkv_paged_attention: max_len must be > 0");
    if (T <= 0) return DKV_OK;
    const size_t need = dkv_paged_attention_workspace(cache, T, n_q_heads, max_len, chunk_keys);
    if (!work || work_bytes < need)
        return dkv::fail(DKV_EWORKSPACE, "dkv_paged_attention: workspace too small (need " + std::to_string(need) + ")");
    const int n_chunks = n_chunks_for(max_len, chunk_keys);
    const int G = n_q_heads / c.n_kv_heads;
    const int n_qtiles = (T * G + dkv::QB - 1) / dkv::QB;
    DKV_REQUIRE((int64_t)n_chunks * n_qtiles < (1LL << 31), "dkv_paged_attention: grid too large");
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(c.head_dim)));
    hipStream_t st = dkv::as_stream(stream);
    // the kernel choice depends on the cache only (never on T), so a verify
    // pass and a one-token decode step take the same arithmetic path
    const bool mfma = c.dtype == DKV_BF16 && c.block_size == 16 && (c.head_dim == 64 || c.head_dim == 128);
    if (mfma) {
        // one wave per q-tile, up to 8 per workgroup (a power of two, so a
        // step's loads split evenly); staged steps plus the chunk's block ids
        const int W = n_qtiles <= 1 ? 1 : n_qtiles <= 2 ? 2 : n_qtiles <= 4 ? 4 : 8;
        const int n_qgroups = (n_qtiles + W - 1) / W;
        DKV_REQUIRE((int64_t)n_chunks * n_qgroups < (1LL << 31), "dkv_paged_attention: grid too large");
        const size_t stage = c.head_dim == 128 ? dkv::VerifyStage<128>::BYTES : dkv::VerifyStage<64>::BYTES;
        const size_t lds = dkv::VERIFY_STAGES * stage + (((size_t)chunk_keys / 16 * 4 + 15) & ~size_t(15));
        // gfx950 gives a workgroup up to 160 KB of LDS
        DKV_REQUIRE(lds <= 160 * 1024, "dkv_paged_attention: chunk_keys too large for the bf16 kernel");
        DKV_REQUIRE((int64_t)c.n_kv_heads * c.batch <= 65535 && n_chunks <= 65535,
                    "dkv_paged_attention: batch x heads or chunk count too large for the grid");
        const dim3 grid(n_qgroups, c.n_kv_heads * c.batch, n_chunks), blk(64 * W);
        float* part = static_cast<float*>(work);
#define DKV_VERIFY(DD, WW)                                                                                         \
    do {                                                                                                           \
        auto kfn = dkv::paged_attn_mfma_kernel<DD, WW>;                                                            \
        static size_t lds_done[16] = {};                                                                           \
        if (!dkv::reserve_lds(reinterpret_cast<const void*>(kfn), lds, lds_done))                                   \
            return dkv::fail(DKV_ELAUNCH, "dkv_paged_attention: cannot reserve " + std::to_string(lds) + " B of LDS"); \
        hipLaunchKernelGGL(kfn, grid, blk, lds, st, c, layer, q, T, n_q_heads, start, count, chunk_keys,          \
                           n_qgroups, n_chunks, n_qtiles, scale, part);                                            \
    } while (0)
        if (c.head_dim == 128) {
            switch (W) {
                case 1: DKV_VERIFY(128, 1); break;
                case 2: DKV_VERIFY(128, 2); break;
                case 4: DKV_VERIFY(128, 4); break;
                default: DKV_VERIFY(128, 8); break;
            }
        } else {
            switch (W) {
                case 1: DKV_VERIFY(64, 1); break;
                case 2: DKV_VERIFY(64, 2); break;
                case 4: DKV_VERIFY(64, 4); break;
                default: DKV_VERIFY(64, 8); break;
            }
        }
#undef DKV_VERIFY
    } else {
        hipLaunchKernelGGL(dkv::paged_attn_kernel, dim3(n_chunks * n_qtiles, c.n_kv_heads, c.batch), dim3(256),
                           dkv::attn_smem(c.head_dim), st, c, layer, q, T, n_q_heads, start, count, chunk_keys,
                           n_chunks, n_qtiles, scale, static_cast<float*>(work));
    }
    int rc = dkv::check_launch("dkv_paged_attention");
    if (rc) return rc;
    hipLaunchKernelGGL(dkv::paged_combine_kernel, dim3(n_q_heads, T, c.batch), dim3(dkv::WAVE * dkv::PCOMB_WAVES), 0, st,
                       static_cast<const float*>(work), T, n_q_heads, c.head_dim, start, count, chunk_keys, n_chunks,
                       out);
    return dkv::check_launch("dkv_paged_attention(combine)");
}
