// bf16 projection GEMM of the model forwards: y[M, N] = x[M, K] . W[N, K]^T
// with float32 accumulation and one rounding to bf16 (or a float32 result).
// Reference: the `x @ W` projections, MLP and LM head of model.py:113-133,
// gpt2.py:191-213, llama.py:187-225 (numpy float32 there).
//
// At decode sizes (M = batch rows, or batch * (gamma + 1) in verify) the
// product is bound by the weight stream: W is read once from HBM, x (a few
// hundred KB) from L2. K is cut into S chunks, S a function of (N, K) only.
// Every output is, per chunk, one in-order chain of
// v_mfma_f32_16x16x32_bf16 over the chunk's 128-k blocks (block step j,
// lane group q: k = 32j + 8q .. +8, the same for W and x), and the chunk
// sums are added in chunk order, either inside the workgroup, or from
// per-chunk partials by the reduce kernel or by the kernel that consumes y
// (DKV_GEMM_DEFER) -- the same float additions in the same order. So an
// output's arithmetic depends neither on M, nor on the launch shape chosen
// for M, nor on the row's place in the batch: a verify row equals the
// one-token decode row bit for bit. W is row-major or tiled
// (DKV_GEMM_WTILED); the layout changes which addresses a lane loads, not
// what it multiplies.
#include "dkv_common.h"

#include <type_traits>

namespace dkv {

typedef __bf16 gbf16x8_t __attribute__((ext_vector_type(8)));
typedef float gf32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t gu32x4_t __attribute__((ext_vector_type(4)));   // a native vector: copies stay in registers

// One 16-byte W load. NT: non-temporal, for workgroups that stream their W
// rows through every K chunk (the long streams: measured 5-7% faster for the
// Llama-3-8B gate/up weight at M = 32 and 96); the short per-chunk streams of
// the split plans measured 12-17% slower that way (their loads wait on
// latency, not bandwidth), so they keep the default policy.
template <bool NT>
__device__ __forceinline__ gu32x4_t load_w(const uint16_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const gu32x4_t*>(p));
    return *reinterpret_cast<const gu32x4_t*>(p);
}

constexpr int GKB = 128;            // k per block: four 32-k MFMA steps
constexpr int GX_ROW = GKB + 8;
     // LDS row of a staged x block (bf16), padded against bank conflicts

__device__ __forceinline__ gbf16x8_t as_bf16x8(gu32x4_t v) { return __builtin_bit_cast(gbf16x8_t, v); }

// bias of outputs n .. n+3 (n % 4 == 0, so one 8-byte load where all four
// exist); zero past N
__device__ __forceinline__ float4 bias4(const uint16_t* b, int64_t n, int N) {
    if (!b) return make_float4(0.f, 0.f, 0.f, 0.f);
    if (n + 3 < N) {
        const uint2 v = *reinterpret_cast<const uint2*>(b + n);
        return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                           __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
    }
    float t[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = n + e < N ? __uint_as_float((uint32_t)b[n + e] << 16) : 0.0f;
    return make_float4(t[0], t[1], t[2], t[3]);
}

__device__ __forceinline__ uint32_t bf16_pair_rne(float lo, float hi) {
    const __bf16 a = (__bf16)lo, b = (__bf16)hi;   // v_cvt_pk_bf16_f32: round to nearest even
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// x operands: 8 consecutive elements of a row, bf16 (16 bytes) or float32
// (32 bytes, kept raw in registers until used, then rounded to bf16 to
// nearest even -- the rounding of a float32 -> bf16 tensor conversion)
typedef uint32_t gu32x8_t __attribute__((ext_vector_type(8)));
template <bool XF32>
using XRaw = typename std::conditional<XF32, gu32x8_t, gu32x4_t>::type;

template <bool XF32>
__device__ __forceinline__ XRaw<XF32> load_x8(const void* base, int64_t elem) {
    if constexpr (XF32) return *reinterpret_cast<const gu32x8_t*>(static_cast<const float*>(base) + elem);
    else return *reinterpret_cast<const gu32x4_t*>(static_cast<const uint16_t*>(base) + elem);
}

// SwiGLU of one (gate, up) pair of outputs, both first rounded to bf16 as the
// unfused GEMM would store them, then g / (1 + exp(-g)) * u in float32 (the
// SwiGLU kernel's arithmetic) rounded to bf16
__device__ __forceinline__ float bf16_round(float v) { return __uint_as_float((uint32_t)f32_to_bf16_rne(v) << 16); }
__device__ __forceinline__ uint32_t swiglu_pair(float g0, float u0, float g1, float u1) {
    const float a = bf16_round(g0), b = bf16_round(u0), c = bf16_round(g1), d = bf16_round(u1);
    return (uint32_t)f32_to_bf16_rne(a / (1.0f + __expf(-a)) * b) |
           ((uint32_t)f32_to_bf16_rne(c / (1.0f + __expf(-c)) * d) << 16);
}

template <bool XF32>
__device__ __forceinline__ gu32x4_t x8_bf16(const XRaw<XF32>& r) {
    if constexpr (XF32)
        return gu32x4_t{bf16_pair_rne(__uint_as_float(r[0]), __uint_as_float(r[1])),
                        bf16_pair_rne(__uint_as_float(r[2]), __uint_as_float(r[3])),
                        bf16_pair_rne(__uint_as_float(r[4]), __uint_as_float(r[5])),
                        bf16_pair_rne(__uint_as_float(r[6]), __uint_as_float(r[7]))};
    else return r;
}

// y[m][n .. n+3] = t for a row-major y of N columns: one vector store when
// N % 4 == 0 (the row, and so the four outputs, are aligned; n < N then
// implies n + 3 < N), else element by element up to column N - 1
__device__ __forceinline__ void store_y4(void* y, int y_f32, int64_t m, int n, int N, const gf32x4_t& t) {
    const int64_t o = m * N + n;
    if ((N & 3) == 0) {
        if (y_f32) *reinterpret_cast<float4*>(static_cast<float*>(y) + o) = make_float4(t[0], t[1], t[2], t[3]);
        else
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + o) =
                make_uint2(bf16_pair_rne(t[0], t[1]), bf16_pair_rne(t[2], t[3]));
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (n + e >= N) break;
        if (y_f32) static_cast<float*>(y)[o + e] = t[e];
        else static_cast<uint16_t*>(y)[o + e] = f32_to_bf16_rne(t[e]);
    }
}

struct GemmArgs {
    const void* x;       // [M, K], bf16 or float32 (x_f32)
    int x_f32;
    const uint16_t* w;   // [N, K]
    const uint16_t* bias;   // [N] bf16 or null, added after the chunk sums
    int M, N, K;
    int KC;              // chunk length: K = S * KC, KC % 32 == 0
    int S;               // chunks
    int c_per;           // chunks per workgroup: S (summed in order here) or 1 (one partial per chunk)
    int units;           // n_tiles * (S / c_per)
    int m_tiles;
    float* part;         // [S][M][N] float32 partials when c_per == 1 < S
    void* y;
    int y_f32;
    int swiglu;          // rows of W interleave (gate_i, up_i); y[m][i] = silu(gate) * up, bf16, N / 2 columns
};

// W stored in tiles (DKV_GEMM_WTILED): 16 rows x 128 k per 4 KB tile, the
// tiles of a 16-row fragment consecutive along k, and inside a tile the
// MFMA A-operand order of the block's four 32-k steps: element (row 16 fn + c,
// k 128 kb + 32 j + 8 q + e) at ((fn * K/128 + kb) * 4 + j) * 512 + (16 q + c) * 8 + e.
// A wave's load of one step is then 1 KB contiguous (16 B per lane, lane
// 16 q + c), and a fragment streams as one run; row-major W makes each load
// 16 rows x 64 B. The arithmetic is the same either way.
// Row-major W may end inside a fragment (N % 16 != 0): its lanes past row N-1
// reread row N-1, whose products land in outputs that are never stored.
template <bool WT>
__device__ __forceinline__ const uint16_t* w_lane_base(const uint16_t* w, int64_t frag_row0, int col, int q, int lane,
                                                       int K, int N) {
    if constexpr (WT) return w + frag_row0 * K + 8 * lane;
    else return w + min(frag_row0 + col, (int64_t)N - 1) * K + 8 * q;
}
// offset of step j of the block starting at k (elements, from the lane base)
template <bool WT>
__device__ __forceinline__ int64_t w_step_off(int k, int j) {
    if constexpr (WT) return 16 * (int64_t)k + 512 * j;
    else return k + 32 * j;
}

// One workgroup: WV waves, 16*NW*WV rows of W (16*NW per wave), against a
// tile of 16*MB rows of x, over c_per consecutive K chunks. Per 128-k block the tile's x
// is staged once in LDS (shared by the waves); each lane streams its W
// rows straight into registers PD - 1 blocks ahead (PD register sets in
// rotation). MULTI: the chunks' sums are added in chunk order here (the same
// additions, in the same order, as the reduce kernel applies to partials).
// PARTIAL: chunks may end in a block of fewer than four 32-k steps (K not a
// multiple of 128); otherwise every block is whole.
template <int NW, int MB, bool MULTI, bool PARTIAL, int PD, bool XF32, int WV, bool WT>
__global__ void __launch_bounds__(64 * WV) gemm_bf16_kernel(GemmArgs a) {
    // x of block gb + 1 waits in registers to be staged while block gb + PD - 1 is fetched: two sets apart
    static_assert(PD >= 3, "x needs a register set between its fetch and its staging");
    constexpr int TM = 16 * MB;
    constexpr int NT = 64 * WV;                               // threads
    constexpr int NXI = (16 * TM + NT - 1) / NT;             // x pieces (8 elements) per thread per block
    __shared__ __align__(16) uint16_t xs[2][TM][GX_ROW];
    // XCD-aware order: workgroup g runs on XCD g % 8; the m tiles of one unit
    // (a W row block and chunk range) take consecutive slots of one XCD, so
    // its W rows are fetched from HBM once and reread from that XCD's L2.
    const int g = blockIdx.x, slot = g >> 3;
    const int u = (slot / a.m_tiles) * 8 + (g & 7), mt = slot % a.m_tiles;
    if (u >= a.units) return;   // whole workgroup
    const int splits = a.S / a.c_per;
    const int nt = u / splits, c0 = (u % splits) * a.c_per;
    const int m0 = mt * TM, mrows = min(TM, a.M - m0);
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int col = lane % 16, q = lane / 16;
    const int n0 = nt * 16 * NW * WV + 16 * NW * wave;
    const bool live = n0 < a.N;   // wave-uniform; NW == 2 only where N % 32 == 0
    const int K = a.K, KC = a.KC;
    const int nb = (KC + GKB - 1) / GKB, G = nb * a.c_per;
    const uint16_t* wrow[NW];
#pragma unroll
    for (int f = 0; f < NW; ++f) wrow[f] = w_lane_base<WT>(a.w, live ? n0 + 16 * f : 0, col, q, lane, K, a.N);
    // x piece i of this thread: tile row xr_row[i], k offset 8 xr_c[i] in the block. Tile rows past M
    // reread row M-1 (their outputs are dropped), so every load and LDS write is unconditional.
    // (pieces past the tile, when the thread count does not divide it, repeat
    // the tile's last piece: the same load and the same LDS bytes)
    int64_t xsrc[NXI];   // element offset of the piece's row in x
    uint32_t xdst[NXI];
    int xc[NXI];
#pragma unroll
    for (int i = 0; i < NXI; ++i) {
        const int p = min(tid + NT * i, 16 * TM - 1), r = p / 16;
        xc[i] = p % 16;
        xsrc[i] = (int64_t)(m0 + min(r, mrows - 1)) * K;
        xdst[i] = (uint32_t)(r * GX_ROW);
    }

    // block gb of this workgroup: k start and number of 32-k steps
    auto blk_k = [&](int gb) {
        const int cl = gb / nb;
        return (c0 + cl) * KC + (gb - cl * nb) * GKB;
    };
    auto blk_steps = [&](int gb) {
        if constexpr (!PARTIAL) return 4;
        const int cl = gb / nb;
        return min(4, (KC - (gb - cl * nb) * GKB) / 32);
    };

    // Every load below is unconditional (addresses clamped into the operands), so that the compiler's
    // wait counts see the same sequence of loads on every path and keep two blocks in flight.
#define DKV_LOAD_W(DST, GB)                                                                                     \
    do {                                                                                                        \
        const int k_ = blk_k(GB), st_ = blk_steps(GB);                                                         \
        _Pragma("unroll") for (int f_ = 0; f_ < NW; ++f_) _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_)       \
            DST[f_][j_] = load_w<MULTI>(wrow[f_] + w_step_off<WT>(k_, PARTIAL ? min(j_, st_ - 1) : j_));        \
    } while (0)
#define DKV_LOAD_X(XD, GB)                                                                                      \
    do {                                                                                                        \
        const int k_ = blk_k(GB), st_ = blk_steps(GB);                                                         \
        _Pragma("unroll") for (int i_ = 0; i_ < NXI; ++i_) XD[i_] =                                             \
            load_x8<XF32>(a.x, xsrc[i_] + k_ + 8 * (PARTIAL ? min(xc[i_], 4 * st_ - 1) : xc[i_]));               \
    } while (0)
#define DKV_STORE_X(XS, BUF)                                                                                    \
    do {                                                                                                        \
        _Pragma("unroll") for (int i_ = 0; i_ < NXI; ++i_)                                                       \
            *reinterpret_cast<gu32x4_t*>(&xs[BUF][0][0] + xdst[i_] + 8 * xc[i_]) = x8_bf16<XF32>(XS[i_]);       \
    } while (0)

    gf32x4_t acc[NW][MB], tot[MULTI ? NW : 1][MULTI ? MB : 1];
#pragma unroll
    for (int f = 0; f < NW; ++f)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[f][mb] = gf32x4_t{0.f, 0.f, 0.f, 0.f};

    // PD register sets of W and of x in rotation: block gb + PD - 1 is fetched while block gb is
    // multiplied. x is fetched as far ahead as W: loads complete in issue order, so waiting for
    // x(gb + 1) also waits for every W load issued before it.
    gu32x4_t wr[PD][NW][4];
    XRaw<XF32> xr[PD][NXI];
    DKV_LOAD_X(xr[0], 0);
    DKV_STORE_X(xr[0], 0);
#pragma unroll
    for (int pb = 1; pb < PD; ++pb) {
        DKV_LOAD_X(xr[pb], min(pb, G - 1));
        DKV_LOAD_W(wr[pb - 1], min(pb - 1, G - 1));
    }
    __syncthreads();

    // one block: stage x(gb+1), fetch block gb+PD-1 (the last block again past the end), multiply
    // block gb
#define DKV_BLOCK(CUR, XNEXT, NXT, XFETCH)                                                                      \
    do {                                                                                                        \
        const int gb = g0 + v_;                                                                                 \
        if (gb + 1 < G) DKV_STORE_X(XNEXT, (gb + 1) & 1);                                                       \
        DKV_LOAD_X(XFETCH, min(gb + PD - 1, G - 1));                                                            \
        DKV_LOAD_W(NXT, min(gb + PD - 1, G - 1));                                                               \
        const int st = blk_steps(min(gb, G - 1));                                                               \
        if (live && gb < G) {                                                                                   \
            const uint16_t* xb = &xs[gb & 1][0][0] + col * GX_ROW + 8 * q;                                      \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                                     \
                if (!PARTIAL || j < st) {                                                                       \
                    gbf16x8_t bx[MB];                                                                           \
                    _Pragma("unroll") for (int mb = 0; mb < MB; ++mb) bx[mb] =                                  \
                        as_bf16x8(*reinterpret_cast<const gu32x4_t*>(xb + 16 * mb * GX_ROW + 32 * j));             \
                    _Pragma("unroll") for (int f = 0; f < NW; ++f) _Pragma("unroll") for (int mb = 0; mb < MB;  \
                                                                                          ++mb) acc[f][mb] =    \
                        __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(CUR[f][j]), bx[mb], acc[f][mb], 0, 0, 0); \
                }                                                                                               \
            }                                                                                                   \
        }                                                                                                       \
        if constexpr (MULTI) {                                                                                  \
            if (gb < G && (gb + 1) % nb == 0) { /* a chunk ends: add its sum in chunk order */                 \
                _Pragma("unroll") for (int f = 0; f < NW; ++f) _Pragma("unroll") for (int mb = 0; mb < MB;      \
                                                                                      ++mb) {                   \
                    if (gb + 1 == nb) tot[f][mb] = acc[f][mb];                                                  \
                    else                                                                                        \
                        _Pragma("unroll") for (int e = 0; e < 4; ++e) tot[f][mb][e] =                           \
                            tot[f][mb][e] + acc[f][mb][e];                                                      \
                    acc[f][mb] = gf32x4_t{0.f, 0.f, 0.f, 0.f};                                                  \
                }                                                                                               \
            }                                                                                                   \
        }                                                                                                       \
        __syncthreads();                                                                                        \
    } while (0)

    for (int g0 = 0; g0 < G; g0 += PD) {
#pragma unroll
        for (int v_ = 0; v_ < PD; ++v_)
            DKV_BLOCK(wr[v_], xr[(v_ + 1) % PD], wr[(v_ + PD - 1) % PD], xr[(v_ + PD - 1) % PD]);
    }
#undef DKV_BLOCK
#undef DKV_STORE_X
#undef DKV_LOAD_X
#undef DKV_LOAD_W
    if (!live) return;
    // lane holds C[4q + r][col]: outputs (m, n + 4q .. 4q + 3), m = m0 + 16 mb + col
    const bool to_part = !MULTI && a.S > 1;
#pragma unroll
    for (int f = 0; f < NW; ++f)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int m = m0 + 16 * mb + col;
            if (m >= a.M) continue;
            gf32x4_t t;
            if constexpr (MULTI) t = tot[f][mb];
            else t = acc[f][mb];
            const int n = n0 + 16 * f + 4 * q;
            if (n >= a.N) continue;   // a fragment past the end of W (N % 16 != 0)
            const int64_t o = (int64_t)m * a.N + n;
            if (!to_part && a.bias) {
                const float4 bv = bias4(a.bias, n, a.N);
                t[0] = t[0] + bv.x;
                t[1] = t[1] + bv.y;
                t[2] = t[2] + bv.z;
                t[3] = t[3] + bv.w;
            }
            if (to_part) {   // partials only where N % 16 == 0
                *reinterpret_cast<float4*>(a.part + (int64_t)c0 * a.M * a.N + o) = make_float4(t[0], t[1], t[2], t[3]);
            } else if (a.swiglu) {   // rows n .. n+3 are (gate, up) of outputs n/2 and n/2 + 1
                *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.y) + (int64_t)m * (a.N / 2) + n / 2) =
                    swiglu_pair(t[0], t[1], t[2], t[3]);
            } else {
                store_y4(a.y, a.y_f32, m, n, a.N, t);
            }
        }
}

// Small M (x tile of 16*MB rows, M <= 16*MB): a workgroup of RW*CW waves owns
// RW 16-row fragments of W; the CW waves of a fragment take its chunks
// cg, cg + CW, ... and stream each chunk's W rows and x straight into
// registers, PD blocks ahead. Each chunk's sum goes to LDS; the fragment's
// first wave adds them in chunk order (then the bias) and writes y -- the
// same additions as the other plans, with no partials in HBM and no second
// kernel. Requires S % CW == 0 and chunks of whole 128-k blocks.
template <int RW, int CW, int MB, bool XF32, bool WT>
__global__ void __launch_bounds__(64 * RW * CW) gemm_bf16_small_kernel(GemmArgs a) {
    constexpr int PD = 4;
    extern __shared__ __align__(16) float red[];   // [S][RW][MB][64 lanes][4]
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE), lane = tid % WAVE;
    const int fr = wave % RW, cg = wave / RW;
    const int col = lane % 16, q = lane / 16;
    const int n0 = (blockIdx.x * RW + fr) * 16;
    const bool live = n0 < a.N;   // wave-uniform
    const int K = a.K, KC = a.KC, S = a.S;
    const int nb = KC / GKB, G = nb * (S / CW);
    const uint16_t* wrow = w_lane_base<WT>(a.w, live ? n0 : 0, col, q, lane, K, a.N);
    int64_t xrow[MB];   // element offset of the lane's x row and lane group
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xrow[mb] = (int64_t)min(16 * mb + col, a.M - 1) * K + 8 * q;
    // block gb of this wave: chunk cg + CW * (gb / nb), k start, 32-k steps
    auto blk_k = [&](int gb) {
        const int cl = gb / nb;
        return (cg + CW * cl) * KC + (gb - cl * nb) * GKB;
    };
    // unconditional loads (clamped), as in gemm_bf16_kernel
#define DKV_SLOAD(WD, XD, GB)                                                                                   \
    do {                                                                                                        \
        const int k_ = blk_k(GB);                                                                               \
        _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_) {                                                     \
            const int kj = k_ + 32 * j_;                                                                        \
            WD[j_] = *reinterpret_cast<const gu32x4_t*>(wrow + w_step_off<WT>(k_, j_));                       \
            _Pragma("unroll") for (int m_ = 0; m_ < MB; ++m_) XD[m_][j_] = load_x8<XF32>(a.x, xrow[m_] + kj);  \
        }                                                                                                       \
    } while (0)
    gu32x4_t w0[4], w1[4], w2[4], w3[4];
    XRaw<XF32> x0[MB][4], x1[MB][4], x2[MB][4], x3[MB][4];
    gf32x4_t acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = gf32x4_t{0.f, 0.f, 0.f, 0.f};
    DKV_SLOAD(w0, x0, 0);
    DKV_SLOAD(w1, x1, min(1, G - 1));
    DKV_SLOAD(w2, x2, min(2, G - 1));
#define DKV_SBLOCK(WC, XC, WN, XN)                                                                              \
    do {                                                                                                        \
        const int gb = g0 + v_;                                                                                 \
        DKV_SLOAD(WN, XN, min(gb + PD - 1, G - 1));                                                             \
        if (gb < G) {                                                                                           \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                                     \
                _Pragma("unroll") for (int mb = 0; mb < MB; ++mb) acc[mb] =                                     \
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(WC[j]), as_bf16x8(x8_bf16<XF32>(XC[mb][j])), \
                                                            acc[mb], 0, 0, 0);                                  \
            }                                                                                                   \
            if ((gb + 1) % nb == 0) { /* a chunk ends: park its sum */                                         \
                const int c = cg + CW * (gb / nb);                                                              \
                _Pragma("unroll") for (int mb = 0; mb < MB; ++mb) {                                             \
                    *reinterpret_cast<gf32x4_t*>(red + ((((int64_t)c * RW + fr) * MB + mb) * WAVE + lane) * 4) = \
                        acc[mb];                                                                                \
                    acc[mb] = gf32x4_t{0.f, 0.f, 0.f, 0.f};                                                     \
                }                                                                                               \
            }                                                                                                   \
        }                                                                                                       \
    } while (0)
    for (int g0 = 0; g0 < G; g0 += PD) {
        {
            constexpr int v_ = 0;
            DKV_SBLOCK(w0, x0, w3, x3);
        }
        {
            constexpr int v_ = 1;
            DKV_SBLOCK(w1, x1, w0, x0);
        }
        {
            constexpr int v_ = 2;
            DKV_SBLOCK(w2, x2, w1, x1);
        }
        {
            constexpr int v_ = 3;
            DKV_SBLOCK(w3, x3, w2, x2);
        }
    }
#undef DKV_SBLOCK
#undef DKV_SLOAD
    __syncthreads();
    if (!live || cg != 0) return;
    // outputs (m, n0 + 4q .. 4q + 3), m = 16 mb + col: the chunk sums in chunk order, then the bias
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = 16 * mb + col;
        gf32x4_t t = *reinterpret_cast<const gf32x4_t*>(red + (((int64_t)fr * MB + mb) * WAVE + lane) * 4);
        for (int c = 1; c < S; ++c) {
            const gf32x4_t u =
                *reinterpret_cast<const gf32x4_t*>(red + ((((int64_t)c * RW + fr) * MB + mb) * WAVE + lane) * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) t[e] = t[e] + u[e];
        }
        const int n = n0 + 4 * q;
        if (m >= a.M || n >= a.N) continue;
        if (a.bias) {
            const float4 bv = bias4(a.bias, n, a.N);
            t[0] = t[0] + bv.x;
            t[1] = t[1] + bv.y;
            t[2] = t[2] + bv.z;
            t[3] = t[3] + bv.w;
        }
        if (a.swiglu) {
            *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.y) + (int64_t)m * (a.N / 2) + n / 2) =
                swiglu_pair(t[0], t[1], t[2], t[3]);
        } else {
            store_y4(a.y, a.y_f32, m, n, a.N, t);
        }
    }
}

// y = sum of the K chunks' partials, in chunk order, then the bias; 4 outputs per thread
__global__ void __launch_bounds__(256) gemm_reduce_kernel(const float* __restrict__ part, int64_t MN, int S, int N,
                                                          const uint16_t* __restrict__ bias, void* __restrict__ y,
                                                          int y_f32, int swiglu) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= MN) return;
    float4 t = *reinterpret_cast<const float4*>(part + i);
    for (int s = 1; s < S; ++s) {
        const float4 u = *reinterpret_cast<const float4*>(part + (int64_t)s * MN + i);
        t.x += u.x;
        t.y += u.y;
        t.z += u.z;
        t.w += u.w;
    }
    if (bias) {   // the four outputs share a row (partials only where N % 16 == 0)
        const float4 bv = bias4(bias, i % N, N);
        t.x += bv.x;
        t.y += bv.y;
        t.z += bv.z;
        t.w += bv.w;
    }
    if (swiglu) *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(y) + i / 2) = swiglu_pair(t.x, t.y, t.z, t.w);
    else if (y_f32) *reinterpret_cast<float4*>(static_cast<float*>(y) + i) = t;
    else *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + i) = make_uint2(bf16_pair_rne(t.x, t.y),
                                                                               bf16_pair_rne(t.z, t.w));
}

// K chunks: a function of (N, K) only, never of M, so that an output's
// additions are the same for every batch. Enough chunks for about 512
// workgroups of 64 W rows when M is small, each chunk a whole number of
// 128-k blocks and at least 1024 long (Llama-3-8B layer: qkv and o at K =
// 4096 in 4 chunks, not 8 of 512, measured 18.4 -> 15.7 and 15.3 -> 12.9 us
// at M = 32, 26.3 -> 21.6 and 20.5 -> 22.3 us at M = 96; gate/up (2 chunks)
// and down (8 of 1792) as before, both slower with fewer chunks).
static int gemm_chunks(int N, int K) {
    const int64_t wgs = (N + 63) / 64;
    int S = 1;
    while (wgs * S < 512 && K % (2 * S * GKB) == 0 && K / (2 * S) >= 1024) S *= 2;
    return S;
}

// Launch shape, free to depend on M (the arithmetic does not): W rows per
// wave, x rows per tile, and whether the chunks are split across workgroups.
struct GemmPlan {
    int nw, mb, m_tiles, n_tiles, c_per;
    int wv;              // waves per workgroup (4, or 7 where that tiles N into whole rounds of 256 CUs)
    int small, rw, cw;   // gemm_bf16_small_kernel: RW fragments x CW chunk groups per workgroup
};

static GemmPlan gemm_plan(int M, int N, int K) {
    GemmPlan p;
    const int S = gemm_chunks(N, K);
    p.small = 0;
    p.wv = 4;
    if (M <= 8 && S >= 4) {   // a few rows and a chunked K: split K inside the workgroup
        p.small = 1, p.nw = 1, p.mb = 1, p.m_tiles = 1, p.c_per = S;
        p.cw = 4, p.rw = 1;
        p.n_tiles = (N + 15) / 16;
        return p;
    }
    // from M = 33 on, two W fragments per wave (each x fragment read from LDS feeds two MFMAs) wherever
    // whole 32-row fragments and 128-k blocks allow; the x tile just covers M up to 128 rows (measured
    // on the Llama-3-8B projection and head shapes, weights streamed cold from HBM)
    p.nw = (N % 32 == 0 && K % GKB == 0 && M > 32) ? 2 : 1;
    p.mb = M <= 16 ? 1 : M <= 32 ? 2 : (M <= 64 || p.nw == 1) ? 4 : 8;
    p.m_tiles = (M + 16 * p.mb - 1) / (16 * p.mb);
    if (p.nw == 2 && M > 64) {   // tiles of up to 128 rows, as even as 16-row fragments allow (M = 96: one tile of
                                 // 96, not 128; M = 288: three of 96, not 128 + 128 + 32)
        const int rows = (M + p.m_tiles - 1) / p.m_tiles;
        p.mb = (rows + 15) / 16;
    }
    p.n_tiles = (N + 64 * p.nw - 1) / (64 * p.nw);
    // split the chunks over workgroups only when the tiles alone leave most of the chip idle
    // (partials need whole 16-row fragments: N % 16 == 0)
    p.c_per = (S > 1 && (int64_t)p.n_tiles * p.m_tiles < 128 && N % 16 == 0) ? 1 : S;
    // 7-wave workgroups when they cut W into whole rounds of 256 tiles and 4-wave ones do not
    // (the Llama-3-8B gate/up weight, 28672 rows: 448 tiles of 64 leave the CUs unevenly loaded,
    // 256 of 112 give every CU one); one fragment per wave, x tiles up to 128 rows (one m tile;
    // at M = 96 the gate/up GEMM measured 49 -> 46 us against 224 two-fragment workgroups)
    const int r7 = 16 * (p.mb <= 2 ? p.nw : 1) * 7;
    if (p.c_per == S && (p.mb <= 2 || p.m_tiles == 1) && K % GKB == 0 && N % r7 == 0 && (N / r7 * p.m_tiles) % 256 == 0 &&
        (p.n_tiles * p.m_tiles) % 256 != 0) {
        p.wv = 7;
        if (p.mb > 2) p.nw = 1;
        p.n_tiles = N / r7;
    }
    return p;
}

}  // namespace dkv

using namespace dkv;

extern "C" int32_t dkv_gemm_bf16_partials(int32_t M, int32_t N, int32_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int S = gemm_chunks(N, K);
    const GemmPlan p = gemm_plan(M, N, K);
    return !p.small && p.c_per == 1 && S > 1 ? S : 0;
}

extern "C" size_t dkv_gemm_bf16_workspace(int32_t M, int32_t N, int32_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int S = gemm_chunks(N, K);
    const GemmPlan p = gemm_plan(M, N, K);
    return !p.small && p.c_per == 1 && S > 1 ? sizeof(float) * (size_t)S * M * N : 0;
}

template <int RW, int CW, int MB, bool WT>
static void launch_small(const GemmArgs& a, int n_wg, hipStream_t st) {
    const size_t lds = sizeof(float) * 4 * WAVE * (size_t)a.S * RW * MB;
    if (a.x_f32)
        hipLaunchKernelGGL((gemm_bf16_small_kernel<RW, CW, MB, true, WT>), dim3(n_wg), dim3(64 * RW * CW), lds, st, a);
    else
        hipLaunchKernelGGL((gemm_bf16_small_kernel<RW, CW, MB, false, WT>), dim3(n_wg), dim3(64 * RW * CW), lds, st, a);
}

template <int NW, int MB, bool PARTIAL, int WV, bool WT>
static void launch_gemm(const GemmArgs& a, dim3 grid, hipStream_t st) {
    constexpr int PD = 3;   // register sets in rotation (4 measured no faster: fewer waves fit)
    const dim3 blk(64 * WV);
    if (a.x_f32) {
        if (a.c_per > 1) hipLaunchKernelGGL((gemm_bf16_kernel<NW, MB, true, PARTIAL, PD, true, WV, WT>), grid, blk, 0, st, a);
        else hipLaunchKernelGGL((gemm_bf16_kernel<NW, MB, false, PARTIAL, PD, true, WV, WT>), grid, blk, 0, st, a);
    } else {
        if (a.c_per > 1) hipLaunchKernelGGL((gemm_bf16_kernel<NW, MB, true, PARTIAL, PD, false, WV, WT>), grid, blk, 0, st, a);
        else hipLaunchKernelGGL((gemm_bf16_kernel<NW, MB, false, PARTIAL, PD, false, WV, WT>), grid, blk, 0, st, a);
    }
}

// the plan's kernel; tiled W always comes in whole 128-k blocks
template <bool WT>
static void launch_plan(const GemmPlan& p, const GemmArgs& a, dim3 grid, hipStream_t st) {
    const bool whole = WT || a.KC % GKB == 0;
    if (p.wv == 7) {   // one fragment per wave, an x tile of 16 to 128 rows, whole 128-k blocks (the plan's test)
        if (p.mb == 2) launch_gemm<1, 2, false, 7, WT>(a, grid, st);
        else if (p.mb == 3) launch_gemm<1, 3, false, 7, WT>(a, grid, st);
        else if (p.mb == 4) launch_gemm<1, 4, false, 7, WT>(a, grid, st);
        else if (p.mb == 5) launch_gemm<1, 5, false, 7, WT>(a, grid, st);
        else if (p.mb == 6) launch_gemm<1, 6, false, 7, WT>(a, grid, st);
        else if (p.mb == 7) launch_gemm<1, 7, false, 7, WT>(a, grid, st);
        else if (p.mb == 8) launch_gemm<1, 8, false, 7, WT>(a, grid, st);
        else launch_gemm<1, 1, false, 7, WT>(a, grid, st);
    } else if (p.nw == 2 && p.mb == 5) {   // two fragments (K % 128 == 0), x tiles of 80 to 112 rows
        launch_gemm<2, 5, false, 4, WT>(a, grid, st);
    } else if (p.nw == 2 && p.mb == 6) {
        launch_gemm<2, 6, false, 4, WT>(a, grid, st);
    } else if (p.nw == 2 && p.mb == 7) {
        launch_gemm<2, 7, false, 4, WT>(a, grid, st);
    } else if (p.nw == 2 && p.mb == 4) {   // K % 128 == 0 with two fragments
        launch_gemm<2, 4, false, 4, WT>(a, grid, st);
    } else if (p.nw == 2) {
        launch_gemm<2, 8, false, 4, WT>(a, grid, st);
    } else if (p.mb == 1) {
        if (whole) launch_gemm<1, 1, false, 4, WT>(a, grid, st);
        else launch_gemm<1, 1, true, 4, false>(a, grid, st);
    } else if (p.mb == 2) {
        if (whole) launch_gemm<1, 2, false, 4, WT>(a, grid, st);
        else launch_gemm<1, 2, true, 4, false>(a, grid, st);
    } else {
        if (whole) launch_gemm<1, 4, false, 4, WT>(a, grid, st);
        else launch_gemm<1, 4, true, 4, false>(a, grid, st);
    }
}

extern "C" int dkv_gemm_bf16(const void* x, int32_t x_dtype, const void* w, const void* bias, int32_t M, int32_t N,
                             int32_t K, void* y, int32_t y_dtype, int32_t flags, void* work, size_t work_bytes,
                             dkv_stream_t stream) {
    DKV_REQUIRE(x && w && y, "dkv_gemm_bf16: NULL argument");
    DKV_REQUIRE(M >= 0 && N > 0 && K > 0, "dkv_gemm_bf16: bad sizes");
    DKV_REQUIRE(K % 32 == 0, "dkv_gemm_bf16: K must be a multiple of 32");
    DKV_REQUIRE(y_dtype == DKV_BF16 || y_dtype == DKV_F32, "dkv_gemm_bf16: y must be bf16 or float32");
    DKV_REQUIRE(x_dtype == DKV_BF16 || x_dtype == DKV_F32, "dkv_gemm_bf16: x must be bf16 or float32");
    DKV_REQUIRE((flags & ~(DKV_GEMM_SWIGLU | DKV_GEMM_DEFER | DKV_GEMM_WTILED)) == 0, "dkv_gemm_bf16: unknown flags");
    const int swiglu = (flags & DKV_GEMM_SWIGLU) != 0;
    const int defer = (flags & DKV_GEMM_DEFER) != 0;
    const bool wt = (flags & DKV_GEMM_WTILED) != 0;
    DKV_REQUIRE(!wt || (K % GKB == 0 && N % 16 == 0), "dkv_gemm_bf16: tiled W needs K % 128 == 0 and N % 16 == 0");
    DKV_REQUIRE(!swiglu || N % 16 == 0, "dkv_gemm_bf16: the SwiGLU epilogue needs N a multiple of 16");
    DKV_REQUIRE(!defer || (!swiglu && !bias && y_dtype == DKV_BF16),
                "dkv_gemm_bf16: deferred partials are for a bf16 y without bias or SwiGLU");
    DKV_REQUIRE(!swiglu || (y_dtype == DKV_BF16 && !bias),
                "dkv_gemm_bf16: the SwiGLU epilogue writes bf16 and takes no bias");
    DKV_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(y) % 16 == 0,
                "dkv_gemm_bf16: x, w and y must be 16-byte aligned");
    DKV_REQUIRE(reinterpret_cast<uintptr_t>(bias) % 8 == 0, "dkv_gemm_bf16: bias must be 8-byte aligned");
    if (M == 0) return DKV_OK;
    const int S = gemm_chunks(N, K);
    const GemmPlan p = gemm_plan(M, N, K);
    const size_t need = dkv_gemm_bf16_workspace(M, N, K);
    if (need && (!work || work_bytes < need))
        return fail(DKV_EWORKSPACE, "dkv_gemm_bf16: workspace too small (need " + std::to_string(need) + ")");
    DKV_REQUIRE(reinterpret_cast<uintptr_t>(work) % 16 == 0, "dkv_gemm_bf16: workspace must be 16-byte aligned");
    GemmArgs a;
    a.x = x;
    a.x_f32 = x_dtype == DKV_F32;
    a.w = static_cast<const uint16_t*>(w);
    a.bias = static_cast<const uint16_t*>(bias);
    a.M = M, a.N = N, a.K = K, a.S = S, a.KC = K / S, a.c_per = p.c_per;
    a.units = p.n_tiles * (S / p.c_per);
    a.m_tiles = p.m_tiles;
    a.part = need ? static_cast<float*>(work) : nullptr;
    a.y = y;
    a.y_f32 = y_dtype == DKV_F32;
    a.swiglu = swiglu;
    hipStream_t st = as_stream(stream);
    if (p.small) {
        DKV_REQUIRE((int64_t)S * p.rw * p.mb * 4 * WAVE * sizeof(float) <= 64 * 1024, "dkv_gemm_bf16: too many K chunks");
        if (wt) launch_small<1, 4, 1, true>(a, p.n_tiles, st);   // S >= 4, a power of two; chunks of whole 128-k blocks
        else launch_small<1, 4, 1, false>(a, p.n_tiles, st);
        return check_launch("dkv_gemm_bf16");
    }
    const int64_t nwg = (int64_t)(a.units + 7) / 8 * 8 * p.m_tiles;
    DKV_REQUIRE(nwg < (int64_t)1 << 31, "dkv_gemm_bf16: too many workgroups");
    const dim3 grid((unsigned)nwg);
    if (wt) launch_plan<true>(p, a, grid, st);
    else launch_plan<false>(p, a, grid, st);
    int rc = check_launch("dkv_gemm_bf16");
    if (rc || !need || defer) return rc;   // deferred: the consumer sums the partials
    const int64_t MN = (int64_t)M * N;   // a multiple of 16
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0, st, a.part, MN, S, N,
                       a.bias, y, a.y_f32, a.swiglu);
    return check_launch("dkv_gemm_bf16(reduce)");
}
