// Sampling and the verify decision.
// Reference: draftkv/engine.py:36-41 (`_probs`), :101-106 (`_sample`),
// :176-179 (the drafter's kept distributions), :188-213 (accept loop, bonus
// token, residual resample).
//
// Three launches (rows of `vocab` float32 logits; every exp in float64 by the
// table-driven dexp below):
//   1. stats   persistent waves, one chunk of SCH logits of one row at a
//              time: chunk max and the float64 sum exp(x/T - max/T) (greedy:
//              the max and its first index). Draft rows whose normalisers the
//              caller kept from the draft steps' samples are skipped.
//   2. finish  grid (pick chunk of PCH logits, sequence): every block of a
//              sequence merges the chunk statistics of the rows it tests and
//              runs the accept tests with the supplied uniforms, one lane per
//              drafted position and a ballot for the first rejection (the
//              same decisions in every block: the arithmetic is
//              deterministic). Then the draw from the final distribution, the
//              first index whose cumulative mass exceeds u * total (numpy
//              Generator.choice semantics: searchsorted 'right'): for p (every
//              position accepted) the chunk masses follow from the row
//              statistics, so every block knows the chosen chunk and the block
//              holding it draws; for the residual clip(p - q) each block sums
//              its chunk and stores its threads' sums. Greedy: argmax
//              comparisons, one block per sequence.
//   3. pick    grid (sequence), the residual only: the chunk from the chunk
//              sums, the crossing thread from its stored sums, and the draw
//              among that thread's masses; an all-zero residual falls back to p
//              (engine.py:210-211).
// Sampling one row (dkv_sample) is the gamma = 0 case: the bonus row is it,
// and its normaliser can be handed back to dkv_accept as a draft row's.
#include "dkv_common.h"

#include <algorithm>
#include <atomic>
#include <mutex>

namespace dkv {

constexpr int SCH = 1024;    // logits per stats chunk (one wave, 16 per lane)
constexpr int PCH = 4096;    // logits per pick chunk (one block, 16 consecutive per thread)
constexpr int ABLK = 256;
static_assert(PCH % SCH == 0 && PCH / ABLK == SCH / WAVE, "a pick chunk is whole stats chunks");

struct ChunkStat {
    float mx;
    int arg;
    double sum;   // sum exp((x - mx)/T) over the chunk (T > 0)
};

// ---- float64 exp, Tang's table-driven method (ACM TOMS 15(2), 1989):
// y = (256 e + j) ln2/256 + r with |r| <= ln2/512, exp(y) = 2^e 2^(j/256) exp(r),
// 2^(j/256) from a table of correctly rounded doubles, exp(r) - 1 by its
// degree-4 Taylor polynomial (truncation below 4e-17 relative). Within one
// ulp of a correctly rounded exp for y >= -746; arguments below (and -inf)
// are clamped to -746, whose exp rounds to 0. No branch: the exps of a
// lane's elements interleave.
constexpr int EXP_TAB = 256;
__constant__ double kExp2Tab[EXP_TAB] = {
    0x1.0000000000000p+0, 0x1.00b1afa5abcbfp+0, 0x1.0163da9fb3335p+0, 0x1.02168143b0281p+0,
    0x1.02c9a3e778061p+0, 0x1.037d42e11bbccp+0, 0x1.04315e86e7f85p+0, 0x1.04e5f72f654b1p+0,
    0x1.059b0d3158574p+0, 0x1.0650a0e3c1f89p+0, 0x1.0706b29ddf6dep+0, 0x1.07bd42b72a836p+0,
    0x1.0874518759bc8p+0, 0x1.092bdf66607e0p+0, 0x1.09e3ecac6f383p+0, 0x1.0a9c79b1f3919p+0,
    0x1.0b5586cf9890fp+0, 0x1.0c0f145e46c85p+0, 0x1.0cc922b7247f7p+0, 0x1.0d83b23395decp+0,
    0x1.0e3ec32d3d1a2p+0, 0x1.0efa55fdfa9c5p+0, 0x1.0fb66affed31bp+0, 0x1.1073028d7233ep+0,
    0x1.11301d0125b51p+0, 0x1.11edbab5e2ab6p+0, 0x1.12abdc06c31ccp+0, 0x1.136a814f204abp+0,
    0x1.1429aaea92de0p+0, 0x1.14e95934f312ep+0, 0x1.15a98c8a58e51p+0, 0x1.166a45471c3c2p+0,
    0x1.172b83c7d517bp+0, 0x1.17ed48695bbc0p+0, 0x1.18af9388c8deap+0, 0x1.1972658375d2fp+0,
    0x1.1a35beb6fcb75p+0, 0x1.1af99f8138a1cp+0, 0x1.1bbe084045cd4p+0, 0x1.1c82f95281c6bp+0,
    0x1.1d4873168b9aap+0, 0x1.1e0e75eb44027p+0, 0x1.1ed5022fcd91dp+0, 0x1.1f9c18438ce4dp+0,
    0x1.2063b88628cd6p+0, 0x1.212be3578a819p+0, 0x1.21f49917ddc96p+0, 0x1.22bdda27912d1p+0,
    0x1.2387a6e756238p+0, 0x1.2451ffb82140ap+0, 0x1.251ce4fb2a63fp+0, 0x1.25e85711ece75p+0,
    0x1.26b4565e27cddp+0, 0x1.2780e341ddf29p+0, 0x1.284dfe1f56381p+0, 0x1.291ba7591bb70p+0,
    0x1.29e9df51fdee1p+0, 0x1.2ab8a66d10f13p+0, 0x1.2b87fd0dad990p+0, 0x1.2c57e39771b2fp+0,
    0x1.2d285a6e4030bp+0, 0x1.2df961f641589p+0, 0x1.2ecafa93e2f56p+0, 0x1.2f9d24abd886bp+0,
    0x1.306fe0a31b715p+0, 0x1.31432edeeb2fdp+0, 0x1.32170fc4cd831p+0, 0x1.32eb83ba8ea32p+0,
    0x1.33c08b26416ffp+0, 0x1.3496266e3fa2dp+0, 0x1.356c55f929ff1p+0, 0x1.36431a2de883bp+0,
    0x1.371a7373aa9cbp+0, 0x1.37f26231e754ap+0, 0x1.38cae6d05d866p+0, 0x1.39a401b7140efp+0,
    0x1.3a7db34e59ff7p+0, 0x1.3b57fbfec6cf4p+0, 0x1.3c32dc313a8e5p+0, 0x1.3d0e544ede173p+0,
    0x1.3dea64c123422p+0, 0x1.3ec70df1c5175p+0, 0x1.3fa4504ac801cp+0, 0x1.40822c367a024p+0,
    0x1.4160a21f72e2ap+0, 0x1.423fb2709468ap+0, 0x1.431f5d950a897p+0, 0x1.43ffa3f84b9d4p+0,
    0x1.44e086061892dp+0, 0x1.45c2042a7d232p+0, 0x1.46a41ed1d0057p+0, 0x1.4786d668b3237p+0,
    0x1.486a2b5c13cd0p+0, 0x1.494e1e192aed2p+0, 0x1.4a32af0d7d3dep+0, 0x1.4b17dea6db7d7p+0,
    0x1.4bfdad5362a27p+0, 0x1.4ce41b817c114p+0, 0x1.4dcb299fddd0dp+0, 0x1.4eb2d81d8abffp+0,
    0x1.4f9b2769d2ca7p+0, 0x1.508417f4531eep+0, 0x1.516daa2cf6642p+0, 0x1.5257de83f4eefp+0,
    0x1.5342b569d4f82p+0, 0x1.542e2f4f6ad27p+0, 0x1.551a4ca5d920fp+0, 0x1.56070dde910d2p+0,
    0x1.56f4736b527dap+0, 0x1.57e27dbe2c4cfp+0, 0x1.58d12d497c7fdp+0, 0x1.59c0827ff07ccp+0,
    0x1.5ab07dd485429p+0, 0x1.5ba11fba87a03p+0, 0x1.5c9268a5946b7p+0, 0x1.5d84590998b93p+0,
    0x1.5e76f15ad2148p+0, 0x1.5f6a320dceb71p+0, 0x1.605e1b976dc09p+0, 0x1.6152ae6cdf6f4p+0,
    0x1.6247eb03a5585p+0, 0x1.633dd1d1929fdp+0, 0x1.6434634ccc320p+0, 0x1.652b9febc8fb7p+0,
    0x1.6623882552225p+0, 0x1.671c1c70833f6p+0, 0x1.68155d44ca973p+0, 0x1.690f4b19e9538p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6b052fa75173ep+0, 0x1.6c012750bdabfp+0, 0x1.6cfdcddd47645p+0,
    0x1.6dfb23c651a2fp+0, 0x1.6ef9298593ae5p+0, 0x1.6ff7df9519484p+0, 0x1.70f7466f42e87p+0,
    0x1.71f75e8ec5f74p+0, 0x1.72f8286ead08ap+0, 0x1.73f9a48a58174p+0, 0x1.74fbd35d7cbfdp+0,
    0x1.75feb564267c9p+0, 0x1.77024b1ab6e09p+0, 0x1.780694fde5d3fp+0, 0x1.790b938ac1cf6p+0,
    0x1.7a11473eb0187p+0, 0x1.7b17b0976cfdbp+0, 0x1.7c1ed0130c132p+0, 0x1.7d26a62ff86f0p+0,
    0x1.7e2f336cf4e62p+0, 0x1.7f3878491c491p+0, 0x1.80427543e1a12p+0, 0x1.814d2add106d9p+0,
    0x1.82589994cce13p+0, 0x1.8364c1eb941f7p+0, 0x1.8471a4623c7adp+0, 0x1.857f4179f5b21p+0,
    0x1.868d99b4492edp+0, 0x1.879cad931a436p+0, 0x1.88ac7d98a6699p+0, 0x1.89bd0a478580fp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8be05bad61778p+0, 0x1.8cf3216b5448cp+0, 0x1.8e06a5e0866d9p+0,
    0x1.8f1ae99157736p+0, 0x1.902fed0282c8ap+0, 0x1.9145b0b91ffc6p+0, 0x1.925c353aa2fe2p+0,
    0x1.93737b0cdc5e5p+0, 0x1.948b82b5f98e5p+0, 0x1.95a44cbc8520fp+0, 0x1.96bdd9a7670b3p+0,
    0x1.97d829fde4e50p+0, 0x1.98f33e47a22a2p+0, 0x1.9a0f170ca07bap+0, 0x1.9b2bb4d53fe0dp+0,
    0x1.9c49182a3f090p+0, 0x1.9d674194bb8d5p+0, 0x1.9e86319e32323p+0, 0x1.9fa5e8d07f29ep+0,
    0x1.a0c667b5de565p+0, 0x1.a1e7aed8eb8bbp+0, 0x1.a309bec4a2d33p+0, 0x1.a42c980460ad8p+0,
    0x1.a5503b23e255dp+0, 0x1.a674a8af46052p+0, 0x1.a799e1330b358p+0, 0x1.a8bfe53c12e59p+0,
    0x1.a9e6b5579fdbfp+0, 0x1.ab0e521356ebap+0, 0x1.ac36bbfd3f37ap+0, 0x1.ad5ff3a3c2774p+0,
    0x1.ae89f995ad3adp+0, 0x1.afb4ce622f2ffp+0, 0x1.b0e07298db666p+0, 0x1.b20ce6c9a8952p+0,
    0x1.b33a2b84f15fbp+0, 0x1.b468415b749b1p+0, 0x1.b59728de5593ap+0, 0x1.b6c6e29f1c52ap+0,
    0x1.b7f76f2fb5e47p+0, 0x1.b928cf22749e4p+0, 0x1.ba5b030a1064ap+0, 0x1.bb8e0b79a6f1fp+0,
    0x1.bcc1e904bc1d2p+0, 0x1.bdf69c3f3a207p+0, 0x1.bf2c25bd71e09p+0, 0x1.c06286141b33dp+0,
    0x1.c199bdd85529cp+0, 0x1.c2d1cd9fa652cp+0, 0x1.c40ab5fffd07ap+0, 0x1.c544778fafb22p+0,
    0x1.c67f12e57d14bp+0, 0x1.c7ba88988c933p+0, 0x1.c8f6d9406e7b5p+0, 0x1.ca3405751c4dbp+0,
    0x1.cb720dcef9069p+0, 0x1.ccb0f2e6d1675p+0, 0x1.cdf0b555dc3fap+0, 0x1.cf3155b5bab74p+0,
    0x1.d072d4a07897cp+0, 0x1.d1b532b08c968p+0, 0x1.d2f87080d89f2p+0, 0x1.d43c8eacaa1d6p+0,
    0x1.d5818dcfba487p+0, 0x1.d6c76e862e6d3p+0, 0x1.d80e316c98398p+0, 0x1.d955d71ff6075p+0,
    0x1.da9e603db3285p+0, 0x1.dbe7cd63a8315p+0, 0x1.dd321f301b460p+0, 0x1.de7d5641c0658p+0,
    0x1.dfc97337b9b5fp+0, 0x1.e11676b197d17p+0, 0x1.e264614f5a129p+0, 0x1.e3b333b16ee12p+0,
    0x1.e502ee78b3ff6p+0, 0x1.e653924676d76p+0, 0x1.e7a51fbc74c83p+0, 0x1.e8f7977cdb740p+0,
    0x1.ea4afa2a490dap+0, 0x1.eb9f4867cca6ep+0, 0x1.ecf482d8e67f1p+0, 0x1.ee4aaa2188510p+0,
    0x1.efa1bee615a27p+0, 0x1.f0f9c1cb6412ap+0, 0x1.f252b376bba97p+0, 0x1.f3ac948dd7274p+0,
    0x1.f50765b6e4540p+0, 0x1.f6632798844f8p+0, 0x1.f7bfdad9cbe14p+0, 0x1.f91d802243c89p+0,
    0x1.fa7c1819e90d8p+0, 0x1.fbdba3692d514p+0, 0x1.fd3c22b8f71f1p+0, 0x1.fe9d96b2a23d9p+0
};

// the table in a block's LDS (callers synchronise before the first dexp)
__device__ __forceinline__ void load_exp_tab(double* tab) {
    for (int i = threadIdx.x; i < EXP_TAB; i += blockDim.x) tab[i] = kExp2Tab[i];
}

// dexp of N arguments at once, stage by stage across the N: the N table
// reads are in flight together and the float64 chains interleave
template <int N>
__device__ __forceinline__ void dexp_n(const double* y, double* out, const double* tab) {
    double r[N], t[N];
    int e[N];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const double yc = fmax(y[k], -746.0);
        const double n = __builtin_rint(yc * 0x1.71547652b82fep+8);   // y * 256 / ln2, to nearest
        // ln2/256 in two parts: n * hi is exact for |n| < 2^19
        r[k] = fma(-n, 0x1.cf79abc9e3b3ap-48, fma(-n, 0x1.62e42fefa0000p-9, yc));
        const int ni = (int)n;
        e[k] = ni >> 8;
        t[k] = tab[ni & (EXP_TAB - 1)];
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const double q = fma(fma(0x1.5555555555555p-5, r[k], 0x1.5555555555555p-3), r[k], 0.5);   // 1/24, 1/6
        const double p = fma(q, r[k] * r[k], r[k]);                                              // exp(r) - 1
        out[k] = ldexp(fma(t[k], p, t[k]), e[k]);
    }
}

__device__ __forceinline__ double dexp(double y, const double* tab) {
    double v;
    dexp_n<1>(&y, &v, tab);
    return v;
}

// rows 0..gamma: target [batch][gamma+1][vocab]; gamma+1..2*gamma: draft rows
// 0..gamma-1 of draft [gamma][batch][vocab] (step-major, as the draft steps
// produce them)
__device__ __forceinline__ const float* row_ptr(const float* target, const float* draft, int s, int row, int gamma,
                                                int vocab, int batch) {
    if (row <= gamma) return target + ((int64_t)s * (gamma + 1) + row) * vocab;
    return draft + ((int64_t)(row - gamma - 1) * batch + s) * vocab;
}

// ---- stats: one wave per chunk of SCH logits of one row, the chunk held
// in registers: its max (first index on ties), then the float64 sum of
// exp(x/T - max/T) (x/T as x * (1/T): a normaliser needs no correctly
// rounded quotient). A lane holds elements i0 + 256 k + 4 lane + e (k, e in
// 0..3; its indices rise with its register index): VEC (rows start 16-byte
// aligned and vocab % 4 == 0) reads them as four float4, each wave load 1 KB
// contiguous, else as 16 floats. SAMP: the exp sum and no index (sampling
// reads none); else the first index of the max and no sum. Waves are
// persistent: each takes chunks n_waves apart and fetches its next chunk
// before reducing the current one.
template <bool VEC>
__device__ __forceinline__ void load_chunk(const float* x, int i0, int i1, int lane, float (&xv)[SCH / WAVE]) {
    // lane l, register k holds element i0 + 256 (k / 4) + 4 l + k % 4 in both
    // paths (the float64 sums then add the same values in the same order
    // whether the row is read with float4 or float loads)
    if constexpr (VEC) {
#pragma unroll
        for (int k = 0; k < SCH / WAVE / 4; ++k) {
            const int i = i0 + 256 * k + 4 * lane;   // i1 % 4 == 0: the float4 is whole or past the end
            const float4 v = i < i1 ? *reinterpret_cast<const float4*>(x + i)
                                    : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            xv[4 * k] = v.x;
            xv[4 * k + 1] = v.y;
            xv[4 * k + 2] = v.z;
            xv[4 * k + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < SCH / WAVE; ++k) {
            const int i = i0 + 256 * (k / 4) + 4 * lane + k % 4;
            xv[k] = i < i1 ? x[i] : -INFINITY;
        }
    }
}

template <bool VEC, bool SAMP>
__global__ void __launch_bounds__(ABLK) stats_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                     int gamma, int vocab, int batch, float T, int nsc, int rows,
                                                     int n_items, ChunkStat* __restrict__ stats) {
    constexpr int PER = SCH / WAVE;
    const int lane = threadIdx.x % WAVE;
    const int nw = gridDim.x * (ABLK / WAVE);
    __shared__ double tab[EXP_TAB];
    if constexpr (SAMP) {
        load_exp_tab(tab);
        __syncthreads();
    }
    auto row_of = [&](int it, int& s, int& r, int& c) {
        c = it % nsc;
        r = (it / nsc) % rows;
        s = it / (nsc * rows);
    };
    auto idx = [&](int k) { return 256 * (k / 4) + 4 * lane + k % 4; };
    int it = blockIdx.x * (ABLK / WAVE) + (int)threadIdx.x / WAVE;
    float xn[PER];
    if (it < n_items) {
        int s, r, c;
        row_of(it, s, r, c);
        load_chunk<VEC>(row_ptr(target, draft, s, r, gamma, vocab, batch), c * SCH, min(vocab, c * SCH + SCH), lane, xn);
    }
    for (; it < n_items; it += nw) {
        float xv[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) xv[k] = xn[k];
        if (it + nw < n_items) {   // the next chunk's loads are in flight while this one is reduced
            int s, r, c;
            row_of(it + nw, s, r, c);
            load_chunk<VEC>(row_ptr(target, draft, s, r, gamma, vocab, batch), c * SCH, min(vocab, c * SCH + SCH), lane,
                            xn);
        }
        int s, r, c;
        row_of(it, s, r, c);
        float mx = -INFINITY;
        int arg = INT_MAX;
        double sum = 0.0;
        if constexpr (SAMP) {   // the max alone (no index: sampling reads none)
#pragma unroll
            for (int k = 0; k < PER; ++k) mx = fmaxf(mx, xv[k]);
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            const double iT = 1.0 / (double)T, mT = (double)mx * iT;
            double y[PER], ex[PER];
#pragma unroll
            for (int k = 0; k < PER; ++k) y[k] = (double)xv[k] * iT - mT;   // past the row: -inf, exp 0
            dexp_n<PER>(y, ex, tab);
#pragma unroll
            for (int k = 0; k < PER; ++k) sum += ex[k];
            sum = wave_sum_d(sum);
        } else {   // the max and its first index
            const int i0 = c * SCH;
#pragma unroll
            for (int k = 0; k < PER; ++k)   // indices rise with k: the lane's first maximum is kept
                if (xv[k] > mx) {
                    mx = xv[k];
                    arg = i0 + idx(k);
                }
            for (int o = 32; o > 0; o >>= 1) {
                const float om = __shfl_xor(mx, o);
                const int oa = __shfl_xor(arg, o);
                if (om > mx || (om == mx && oa < arg)) {
                    mx = om;
                    arg = oa;
                }
            }
        }
        if (lane == 0) {
            ChunkStat& cs = stats[((int64_t)s * (2 * gamma + 1) + r) * nsc + c];
            cs.mx = mx;
            cs.arg = arg;
            cs.sum = sum;
        }
    }
}

struct RowNorm {   // the layout of dkv_row_stats_t
    double m;   // max(x)/T
    double S;   // sum exp(x/T - m)
    double iS;  // 1 / S
    int arg;
    int reserved;
};
static_assert(sizeof(RowNorm) == sizeof(dkv_row_stats_t) && alignof(RowNorm) == alignof(dkv_row_stats_t),
              "RowNorm is dkv_row_stats_t");

// what the pick kernel needs of a sequence whose final distribution is the residual
struct PickRec {
    int mode;   // 2: residual of target row `row` against draft row `row`; else nothing to pick
    int row;
    double u;
    RowNorm pn, qn;
};

// p(x) = exp(x/T - m) / S with x/T as x * (1/T) and the division by S as a
// product with its reciprocal (each within an ulp of the quotient). The
// product is rounded on its own (no contraction into a following add), so
// equal rows give equal probabilities and p - q is exactly 0 where p == q.
__device__ __forceinline__ double prob(float x, const RowNorm& r, float T, const double* tab) {
#pragma clang fp contract(off)
    return dexp((double)x * (1.0 / (double)T) - r.m, tab) * r.iS;
}

__device__ __forceinline__ double mul_rn(double a, double b) {
#pragma clang fp contract(off)
    return a * b;
}

__device__ __forceinline__ double resid(double p, double q) {
#pragma clang fp contract(off)
    const double r = p - q;
    return r > 0.0 ? r : 0.0;
}

// Masses of the PER consecutive indices b0 = i0 + PER t .. b0+PER-1 of thread
// t (those below i1; i1 - i0 <= PCH) under the final distribution: p (mode 1)
// or clip(p - q) (mode 2). The range is read with coalesced loads (each wave
// load one contiguous KB: float4 at i0 + 4 (t + 256 j); VEC) into the LDS
// stage, then each thread takes its PER consecutive values from there. Every
// thread of the block calls it.
template <bool VEC>
__device__ __forceinline__ double range_masses(const float* pr, const float* qr, const RowNorm& pn, const RowNorm& qn,
                                               int mode, int i0, int i1, float T, const double* tab, float* stage,
                                               double* v) {
    constexpr int PER = PCH / ABLK;
    const int tid = threadIdx.x, b0 = i0 + PER * tid;
    float* sp = stage;
    float* sq = stage + PCH;
    // unconditional loads (an index past i1 reads the last float4 or float
    // before it; those values are replaced by -inf below): all in flight together
    if constexpr (VEC) {   // i0 % 4 == 0 and i1 % 4 == 0
#pragma unroll
        for (int j = 0; j < PCH / (4 * ABLK); ++j) {
            const int o = 4 * (tid + ABLK * j), i = min(i0 + o, i1 - 4);
            const float4 a = *reinterpret_cast<const float4*>(pr + i);
            *reinterpret_cast<float4*>(sp + o) = a;
            if (mode == 2) *reinterpret_cast<float4*>(sq + o) = *reinterpret_cast<const float4*>(qr + i);
        }
    } else {
#pragma unroll
        for (int j = 0; j < PCH / ABLK; ++j) {
            const int o = tid + ABLK * j, i = min(i0 + o, i1 - 1);
            sp[o] = pr[i];
            if (mode == 2) sq[o] = qr[i];
        }
    }
    __syncthreads();
    float xp[PER], xq[PER];
#pragma unroll
    for (int k = 0; k < PER; k += 4) {
        const float4 a = *reinterpret_cast<const float4*>(sp + PER * tid + k);
        const float4 b = mode == 2 ? *reinterpret_cast<const float4*>(sq + PER * tid + k) : a;
        const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool in = b0 + k + e < i1;
            xp[k + e] = in ? av[e] : -INFINITY;
            xq[k + e] = in ? bv[e] : -INFINITY;
        }
    }
    __syncthreads();   // the stage is free again when the function returns
    // past i1 both logits are -inf: mass 0. p(x) = exp(x/T - m) * (1/S) as prob() computes it.
    // Eight at a time (the exps of eight interleave; fewer registers than sixteen).
    constexpr int H = 8;
    const double iT = 1.0 / (double)T;
    double loc = 0.0;
#pragma unroll
    for (int h = 0; h < PER; h += H) {
        double y[H], ep[H];
#pragma unroll
        for (int k = 0; k < H; ++k) y[k] = (double)xp[h + k] * iT - pn.m;
        dexp_n<H>(y, ep, tab);
        if (mode == 1) {
#pragma unroll
            for (int k = 0; k < H; ++k) v[h + k] = mul_rn(ep[k], pn.iS);
        } else {
            double eq[H];
#pragma unroll
            for (int k = 0; k < H; ++k) y[k] = (double)xq[h + k] * iT - qn.m;
            dexp_n<H>(y, eq, tab);
#pragma unroll
            for (int k = 0; k < H; ++k) v[h + k] = resid(mul_rn(ep[k], pn.iS), mul_rn(eq[k], qn.iS));
        }
#pragma unroll
        for (int k = 0; k < H; ++k) loc += v[h + k];
    }
    return loc;
}

// Draw within [i0, i1) (at most PCH indices; thread t owns PER consecutive
// ones from i0 + PER t, with masses v and their sum loc): the first index
// whose running mass, from `before` at i0, exceeds tgt. One block-wide
// exclusive scan of the threads' sums; the thread whose range crosses the
// target walks its own indices. A draw that rounding pushes past the end
// takes the last index with positive mass (the reference's cdf ends at
// exactly 1). Every thread of the block calls it; thread 0 returns the index.
__device__ __forceinline__ int scan_draw(const double* v, double loc, int i0, int i1, double before, double tgt,
                                         double* wsum, int* found, int* last_pos) {
    constexpr int PER = PCH / ABLK;
    const int tid = threadIdx.x, lane = tid % WAVE, w = tid / WAVE;
    const int b0 = i0 + PER * tid;
    double x = loc;
    for (int o = 1; o < WAVE; o <<= 1) {
        const double y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == WAVE - 1) wsum[w] = x;
    if (tid == 0) {
        *found = INT_MAX;
        *last_pos = -1;
    }
    __syncthreads();
    double off = before + (x - loc);
    for (int k = 0; k < w; ++k) off += wsum[k];
    int hit = INT_MAX, lastp = -1;
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (v[k] > 0.0) lastp = b0 + k;
    if (off + loc > tgt) {
        double run = off;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            run += v[k];
            if (hit == INT_MAX && v[k] > 0.0 && run > tgt) hit = b0 + k;
        }
    }
    if (hit != INT_MAX) atomicMin(found, hit);
    if (lastp >= 0) atomicMax(last_pos, lastp);
    __syncthreads();
    return *found != INT_MAX ? *found : (*last_pos >= 0 ? *last_pos : i1 - 1);
}

// The first of n masses cm[0..n) (n <= 1024) whose running sum exceeds
// u * total, by one wave (every lane of it calls this): lane l sums a run of
// g = ceil(n/64) consecutive masses in order, a wave scan of the run sums
// gives each run's start and the total, and the first run that crosses the
// target walks its masses in order. Returns the index (every lane), with the
// running sum before it and the target; rounding that carries the draw past
// the end takes the last one, scanned from its start. Deterministic: the
// same masses give the same choice.
__device__ __forceinline__ int choose(const double* cm, int n, double u, double& before, double& tgt, double& total) {
    const int lane = threadIdx.x % WAVE, g = (n + WAVE - 1) / WAVE, c0 = min(n, lane * g), c1 = min(n, c0 + g);
    double loc = 0.0;
    for (int c = c0; c < c1; ++c) loc += cm[c];
    double x = loc;
    for (int o = 1; o < WAVE; o <<= 1) {
        const double y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    total = __shfl(x, WAVE - 1);
    tgt = u * total;
    double run = x - loc;
    int hit = INT_MAX;
    double hit_before = 0.0;
    if (run + loc > tgt) {
        for (int c = c0; c < c1; ++c) {
            if (run + cm[c] > tgt) {
                hit = c;
                hit_before = run;
                break;
            }
            run += cm[c];
        }
    }
    const uint64_t m = __ballot(hit != INT_MAX);
    if (m) {
        const int src_lane = __ffsll((unsigned long long)m) - 1;
        before = __shfl(hit_before, src_lane);
        return __shfl(hit, src_lane);
    }
    before = total - cm[n - 1];
    return n - 1;
}

// p's masses per stats chunk from the row statistics (no pass over the row)
__device__ __forceinline__ void p_chunk_masses(const ChunkStat* pst, int nsc, const RowNorm& pn, float T,
                                               const double* tab, double* cm) {
    const double iT = 1.0 / (double)T;
    for (int c = threadIdx.x; c < nsc; c += ABLK) cm[c] = pst[c].sum * dexp((double)pst[c].mx * iT - pn.m, tab) * pn.iS;
}

constexpr int FWAVES = ABLK / WAVE;          // waves of a finish block
constexpr int WALK = 8;                      // drafted positions tested per round of row merges
constexpr int MROWS = (2 * WALK + 1 + FWAVES - 1) / FWAVES;   // rows one wave merges per round
constexpr int PICK_MAX_CHUNKS = 1024;        // stats chunks: vocab up to 1M

// Row norms of up to MROWS rows (row ids rid[0..nr)) from their chunk
// statistics, by one wave, in two phases: merge_max, the row max with the
// first index on ties (lanes over chunks 64 apart, the loads of all the
// wave's rows in flight together); merge_sum, the float64 sum of the chunk
// sums rescaled to the row max and a butterfly sum, lane 0 storing row r's
// norm at out[r]. Slots past nr read row rid 0 and are dropped.
struct MergeMax {
    float mx[MROWS];
    int arg[MROWS];
};

__device__ __forceinline__ MergeMax merge_max(const ChunkStat* __restrict__ st, const int* rid, int nr, int nsc,
                                              int lane) {
    MergeMax m;
#pragma unroll
    for (int r = 0; r < MROWS; ++r) {
        m.mx[r] = -INFINITY;
        m.arg[r] = INT_MAX;
    }
    for (int c = lane; c < nsc; c += WAVE) {
        ChunkStat v[MROWS];
#pragma unroll
        for (int r = 0; r < MROWS; ++r) v[r] = st[(int64_t)rid[r] * nsc + c];
#pragma unroll
        for (int r = 0; r < MROWS; ++r)
            if (r < nr && (v[r].mx > m.mx[r] || (v[r].mx == m.mx[r] && v[r].arg < m.arg[r]))) {
                m.mx[r] = v[r].mx;
                m.arg[r] = v[r].arg;
            }
    }
#pragma unroll
    for (int r = 0; r < MROWS; ++r) {
        if (r < nr) {
            for (int o = WAVE / 2; o > 0; o >>= 1) {
                const float om = __shfl_xor(m.mx[r], o);
                const int oa = __shfl_xor(m.arg[r], o);
                if (om > m.mx[r] || (om == m.mx[r] && oa < m.arg[r])) {
                    m.mx[r] = om;
                    m.arg[r] = oa;
                }
            }
        }
    }
    return m;
}

__device__ __forceinline__ void merge_sum(const ChunkStat* __restrict__ st, const int* rid, int nr, int nsc,
                                          const MergeMax& m, bool samp, float T, const double* tab, int lane,
                                          RowNorm** out) {
    double S[MROWS];
    const double iT = samp ? 1.0 / (double)T : 0.0;
#pragma unroll
    for (int r = 0; r < MROWS; ++r) S[r] = 0.0;
    if (samp) {   // every slot computes: no branches
        for (int c = lane; c < nsc; c += WAVE) {
            double y[MROWS], ex[MROWS], cs[MROWS];
#pragma unroll
            for (int r = 0; r < MROWS; ++r) {
                const ChunkStat v = st[(int64_t)rid[r] * nsc + c];
                y[r] = (double)v.mx * iT - (double)m.mx[r] * iT;
                cs[r] = v.sum;
            }
            dexp_n<MROWS>(y, ex, tab);
#pragma unroll
            for (int r = 0; r < MROWS; ++r) S[r] += cs[r] * ex[r];
        }
    }
#pragma unroll
    for (int r = 0; r < MROWS; ++r) {
        if (r < nr) {
            RowNorm rn{0.0, 0.0, 0.0, m.arg[r], 0};
            if (samp) {
                rn.m = (double)m.mx[r] * iT;
                rn.S = wave_sum_d(S[r]);
                rn.iS = 1.0 / rn.S;
            }
            if (lane == 0) *out[r] = rn;
        }
    }
}

// One block per (pick chunk of PCH indices, sequence); greedy launches chunk
// 0 only. Every block of a sequence makes the same decisions. Then: greedy,
// the outputs; p (every drafted position accepted), the chunk choice over the
// stats chunks' masses and the draw inside the chosen one by the block that
// holds it; the residual, this block's chunk sum (csum) and, from block 0, the
// sequence's PickRec for pick_kernel.
template <bool VEC>
__global__ void __launch_bounds__(ABLK) finish_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                      const int32_t* __restrict__ draft_tokens, int gamma, int vocab,
                                                      float T, const double* __restrict__ u,
                                                      const RowNorm* __restrict__ dstats, RowNorm* __restrict__ row_out,
                                                      int nsc, int npc,
                                                      const ChunkStat* __restrict__ stats, double* __restrict__ csum,
                                                      double* __restrict__ part, PickRec* __restrict__ recs,
                                                      int32_t* __restrict__ accepted,
                                                      int32_t* __restrict__ next_token,
                                                      int32_t* __restrict__ n_uniforms) {
    constexpr int PER = PCH / ABLK;
    const int chunk = blockIdx.x, s = blockIdx.y, batch = gridDim.y;
    const int tid = threadIdx.x, lane = tid % WAVE, w = tid / WAVE;
    const bool samp = T > 0.0f;
    const int R = 2 * gamma + 1;
    const ChunkStat* st = stats + (int64_t)s * R * nsc;
    const double* us = u + (int64_t)s * (gamma + 1);
    __shared__ double tab[EXP_TAB];
    __shared__ RowNorm tn[WALK + 1], dn[WALK];   // norms of this round's target and draft rows
    __shared__ double su[WALK + 1];              // this round's uniforms, and the one after them
    __shared__ int s_stop, s_chunk, found, last_pos;
    __shared__ double s_before, s_target;
    // the chunk masses of a choice and the range stage are never live together
    __shared__ __align__(16) float stage[2 * PCH];
    static_assert(PICK_MAX_CHUNKS * sizeof(double) <= sizeof(float) * 2 * PCH, "s_cm fits the stage");
    double* s_cm = reinterpret_cast<double*>(stage);
    __shared__ double wsum[FWAVES];
    // the exp table is fetched into registers first and stored once the first merge loads are in flight
    double tab_v = 0.0;
    if (samp && tid < EXP_TAB) tab_v = kExp2Tab[tid];
    static_assert(EXP_TAB <= ABLK, "one table entry per thread");

    // ---- the tests, WALK positions per round. Wave 0's lanes fetch the
    // round's drafted tokens, their logits and uniforms while every wave merges
    // the round's rows (target rows base.., the bonus row gamma with the last
    // round, and, sampling, the draft rows); then each lane decides its own
    // position and a ballot finds the first rejection. Every tested position
    // takes one uniform when sampling, so the draws used follow from it.
    int base = 0, n = 0, acc = 0;
    if (tid == 0) s_stop = 0;   // (gamma 0: no test writes it)
    for (;; base += WALK) {
        n = min(WALK, gamma - base);
        const bool last = base + n == gamma;
        const int nt = n + (last ? 1 : 0), nd = samp && !dstats ? n : 0;   // draft rows to merge
        int d = -1;
        float xp = 0.0f, xq = 0.0f;
        if (w == 0 && lane <= n) {
            const int i = base + lane;
            if (samp) su[lane] = us[i];
            if (lane < n) {
                d = draft_tokens[(int64_t)s * gamma + i];
                if (samp && d >= 0 && d < vocab) {   // never read past the row
                    xp = row_ptr(target, draft, s, i, gamma, vocab, batch)[d];
                    xq = row_ptr(target, draft, s, gamma + 1 + i, gamma, vocab, batch)[d];
                }
            }
        }
        int rid[MROWS];
        RowNorm* out[MROWS];
        int nr = 0;
#pragma unroll
        for (int r = 0; r < MROWS; ++r) {
            const int j = w + FWAVES * r;   // the round's j-th row: target rows first
            rid[r] = 0;
            out[r] = tn;
            if (j < nt) {
                rid[r] = base + j;
                out[r] = tn + j;
                nr = r + 1;
            } else if (j < nt + nd) {
                rid[r] = gamma + 1 + base + (j - nt);
                out[r] = dn + (j - nt);
                nr = r + 1;
            }
        }
        const MergeMax mm = merge_max(st, rid, nr, nsc, lane);
        if (base == 0) {
            if (samp && tid < EXP_TAB) tab[tid] = tab_v;
            __syncthreads();
        }
        merge_sum(st, rid, nr, nsc, mm, samp, T, tab, lane, out);
        if (samp && dstats && w == 1 && lane < n) dn[lane] = dstats[(int64_t)(base + lane) * batch + s];
        __syncthreads();
        if (w == 0 && n > 0) {
            bool ok = true;   // lanes past the round pass
            if (lane < n) {
                if (d < 0 || d >= vocab) {
                    ok = false;   // not a token of this vocabulary
                } else if (!samp) {
                    ok = tn[lane].arg == d;
                } else {
                    const double p = prob(xp, tn[lane], T, tab), q = prob(xq, dn[lane], T, tab);
                    const double ratio = q > 0.0 ? p / q : 0.0;
                    ok = su[lane] < fmin(1.0, ratio);
                }
            }
            const uint64_t fail = __ballot(!ok);
            if (lane == 0) s_stop = fail ? base + __ffsll((unsigned long long)fail) : 0;   // 1 + the rejected position
        }
        __syncthreads();
        if (s_stop) {
            acc = s_stop - 1;
            break;
        }
        if (last) {
            acc = gamma;
            break;
        }
    }
    const int used = samp ? min(acc + 1, gamma) : 0;   // uniforms the tests took
    const RowNorm pn = tn[acc - base];   // the final row: rejected position acc, or the bonus row gamma
    if (row_out && chunk == 0 && tid == 0) row_out[s] = pn;   // (one row: dkv_sample's statistics out)

    if (!samp) {
        if (tid == 0) {
            next_token[s] = pn.arg;
            accepted[s] = acc;
            n_uniforms[s] = acc == gamma ? 1 : 0;   // the bonus draw is taken even though p is one-hot
        }
        return;
    }
    const double uf = su[used - base];
    if (chunk == 0 && tid == 0) {
        accepted[s] = acc;
        n_uniforms[s] = used + 1;
    }
    double v[PER];
    if (acc == gamma) {
        // p: every block finds the same stats chunk; the block whose pick chunk holds it draws
        p_chunk_masses(st + (int64_t)acc * nsc, nsc, pn, T, tab, s_cm);
        __syncthreads();
        if (w == 0) {
            double before, tgt, total;
            const int c = choose(s_cm, nsc, uf, before, tgt, total);
            if (lane == 0) s_chunk = c, s_before = before, s_target = tgt;
        }
        __syncthreads();
        const int c = s_chunk;
        if (c / (PCH / SCH) != chunk) return;
        const int i0 = c * SCH, i1 = min(vocab, i0 + SCH);
        const float* pr = row_ptr(target, draft, s, acc, gamma, vocab, batch);
        const double loc = range_masses<VEC>(pr, pr, pn, pn, 1, i0, i1, T, tab, stage, v);
        const int tok = scan_draw(v, loc, i0, i1, s_before, s_target, wsum, &found, &last_pos);
        if (tid == 0) next_token[s] = tok;
        return;
    }
    // the residual of row acc: this block's chunk sum, summed in the draw's order
    const RowNorm qn = dn[acc - base];
    if (chunk == 0 && tid == 0) recs[s] = PickRec{2, acc, uf, pn, qn};
    const int i0 = chunk * PCH, i1 = min(vocab, i0 + PCH);
    const float* pr = row_ptr(target, draft, s, acc, gamma, vocab, batch);
    const float* qr = row_ptr(target, draft, s, gamma + 1 + acc, gamma, vocab, batch);
    const double loc = range_masses<VEC>(pr, qr, pn, qn, 2, i0, i1, T, tab, stage, v);
    part[((int64_t)s * npc + chunk) * ABLK + tid] = loc;   // the thread's sum, for pick_kernel's scan
    double x = loc;
    for (int o = 1; o < WAVE; o <<= 1) {
        const double y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == WAVE - 1) wsum[w] = x;
    __syncthreads();
    if (tid == 0) {
        double t = wsum[0];
        for (int k = 1; k < FWAVES; ++k) t += wsum[k];
        csum[(int64_t)s * npc + chunk] = t;
    }
}

// The residual draw, one block per sequence (after finish_kernel): the pick
// chunk from the chunk sums, then, from the threads' sums finish_kernel
// stored, the thread whose range crosses the target (the scan scan_draw
// makes, on the same values); only that thread's PER masses are recomputed
// and walked. Where that walk finds no index (rounding), the whole chunk is
// scanned as scan_draw does. An all-zero residual falls back to p itself
// (engine.py:210-211), drawn over the stats chunks' masses of p as
// finish_kernel draws p.
template <bool VEC>
__global__ void __launch_bounds__(ABLK) pick_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                    int gamma, int vocab, float T, int nsc, int npc,
                                                    const ChunkStat* __restrict__ stats,
                                                    const double* __restrict__ csum, const double* __restrict__ part,
                                                    const int32_t* __restrict__ accepted,
                                                    const PickRec* __restrict__ recs, int32_t* __restrict__ next_token) {
    constexpr int PER = PCH / ABLK;
    const int s = blockIdx.x, batch = gridDim.x, tid = threadIdx.x, lane = tid % WAVE, w = tid / WAVE;
    if (accepted[s] == gamma) return;   // drawn from p by finish_kernel
    const PickRec rec = recs[s];
    __shared__ double tab[EXP_TAB];
    // the chunk masses of a choice and the range stage are never live together
    __shared__ __align__(16) float stage[2 * PCH];
    static_assert(PICK_MAX_CHUNKS * sizeof(double) <= sizeof(float) * 2 * PCH, "s_cm fits the stage");
    double* s_cm = reinterpret_cast<double*>(stage);
    __shared__ double wsum[FWAVES], sv[PER];
    __shared__ int s_chunk, s_mode, found, last_pos, first_t, s_hit;
    __shared__ double s_before, s_target, s_off;
    load_exp_tab(tab);
    for (int c = tid; c < npc; c += ABLK) s_cm[c] = csum[(int64_t)s * npc + c];
    if (tid == 0) first_t = INT_MAX;
    __syncthreads();
    if (w == 0) {   // an all-zero residual (total 0) falls back to p below
        double before, tgt, total;
        const int c = choose(s_cm, npc, rec.u, before, tgt, total);
        if (lane == 0) s_mode = total > 0.0 ? 2 : 1, s_chunk = c, s_before = before, s_target = tgt;
    }
    __syncthreads();
    const int mode = s_mode;
    const float* pr = row_ptr(target, draft, s, rec.row, gamma, vocab, batch);
    const float* qr = row_ptr(target, draft, s, gamma + 1 + rec.row, gamma, vocab, batch);
    if (mode == 2) {
        const int c = s_chunk, i0 = c * PCH;
        const double tgt = s_target;
        const double loc = part[((int64_t)s * npc + c) * ABLK + tid];
        double x = loc;   // scan_draw's scan of the threads' sums
        for (int o = 1; o < WAVE; o <<= 1) {
            const double y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        if (lane == WAVE - 1) wsum[w] = x;
        __syncthreads();
        double off = s_before + (x - loc);
        for (int k = 0; k < w; ++k) off += wsum[k];
        if (off + loc > tgt) atomicMin(&first_t, tid);
        __syncthreads();
        const int t = first_t;
        if (tid == t) s_off = off;
        if (tid == 0) s_hit = INT_MAX;
        __syncthreads();
        if (t != INT_MAX && w == 0) {
            // lane k < PER: mass k of thread t's range, as range_masses computes it
            const int i = i0 + PER * t + min(lane, PER - 1), i1 = min(vocab, i0 + PCH);
            const double iT = 1.0 / (double)T;
            const float a = pr[min(i, i1 - 1)], b = qr[min(i, i1 - 1)];
            double y[2] = {(double)(i < i1 ? a : -INFINITY) * iT - rec.pn.m,
                           (double)(i < i1 ? b : -INFINITY) * iT - rec.qn.m};
            double e[2];
            dexp_n<2>(y, e, tab);
            if (lane < PER) sv[lane] = resid(mul_rn(e[0], rec.pn.iS), mul_rn(e[1], rec.qn.iS));
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (lane == 0) {
                double run = s_off;
                for (int k = 0; k < PER; ++k) {
                    run += sv[k];
                    if (sv[k] > 0.0 && run > tgt) {
                        s_hit = i0 + PER * t + k;
                        break;
                    }
                }
            }
        }
        __syncthreads();
        if (s_hit != INT_MAX) {
            if (tid == 0) next_token[s] = s_hit;
            return;
        }
        // no crossing found in the stored sums' thread: the chunk's full scan
        const int i1 = min(vocab, i0 + PCH);
        double v[PER];
        const double l2 = range_masses<VEC>(pr, qr, rec.pn, rec.qn, 2, i0, i1, T, tab, stage, v);
        const int tok = scan_draw(v, l2, i0, i1, s_before, tgt, wsum, &found, &last_pos);
        if (tid == 0) next_token[s] = tok;
        return;
    }
    p_chunk_masses(stats + ((int64_t)s * (2 * gamma + 1) + rec.row) * nsc, nsc, rec.pn, T, tab, s_cm);
    __syncthreads();
    if (w == 0) {
        double before, tgt, total;
        const int c = choose(s_cm, nsc, rec.u, before, tgt, total);
        if (lane == 0) s_chunk = c, s_before = before, s_target = tgt;
    }
    __syncthreads();
    const int i0 = s_chunk * SCH, i1 = min(vocab, i0 + SCH);
    double v[PER];
    const double loc = range_masses<VEC>(pr, pr, rec.pn, rec.pn, 1, i0, i1, T, tab, stage, v);
    const int tok = scan_draw(v, loc, i0, i1, s_before, s_target, wsum, &found, &last_pos);
    if (tid == 0) next_token[s] = tok;
}

}  // namespace dkv

using namespace dkv;

static int stats_chunks(int vocab) { return (vocab + SCH - 1) / SCH; }
static int pick_chunks(int vocab) { return (vocab + PCH - 1) / PCH; }

extern "C" size_t dkv_accept_workspace(int32_t batch, int32_t gamma, int32_t vocab) {
    if (batch <= 0 || gamma < 0 || vocab <= 0) return 0;
    const size_t nsc = stats_chunks(vocab), npc = pick_chunks(vocab), R = 2 * (size_t)gamma + 1;
    return sizeof(ChunkStat) * batch * R * nsc + sizeof(double) * batch * npc * (1 + ABLK) + sizeof(PickRec) * batch +
           256;
}

// dkv_accept, and dkv_sample as its gamma-0 case writing the row's statistics to row_out
static int accept_impl(const float* target, const float* draft, const int32_t* draft_tokens, int32_t batch,
                       int32_t gamma, int32_t vocab, float temperature, const double* u,
                       const dkv_row_stats_t* draft_stats, dkv_row_stats_t* row_out, int32_t* accepted,
                       int32_t* next_token, int32_t* n_uniforms, void* work, size_t work_bytes, dkv_stream_t stream) {
    DKV_REQUIRE(target && accepted && next_token && n_uniforms && u, "dkv_accept: NULL argument");
    DKV_REQUIRE(batch > 0 && gamma >= 0 && vocab > 0, "dkv_accept: bad sizes");
    DKV_REQUIRE(stats_chunks(vocab) <= PICK_MAX_CHUNKS, "dkv_accept: vocab too large");
    DKV_REQUIRE(2 * (int64_t)gamma + 1 <= 65535 && batch <= 65535, "dkv_accept: gamma or batch too large for the grid");
    DKV_REQUIRE(gamma == 0 || draft_tokens, "dkv_accept: draft_tokens is NULL");
    DKV_REQUIRE(temperature <= 0.0f || gamma == 0 || draft, "dkv_accept: draft logits needed when T > 0");
    const size_t need = dkv_accept_workspace(batch, gamma, vocab);
    if (!work || work_bytes < need)
        return fail(DKV_EWORKSPACE, "dkv_accept: workspace too small (need " + std::to_string(need) + ")");
    DKV_REQUIRE(reinterpret_cast<uintptr_t>(work) % 16 == 0, "dkv_accept: workspace must be 16-byte aligned");
    const int nsc = stats_chunks(vocab), npc = pick_chunks(vocab), R = 2 * gamma + 1;
    char* w = static_cast<char*>(work);
    ChunkStat* stats = reinterpret_cast<ChunkStat*>(w);
    w += sizeof(ChunkStat) * batch * R * nsc;
    double* csum = reinterpret_cast<double*>(w);
    w += sizeof(double) * batch * npc;
    double* part = reinterpret_cast<double*>(w);
    w += sizeof(double) * batch * npc * ABLK;
    PickRec* recs = reinterpret_cast<PickRec*>(w);
    hipStream_t st = as_stream(stream);
    const bool samp = temperature > 0.0f;
    const RowNorm* dstats = reinterpret_cast<const RowNorm*>(draft_stats);
    const int rows = samp && !dstats ? R : gamma + 1;   // the draft rows' statistics, when given, are not recomputed
    const bool vec = vocab % 4 == 0 && reinterpret_cast<uintptr_t>(target) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(draft) % 16 == 0;
    const int64_t items = (int64_t)batch * rows * nsc;
    DKV_REQUIRE(items < ((int64_t)1 << 31), "dkv_accept: too many logits");
    int n_items = (int)items;
    // persistent waves: as many workgroups as fit on the device at once, each wave a few chunks
    const int kind = (samp ? 2 : 0) + (vec ? 1 : 0);
    const void* sk[4] = {reinterpret_cast<const void*>(stats_kernel<false, false>),
                         reinterpret_cast<const void*>(stats_kernel<true, false>),
                         reinterpret_cast<const void*>(stats_kernel<false, true>),
                         reinterpret_cast<const void*>(stats_kernel<true, true>)};
    static std::atomic<int> resident[4] = {0, 0, 0, 0};   // workgroups per device, per kernel (same on every call)
    if (resident[kind].load(std::memory_order_relaxed) == 0) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sk[kind], ABLK, 0) != hipSuccess || cus <= 0 ||
            per_cu <= 0)
            cus = 256, per_cu = 4;
        resident[kind].store(cus * per_cu, std::memory_order_relaxed);
    }
    const int grid = (int)std::min<int64_t>(resident[kind].load(std::memory_order_relaxed),
                                            (items + ABLK / WAVE - 1) / (ABLK / WAVE));
#define DKV_STATS(V, S)                                                                                          \
    hipLaunchKernelGGL((stats_kernel<V, S>), dim3(grid), dim3(ABLK), 0, st, target, draft, gamma, vocab, batch,     \
                       temperature, nsc, rows, n_items, stats)
    switch (kind) {
        case 0: DKV_STATS(false, false); break;
        case 1: DKV_STATS(true, false); break;
        case 2: DKV_STATS(false, true); break;
        default: DKV_STATS(true, true); break;
    }
#undef DKV_STATS
    int rc = check_launch("dkv_accept(stats)");
    if (rc) return rc;
    const dim3 fgrid(samp ? npc : 1, batch);
    if (vec)
        hipLaunchKernelGGL(finish_kernel<true>, fgrid, dim3(ABLK), 0, st, target, draft, draft_tokens, gamma, vocab,
                           temperature, u, dstats, reinterpret_cast<RowNorm*>(row_out), nsc, npc, stats, csum, part, recs,
                           accepted, next_token, n_uniforms);
    else
        hipLaunchKernelGGL(finish_kernel<false>, fgrid, dim3(ABLK), 0, st, target, draft, draft_tokens, gamma, vocab,
                           temperature, u, dstats, reinterpret_cast<RowNorm*>(row_out), nsc, npc, stats, csum, part, recs,
                           accepted, next_token, n_uniforms);
    if ((rc = check_launch("dkv_accept(finish)"))) return rc;
    if (!samp || gamma == 0) return DKV_OK;   // greedy, or a plain sample: nothing left to draw
    if (vec)
        hipLaunchKernelGGL(pick_kernel<true>, dim3(batch), dim3(ABLK), 0, st, target, draft, gamma, vocab, temperature,
                           nsc, npc, stats, csum, part, accepted, recs, next_token);
    else
        hipLaunchKernelGGL(pick_kernel<false>, dim3(batch), dim3(ABLK), 0, st, target, draft, gamma, vocab,
                           temperature, nsc, npc, stats, csum, part, accepted, recs, next_token);
    return check_launch("dkv_accept(pick)");
}

extern "C" int dkv_accept(const float* target, const float* draft, const int32_t* draft_tokens, int32_t batch,
                          int32_t gamma, int32_t vocab, float temperature, const double* u,
                          const dkv_row_stats_t* draft_stats, int32_t* accepted, int32_t* next_token,
                          int32_t* n_uniforms, void* work, size_t work_bytes, dkv_stream_t stream) {
    DKV_REQUIRE(reinterpret_cast<uintptr_t>(draft_stats) % alignof(dkv_row_stats_t) == 0,
                "dkv_accept: draft_stats must be 8-byte aligned");
    return accept_impl(target, draft, draft_tokens, batch, gamma, vocab, temperature, u, draft_stats, nullptr,
                       accepted, next_token, n_uniforms, work, work_bytes, stream);
}

extern "C" size_t dkv_sample_workspace(int32_t batch, int32_t vocab) {
    // gamma = 0 accept plus room for the per-row counters it returns
    return dkv_accept_workspace(batch, 0, vocab) + 2 * sizeof(int32_t) * (size_t)batch + 256;
}

extern "C" int dkv_sample(const float* logits, int64_t row_stride, int32_t batch, int32_t vocab, float temperature,
                          const double* u, int32_t* tokens, dkv_row_stats_t* row_stats, void* work, size_t work_bytes,
                          dkv_stream_t stream) {
    DKV_REQUIRE(logits && u && tokens, "dkv_sample: NULL argument");
    DKV_REQUIRE(row_stride == vocab, "dkv_sample: rows must be contiguous (row_stride == vocab)");
    const size_t need = dkv_sample_workspace(batch, vocab);
    if (!work || work_bytes < need)
        return fail(DKV_EWORKSPACE, "dkv_sample: workspace too small (need " + std::to_string(need) + ")");
    char* w = static_cast<char*>(work);
    const size_t acc_ws = dkv_accept_workspace(batch, 0, vocab);
    int32_t* scratch_i = reinterpret_cast<int32_t*>(w + ((acc_ws + 255) / 256) * 256);
    DKV_REQUIRE(reinterpret_cast<uintptr_t>(row_stats) % alignof(dkv_row_stats_t) == 0,
                "dkv_sample: row_stats must be 8-byte aligned");
    return accept_impl(logits, nullptr, nullptr, batch, 0, vocab, temperature, u, nullptr, row_stats, scratch_i, tokens,
                       scratch_i + batch, work, acc_ws, stream);
}

// ---------------------------------------------------------------- no allocation
// dkv_accept for callers that cannot allocate (code under stream capture,
// serving loops that forbid it): the workspace is this file-scope device
// array, one copy per GPU for the life of the process. Its address on a
// device comes from hipGetSymbolAddress, taken once per device with that
// device current; the array's name is never used as a device address on the
// host. Every call on a GPU shares that GPU's array, so calls that overlap on
// one GPU (two streams, two host threads) race. The kernels write every
// workspace entry before they read it, so nothing needs clearing between
// calls.
static __device__ __align__(256) unsigned char scratch[DKV_ACCEPT_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

int scratch_of_current_device(void** out, const char* who) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return dkv::fail(DKV_ELAUNCH, std::string(who) + ": hipGetDevice: " + hipGetErrorString(e));
    if (dev < 0 || dev >= 64) return dkv::fail(DKV_EINVAL, std::string(who) + ": device id out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return dkv::fail(DKV_ELAUNCH, std::string(who) + ": hipGetSymbolAddress(scratch): " +
                                              (e != hipSuccess ? hipGetErrorString(e) : "null address"));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DKV_OK;
}
}  // namespace

extern "C" int dkv_accept_noalloc(const float* target, const float* draft, const int32_t* draft_tokens,
                                  int32_t batch, int32_t gamma, int32_t vocab, float temperature, const double* u,
                                  const dkv_row_stats_t* draft_stats, int32_t* accepted, int32_t* next_token,
                                  int32_t* n_uniforms, dkv_stream_t stream) {
    DKV_REQUIRE(batch > 0 && gamma >= 0 && vocab > 0, "dkv_accept_noalloc: bad sizes");
    const size_t need = dkv_accept_workspace(batch, gamma, vocab);
    if (need > DKV_ACCEPT_SCRATCH_BYTES)
        return dkv::fail(DKV_ECAPACITY, "dkv_accept_noalloc: batch " + std::to_string(batch) + ", gamma " +
                                            std::to_string(gamma) + ", vocab " + std::to_string(vocab) + " need " +
                                            std::to_string(need) + " B of workspace; the static scratch holds " +
                                            std::to_string((size_t)DKV_ACCEPT_SCRATCH_BYTES));
    void* ws = nullptr;
    int rc = scratch_of_current_device(&ws, "dkv_accept_noalloc");
    if (rc) return rc;
    return dkv_accept(target, draft, draft_tokens, batch, gamma, vocab, temperature, u, draft_stats, accepted,
                      next_token, n_uniforms, ws, DKV_ACCEPT_SCRATCH_BYTES, stream);
}
