// Sampling and the verify decision.
// Reference: draftkv/engine.py:36-41 (`_probs`), :101-106 (`_sample`),
// :188-213 (accept loop, bonus token, residual resample).
//
// Pipeline (rows of `vocab` float32 logits, cut in chunks of VCH; every
// exp in float64 by the table-driven dexp below):
//   1. stats   grid (chunk, row, seq): chunk max, first argmax and
//              sum exp(x/T - max/T) in float64.
//   2. decide  grid (seq): merge chunk stats per row, run the accept tests
//              with the supplied uniforms, choose the final distribution:
//              p of the bonus row, or the residual clip(p - q) (falling back
//              to p when it sums to 0); greedy mode: argmax comparisons.
//   3. sums    grid (chunk, seq): per chunk mass of the final distribution.
//   4. pick    grid (seq): first index whose cumulative mass exceeds u*total
//              (numpy Generator.choice semantics: searchsorted 'right').
// Sampling one row (dkv_sample) is the gamma = 0 case: the bonus row is it.
#include "dkv_common.h"

#include <mutex>

namespace dkv {

constexpr int VCH = 4096;
constexpr int ABLK = 256;
static_assert(VCH % ABLK == 0, "pick: every thread owns VCH / ABLK elements");

struct ChunkStat {
    float mx;
    int arg;
    double sum;   // sum exp((x - mx)/T) over the chunk (T > 0)
};

struct SeqState {
    int mode;        // 0: done (greedy), 1: sample p of row `row`, 2: residual of row `row`
    int row;
    double u;        // uniform for the final draw
};

// ---- float64 exp, Tang's table-driven method (ACM TOMS 15(2), 1989):
// y = (64 e + j) ln2/64 + r with |r| <= ln2/128, exp(y) = 2^e 2^(j/64) exp(r),
// 2^(j/64) from a table of correctly rounded doubles, exp(r) - 1 by its
// degree-6 Taylor polynomial (truncation below 3e-20 relative). Within one
// ulp of a correctly rounded exp for y in [-745, 709]; 0 below (and for
// -inf). About 15 float64 operations against ~35 for the library's.
__constant__ double kExp2Tab[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0};

// the table in a block's LDS (callers synchronise before the first dexp)
__device__ __forceinline__ void load_exp_tab(double* tab) {
    for (int i = threadIdx.x; i < 64; i += blockDim.x) tab[i] = kExp2Tab[i];
}

__device__ __forceinline__ double dexp(double y, const double* tab) {
    if (!(y > -745.5)) return 0.0;
    const double n = __builtin_rint(y * 0x1.71547652b82fep+6);   // y * 64 / ln2, to nearest
    double r = fma(-n, 0x1.62e42fefa0000p-7, y);                  // ln2/64 in two parts: n * hi is exact
    r = fma(-n, 0x1.cf79abc9e3b3ap-46, r);
    const int ni = (int)n, j = ni & 63, e = (ni - j) >> 6;
    double q = fma(0x1.6c16c16c16c17p-10, r, 0x1.1111111111111p-7);   // 1/720, 1/120
    q = fma(q, r, 0x1.5555555555555p-5);                              // 1/24
    q = fma(q, r, 0x1.5555555555555p-3);                              // 1/6
    q = fma(q, r, 0.5);
    const double p = fma(q, r * r, r);                                // exp(r) - 1
    const double t = tab[j];
    return ldexp(fma(t, p, t), e);
}

__device__ __forceinline__ const float* row_ptr(const float* target, const float* draft, int s, int row, int gamma,
                                                int vocab) {
    // rows 0..gamma: target; gamma+1..2*gamma: draft rows 0..gamma-1
    if (row <= gamma) return target + ((int64_t)s * (gamma + 1) + row) * vocab;
    return draft + ((int64_t)s * gamma + (row - gamma - 1)) * vocab;
}

// One read of the chunk, held in registers: the block's max (first index on
// ties), then the float64 sum of exp(x/T - max/T) (x/T as x * (1/T): a
// normaliser needs no correctly rounded quotient).
__global__ void __launch_bounds__(ABLK) stats_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                     int gamma, int vocab, float T, int n_chunks,
                                                     ChunkStat* __restrict__ stats) {
    constexpr int PER = VCH / ABLK;
    const int chunk = blockIdx.x, row = blockIdx.y, s = blockIdx.z;
    const bool samp = T > 0.0f;
    const int n_rows = samp ? 2 * gamma + 1 : gamma + 1;
    if (row >= n_rows) return;
    __shared__ double tab[64];
    load_exp_tab(tab);   // (the max's barrier below precedes every use)
    const float* x = row_ptr(target, draft, s, row, gamma, vocab);
    const int i0 = chunk * VCH, i1 = min(vocab, i0 + VCH);
    __shared__ float smx[ABLK / WAVE];
    __shared__ int sarg[ABLK / WAVE];
    __shared__ double ssum[ABLK / WAVE];
    float xv[PER];
    float mx = -INFINITY;
    int arg = INT_MAX;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = i0 + threadIdx.x + k * ABLK;
        xv[k] = i < i1 ? x[i] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k)   // a thread's indices rise with k: its first maximum is kept
        if (xv[k] > mx) {
            mx = xv[k];
            arg = i0 + threadIdx.x + k * ABLK;
        }
    for (int o = 32; o > 0; o >>= 1) {
        const float om = __shfl_xor(mx, o);
        const int oa = __shfl_xor(arg, o);
        if (om > mx || (om == mx && oa < arg)) {
            mx = om;
            arg = oa;
        }
    }
    const int w = threadIdx.x / WAVE;
    if (threadIdx.x % WAVE == 0) {
        smx[w] = mx;
        sarg[w] = arg;
    }
    __syncthreads();
    mx = smx[0];
    arg = sarg[0];
    for (int i = 1; i < ABLK / WAVE; ++i)
        if (smx[i] > mx || (smx[i] == mx && sarg[i] < arg)) {
            mx = smx[i];
            arg = sarg[i];
        }
    double sum = 0.0;
    if (samp) {
        const double iT = 1.0 / (double)T, mT = (double)mx * iT;
#pragma unroll
        for (int k = 0; k < PER; ++k)
            if (xv[k] > -INFINITY) sum += dexp((double)xv[k] * iT - mT, tab);
        sum = wave_sum_d(sum);
        if (threadIdx.x % WAVE == 0) ssum[w] = sum;
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        double t = 0.0;
        if (samp)
            for (int i = 0; i < ABLK / WAVE; ++i) t += ssum[i];
        ChunkStat& cs = stats[((int64_t)s * (2 * gamma + 1) + row) * n_chunks + chunk];
        cs.mx = mx;
        cs.arg = arg;
        cs.sum = t;
    }
}

struct RowNorm {
    double m;   // max(x)/T
    double S;   // sum exp(x/T - m)
    double iS;  // 1 / S
    int arg;
};

// p(x) = exp(x/T - m) / S with x/T as x * (1/T) and the division by S as a
// product with its reciprocal (each within an ulp of the quotient)
__device__ __forceinline__ double prob(float x, const RowNorm& r, float T, const double* tab) {
    return dexp((double)x * (1.0 / (double)T) - r.m, tab) * r.iS;
}

// One block per sequence, one wave per row (rows w, w + DECIDE_WAVES, ...):
// each wave merges its row's chunk statistics into the row's norm. Then wave
// 0 takes the drafted positions 64 at a time: its lanes fetch the accept
// test's inputs of 64 positions at once (the argmax, or p and q of the
// drafted token: the scattered reads in flight together), and lane 0 walks
// those tests in order -- the same decisions, in the same order, as one lane
// reading as it goes -- until one fails. Any gamma.
constexpr int DECIDE_WAVES = 16;
constexpr int PICK_MAX_CHUNKS = 1024;   // vocab up to 4M
__global__ void __launch_bounds__(WAVE * DECIDE_WAVES) decide_kernel(const float* __restrict__ target,
                                                                     const float* __restrict__ draft,
                                                                     const int32_t* __restrict__ draft_tokens,
                                                                     int gamma, int vocab, float T,
                                                                     const double* __restrict__ u, int n_chunks,
                                                                     const ChunkStat* __restrict__ stats,
                                                                     RowNorm* __restrict__ norms,
                                                                     SeqState* __restrict__ state, int32_t* accepted,
                                                                     int32_t* next_token, int32_t* n_uniforms) {
    const int s = blockIdx.x, lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const bool samp = T > 0.0f;
    const int R = 2 * gamma + 1;
    const ChunkStat* st = stats + (int64_t)s * R * n_chunks;
    const int n_rows = samp ? R : gamma + 1;
    RowNorm* nr = norms + (int64_t)s * R;
    __shared__ double sp[WAVE], sq[WAVE];
    __shared__ int sarg[WAVE];
    __shared__ double tab[64];
    load_exp_tab(tab);
    __syncthreads();
    for (int r = w; r < n_rows; r += DECIDE_WAVES) {
        const ChunkStat* sr = st + (int64_t)r * n_chunks;
        float mx = -INFINITY;
        int arg = INT_MAX;
        for (int c = lane; c < n_chunks; c += WAVE)
            if (sr[c].mx > mx || (sr[c].mx == mx && sr[c].arg < arg)) {
                mx = sr[c].mx;
                arg = sr[c].arg;
            }
        for (int o = WAVE / 2; o > 0; o >>= 1) {
            const float om = __shfl_xor(mx, o);
            const int oa = __shfl_xor(arg, o);
            if (om > mx || (om == mx && oa < arg)) {
                mx = om;
                arg = oa;
            }
        }
        RowNorm rn{0.0, 0.0, 0.0, arg};
        if (samp) {
            const double iT = 1.0 / (double)T;
            rn.m = (double)mx * iT;
            double S = 0.0;
            for (int c = lane; c < n_chunks; c += WAVE) S += sr[c].sum * dexp((double)sr[c].mx * iT - rn.m, tab);
            rn.S = wave_sum_d(S);
            rn.iS = 1.0 / rn.S;
        }
        if (lane == 0) nr[r] = rn;
    }
    __syncthreads();   // the norms written by every wave are visible to wave 0
    if (w != 0) return;
    const double* us = u + (int64_t)s * (gamma + 1);
    int acc = 0, used = 0;
    bool stop = false;
    for (int base = 0; base < gamma && !stop; base += WAVE) {
        const int i = base + lane;
        if (i < gamma) {   // lane: the inputs of position i's test
            const int d = draft_tokens[(int64_t)s * gamma + i];
            if (samp) {
                double p = 0.0, q = 0.0;
                if (d >= 0 && d < vocab) {
                    p = prob(row_ptr(target, draft, s, i, gamma, vocab)[d], nr[i], T, tab);
                    q = prob(row_ptr(target, draft, s, gamma + 1 + i, gamma, vocab)[d], nr[gamma + 1 + i], T, tab);
                }
                sp[lane] = p;
                sq[lane] = q;
            } else {
                sarg[lane] = nr[i].arg;
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane == 0) {
            for (int j = base; j < min(gamma, base + WAVE); ++j) {
                const int d = draft_tokens[(int64_t)s * gamma + j];
                bool ok;
                if (d < 0 || d >= vocab) {
                    ok = false;              // not a token of this vocabulary: never read past the row
                    if (samp) ++used;
                } else if (!samp) {
                    ok = sarg[j - base] == d;
                } else {
                    const double ratio = sq[j - base] > 0.0 ? sp[j - base] / sq[j - base] : 0.0;
                    ok = us[used] < fmin(1.0, ratio);
                    ++used;
                }
                if (!ok) {
                    stop = true;
                    break;
                }
                ++acc;
            }
        }
        stop = __shfl(stop ? 1 : 0, 0) != 0;
        __builtin_amdgcn_wave_barrier();   // lane 0 is done with this block before the lanes refill it
    }
    if (lane != 0) return;
    SeqState ss{0, acc, 0.0};
    if (!samp) {
        next_token[s] = nr[acc].arg;
        if (acc == gamma) ++used;   // the bonus draw is taken even though p is one-hot
    } else {
        ss.mode = (acc == gamma) ? 1 : 2;
        ss.u = us[used];
        ++used;
    }
    state[s] = ss;
    accepted[s] = acc;
    n_uniforms[s] = used;
}

// probability of index i under the final distribution of sequence s
__device__ __forceinline__ double final_mass(const float* p_row, const float* q_row, const RowNorm& pn,
                                             const RowNorm& qn, int mode, int i, float T, const double* tab) {
    const double p = prob(p_row[i], pn, T, tab);
    if (mode == 1) return p;
    const double r = p - prob(q_row[i], qn, T, tab);
    return r > 0.0 ? r : 0.0;
}

__global__ void __launch_bounds__(ABLK) sums_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                    int gamma, int vocab, float T, int n_chunks,
                                                    const RowNorm* __restrict__ norms,
                                                    const SeqState* __restrict__ state, double* __restrict__ csum) {
    const int chunk = blockIdx.x, s = blockIdx.y;
    const SeqState ss = state[s];
    if (ss.mode == 0) return;
    const int R = 2 * gamma + 1;
    const RowNorm* nr = norms + (int64_t)s * R;
    const float* pr = row_ptr(target, draft, s, ss.row, gamma, vocab);
    const float* qr = ss.mode == 2 ? row_ptr(target, draft, s, gamma + 1 + ss.row, gamma, vocab) : pr;
    const RowNorm pn = nr[ss.row], qn = ss.mode == 2 ? nr[gamma + 1 + ss.row] : pn;
    const int i0 = chunk * VCH, i1 = min(vocab, i0 + VCH);
    __shared__ double tab[64];
    load_exp_tab(tab);
    __syncthreads();
    double sum = 0.0;
    for (int i = i0 + threadIdx.x; i < i1; i += ABLK) sum += final_mass(pr, qr, pn, qn, ss.mode, i, T, tab);
    sum = wave_sum_d(sum);
    __shared__ double ssum[ABLK / WAVE];
    if (threadIdx.x % WAVE == 0) ssum[threadIdx.x / WAVE] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int i = 0; i < ABLK / WAVE; ++i) t += ssum[i];
        csum[(int64_t)s * n_chunks + chunk] = t;
    }
}

__global__ void __launch_bounds__(ABLK) pick_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                    int gamma, int vocab, float T, int n_chunks,
                                                    const ChunkStat* __restrict__ stats,
                                                    const RowNorm* __restrict__ norms,
                                                    const SeqState* __restrict__ state,
                                                    const double* __restrict__ csum, int32_t* next_token) {
    const int s = blockIdx.x;
    const SeqState ss = state[s];
    if (ss.mode == 0) return;
    const int R = 2 * gamma + 1;
    const RowNorm* nr = norms + (int64_t)s * R;
    const double* cs = csum + (int64_t)s * n_chunks;
    const ChunkStat* pst = stats + ((int64_t)s * R + ss.row) * n_chunks;
    __shared__ int s_chunk, s_mode;
    __shared__ double s_before, s_target;
    // the chunk masses, read (and for p, computed) by all threads at once; the
    // sums over them stay sequential in chunk order on thread 0
    __shared__ double s_cs[PICK_MAX_CHUNKS], s_pm[PICK_MAX_CHUNKS];
    __shared__ double tab[64];
    load_exp_tab(tab);
    __syncthreads();
    {
        const RowNorm pn = nr[ss.row];
        for (int c = threadIdx.x; c < n_chunks; c += blockDim.x) {
            s_cs[c] = cs[c];
            s_pm[c] = pst[c].sum * dexp((double)pst[c].mx * (1.0 / (double)T) - pn.m, tab) * pn.iS;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int mode = ss.mode;
        double total = 0.0;
        for (int c = 0; c < n_chunks; ++c) total += s_cs[c];
        // an all-zero residual falls back to p itself (engine.py:210-211); p's
        // chunk masses then come from the row statistics
        const bool from_p = (mode == 2 && !(total > 0.0));
        if (from_p) mode = 1;
        const double* cmass = from_p ? s_pm : s_cs;
        if (from_p) {
            total = 0.0;
            for (int c = 0; c < n_chunks; ++c) total += cmass[c];
        }
        const double tgt = ss.u * total;
        double run = 0.0;
        int chosen = n_chunks - 1;
        bool hit = false;
        for (int c = 0; c < n_chunks; ++c) {
            const double cm = cmass[c];
            if (run + cm > tgt) {
                chosen = c;
                hit = true;
                break;
            }
            run += cm;
        }
        // rounding carried the draw past the end: scan the last chunk from its start
        if (!hit) run -= cmass[chosen];
        s_chunk = chosen;
        s_mode = mode;
        s_before = run;
        s_target = tgt;
    }
    __syncthreads();
    const int mode = s_mode;
    const float* pr = row_ptr(target, draft, s, ss.row, gamma, vocab);
    const float* qr = mode == 2 ? row_ptr(target, draft, s, gamma + 1 + ss.row, gamma, vocab) : pr;
    const RowNorm pn = nr[ss.row], qn = mode == 2 ? nr[gamma + 1 + ss.row] : pn;
    const int c = s_chunk;
    const int i0 = c * VCH, i1 = min(vocab, i0 + VCH);
    const double tgt = s_target;
    // Thread t owns PER consecutive elements of the chunk: per-thread masses,
    // one block-wide exclusive scan of them, then the thread whose range
    // crosses the target walks its own elements.
    constexpr int PER = VCH / ABLK;
    __shared__ double wsum[ABLK / WAVE];
    __shared__ int found, last_pos;
    if (threadIdx.x == 0) {
        found = INT_MAX;
        last_pos = -1;
    }
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const int b0 = i0 + PER * threadIdx.x;
    double v[PER];
    double loc = 0.0;
    int lastp = -1;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = b0 + k;
        v[k] = i < i1 ? final_mass(pr, qr, pn, qn, mode, i, T, tab) : 0.0;
        loc += v[k];
        if (v[k] > 0.0) lastp = i;
    }
    double x = loc;   // inclusive scan within the wave
    for (int o = 1; o < WAVE; o <<= 1) {
        const double y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == WAVE - 1) wsum[w] = x;
    __syncthreads();
    double off = s_before + (x - loc);
    for (int k = 0; k < w; ++k) off += wsum[k];
    int hit = INT_MAX;
    if (off + loc > tgt) {
        double run = off;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            run += v[k];
            if (hit == INT_MAX && v[k] > 0.0 && run > tgt) hit = b0 + k;
        }
    }
    if (hit != INT_MAX) atomicMin(&found, hit);
    if (lastp >= 0) atomicMax(&last_pos, lastp);
    __syncthreads();
    if (threadIdx.x == 0) {
        // a draw that rounding pushes past the end of the cdf takes the last
        // index with positive mass (the reference's cdf ends at exactly 1)
        next_token[s] = found != INT_MAX ? found : (last_pos >= 0 ? last_pos : i1 - 1);
    }
}

}  // namespace dkv

using namespace dkv;

static int chunks_of(int vocab) { return (vocab + VCH - 1) / VCH; }

extern "C" size_t dkv_accept_workspace(int32_t batch, int32_t gamma, int32_t vocab) {
    if (batch <= 0 || gamma < 0 || vocab <= 0) return 0;
    const size_t nc = chunks_of(vocab), R = 2 * (size_t)gamma + 1;
    return sizeof(ChunkStat) * batch * R * nc + sizeof(RowNorm) * batch * R + sizeof(SeqState) * batch +
           sizeof(double) * batch * nc + 256;
}

extern "C" int dkv_accept(const float* target, const float* draft, const int32_t* draft_tokens, int32_t batch,
                          int32_t gamma, int32_t vocab, float temperature, const double* u, int32_t* accepted,
                          int32_t* next_token, int32_t* n_uniforms, void* work, size_t work_bytes,
                          dkv_stream_t stream) {
    DKV_REQUIRE(target && accepted && next_token && n_uniforms && u, "dkv_accept: NULL argument");
    DKV_REQUIRE(batch > 0 && gamma >= 0 && vocab > 0, "dkv_accept: bad sizes");
    DKV_REQUIRE(chunks_of(vocab) <= PICK_MAX_CHUNKS, "dkv_accept: vocab too large");
    DKV_REQUIRE(2 * (int64_t)gamma + 1 <= 65535 && batch <= 65535, "dkv_accept: gamma or batch too large for the grid");
    DKV_REQUIRE(gamma == 0 || draft_tokens, "dkv_accept: draft_tokens is NULL");
    DKV_REQUIRE(temperature <= 0.0f || gamma == 0 || draft, "dkv_accept: draft logits needed when T > 0");
    const size_t need = dkv_accept_workspace(batch, gamma, vocab);
    if (!work || work_bytes < need)
        return fail(DKV_EWORKSPACE, "dkv_accept: workspace too small (need " + std::to_string(need) + ")");
    const int nc = chunks_of(vocab), R = 2 * gamma + 1;
    char* w = static_cast<char*>(work);
    ChunkStat* stats = reinterpret_cast<ChunkStat*>(w);
    w += sizeof(ChunkStat) * batch * R * nc;
    RowNorm* norms = reinterpret_cast<RowNorm*>(w);
    w += sizeof(RowNorm) * batch * R;
    SeqState* state = reinterpret_cast<SeqState*>(w);
    w += sizeof(SeqState) * batch;
    double* csum = reinterpret_cast<double*>(w);
    hipStream_t st = as_stream(stream);
    const int rows = temperature > 0.0f ? R : gamma + 1;
    hipLaunchKernelGGL(stats_kernel, dim3(nc, rows, batch), dim3(ABLK), 0, st, target, draft, gamma, vocab,
                       temperature, nc, stats);
    int rc = check_launch("dkv_accept(stats)");
    if (rc) return rc;
    hipLaunchKernelGGL(decide_kernel, dim3(batch), dim3(WAVE * DECIDE_WAVES), 0, st, target, draft, draft_tokens,
                       gamma, vocab,
                       temperature, u, nc, stats, norms, state, accepted, next_token, n_uniforms);
    if ((rc = check_launch("dkv_accept(decide)"))) return rc;
    if (temperature <= 0.0f) return DKV_OK;
    hipLaunchKernelGGL(sums_kernel, dim3(nc, batch), dim3(ABLK), 0, st, target, draft, gamma, vocab, temperature, nc,
                       norms, state, csum);
    if ((rc = check_launch("dkv_accept(sums)"))) return rc;
    hipLaunchKernelGGL(pick_kernel, dim3(batch), dim3(ABLK), 0, st, target, draft, gamma, vocab, temperature, nc,
                       stats, norms, state, csum, next_token);
    return check_launch("dkv_accept(pick)");
}

extern "C" size_t dkv_sample_workspace(int32_t batch, int32_t vocab) {
    // gamma = 0 accept plus room for the per-row counters it returns
    return dkv_accept_workspace(batch, 0, vocab) + 2 * sizeof(int32_t) * (size_t)batch + 256;
}

extern "C" int dkv_sample(const float* logits, int64_t row_stride, int32_t batch, int32_t vocab, float temperature,
                          const double* u, int32_t* tokens, void* work, size_t work_bytes, dkv_stream_t stream) {
    DKV_REQUIRE(logits && u && tokens, "dkv_sample: NULL argument");
    DKV_REQUIRE(row_stride == vocab, "dkv_sample: rows must be contiguous (row_stride == vocab)");
    const size_t need = dkv_sample_workspace(batch, vocab);
    if (!work || work_bytes < need)
        return fail(DKV_EWORKSPACE, "dkv_sample: workspace too small (need " + std::to_string(need) + ")");
    char* w = static_cast<char*>(work);
    const size_t acc_ws = dkv_accept_workspace(batch, 0, vocab);
    int32_t* scratch_i = reinterpret_cast<int32_t*>(w + ((acc_ws + 255) / 256) * 256);
    return dkv_accept(logits, nullptr, nullptr, batch, 0, vocab, temperature, u, scratch_i, tokens,
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
                                  int32_t* accepted, int32_t* next_token, int32_t* n_uniforms,
                                  dkv_stream_t stream) {
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
    return dkv_accept(target, draft, draft_tokens, batch, gamma, vocab, temperature, u, accepted, next_token,
                      n_uniforms, ws, DKV_ACCEPT_SCRATCH_BYTES, stream);
}
