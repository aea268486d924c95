// Drafter mirror maintenance: append + evict, truncate and
// per-round resync, rebuild under a new arm, and a gather for `read`.
// Reference: draftkv/compress.py:95-241.
//
// Storage (mirror_layout.h): per (sequence, layer, kv head) a dense run of
// 32-row pages; rows 0..n_rows-1 are live, in no particular order (attention
// is order-free and the eviction order is defined on (score, position), not
// on slots). Eviction and truncation keep the run dense by moving surviving
// rows from the tail into the holes ("eviction compaction").
#include <climits>
#include <type_traits>

#include "mirror_layout.h"

namespace dkv {

constexpr int BLK = 256;
constexpr int NWAVES = BLK / WAVE;
constexpr int MAXMOVE = 1024;     // hole/mover pairs handled per compaction pass
constexpr int WIN = 4096;         // position window scanned for the sink/recent bounds
constexpr int32_t DEAD = INT_MAX; // position marking an evicted row before compaction

// ------------------------------------------------------------ row quantizer
// A wave quantizes one head-row of D values. Lane l owns channels [8l, 8l+8);
// lanes past D stand for the zero padding of a short last group
// (compress.py:32-35). Group min/max are reduced over the group's group/8
// lanes, so K words (one row's codes) are written whole by one lane. V words
// hold codes of 8 rows, so a V code is a read-modify-write: callers give
// each (sequence, layer, head) segment to one wave at a time.
struct LaneCodes {
    int code[8];
    float raw[8];
    GroupMeta m;
};

// codes and group meta of this lane's 8 channel values (zero past D)
__device__ __forceinline__ void quant_vals(const float (&v)[8], const PageFmt& f, int bits, int lane, LaneCodes& lc) {
    if (f.cb == 32) {
#pragma unroll
        for (int e = 0; e < 8; ++e) lc.raw[e] = v[e];
        return;
    }
    const int gl = f.group / 8;                 // lanes per group
    float mn = INFINITY, mx = -INFINITY;
    if (lane < f.NG * gl) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            mn = fminf(mn, v[e]);
            mx = fmaxf(mx, v[e]);
        }
    }
    for (int o = 1; o < gl; o <<= 1) {
        mn = fminf(mn, __shfl_xor(mn, o));
        mx = fmaxf(mx, __shfl_xor(mx, o));
    }
    lc.m = group_meta(mn, mx, bits, f.meta_f16);
#pragma unroll
    for (int e = 0; e < 8; ++e) lc.code[e] = quant_code(v[e], lc.m, bits);
}

template <class Load>
__device__ __forceinline__ void quant_lane(Load ld, const PageFmt& f, int bits, int lane, LaneCodes& lc) {
    const int d0 = 8 * lane;
    const bool real = d0 < f.D;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = real ? ld(d0 + e) : 0.0f;
    quant_vals(v, f, bits, lane, lc);
}

__device__ __forceinline__ void put_k_lane(uint8_t* page, const PageFmt& f, int i, int lane, const LaneCodes& lc) {
    const int d0 = 8 * lane;
    if (d0 >= f.D) return;
    if (f.cb == 32) {
        float* dst = reinterpret_cast<float*>(page + f.kc) + (int64_t)i * f.D + d0;
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = lc.raw[e];
        return;
    }
    uint32_t* sec = reinterpret_cast<uint32_t*>(page + f.kc);
    if (f.cb == 4) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= static_cast<uint32_t>(lc.code[e]) << code_shift(4, e);
        sec[((int64_t)i * f.D + d0) / 8] = w;
    } else {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            w0 |= static_cast<uint32_t>(lc.code[e]) << code_shift(8, e);
            w1 |= static_cast<uint32_t>(lc.code[4 + e]) << code_shift(8, e);
        }
        sec[k_word(f, i, d0 / 4)] = w0;
        sec[k_word(f, i, d0 / 4 + 1)] = w1;
    }
    if (d0 % f.group == 0) write_meta(page + k_meta_off(f, i, d0 / f.group), lc.m, f.meta_f16);
}

// V codes of this lane's 8 channels for row i (exclusive access to the words)
__device__ __forceinline__ void put_v_lane(uint8_t* page, const PageFmt& f, int i, int lane, const LaneCodes& lc) {
    const int d0 = 8 * lane;
    if (d0 >= f.D) return;
    if (f.cb == 32) {
        float* dst = reinterpret_cast<float*>(page + f.vc) + (int64_t)i * f.D + d0;
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = lc.raw[e];
        return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        int64_t w;
        int sh;
        v_code_loc(f, i, d0 + e, &w, &sh);
        if (f.cb == 8) {
            page[f.vc + w * 4 + sh / 8] = static_cast<uint8_t>(lc.code[e]);
        } else {
            uint32_t* pw = reinterpret_cast<uint32_t*>(page + f.vc) + w;
            *pw = (*pw & ~(0xfu << sh)) | (static_cast<uint32_t>(lc.code[e]) << sh);
        }
    }
    if (d0 % f.group == 0) write_meta(page + v_meta_off(f, i, d0 / f.group), lc.m, f.meta_f16);
}

template <class LoadK, class LoadV>
__device__ __forceinline__ void quant_row(LoadK ldk, LoadV ldv, const PageFmt& f, int bits, uint8_t* page, int i,
                                          int lane) {
    LaneCodes lc;
    quant_lane(ldk, f, bits, lane, lc);
    put_k_lane(page, f, i, lane, lc);
    quant_lane(ldv, f, bits, lane, lc);
    put_v_lane(page, f, i, lane, lc);
}

// the same from this lane's 8 K and 8 V channel values, already loaded
__device__ __forceinline__ void quant_row_vals(const float (&kv)[8], const float (&vv)[8], const PageFmt& f, int bits,
                                               uint8_t* page, int i, int lane) {
    LaneCodes lc;
    quant_vals(kv, f, bits, lane, lc);
    put_k_lane(page, f, i, lane, lc);
    quant_vals(vv, f, bits, lane, lc);
    put_v_lane(page, f, i, lane, lc);
}

// ------------------------------------------------------------ block helpers
// The append/truncate/evict op runs one block of OP_BLK threads per
// (sequence, layer); these helpers and the compaction below assume it.
constexpr int OP_BLK = 1024;
constexpr int OP_WAVES = OP_BLK / WAVE;
constexpr int DEADLIST = 1024;   // dead rows a list compaction takes (more: the general one)

__device__ int block_sum_int(int v, int* red) {
    v = wave_sum_i(v);
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    int t = 0;
    for (int i = 0; i < OP_WAVES; ++i) t += red[i];
    return t;
}

// exclusive prefix of a 0/1 flag over the block (thread order); returns the
// rank and writes the block total to *total
__device__ int block_rank(int flag, int* red, int* total) {
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const unsigned long long ballot = __ballot(flag);
    const int below = __popcll(ballot & ((1ull << lane) - 1ull));
    const int wcount = __popcll(ballot);
    __syncthreads();
    if (lane == 0) red[w] = wcount;
    __syncthreads();
    int off = 0, tot = 0;
    for (int i = 0; i < OP_WAVES; ++i) {
        if (i < w) off += red[i];
        tot += red[i];
    }
    *total = tot;
    return off + below;
}

struct RowCtx {
    const dkv_drafter_t* m;
    int s, L, bits;
    PageFmt f;
    int32_t* pos;     // this (s, L)'s pos array
    double* score;
};

// Copy row slot `from` to slot `to` of head h (codes, meta; pos and score
// with h == 0). One wave per head: the V words it rewrites belong to this
// head's segment only.
__device__ void copy_row_head(const RowCtx& c, int h, int from, int to, int lane) {
    const dkv_drafter_t& m = *c.m;
    const PageFmt& f = c.f;
    const int D = f.D;
    const int fi = from % PAGE, ti = to % PAGE;
    const uint8_t* src = page_ptr(m, c.s, c.L, h, from / PAGE);
    uint8_t* dst = page_ptr(m, c.s, c.L, h, to / PAGE);
    if (f.cb == 32) {
        for (int d = lane; d < D; d += WAVE) {
            reinterpret_cast<float*>(dst + f.kc)[(int64_t)ti * D + d] =
                reinterpret_cast<const float*>(src + f.kc)[(int64_t)fi * D + d];
            reinterpret_cast<float*>(dst + f.vc)[(int64_t)ti * D + d] =
                reinterpret_cast<const float*>(src + f.vc)[(int64_t)fi * D + d];
        }
    } else {
        const int wpr = D * f.cb / 32;   // K words per row
        for (int w = lane; w < wpr; w += WAVE)
            reinterpret_cast<uint32_t*>(dst + f.kc)[k_word(f, ti, w)] =
                reinterpret_cast<const uint32_t*>(src + f.kc)[k_word(f, fi, w)];
        for (int d = lane; d < D; d += WAVE) {
            int64_t ws, wd;
            int ss, sd;
            v_code_loc(f, fi, d, &ws, &ss);
            v_code_loc(f, ti, d, &wd, &sd);
            const int code = read_code(src + f.vc, ws, ss, f.cb);
            if (f.cb == 8) {
                dst[f.vc + wd * 4 + sd / 8] = static_cast<uint8_t>(code);
            } else {
                uint32_t* pw = reinterpret_cast<uint32_t*>(dst + f.vc) + wd;
                *pw = (*pw & ~(0xfu << sd)) | (static_cast<uint32_t>(code) << sd);
            }
        }
        for (int g = lane; g < f.NG; g += WAVE) {
            write_meta(dst + k_meta_off(f, ti, g), read_meta(src + k_meta_off(f, fi, g), f.meta_f16), f.meta_f16);
            write_meta(dst + v_meta_off(f, ti, g), read_meta(src + v_meta_off(f, fi, g), f.meta_f16), f.meta_f16);
        }
    }
    if (h == 0 && lane == 0) {
        c.pos[to] = c.pos[from];
        c.score[to] = c.score[from];
    }
}

// Keep rows with pos < thr: move survivors from [new_n, n) into the holes of
// [0, new_n). Returns new_n. Whole block participates.
__device__ __forceinline__ int compact(const RowCtx& c, int n, int32_t thr, int* red, int* holes, int* movers) {
    int keep = 0;
    for (int r = threadIdx.x; r < n; r += OP_BLK) keep += (c.pos[r] < thr);
    const int new_n = block_sum_int(keep, red);
    if (new_n == n) return n;
    for (int base = 0;; base += MAXMOVE) {
        int seen_h = 0, seen_m = 0;
        __syncthreads();
        for (int r0 = 0; r0 < new_n; r0 += OP_BLK) {
            const int r = r0 + threadIdx.x;
            const int fl = (r < new_n) && (c.pos[r] >= thr);
            int tot;
            const int rk = block_rank(fl, red, &tot) + seen_h;
            if (fl && rk >= base && rk < base + MAXMOVE) holes[rk - base] = r;
            seen_h += tot;
        }
        for (int r0 = new_n; r0 < n; r0 += OP_BLK) {
            const int r = r0 + threadIdx.x;
            const int fl = (r < n) && (c.pos[r] < thr);
            int tot;
            const int rk = block_rank(fl, red, &tot) + seen_m;
            if (fl && rk >= base && rk < base + MAXMOVE) movers[rk - base] = r;
            seen_m += tot;
        }
        const int np = min(min(MAXMOVE, seen_h - base), min(MAXMOVE, seen_m - base));
        __syncthreads();
        if (np <= 0) break;
        // sources (>= new_n) and destinations (< new_n) are disjoint; one wave
        // per head walks the pairs in order
        for (int h = threadIdx.x / WAVE; h < c.m->n_kv_heads; h += OP_WAVES)
            for (int p = 0; p < np; ++p) copy_row_head(c, h, movers[p], holes[p], threadIdx.x % WAVE);
        __syncthreads();
        if (seen_h - base <= MAXMOVE) break;
    }
    return new_n;
}

// LDS working set of the op (one block per (sequence, layer)).
struct OpShared {
    int red[OP_WAVES];
    double redd[OP_WAVES];
    int32_t rpos[OP_WAVES];
    int rslot[OP_WAVES];
    int list[DEADLIST];      // dead slots (truncated rows, then victims), any order
    int sorted[DEADLIST];    // the dead slots ascending / the general compaction's holes
    int movers[DEADLIST];
    unsigned bits_lo[WIN / 32], bits_hi[WIN / 32];
    int count;
    int32_t bounds[2];
};
static_assert(DEADLIST <= OP_BLK && DEADLIST <= MAXMOVE, "a list compaction ranks one slot per thread");

// Compaction when the k dead slots (distinct, below n) are known, in any
// order in list[0..k). Same result as compact(): the holes are the dead
// slots below n - k in slot order, the movers the live slots of [n - k, n)
// in slot order, paired by rank; no pass over the other rows.
__device__ __forceinline__ int compact_list(const RowCtx& c, int n, int k, OpShared& sh) {
    if (k == 0) return n;
    const int new_n = n - k;
    for (int i = threadIdx.x; i < k; i += OP_BLK) {
        const int v = sh.list[i];
        int rk = 0;
        for (int j = 0; j < k; ++j) rk += (sh.list[j] < v);
        sh.sorted[rk] = v;
    }
    __syncthreads();
    // slot new_n + t of the tail, live unless it is among the dead
    const int t = threadIdx.x, r = new_n + t;
    int live = 0;
    if (t < k) {
        int lo = 0, hi = k;
        while (lo < hi) {
            const int mid = (lo + hi) / 2;
            if (sh.sorted[mid] < r) lo = mid + 1; else hi = mid;
        }
        live = !(lo < k && sh.sorted[lo] == r);
    }
    int np;
    const int rk = block_rank(live, sh.red, &np);   // np = dead slots below new_n
    if (live) sh.movers[rk] = r;
    __syncthreads();
    for (int h = threadIdx.x / WAVE; h < c.m->n_kv_heads; h += OP_WAVES)
        for (int p = 0; p < np; ++p) copy_row_head(c, h, sh.movers[p], sh.sorted[p], threadIdx.x % WAVE);
    __syncthreads();
    return new_n;
}

// One pass over the positions of rows [0, n), 16 rows per thread per step
// (four 16-byte loads in flight): rows at or past p0 (when trunc) go to the
// dead list (counted past DEADLIST, not listed); when bits, the other rows'
// positions below WIN and within WIN under maxpos set the window bitmaps.
// Returns the dead count.
__device__ __forceinline__ int scan_rows(const RowCtx& c, int n, bool trunc, int32_t p0, bool bits, int32_t maxpos,
                                         OpShared& sh) {
    if (bits)
        for (int i = threadIdx.x; i < WIN / 32; i += OP_BLK) {
            sh.bits_lo[i] = 0u;
            sh.bits_hi[i] = 0u;
        }
    if (threadIdx.x == 0) sh.count = 0;
    __syncthreads();
    for (int base = 0; base < n; base += 16 * OP_BLK) {
        int4 pv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = base + 4 * ((int)threadIdx.x + j * OP_BLK);
            pv[j] = r < n ? *reinterpret_cast<const int4*>(c.pos + r) : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int32_t pe[4] = {pv[j].x, pv[j].y, pv[j].z, pv[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = base + 4 * ((int)threadIdx.x + j * OP_BLK) + e;
                if (r >= n) continue;
                const int32_t p = pe[e];
                if (trunc && p >= p0) {
                    const int i = atomicAdd(&sh.count, 1);
                    if (i < DEADLIST) sh.list[i] = r;
                } else if (bits) {
                    if (p < WIN) atomicOr(&sh.bits_lo[p / 32], 1u << (p % 32));
                    const int32_t dtop = maxpos - p;
                    if (dtop >= 0 && dtop < WIN) atomicOr(&sh.bits_hi[dtop / 32], 1u << (dtop % 32));
                }
            }
        }
    }
    __syncthreads();
    return sh.count;
}

// The lowest (score, position) row with sink_max < pos < recent_min, marked
// DEAD and put in the dead list at index k; every thread gets its slot (-1
// when no row qualifies). 16 rows per thread per step.
__device__ __forceinline__ int select_victim(const RowCtx& c, int n, int32_t sink_max, int32_t recent_min, int k,
                                             OpShared& sh) {
    double best = INFINITY;
    int32_t bpos = INT_MAX;
    int bslot = -1;
    for (int base = 0; base < n; base += 16 * OP_BLK) {
        int4 pv[4];
        double2 sa[4], sb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = base + 4 * ((int)threadIdx.x + j * OP_BLK);
            if (r < n) {
                pv[j] = *reinterpret_cast<const int4*>(c.pos + r);
                sa[j] = *reinterpret_cast<const double2*>(c.score + r);
                sb[j] = *reinterpret_cast<const double2*>(c.score + r + 2);
            } else {
                pv[j] = make_int4(DEAD, DEAD, DEAD, DEAD);
                sa[j] = sb[j] = make_double2(0.0, 0.0);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int32_t pe[4] = {pv[j].x, pv[j].y, pv[j].z, pv[j].w};
            const double se[4] = {sa[j].x, sa[j].y, sb[j].x, sb[j].y};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = base + 4 * ((int)threadIdx.x + j * OP_BLK) + e;
                const int32_t p = pe[e];
                if (r >= n || p == DEAD || p <= sink_max || p >= recent_min) continue;
                if (se[e] < best || (se[e] == best && p < bpos)) {
                    best = se[e];
                    bpos = p;
                    bslot = r;
                }
            }
        }
    }
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        const double ob = __shfl_xor(best, o);
        const int32_t op = __shfl_xor(bpos, o);
        const int os = __shfl_xor(bslot, o);
        if (ob < best || (ob == best && op < bpos)) {
            best = ob;
            bpos = op;
            bslot = os;
        }
    }
    const int w = threadIdx.x / WAVE;
    __syncthreads();
    if (threadIdx.x % WAVE == 0) {
        sh.redd[w] = best;
        sh.rpos[w] = bpos;
        sh.rslot[w] = bslot;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double b = sh.redd[0];
        int32_t bp = sh.rpos[0];
        int bs = sh.rslot[0];
        for (int i = 1; i < OP_WAVES; ++i)
            if (sh.redd[i] < b || (sh.redd[i] == b && sh.rpos[i] < bp)) {
                b = sh.redd[i];
                bp = sh.rpos[i];
                bs = sh.rslot[i];
            }
        if (bs >= 0) {
            c.pos[bs] = DEAD;
            if (k < DEADLIST) sh.list[k] = bs;
        }
        sh.count = bs;
    }
    __syncthreads();
    const int bs = sh.count;
    __syncthreads();
    return bs;
}

// One victim when the protected windows are the contiguous position ranges
// [0, sink) and [maxpos - recent + 1, maxpos] (every position in them live,
// the usual case of a decode step): one pass over rows [0, n) counts the live
// positions in both windows (`absent` of them are not in those rows yet: the
// rows about to be appended) and finds the lowest (score, position) row
// strictly between them -- the victim select_victim would pick under the
// bounds those windows give. Returns the victim's slot, marked DEAD and
// listed at sh.list[0]; -1 when a window is not whole or no row lies between
// them (the caller then takes the general path; nothing was changed).
__device__ __forceinline__ int select_fast(const RowCtx& c, int n, int sink, int recent, int32_t maxpos, int absent,
                                           OpShared& sh) {
    const int32_t smax = sink - 1, rmin = maxpos - recent + 1;
    double best = INFINITY;
    int32_t bpos = INT_MAX;
    int bslot = -1, cnt = 0;   // cnt: live rows in the two windows
    for (int base = 0; base < n; base += 16 * OP_BLK) {
        int4 pv[4];
        double2 sa[4], sb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = base + 4 * ((int)threadIdx.x + j * OP_BLK);
            if (r < n) {
                pv[j] = *reinterpret_cast<const int4*>(c.pos + r);
                sa[j] = *reinterpret_cast<const double2*>(c.score + r);
                sb[j] = *reinterpret_cast<const double2*>(c.score + r + 2);
            } else {
                pv[j] = make_int4(DEAD, DEAD, DEAD, DEAD);
                sa[j] = sb[j] = make_double2(0.0, 0.0);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int32_t pe[4] = {pv[j].x, pv[j].y, pv[j].z, pv[j].w};
            const double se[4] = {sa[j].x, sa[j].y, sb[j].x, sb[j].y};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = base + 4 * ((int)threadIdx.x + j * OP_BLK) + e;
                const int32_t p = pe[e];
                if (r >= n || p == DEAD) continue;
                if (p <= smax || (p >= rmin && p <= maxpos)) {
                    ++cnt;
                } else if (p > smax && p < rmin && (se[e] < best || (se[e] == best && p < bpos))) {
                    best = se[e];
                    bpos = p;
                    bslot = r;
                }
            }
        }
    }
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        const double ob = __shfl_xor(best, o);
        const int32_t op = __shfl_xor(bpos, o);
        const int os = __shfl_xor(bslot, o);
        cnt += __shfl_xor(cnt, o);
        if (ob < best || (ob == best && op < bpos)) {
            best = ob;
            bpos = op;
            bslot = os;
        }
    }
    const int w = threadIdx.x / WAVE;
    __syncthreads();
    if (threadIdx.x % WAVE == 0) {
        sh.redd[w] = best;
        sh.rpos[w] = bpos;
        sh.rslot[w] = bslot;
        sh.red[w] = cnt;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double b = sh.redd[0];
        int32_t bp = sh.rpos[0];
        int bs = sh.rslot[0], total = sh.red[0];
        for (int i = 1; i < OP_WAVES; ++i) {
            total += sh.red[i];
            if (sh.redd[i] < b || (sh.redd[i] == b && sh.rpos[i] < bp)) {
                b = sh.redd[i];
                bp = sh.rpos[i];
                bs = sh.rslot[i];
            }
        }
        if (total != sink + recent - absent) bs = -1;   // a window is not whole: the general path decides
        if (bs >= 0) {
            c.pos[bs] = DEAD;
            sh.list[0] = bs;
        }
        sh.count = bs;
    }
    __syncthreads();
    const int bs = sh.count;
    __syncthreads();
    return bs;
}

// Evict down to `budget` (compress.py:159-179): protected = the `sink` lowest
// and `recent` highest live positions (recent == 0 protects all); drop the
// n - budget lowest (score, position) of the rest. have_bits: the window
// bitmaps already hold every live row but the `cnt` appended at p0.. (maxpos
// = p0 + cnt - 1).
// (every helper of the op kernel is inlined: a call would give the kernel a
// stack in scratch, whose setup costs more than the eviction itself)
__device__ __forceinline__ int evict(const RowCtx& c, int n, int budget, dkv_qcfg_t cfg, int32_t p0, int cnt,
                                     bool have_bits, OpShared& sh) {
    if (n <= budget || cfg.recent == 0) return n;
    const int n_drop = n - budget;
    const int32_t maxpos = p0 + cnt - 1;
    // the usual decode step: one victim, both windows whole (disjoint, with rows between them)
    if (n_drop == 1 && maxpos - cfg.recent + 1 > cfg.sink &&
        select_fast(c, n, cfg.sink, cfg.recent, maxpos, 0, sh) >= 0)
        return compact_list(c, n, 1, sh);
    // sink-th smallest and recent-th largest live positions, from bitmaps of
    // the windows [0, WIN) and (maxpos - WIN, maxpos]
    if (have_bits) {
        for (int t = threadIdx.x; t < cnt; t += OP_BLK) {
            const int32_t p = p0 + t;
            if (p < WIN) atomicOr(&sh.bits_lo[p / 32], 1u << (p % 32));
            const int32_t dtop = maxpos - p;
            if (dtop >= 0 && dtop < WIN) atomicOr(&sh.bits_hi[dtop / 32], 1u << (dtop % 32));
        }
        __syncthreads();
    } else {
        scan_rows(c, n, false, 0, true, maxpos, sh);
    }
    if (threadIdx.x == 0) {
        int32_t sink_max = -1;          // rows with pos <= sink_max are protected
        int cnt_lo = 0;
        for (int p = 0; p < WIN && cnt_lo < cfg.sink; ++p)
            if (sh.bits_lo[p / 32] >> (p % 32) & 1u) { ++cnt_lo; sink_max = p; }
        int32_t recent_min = INT_MAX;   // rows with pos >= recent_min are protected
        int cnt_hi = 0;
        for (int dt = 0; dt < WIN && cnt_hi < cfg.recent; ++dt)
            if (sh.bits_hi[dt / 32] >> (dt % 32) & 1u) { ++cnt_hi; recent_min = maxpos - dt; }
        sh.bounds[0] = (cnt_hi >= cfg.recent || cnt_hi == n) ? recent_min : -2;   // -2: not within the window
        sh.bounds[1] = sink_max;
    }
    __syncthreads();
    int32_t recent_min = sh.bounds[0];
    const int32_t sink_max = sh.bounds[1];
    if (recent_min == -2) {
        // binary search the recent-th largest live position
        int32_t lo = 0, hi = maxpos;
        while (lo < hi) {
            const int32_t mid = lo + (hi - lo + 1) / 2;
            int cnt_ge = 0;
            for (int r = threadIdx.x; r < n; r += OP_BLK) cnt_ge += (c.pos[r] >= mid);
            cnt_ge = block_sum_int(cnt_ge, sh.red);
            if (cnt_ge >= cfg.recent) lo = mid; else hi = mid - 1;
        }
        recent_min = lo;
    }
    int nv = 0;
    for (; nv < n_drop; ++nv)
        if (select_victim(c, n, sink_max, recent_min, nv, sh) < 0) break;
    if (nv <= DEADLIST) return compact_list(c, n, nv, sh);
    return compact(c, n, DEAD, sh.red, sh.sorted, sh.movers);
}

// ------------------------------------------------------------ fused layer op
// Per (seq, layer): optional truncate (pos >= start), append of `cnt` rows at
// positions start.. from the input tensors or the full cache, then evict.
struct OpArgs {
    dkv_drafter_t m;
    dkv_paged_t full;        // used when src_full
    dkv_qcfg_t cfgs[64];     // per layer arm
    const void* k;           // [batch][T][Hkv][D] when !src_full
    const void* v;
    int in_dtype, T, src_full, do_trunc, layer0;
    const int32_t* start;
    const int32_t* count;    // rows appended per seq (NULL = T) when !src_full
    const int32_t* end;      // end position per seq when src_full
    const int32_t* budget;   // [layer*batch + s], or [s] when budget_per_layer == 0
    int budget_per_layer;
};

__global__ void __launch_bounds__(OP_BLK) drafter_op_kernel(OpArgs a) {
    const int s = blockIdx.x, L = a.layer0 + blockIdx.y;
    const dkv_drafter_t& m = a.m;
    const dkv_qcfg_t cfg = a.cfgs[L];
    const int D = m.head_dim, H = m.n_kv_heads;
    __shared__ OpShared sh;

    RowCtx c{&a.m, s, L, cfg.bits, page_fmt(cfg, D), m.pos + row_index(m, s, L), m.score + row_index(m, s, L)};
    // the one-row append of a decode step: the wave that owns head w loads
    // the row's K and V channels first, with the row count, as neither
    // depends on the mirror's state
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const bool pre = !a.src_full && a.T == 1 && w < H;
    float pk[8], pv[8];
    if (pre) {
        const int64_t src = ((int64_t)s * H + w) * D;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int d = 8 * lane + e;
            pk[e] = d < D ? load_elem(a.k, src + d, a.in_dtype) : 0.0f;
            pv[e] = d < D ? load_elem(a.v, src + d, a.in_dtype) : 0.0f;
        }
    }
    int32_t* nrows_p = m.n_rows + (int64_t)s * m.n_layers + L;
    int n = *nrows_p;
    const int32_t p0 = a.start[s];
    int want = a.src_full ? (a.end[s] - p0) : (a.count ? a.count[s] : a.T);
    if (want < 0) want = 0;
    // When the rows fit without clipping at cap, the eviction window (maxpos
    // = p0 + want - 1) is known before the truncation, and one pass over the
    // positions finds the truncated rows and fills the window bitmaps.
    const bool one_pass = a.do_trunc && want > 0 && n + want <= m.cap && cfg.recent != 0;
    bool have_bits = false;
    if (a.do_trunc) {
        const int nd = scan_rows(c, n, true, p0, one_pass, p0 + want - 1, sh);
        have_bits = one_pass;
        n = (nd <= DEADLIST) ? compact_list(c, n, nd, sh) : compact(c, n, p0, sh.red, sh.sorted, sh.movers);
    }
    int cnt = want;
    if (n + cnt > m.cap) cnt = max(0, m.cap - n);   // the host sizes cap; never write past it
    const int budget = cnt > 0 ? a.budget[a.budget_per_layer ? (L * m.batch + s) : s] : 0;
    // The decode step (one row in, one over budget, both protected windows
    // whole): the victim is found first, over the rows already there (the new
    // row is the newest, protected), and the new row is written into its slot
    // -- what the append, the eviction and the compaction that moves the new
    // row into the hole leave, without the moves.
    int dest = n;   // slot of the first appended row
    bool replaced = false;
    if (!a.do_trunc && cnt == 1 && cfg.recent != 0 && n + 1 - budget == 1 && p0 - cfg.recent + 1 > cfg.sink) {
        const int v = select_fast(c, n, cfg.sink, cfg.recent, p0, 1, sh);
        if (v >= 0) {
            dest = v;
            replaced = true;
        }
    }
    for (int h = w; h < H; h += OP_WAVES) {        // one wave per head segment
        for (int t = 0; t < cnt; ++t) {
            const int slot = dest + t;
            uint8_t* page = page_ptr(m, s, L, h, slot / PAGE);
            const int i = slot % PAGE;
            if (pre && h == w) {   // (T == 1: t == 0) the channels loaded above
                quant_row_vals(pk, pv, c.f, cfg.bits, page, i, lane);
            } else if (a.src_full) {
                const dkv_paged_t& f = a.full;
                const int pos = p0 + t;
                const int32_t blk = paged_block(f, s, L, pos);
                const int off = pos % f.block_size;
                quant_row([&](int d) { return load_elem(f.pool, paged_k_off(f, blk, off, h, d), f.dtype); },
                          [&](int d) { return load_elem(f.pool, paged_v_off(f, blk, off, h, d), f.dtype); }, c.f,
                          cfg.bits, page, i, lane);
            } else {
                const int64_t src = (((int64_t)s * a.T + t) * H + h) * D;
                quant_row([&](int d) { return load_elem(a.k, src + d, a.in_dtype); },
                          [&](int d) { return load_elem(a.v, src + d, a.in_dtype); }, c.f, cfg.bits, page, i, lane);
            }
            if (lane == 0 && h == 0) {
                c.pos[slot] = p0 + t;
                c.score[slot] = 0.0;
            }
        }
    }
    __syncthreads();
    if (!replaced) {
        n += cnt;
        if (cnt > 0) n = evict(c, n, budget, cfg, p0, cnt, have_bits && cnt == want, sh);
    }
    __syncthreads();
    if (threadIdx.x == 0) *nrows_p = n;
}

// ------------------------------------------------------------ rebuild
// grid: x = page, y = sequence, z = index into the changed-layer list. All
// scores restart at 0, so the survivors are the closed form
// [0, sink) u [n - (B - sink), n); only those rows are quantized, densely and
// in position order. One wave per (row, head).
struct RebuildArgs {
    dkv_drafter_t m;
    dkv_paged_t full;
    dkv_qcfg_t cfgs[64];
    int32_t layers[64];
    const int32_t* len;
    const int32_t* budget;
};

__global__ void __launch_bounds__(BLK) drafter_rebuild_kernel(RebuildArgs a) {
    const int s = blockIdx.y, L = a.layers[blockIdx.z];
    const dkv_drafter_t& m = a.m;
    const dkv_paged_t& f = a.full;
    const dkv_qcfg_t cfg = a.cfgs[L];
    const int D = m.head_dim, H = m.n_kv_heads;
    const int n = a.len[s];
    const int B = a.budget[L * m.batch + s];
    int kept, sink;
    if (n <= B || cfg.recent == 0) {
        kept = n;
        sink = n;
    } else {
        kept = B;
        sink = min(cfg.sink, n);
    }
    kept = min(kept, m.cap);
    const PageFmt pf = page_fmt(cfg, D);
    int32_t* pos = m.pos + row_index(m, s, L);
    double* score = m.score + row_index(m, s, L);
    const int page = blockIdx.x;
    if (page == 0 && threadIdx.x == 0) m.n_rows[(int64_t)s * m.n_layers + L] = kept;
    if (page * PAGE >= kept) return;
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const int d0 = 8 * lane;
    // one wave per (page, head); rows visited by V word group j so that a
    // lane's 8 V words (one per channel) collect all their nibbles before
    // being stored whole
    for (int h = w; h < H; h += NWAVES) {
        uint8_t* pg = page_ptr(m, s, L, h, page);
        for (int j = 0; j < 4; ++j) {
            uint32_t vw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
            for (int e = 0; e < 8; ++e) {
                const int i = e < 4 ? 4 * j + e : 16 + 4 * j + (e - 4);
                const int r = page * PAGE + i;
                if (r >= kept) continue;
                const int p = r < sink ? r : n - (kept - sink) + (r - sink);
                const int32_t blk = paged_block(f, s, L, p);
                const int off = p % f.block_size;
                LaneCodes lc;
                quant_lane([&](int d) { return load_elem(f.pool, paged_k_off(f, blk, off, h, d), f.dtype); }, pf,
                           cfg.bits, lane, lc);
                put_k_lane(pg, pf, i, lane, lc);
                quant_lane([&](int d) { return load_elem(f.pool, paged_v_off(f, blk, off, h, d), f.dtype); }, pf,
                           cfg.bits, lane, lc);
                if (pf.cb == 4) {
#pragma unroll
                    for (int x = 0; x < 8; ++x) vw[x] |= static_cast<uint32_t>(lc.code[x]) << code_shift(4, e);
                    if (d0 < D && d0 % pf.group == 0)
                        write_meta(pg + v_meta_off(pf, i, d0 / pf.group), lc.m, pf.meta_f16);
                } else {
                    put_v_lane(pg, pf, i, lane, lc);
                }
                if (lane == 0 && h == 0) {
                    pos[r] = p;
                    score[r] = 0.0;
                }
            }
            if (pf.cb == 4 && d0 < D) {
#pragma unroll
                for (int x = 0; x < 8; ++x) {
                    const int d = d0 + x;
                    reinterpret_cast<uint32_t*>(pg + pf.vc)[((int64_t)(d % 16) * 4 + j) * pf.NDT + d / 16] = vw[x];
                }
            }
        }
    }
}

// Rebuild, one block per few pages of a (head, sequence x changed layer)
// segment, head_dim <= 128. A block walks its pages with the next page's
// source rows in flight while the current page is quantized:
//   1. the page's kept rows of K and V (bf16/f32, from the paged full cache)
//      arrive in registers (coalesced loads, issued one page ahead) and are
//      staged in LDS as float32;
//   2. every lane quantizes 8 channels of one row (group min/max over the
//      group's lanes, zero padding of a short last group included), writes K
//      code words and the (scale, lo) pairs, and leaves V codes in LDS;
//   3. V code words (8 rows per word for 4-bit codes, 4 for bytes) are
//      assembled from LDS and stored whole.
constexpr int RB_MAXD = 128;
// rows padded by 4 floats: the V staging stores walk rows at a fixed channel,
// and a 512-byte row stride would put all 32 rows in one LDS bank (the pad
// keeps rows 16-byte aligned for the vector reads of the quantize step)
constexpr int RB_ROW = RB_MAXD + 4;
struct RebuildSmem {
    float x[2][PAGE][RB_ROW];
    uint8_t vcode[PAGE][RB_MAXD];
    int32_t blk[2][PAGE], off[2][PAGE];   // source block and slot of each row (two pages)
};

// The raw source words of one page held by a thread: K octets (8 channels of
// a row) and V elements (one channel of a row), as loaded.
template <bool BF>
struct RawPage {
    static constexpr int KU = PAGE * (RB_MAXD / 8) / BLK;   // K octets per thread
    static constexpr int VU = PAGE * RB_MAXD / BLK;         // V elements per thread
    using KWord = typename std::conditional<BF, uint4, float4>::type;
    KWord k[KU][BF ? 1 : 2];
    typename std::conditional<BF, uint16_t, float>::type v[VU];
};

template <bool BF>
__device__ __forceinline__ void load_raw(RawPage<BF>& r, const dkv_paged_t& f, int h, int D, int rows,
                                         const int32_t* sblk, const int32_t* soff) {
    using R = RawPage<BF>;
    const int64_t bel = paged_block_elems(f);
    const int64_t vb = (int64_t)f.n_kv_heads * f.block_size * D;
#pragma unroll
    for (int x = 0; x < R::KU; ++x) {
        const int u = threadIdx.x + x * BLK;
        const int i = u / (D / 8), c8 = (u % (D / 8)) * 8;
        if (u < PAGE * (D / 8) && i < rows) {
            const int64_t o = (int64_t)sblk[i] * bel + ((int64_t)h * f.block_size + soff[i]) * D + c8;
            if constexpr (BF) {
                r.k[x][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(f.pool) + o);
            } else {
                const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(f.pool) + o);
                r.k[x][0] = src[0];
                r.k[x][1] = src[1];
            }
        }
    }
#pragma unroll
    for (int x = 0; x < R::VU; ++x) {
        const int u = threadIdx.x + x * BLK;
        const int d = u / PAGE, i = u % PAGE;
        if (u < PAGE * D && i < rows) {
            const int64_t o = (int64_t)sblk[i] * bel + vb + ((int64_t)h * D + d) * f.block_size + soff[i];
            if constexpr (BF) r.v[x] = static_cast<const uint16_t*>(f.pool)[o];
            else r.v[x] = static_cast<const float*>(f.pool)[o];
        }
    }
}

template <bool BF>
__device__ __forceinline__ void stage_raw(const RawPage<BF>& r, RebuildSmem& sm, int D, int rows) {
    using R = RawPage<BF>;
#pragma unroll
    for (int x = 0; x < R::KU; ++x) {
        const int u = threadIdx.x + x * BLK;
        if (u < PAGE * (D / 8)) {
            const int i = u / (D / 8), c8 = (u % (D / 8)) * 8;
            float kv[8];
            if (i < rows) {
                if constexpr (BF) {
                    const uint32_t ww[4] = {r.k[x][0].x, r.k[x][0].y, r.k[x][0].z, r.k[x][0].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kv[2 * e] = bf16_to_f32(ww[e] & 0xffffu);
                        kv[2 * e + 1] = bf16_to_f32(ww[e] >> 16);
                    }
                } else {
                    kv[0] = r.k[x][0].x; kv[1] = r.k[x][0].y; kv[2] = r.k[x][0].z; kv[3] = r.k[x][0].w;
                    kv[4] = r.k[x][1].x; kv[5] = r.k[x][1].y; kv[6] = r.k[x][1].z; kv[7] = r.k[x][1].w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) kv[e] = 0.0f;
            }
            *reinterpret_cast<float4*>(&sm.x[0][i][c8]) = make_float4(kv[0], kv[1], kv[2], kv[3]);
            *reinterpret_cast<float4*>(&sm.x[0][i][c8 + 4]) = make_float4(kv[4], kv[5], kv[6], kv[7]);
        }
    }
#pragma unroll
    for (int x = 0; x < R::VU; ++x) {
        const int u = threadIdx.x + x * BLK;
        if (u < PAGE * D) {
            const int i = u % PAGE;
            float v = 0.0f;
            if (i < rows) {
                if constexpr (BF) v = bf16_to_f32(r.v[x]);
                else v = r.v[x];
            }
            sm.x[1][i][u / PAGE] = v;
        }
    }
}

template <bool BF>
__global__ void __launch_bounds__(BLK) drafter_rebuild_page_kernel(RebuildArgs a) {
    const int h = blockIdx.y;
    const int s = blockIdx.z % a.m.batch, L = a.layers[blockIdx.z / a.m.batch];
    const dkv_drafter_t& m = a.m;
    const dkv_paged_t& f = a.full;
    const dkv_qcfg_t cfg = a.cfgs[L];
    const int D = m.head_dim;
    const int n = a.len[s];
    const int B = a.budget[L * m.batch + s];
    int kept, sink;
    if (n <= B || cfg.recent == 0) {
        kept = n;
        sink = n;
    } else {
        kept = B;
        sink = min(cfg.sink, n);
    }
    kept = min(kept, m.cap);
    if (blockIdx.x == 0 && h == 0 && threadIdx.x == 0) m.n_rows[(int64_t)s * m.n_layers + L] = kept;
    __shared__ RebuildSmem sm;
    const PageFmt pf = page_fmt(cfg, D);
    auto pos_of = [&](int r) { return r < sink ? r : n - (kept - sink) + (r - sink); };
    // source block and slot of the rows of page pg, into table b (threads < PAGE)
    auto lookup = [&](int pg, int b) {
        if (threadIdx.x < PAGE) {
            const int i = threadIdx.x, r = pg * PAGE + i;
            int32_t blk = 0, off = 0;
            if (r < kept) {
                const int p = pos_of(r);
                blk = paged_block(f, s, L, p);
                off = p % f.block_size;
            }
            sm.blk[b][i] = blk;
            sm.off[b][i] = off;
        }
    };
    // each block takes a contiguous run of the segment's pages, so a source
    // block shared by two pages is read twice in a row by one block (the
    // second time from its XCD's L2)
    const int npg = (kept + PAGE - 1) / PAGE;
    const int per = (npg + (int)gridDim.x - 1) / (int)gridDim.x;
    int page = blockIdx.x * per;
    const int pend = min(npg, page + per);
    if (page >= pend) return;
    RawPage<BF> raw;
    lookup(page, 0);
    __syncthreads();
    load_raw<BF>(raw, f, h, D, min(PAGE, kept - page * PAGE), sm.blk[0], sm.off[0]);
    for (int it = 0; page < pend; ++page, ++it) {
        const int r0 = page * PAGE;
        const int rows = min(PAGE, kept - r0);
        const int nxt = page + 1;
        const bool more = nxt < pend;
        uint8_t* pg = page_ptr(m, s, L, h, page);
        __syncthreads();   // the previous page's quantize and packing are done with LDS
        stage_raw<BF>(raw, sm, D, rows);
        if (more) lookup(nxt, (it + 1) & 1);
        __syncthreads();
        // the next page's rows go out now and arrive during this page's work
        if (more) load_raw<BF>(raw, f, h, D, min(PAGE, kept - nxt * PAGE), sm.blk[(it + 1) & 1], sm.off[(it + 1) & 1]);

        // ---- 2. quantize: lane = (tensor, row, octet); a row owns U2 lanes (power of two)
        const int gl = pf.cb == 32 ? 1 : pf.group / 8;         // lanes per group
        const int U = pf.cb == 32 ? D / 8 : pf.NG * gl;          // octets that belong to a group
        int U2 = 1;
        while (U2 < U) U2 <<= 1;
        for (int u = threadIdx.x; u < 2 * PAGE * U2; u += BLK) {
            const int t = u / (PAGE * U2), rem = u % (PAGE * U2);
            const int i = rem / U2, oct = rem % U2, d0 = 8 * oct;
            const bool live = i < rows;
            float v[8];
            if (d0 + 8 <= D) {
                const float4 a0 = *reinterpret_cast<const float4*>(&sm.x[t][i][d0]);
                const float4 a1 = *reinterpret_cast<const float4*>(&sm.x[t][i][d0 + 4]);
                v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
                v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (d0 + e < D) ? sm.x[t][i][d0 + e] : 0.0f;
            }
            if (pf.cb == 32) {
                if (live && d0 < D) {
                    float* dst = reinterpret_cast<float*>(pg + (t ? pf.vc : pf.kc)) + (int64_t)i * D + d0;
#pragma unroll
                    for (int e = 0; e < 8; ++e) dst[e] = v[e];
                }
                continue;
            }
            float mn = INFINITY, mx = -INFINITY;
            if (oct < U) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    mn = fminf(mn, v[e]);
                    mx = fmaxf(mx, v[e]);
                }
            }
            for (int o = 1; o < gl; o <<= 1) {
                mn = fminf(mn, __shfl_xor(mn, o));
                mx = fmaxf(mx, __shfl_xor(mx, o));
            }
            const GroupMeta gm = group_meta(mn, mx, cfg.bits, pf.meta_f16);
            uint32_t code[8];
            quant_codes8(v, gm, cfg.bits, code);
            if (oct >= U || d0 >= D) continue;
            const bool first = d0 % pf.group == 0;
            if (t == 0) {
                if (!live) continue;
                uint32_t* sec = reinterpret_cast<uint32_t*>(pg + pf.kc);
                if (pf.cb == 4) {
                    uint32_t w = 0;
#pragma unroll
                    for (int e = 0; e < 8; ++e) w |= static_cast<uint32_t>(code[e]) << code_shift(4, e);
                    sec[((int64_t)i * D + d0) / 8] = w;
                } else {
                    uint32_t w0 = 0, w1 = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        w0 |= static_cast<uint32_t>(code[e]) << code_shift(8, e);
                        w1 |= static_cast<uint32_t>(code[4 + e]) << code_shift(8, e);
                    }
                    sec[k_word(pf, i, d0 / 4)] = w0;
                    sec[k_word(pf, i, d0 / 4 + 1)] = w1;
                }
                if (first) write_meta(pg + k_meta_off(pf, i, d0 / pf.group), gm, pf.meta_f16);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (d0 + e < D) sm.vcode[i][d0 + e] = static_cast<uint8_t>(code[e]);
                if (live && first) write_meta(pg + v_meta_off(pf, i, d0 / pf.group), gm, pf.meta_f16);
            }
        }
        if (h == 0) {
            int32_t* pos = m.pos + row_index(m, s, L);
            double* score = m.score + row_index(m, s, L);
            for (int i = threadIdx.x; i < rows; i += BLK) {
                pos[r0 + i] = pos_of(r0 + i);
                score[r0 + i] = 0.0;
            }
        }
        if (pf.cb == 32) continue;
        __syncthreads();

        // ---- 3. V code words: word ((a*4 + j)*NDT + t) holds channel d = 16t + a of
        // the rows (j, e) = {4j..4j+3, 16+4j..16+4j+3}; bytes: two words per (a, j, t),
        // placed by v8_word
        uint32_t* vsec = reinterpret_cast<uint32_t*>(pg + pf.vc);
        const int per = pf.cb == 4 ? 8 : 4;                     // rows per word
        const int n_words = 16 * 4 * pf.NDT * (8 / per);
        for (int u = threadIdx.x; u < n_words; u += BLK) {
            const int half = pf.cb == 4 ? 0 : u % 2;
            const int base = pf.cb == 4 ? u : u / 2;
            const int t = base % pf.NDT, aj = base / pf.NDT;
            const int j = aj % 4, acol = aj / 4;
            const int d = 16 * t + acol;
            if (d >= D) continue;
            uint32_t w = 0;
            for (int q = 0; q < per; ++q) {
                const int e = half * 4 + q;
                const int i = e < 4 ? 4 * j + e : 16 + 4 * j + (e - 4);
                const uint32_t code = sm.vcode[i][d];
                w |= code << (pf.cb == 4 ? code_shift(4, e) : code_shift(8, q));
            }
            vsec[pf.cb == 4 ? base : v8_word(pf, aj, t, half)] = w;
        }
    }
}

// ---- the common shape: bf16 source in 16-token blocks, head_dim 128, 4- or
// 8-bit codes, group G. Same output as drafter_rebuild_page_kernel, with the
// work laid out at compile time: thread tid quantizes octet tid % 16 (8
// channels) of rows tid / 16 and tid / 16 + 16 of K and of V; its V loads are
// one channel of one row each (channels tid / 32 + 8x), so all 16 share one
// base address and differ by immediate offsets. V codes are staged by
// channel (vt[d][row]), so a V code word is two 4-byte LDS reads.
constexpr int RF_VT = PAGE + 4;         // bytes per channel of staged V codes
constexpr int RF_ROW = RB_MAXD + 8;     // bf16 per staged row (16-byte aligned rows)
struct RebuildFastSmem {
    uint16_t x[2][PAGE][RF_ROW];        // the page's K and V rows as loaded (bf16)
    uint8_t vt[RB_MAXD][RF_VT];
    int64_t kb[2][PAGE], vb[2][PAGE];   // element offsets of each row's K and V channel 0 (two pages)
};

template <int CB, int G, int MF>
__global__ void __launch_bounds__(BLK) drafter_rebuild_fast_kernel(RebuildArgs a) {
    constexpr int D = 128, BS = 16, GL = G / 8, NG = D / G;
    const int h = blockIdx.y;
    const int s = blockIdx.z % a.m.batch, L = a.layers[blockIdx.z / a.m.batch];
    const dkv_drafter_t& m = a.m;
    const dkv_paged_t& f = a.full;
    const dkv_qcfg_t cfg = a.cfgs[L];
    const int n = a.len[s];
    const int B = a.budget[L * m.batch + s];
    int kept, sink;
    if (n <= B || cfg.recent == 0) {
        kept = n;
        sink = n;
    } else {
        kept = B;
        sink = min(cfg.sink, n);
    }
    kept = min(kept, m.cap);
    if (blockIdx.x == 0 && h == 0 && threadIdx.x == 0) m.n_rows[(int64_t)s * m.n_layers + L] = kept;
    __shared__ RebuildFastSmem sm;
    const PageFmt pf = page_fmt(cfg, D);   // container CB: 4 bits for 2-4-bit codes, bytes for 8
    const int bits = cfg.bits;
    const uint16_t* pool = static_cast<const uint16_t*>(f.pool);
    const int64_t bel = paged_block_elems(f);
    auto pos_of = [&](int r) { return r < sink ? r : n - (kept - sink) + (r - sink); };
    auto lookup = [&](int pg, int b) {
        if (threadIdx.x < PAGE) {
            const int i = threadIdx.x, r = pg * PAGE + i;
            int64_t kb = 0, vb = 0;
            if (r < kept) {
                const int p = pos_of(r);
                const int64_t blk = paged_block(f, s, L, p);
                kb = blk * bel + ((int64_t)h * BS + p % BS) * D;
                vb = blk * bel + (int64_t)f.n_kv_heads * BS * D + (int64_t)h * D * BS + p % BS;
            }
            sm.kb[b][i] = kb;
            sm.vb[b][i] = vb;
        }
    };
    const int tid = threadIdx.x, oct = tid % 16, kr = tid / 16;   // K: rows kr, kr + 16
    const int vi = tid % PAGE, vd = tid / PAGE;                  // V: row vi, channels vd + 8x
    uint4 rk[2];
    uint16_t rv[16];
    auto load = [&](int b, int rows) {
#pragma unroll
        for (int x = 0; x < 2; ++x)
            if (kr + 16 * x < rows) rk[x] = *reinterpret_cast<const uint4*>(pool + sm.kb[b][kr + 16 * x] + 8 * oct);
        if (vi < rows) {
            const uint16_t* p = pool + sm.vb[b][vi] + vd * BS;
#pragma unroll
            for (int x = 0; x < 16; ++x) rv[x] = p[8 * BS * x];
        }
    };
    // rows past the page's live count stage as zeros (their codes are those of 0)
    auto stage = [&](int rows) {
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            const int i = kr + 16 * x;
            *reinterpret_cast<uint4*>(&sm.x[0][i][8 * oct]) = i < rows ? rk[x] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int x = 0; x < 16; ++x) sm.x[1][vi][vd + 8 * x] = vi < rows ? rv[x] : uint16_t(0);
    };

    // each block takes a contiguous run of the segment's pages: a 16-token
    // source block that straddles two pages is then read by one block twice in
    // a row (the second time from its XCD's L2) instead of by two blocks
    const int npg = (kept + PAGE - 1) / PAGE;
    const int per = (npg + (int)gridDim.x - 1) / (int)gridDim.x;
    int page = blockIdx.x * per;
    const int pend = min(npg, page + per);
    if (page >= pend) return;
    lookup(page, 0);
    __syncthreads();
    load(0, min(PAGE, kept - page * PAGE));
    for (int it = 0; page < pend; ++page, ++it) {
        const int r0 = page * PAGE;
        const int rows = min(PAGE, kept - r0);
        const int nxt = page + 1;
        const bool more = nxt < pend;
        uint8_t* pg = page_ptr(m, s, L, h, page);
        __syncthreads();   // the previous page's quantize and packing are done with LDS
        stage(rows);
        if (more) lookup(nxt, (it + 1) & 1);
        __syncthreads();
        if (more) load((it + 1) & 1, min(PAGE, kept - nxt * PAGE));   // lands during this page's work

        // ---- quantize: items (tensor t, row i) = (0, kr), (0, kr+16), (1, kr), (1, kr+16), octet oct
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            const int t = x >> 1, i = kr + 16 * (x & 1);
            const uint4 raw8 = *reinterpret_cast<const uint4*>(&sm.x[t][i][8 * oct]);
            const uint32_t ww[4] = {raw8.x, raw8.y, raw8.z, raw8.w};
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[2 * e] = __uint_as_float(ww[e] << 16);
                v[2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
            }
            float mn = v[0], mx = v[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) {
                mn = fminf(mn, v[e]);
                mx = fmaxf(mx, v[e]);
            }
#pragma unroll
            for (int o = 1; o < GL; o <<= 1) {
                mn = fminf(mn, __shfl_xor(mn, o));
                mx = fmaxf(mx, __shfl_xor(mx, o));
            }
            const GroupMeta gm = group_meta(mn, mx, bits, MF);
            uint32_t code[8];
            quant_codes8(v, gm, bits, code);
            const bool first = oct % GL == 0, live = i < rows;
            if (t == 0) {
                if (live) {
                    uint32_t* sec = reinterpret_cast<uint32_t*>(pg + pf.kc);
                    if (CB == 4) {
                        uint32_t w = 0;
#pragma unroll
                        for (int e = 0; e < 8; ++e) w |= code[e] << code_shift(4, e);
                        sec[i * 16 + oct] = w;
                    } else {
                        uint32_t w0 = 0, w1 = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            w0 |= code[e] << code_shift(8, e);
                            w1 |= code[4 + e] << code_shift(8, e);
                        }
                        // words 2 oct and 2 oct + 1 of the row: adjacent (and 8-byte aligned) in
                        // the lane-order layout too
                        *reinterpret_cast<uint2*>(sec + k_word(pf, i, 2 * oct)) = make_uint2(w0, w1);
                    }
                    if (first) write_meta(pg + k_meta_off(pf, i, oct / GL), gm, MF);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) sm.vt[8 * oct + e][i] = static_cast<uint8_t>(code[e]);
                if (live && first) write_meta(pg + v_meta_off(pf, i, oct / GL), gm, MF);
            }
        }
        if (h == 0) {
            int32_t* pos = m.pos + row_index(m, s, L);
            double* score = m.score + row_index(m, s, L);
            if (tid < rows) {
                pos[r0 + tid] = pos_of(r0 + tid);
                score[r0 + tid] = 0.0;
            }
        }
        __syncthreads();

        // ---- V code words: group (a*4 + j)*8 + t holds channel d = 16t + a of the
        // rows {4j..4j+3} (k-slots 0..3) and {16+4j..16+4j+3} (k-slots 4..7); 4-bit
        // codes one word per group, bytes two (placed by v8_word)
        uint32_t* vsec = reinterpret_cast<uint32_t*>(pg + pf.vc);
#pragma unroll
        for (int y = 0; y < 2; ++y) {
            const int w = tid + BLK * y;   // 512 (a, j, t) triples
            const int t = w % 8, aj = w / 8, j = aj % 4, acol = aj / 4;
            const int d = 16 * t + acol;
            const uint32_t lo = *reinterpret_cast<const uint32_t*>(&sm.vt[d][4 * j]);        // rows 4j..4j+3
            const uint32_t hi = *reinterpret_cast<const uint32_t*>(&sm.vt[d][16 + 4 * j]);   // rows 16+4j..
            // byte k of lo / hi: the code of row 4j + k / 16 + 4j + k
            auto byte = [](uint32_t w, int k) { return (w >> (8 * k)) & 0xFFu; };
            if (CB == 4) {
                // k-slot e (rows 4j+e, then 16+4j+e-4) at code_shift(4, e): even slots
                // at 0, 4, 8, 12, odd ones at 16, 20, 24, 28
                vsec[w] = byte(lo, 0) | (byte(lo, 2) << 4) | (byte(hi, 0) << 8) | (byte(hi, 2) << 12) |
                          (byte(lo, 1) << 16) | (byte(lo, 3) << 20) | (byte(hi, 1) << 24) | (byte(hi, 3) << 28);
            } else {
                // slot q of each 4-row half at code_shift(8, q): q = 0, 2, 1, 3 in bytes 0..3
                vsec[v8_word(pf, aj, t, 0)] =
                    byte(lo, 0) | (byte(lo, 2) << 8) | (byte(lo, 1) << 16) | (byte(lo, 3) << 24);
                vsec[v8_word(pf, aj, t, 1)] =
                    byte(hi, 0) | (byte(hi, 2) << 8) | (byte(hi, 1) << 16) | (byte(hi, 3) << 24);
            }
        }
    }
}

// ------------------------------------------------------------ gather
struct GatherOut {
    uint8_t* codes;
    float* scale;
    float* lo;
    float* deq;
};

__global__ void __launch_bounds__(BLK) drafter_gather_kernel(dkv_drafter_t m, int s, int L, dkv_qcfg_t cfg, int rows,
                                                             GatherOut ko, GatherOut vo, int32_t* pos_out) {
    const int r = blockIdx.x;
    const int D = m.head_dim, H = m.n_kv_heads;
    const PageFmt f = page_fmt(cfg, D);
    const int p = r / PAGE, i = r % PAGE;
    if (threadIdx.x == 0 && pos_out) pos_out[r] = m.pos[row_index(m, s, L) + r];
    for (int x = threadIdx.x; x < 2 * H * D; x += blockDim.x) {
        const int is_v = x / (H * D), h = (x / D) % H, d = x % D;
        const uint8_t* pg = page_ptr(m, s, L, h, p);
        const GatherOut& o = is_v ? vo : ko;
        const int64_t oi = ((int64_t)r * H + h) * D + d;
        if (f.cb == 32) {
            const float val = reinterpret_cast<const float*>(pg + (is_v ? f.vc : f.kc))[(int64_t)i * D + d];
            if (o.codes) o.codes[oi] = 0;
            if (o.deq) o.deq[oi] = val;
            continue;
        }
        const int g = d / cfg.group;
        const GroupMeta mt = read_meta(pg + (is_v ? v_meta_off(f, i, g) : k_meta_off(f, i, g)), f.meta_f16);
        int64_t w;
        int sh;
        if (is_v) v_code_loc(f, i, d, &w, &sh); else k_code_loc(f, i, d, &w, &sh);
        const int code = read_code(pg + (is_v ? f.vc : f.kc), w, sh, f.cb);
        if (o.codes) o.codes[oi] = static_cast<uint8_t>(code);
        if (o.deq) o.deq[oi] = dequant(code, mt);
        if (d % cfg.group == 0) {
            const int64_t gi = ((int64_t)r * H + h) * f.NG + g;
            if (o.scale) o.scale[gi] = mt.scale;
            if (o.lo) o.lo[gi] = mt.lo;
        }
    }
}

// ------------------------------------------------------------ host checks
int check_mirror(const dkv_drafter_t* m, const char* fn) {
    DKV_REQUIRE(m != nullptr, std::string(fn) + ": mirror is NULL");
    DKV_REQUIRE(m->pages && m->pos && m->score && m->n_rows, std::string(fn) + ": mirror has a NULL buffer");
    // the row scans read pos and score with 16-byte loads
    DKV_REQUIRE(reinterpret_cast<uintptr_t>(m->pos) % 16 == 0 && reinterpret_cast<uintptr_t>(m->score) % 16 == 0,
                std::string(fn) + ": pos and score must be 16-byte aligned");
    DKV_REQUIRE(m->batch > 0 && m->n_layers > 0 && m->n_layers <= 64 && m->n_kv_heads > 0 && m->cap > 0 &&
                    m->cap % PAGE == 0,
                std::string(fn) + ": bad mirror shape (n_layers 1..64, cap a positive multiple of 32)");
    DKV_REQUIRE(m->head_dim == 8 || (m->head_dim > 0 && m->head_dim % 16 == 0),
                std::string(fn) + ": head_dim must be 8 or a multiple of 16");
    return DKV_OK;
}

int check_cfg(const dkv_drafter_t* m, const dkv_qcfg_t& c, const char* fn) {
    DKV_REQUIRE(c.bits == 2 || c.bits == 3 || c.bits == 4 || c.bits == 8 || c.bits == 16,
                std::string(fn) + ": bits must be 2, 3, 4, 8 or 16");
    DKV_REQUIRE(c.bits >= 16 || (c.group >= 8 && (c.group & (c.group - 1)) == 0 &&
                                  n_groups(m->head_dim, c.group) * c.group <= 512),
                std::string(fn) + ": group must be a power of two >= 8 with ceil(d/group)*group <= 512");
    DKV_REQUIRE(c.sink >= 0 && c.recent >= 0, std::string(fn) + ": sink/recent must be >= 0");
    DKV_REQUIRE(page_fmt(c, m->head_dim).bytes <= m->page_stride,
                std::string(fn) + ": arm needs more bytes per page than the mirror reserves");
    return DKV_OK;
}

}  // namespace dkv

using namespace dkv;

extern "C" int64_t dkv_page_bytes(int32_t bits, int32_t head_dim, int32_t group, int32_t meta_f16) {
    if (head_dim <= 0 || (bits < 16 && group <= 0)) return -1;
    return page_fmt(bits, head_dim, group, meta_f16).bytes;
}

extern "C" int dkv_drafter_append(const dkv_drafter_t* mirror, int32_t layer, dkv_qcfg_t cfg, const void* k,
                                  const void* v, int32_t in_dtype, int32_t T, const int32_t* start,
                                  const int32_t* count, const int32_t* budget, dkv_stream_t stream) {
    int rc = check_mirror(mirror, "dkv_drafter_append");
    if (rc) return rc;
    if ((rc = check_cfg(mirror, cfg, "dkv_drafter_append"))) return rc;
    DKV_REQUIRE(layer >= 0 && layer < mirror->n_layers, "dkv_drafter_append: layer out of range");
    DKV_REQUIRE(k && v && start && budget, "dkv_drafter_append: NULL argument");
    DKV_REQUIRE(in_dtype == DKV_F32 || in_dtype == DKV_BF16, "dkv_drafter_append: bad input dtype");
    if (T <= 0) return DKV_OK;
    OpArgs a{};
    a.m = *mirror;
    a.cfgs[layer] = cfg;
    a.k = k;
    a.v = v;
    a.in_dtype = in_dtype;
    a.T = T;
    a.layer0 = layer;
    a.start = start;
    a.count = count;
    a.budget = budget;
    hipLaunchKernelGGL(drafter_op_kernel, dim3(mirror->batch, 1), dim3(OP_BLK), 0, as_stream(stream), a);
    return check_launch("dkv_drafter_append");
}

extern "C" int dkv_drafter_truncate(const dkv_drafter_t* mirror, const dkv_qcfg_t* cfgs, const int32_t* start,
                                    dkv_stream_t stream) {
    int rc = check_mirror(mirror, "dkv_drafter_truncate");
    if (rc) return rc;
    DKV_REQUIRE(cfgs && start, "dkv_drafter_truncate: NULL argument");
    OpArgs a{};
    a.m = *mirror;
    for (int L = 0; L < mirror->n_layers; ++L) {
        if ((rc = check_cfg(mirror, cfgs[L], "dkv_drafter_truncate"))) return rc;
        a.cfgs[L] = cfgs[L];
    }
    a.do_trunc = 1;
    a.T = 0;              // nothing appended, so no eviction and budget is never read
    a.start = start;
    a.budget = start;
    hipLaunchKernelGGL(drafter_op_kernel, dim3(mirror->batch, mirror->n_layers), dim3(OP_BLK), 0, as_stream(stream), a);
    return check_launch("dkv_drafter_truncate");
}

static int same_shape(const dkv_drafter_t* m, const dkv_paged_t* f) {
    return f->n_layers == m->n_layers && f->n_kv_heads == m->n_kv_heads && f->head_dim == m->head_dim &&
           f->batch == m->batch;
}

extern "C" int dkv_drafter_sync(const dkv_drafter_t* mirror, const dkv_paged_t* full, const dkv_qcfg_t* cfgs,
                                const int32_t* start, const int32_t* end, const int32_t* budget,
                                dkv_stream_t stream) {
    int rc = check_mirror(mirror, "dkv_drafter_sync");
    if (rc) return rc;
    DKV_REQUIRE(full && cfgs && start && end && budget, "dkv_drafter_sync: NULL argument");
    DKV_REQUIRE(same_shape(mirror, full), "dkv_drafter_sync: full cache and mirror shapes differ");
    OpArgs a{};
    a.m = *mirror;
    a.full = *full;
    for (int L = 0; L < mirror->n_layers; ++L) {
        if ((rc = check_cfg(mirror, cfgs[L], "dkv_drafter_sync"))) return rc;
        a.cfgs[L] = cfgs[L];
    }
    a.src_full = 1;
    a.do_trunc = 1;
    a.start = start;
    a.end = end;
    a.budget = budget;
    a.budget_per_layer = 1;
    hipLaunchKernelGGL(drafter_op_kernel, dim3(mirror->batch, mirror->n_layers), dim3(OP_BLK), 0, as_stream(stream), a);
    return check_launch("dkv_drafter_sync");
}

extern "C" int dkv_drafter_rebuild(const dkv_drafter_t* mirror, const dkv_paged_t* full, const int32_t* layers,
                                   int32_t n_changed, const dkv_qcfg_t* cfgs, const int32_t* len,
                                   const int32_t* budget, dkv_stream_t stream) {
    int rc = check_mirror(mirror, "dkv_drafter_rebuild");
    if (rc) return rc;
    DKV_REQUIRE(full && layers && cfgs && len && budget, "dkv_drafter_rebuild: NULL argument");
    DKV_REQUIRE(same_shape(mirror, full), "dkv_drafter_rebuild: full cache and mirror shapes differ");
    DKV_REQUIRE(n_changed >= 0 && n_changed <= mirror->n_layers, "dkv_drafter_rebuild: bad layer count");
    if (n_changed == 0) return DKV_OK;
    RebuildArgs a{};
    a.m = *mirror;
    a.full = *full;
    for (int L = 0; L < mirror->n_layers; ++L) a.cfgs[L] = cfgs[L];
    for (int i = 0; i < n_changed; ++i) {
        DKV_REQUIRE(layers[i] >= 0 && layers[i] < mirror->n_layers, "dkv_drafter_rebuild: layer out of range");
        if ((rc = check_cfg(mirror, cfgs[layers[i]], "dkv_drafter_rebuild"))) return rc;
        a.layers[i] = layers[i];
    }
    a.len = len;
    a.budget = budget;
    if (mirror->head_dim <= RB_MAXD && mirror->head_dim % 8 == 0) {
        DKV_REQUIRE((int64_t)mirror->batch * n_changed <= 65535, "dkv_drafter_rebuild: batch x layers too large");
        // a few blocks per (sequence, layer, head) segment, about 4096 in all;
        // each walks its segment's pages while they hold rows
        const int segs = mirror->n_kv_heads * mirror->batch * n_changed;
        const int per_seg = std::min(mirror->cap / PAGE, std::max(1, (4096 + segs - 1) / segs));
        const dim3 grid(per_seg, mirror->n_kv_heads, mirror->batch * n_changed);
        // the compile-time kernel when every changed layer has the common shape
        bool fast = full->dtype == DKV_BF16 && full->block_size == 16 && mirror->head_dim == 128;
        int key = -1;
        for (int i = 0; i < n_changed && fast; ++i) {
            const dkv_qcfg_t& c = cfgs[layers[i]];
            const int k = (c.bits == 8 ? 8 : 0) | (c.group == 16 ? 0 : c.group == 32 ? 1 : c.group == 64 ? 2 : 3) << 1 |
                          (c.meta_f16 ? 1 : 0);
            fast = c.bits < 16 && (c.group == 16 || c.group == 32 || c.group == 64 || c.group == 128) &&
                   (key < 0 || key == k);
            key = k;
        }
        if (fast) {
#define DKV_RBF(CB, G, MF) hipLaunchKernelGGL((drafter_rebuild_fast_kernel<CB, G, MF>), grid, dim3(BLK), 0, \
                                              as_stream(stream), a)
            switch (key) {
                case 0: DKV_RBF(4, 16, 0); break;   case 1: DKV_RBF(4, 16, 1); break;
                case 2: DKV_RBF(4, 32, 0); break;   case 3: DKV_RBF(4, 32, 1); break;
                case 4: DKV_RBF(4, 64, 0); break;   case 5: DKV_RBF(4, 64, 1); break;
                case 6: DKV_RBF(4, 128, 0); break;  case 7: DKV_RBF(4, 128, 1); break;
                case 8: DKV_RBF(8, 16, 0); break;   case 9: DKV_RBF(8, 16, 1); break;
                case 10: DKV_RBF(8, 32, 0); break;  case 11: DKV_RBF(8, 32, 1); break;
                case 12: DKV_RBF(8, 64, 0); break;  case 13: DKV_RBF(8, 64, 1); break;
                case 14: DKV_RBF(8, 128, 0); break; default: DKV_RBF(8, 128, 1); break;
            }
#undef DKV_RBF
        } else if (full->dtype == DKV_BF16) {
            hipLaunchKernelGGL(drafter_rebuild_page_kernel<true>, grid, dim3(BLK), 0, as_stream(stream), a);
        } else {
            hipLaunchKernelGGL(drafter_rebuild_page_kernel<false>, grid, dim3(BLK), 0, as_stream(stream), a);
        }
    } else {
        hipLaunchKernelGGL(drafter_rebuild_kernel, dim3(mirror->cap / PAGE, mirror->batch, n_changed), dim3(BLK), 0,
                           as_stream(stream), a);
    }
    return check_launch("dkv_drafter_rebuild");
}

extern "C" int dkv_drafter_gather(const dkv_drafter_t* mirror, int32_t seq, int32_t layer, dkv_qcfg_t cfg,
                                  int32_t rows, uint8_t* k_codes, float* k_scale, float* k_lo, float* k_deq,
                                  uint8_t* v_codes, float* v_scale, float* v_lo, float* v_deq, int32_t* pos,
                                  dkv_stream_t stream) {
    int rc = check_mirror(mirror, "dkv_drafter_gather");
    if (rc) return rc;
    if ((rc = check_cfg(mirror, cfg, "dkv_drafter_gather"))) return rc;
    DKV_REQUIRE(seq >= 0 && seq < mirror->batch && layer >= 0 && layer < mirror->n_layers,
                "dkv_drafter_gather: seq/layer out of range");
    DKV_REQUIRE(rows >= 0 && rows <= mirror->cap, "dkv_drafter_gather: rows out of range");
    if (rows == 0) return DKV_OK;
    hipLaunchKernelGGL(drafter_gather_kernel, dim3(rows), dim3(BLK), 0, as_stream(stream), *mirror, seq, layer, cfg,
                       rows, GatherOut{k_codes, k_scale, k_lo, k_deq}, GatherOut{v_codes, v_scale, v_lo, v_deq}, pos);
    return check_launch("dkv_drafter_gather");
}
