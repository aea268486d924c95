// Drafter mirror maintenance: (a1,a3,a4) append + evict, (a9) truncate and
// per-round resync, (c) rebuild under a new arm, and a gather for `read`.
// Reference: draftkv/compress.py:95-241.
//
// Storage: per (seq, layer, kv head) a dense segment of row slots; rows
// 0..n_rows-1 are live, in no particular order (attention is order-free and
// the eviction order is defined on (score, position), not on slots). Both
// eviction and truncation keep the segment dense by moving surviving rows
// from the tail into the holes ("eviction compaction").
#include <climits>

#include "dkv_common.h"

namespace dkv {

constexpr int BLK = 256;
constexpr int NWAVES = BLK / WAVE;
constexpr int MAXMOVE = 1024;     // hole/mover pairs handled per compaction pass
constexpr int WIN = 4096;         // position window scanned for the sink/recent bounds
constexpr int32_t DEAD = INT_MAX; // position marking an evicted row before compaction

// ------------------------------------------------------------ row quantizer
// One wave quantizes one head-row of D values fetched by `ld(j)` and writes
// its packed codes and (scale, lo) pairs.
template <class Load>
__device__ void quant_head_row(Load ld, int D, dkv_qcfg_t cfg, uint8_t* crow, uint8_t* mrow, int lane) {
    if (cfg.bits >= 16) {
        float* f = reinterpret_cast<float*>(crow);
        for (int j = lane; j < D; j += WAVE) f[j] = ld(j);
        return;
    }
    const int ng = n_groups(D, cfg.group);
    for (int g = 0; g < ng; ++g) {
        float mn = INFINITY, mx = -INFINITY;
        for (int e = lane; e < cfg.group; e += WAVE) {
            const int j = g * cfg.group + e;
            const float v = j < D ? ld(j) : 0.0f;
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        mn = wave_min(mn);
        mx = wave_max(mx);
        const GroupMeta m = group_meta(mn, mx, cfg.bits, cfg.meta_f16);
        if (lane == 0) put_meta(mrow, g, m, cfg.meta_f16);
        const int j0 = g * cfg.group, j1 = min(D, j0 + cfg.group);
        if (cfg.bits == 8) {
            for (int j = j0 + lane; j < j1; j += WAVE) crow[j] = static_cast<uint8_t>(quant_code(ld(j), m, 8));
        } else {
            // two codes per byte; groups start on even elements (group is even or
            // the row holds a single group)
            for (int j = j0 + 2 * lane; j < j1; j += 2 * WAVE) {
                const int lo_c = quant_code(ld(j), m, cfg.bits);
                const int hi_c = (j + 1 < j1) ? quant_code(ld(j + 1), m, cfg.bits) : 0;
                crow[j >> 1] = static_cast<uint8_t>(lo_c | (hi_c << 4));
            }
        }
    }
}

// ------------------------------------------------------------ block helpers
__device__ int block_sum_int(int v, int* red) {
    v = wave_sum_i(v);
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    int t = 0;
    for (int i = 0; i < NWAVES; ++i) t += red[i];
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
    for (int i = 0; i < NWAVES; ++i) {
        if (i < w) off += red[i];
        tot += red[i];
    }
    *total = tot;
    return off + below;
}

struct RowCtx {
    const dkv_drafter_t* m;
    int s, L;
    int64_t crow_bytes, mrow_bytes;   // bytes per head-row for this layer's arm
    int32_t* pos;                     // this (s, L)'s pos array
    double* score;
};

// copy one row slot to another (all heads, K and V, codes and meta, pos, score)
__device__ void copy_row(const RowCtx& c, int from, int to, int part, int nparts) {
    const dkv_drafter_t& m = *c.m;
    const int H = m.n_kv_heads;
    const int64_t cw = c.crow_bytes / 4, mw = c.mrow_bytes / 4;
    const int64_t per_head = 2 * (cw + mw);
    for (int64_t i = part; i < H * per_head; i += nparts) {
        const int h = i / per_head;
        int64_t r = i % per_head;
        Seg sg = seg_of(m, c.s, c.L, h);
        uint8_t* base;
        int64_t rb;
        if (r < cw) { base = sg.kc; rb = c.crow_bytes; }
        else if ((r -= cw) < cw) { base = sg.vc; rb = c.crow_bytes; }
        else if ((r -= cw) < mw) { base = sg.km; rb = c.mrow_bytes; }
        else { r -= mw; base = sg.vm; rb = c.mrow_bytes; }
        uint32_t* dst = reinterpret_cast<uint32_t*>(base + (int64_t)to * rb);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(base + (int64_t)from * rb);
        dst[r] = src[r];
    }
    if (part == 0) {
        c.pos[to] = c.pos[from];
        c.score[to] = c.score[from];
    }
}

// Keep rows with pos < thr: move survivors from [new_n, n) into the holes of
// [0, new_n). Returns new_n. Whole block participates.
__device__ int compact(const RowCtx& c, int n, int32_t thr, int* red, int* holes, int* movers) {
    int keep = 0;
    for (int r = threadIdx.x; r < n; r += BLK) keep += (c.pos[r] < thr);
    const int new_n = block_sum_int(keep, red);
    if (new_n == n) return n;
    // ranks of holes in [0, new_n) and movers in [new_n, n), processed in
    // windows of MAXMOVE pairs
    for (int base = 0;; base += MAXMOVE) {
        int nh = 0, nm = 0, seen_h = 0, seen_m = 0;
        __syncthreads();
        for (int r0 = 0; r0 < new_n; r0 += BLK) {
            const int r = r0 + threadIdx.x;
            const int f = (r < new_n) && (c.pos[r] >= thr);
            int tot;
            const int rk = block_rank(f, red, &tot) + seen_h;
            if (f && rk >= base && rk < base + MAXMOVE) holes[rk - base] = r;
            seen_h += tot;
        }
        for (int r0 = new_n; r0 < n; r0 += BLK) {
            const int r = r0 + threadIdx.x;
            const int f = (r < n) && (c.pos[r] < thr);
            int tot;
            const int rk = block_rank(f, red, &tot) + seen_m;
            if (f && rk >= base && rk < base + MAXMOVE) movers[rk - base] = r;
            seen_m += tot;
        }
        nh = min(MAXMOVE, seen_h - base);
        nm = min(MAXMOVE, seen_m - base);
        __syncthreads();
        const int np = min(nh, nm);
        if (np <= 0) break;
        // each pair is copied by a slice of the block
        for (int p = 0; p < np; ++p) copy_row(c, movers[p], holes[p], threadIdx.x, BLK);
        __syncthreads();
        if (seen_h - base <= MAXMOVE) break;
    }
    return new_n;
}

// Evict down to `budget` (compress.py:159-179): protected = the `sink` lowest
// and `recent` highest live positions (recent == 0 protects all); drop the
// n - budget lowest (score, position) of the rest.
__device__ int evict(const RowCtx& c, int n, int budget, dkv_qcfg_t cfg, int32_t maxpos, int* red,
                     int* holes, int* movers, unsigned* bits_lo, unsigned* bits_hi, double* redd) {
    if (n <= budget || cfg.recent == 0) return n;
    const int n_drop = n - budget;
    // bounds: sink-th smallest and recent-th largest live positions, from
    // bitmaps of the windows [0, WIN) and (maxpos - WIN, maxpos]
    for (int i = threadIdx.x; i < WIN / 32; i += BLK) {
        bits_lo[i] = 0u;
        bits_hi[i] = 0u;
    }
    __syncthreads();
    for (int r = threadIdx.x; r < n; r += BLK) {
        const int32_t p = c.pos[r];
        if (p < WIN) atomicOr(&bits_lo[p / 32], 1u << (p % 32));
        const int32_t dtop = maxpos - p;
        if (dtop >= 0 && dtop < WIN) atomicOr(&bits_hi[dtop / 32], 1u << (dtop % 32));
    }
    __syncthreads();
    __shared__ int32_t s_bounds[2];
    if (threadIdx.x == 0) {
        int32_t sink_max = -1;          // rows with pos <= sink_max are protected
        int cnt = 0;
        for (int p = 0; p < WIN && cnt < cfg.sink; ++p)
            if (bits_lo[p / 32] >> (p % 32) & 1u) { ++cnt; sink_max = p; }
        int32_t recent_min = INT_MAX;   // rows with pos >= recent_min are protected
        cnt = 0;
        for (int dt = 0; dt < WIN && cnt < cfg.recent; ++dt)
            if (bits_hi[dt / 32] >> (dt % 32) & 1u) { ++cnt; recent_min = maxpos - dt; }
        s_bounds[0] = (cnt >= cfg.recent || cnt == n) ? recent_min : -2;   // -2: not found in window
        s_bounds[1] = sink_max;
    }
    __syncthreads();
    int32_t recent_min = s_bounds[0];
    const int32_t sink_max = s_bounds[1];
    if (recent_min == -2) {
        // fall back: binary search the recent-th largest position
        int32_t lo = 0, hi = maxpos;   // answer in [lo, hi]
        while (lo < hi) {
            const int32_t mid = lo + (hi - lo + 1) / 2;
            int cnt = 0;
            for (int r = threadIdx.x; r < n; r += BLK) cnt += (c.pos[r] >= mid);
            cnt = block_sum_int(cnt, red);
            if (cnt >= cfg.recent) lo = mid; else hi = mid - 1;
        }
        recent_min = lo;
    }
    // select victims one at a time: lowest (score, pos) among unprotected
    __shared__ int s_slot[NWAVES];
    __shared__ int32_t s_pos[NWAVES];
    for (int k = 0; k < n_drop; ++k) {
        double best = INFINITY;
        int32_t bpos = INT_MAX;
        int bslot = -1;
        for (int r = threadIdx.x; r < n; r += BLK) {
            const int32_t p = c.pos[r];
            if (p == DEAD || p <= sink_max || p >= recent_min) continue;
            const double sc = c.score[r];
            if (sc < best || (sc == best && p < bpos)) { best = sc; bpos = p; bslot = r; }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const double ob = __shfl_xor(best, o);
            const int32_t op = __shfl_xor(bpos, o);
            const int os = __shfl_xor(bslot, o);
            if (ob < best || (ob == best && op < bpos)) { best = ob; bpos = op; bslot = os; }
        }
        const int w = threadIdx.x / WAVE;
        __syncthreads();
        if (threadIdx.x % WAVE == 0) { redd[w] = best; s_pos[w] = bpos; s_slot[w] = bslot; }
        __syncthreads();
        if (threadIdx.x == 0) {
            double b = redd[0];
            int32_t bp = s_pos[0];
            int bs = s_slot[0];
            for (int i = 1; i < NWAVES; ++i)
                if (redd[i] < b || (redd[i] == b && s_pos[i] < bp)) { b = redd[i]; bp = s_pos[i]; bs = s_slot[i]; }
            if (bs >= 0) c.pos[bs] = DEAD;
        }
        __syncthreads();
    }
    return compact(c, n, DEAD, red, holes, movers);
}

// ------------------------------------------------------------ fused layer op
// Per (seq, layer): optional truncate (pos >= trunc_at), append of `cnt`
// rows at positions p0.. from either the input tensors or the full cache,
// then evict to budget.
struct OpArgs {
    dkv_drafter_t m;
    dkv_paged_t full;        // used when src_full
    dkv_qcfg_t cfgs[64];     // per layer arm (layer index < 64)
    const void* k;           // [batch][T][Hkv][D] when !src_full
    const void* v;
    int in_dtype, T, src_full, do_trunc, layer0;   // layer0: first layer (grid.y offset)
    const int32_t* start;    // first appended position per seq (also truncate point)
    const int32_t* count;    // rows appended per seq (NULL = T) when !src_full
    const int32_t* end;      // end position per seq when src_full
    const int32_t* budget;   // [layer*batch + s] or [s] when budget_per_layer == 0
    int budget_per_layer;
};

__global__ void __launch_bounds__(BLK) drafter_op_kernel(OpArgs a) {
    const int s = blockIdx.x, L = a.layer0 + blockIdx.y;
    const dkv_drafter_t& m = a.m;
    const dkv_qcfg_t cfg = a.cfgs[L];
    const int D = m.head_dim, H = m.n_kv_heads;
    __shared__ int red[NWAVES];
    __shared__ double redd[NWAVES];
    __shared__ int holes[MAXMOVE], movers[MAXMOVE];
    __shared__ unsigned bits_lo[WIN / 32], bits_hi[WIN / 32];

    RowCtx c{&a.m, s, L, code_row_bytes(cfg.bits, D), meta_row_bytes(cfg.bits, D, cfg.group, cfg.meta_f16),
             m.pos + row_index(m, s, L), m.score + row_index(m, s, L)};
    int32_t* nrows_p = m.n_rows + (int64_t)s * m.n_layers + L;
    int n = *nrows_p;
    const int32_t p0 = a.start[s];
    if (a.do_trunc) {
        __syncthreads();
        n = compact(c, n, p0, red, holes, movers);
    }
    int cnt = a.src_full ? (a.end[s] - p0) : (a.count ? a.count[s] : a.T);
    if (cnt < 0) cnt = 0;
    if (n + cnt > m.cap) cnt = max(0, m.cap - n);   // host sizes cap; never write past it
    // append: one wave per (row, head)
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    for (int item = w; item < cnt * H; item += NWAVES) {
        const int t = item / H, h = item % H;
        const int slot = n + t;
        Seg sg = seg_of(m, s, L, h);
        uint8_t* kr = sg.kc + (int64_t)slot * c.crow_bytes;
        uint8_t* vr = sg.vc + (int64_t)slot * c.crow_bytes;
        uint8_t* kmr = sg.km + (int64_t)slot * c.mrow_bytes;
        uint8_t* vmr = sg.vm + (int64_t)slot * c.mrow_bytes;
        if (a.src_full) {
            const dkv_paged_t& f = a.full;
            const int pos = p0 + t;
            const int32_t blk = paged_block(f, s, L, pos);
            const int off = pos % f.block_size;
            quant_head_row([&](int j) { return load_elem(f.pool, paged_k_off(f, blk, off, h, j), f.dtype); }, D, cfg,
                           kr, kmr, lane);
            quant_head_row([&](int j) { return load_elem(f.pool, paged_v_off(f, blk, off, h, j), f.dtype); }, D, cfg,
                           vr, vmr, lane);
        } else {
            const int64_t src = (((int64_t)s * a.T + t) * H + h) * D;
            quant_head_row([&](int j) { return load_elem(a.k, src + j, a.in_dtype); }, D, cfg, kr, kmr, lane);
            quant_head_row([&](int j) { return load_elem(a.v, src + j, a.in_dtype); }, D, cfg, vr, vmr, lane);
        }
        if (lane == 0 && h == 0) {
            c.pos[slot] = p0 + t;
            c.score[slot] = 0.0;
        }
    }
    __syncthreads();
    n += cnt;
    if (cnt > 0) {
        const int budget = a.budget[a.budget_per_layer ? (L * m.batch + s) : s];
        n = evict(c, n, budget, cfg, p0 + cnt - 1, red, holes, movers, bits_lo, bits_hi, redd);
    }
    __syncthreads();
    if (threadIdx.x == 0) *nrows_p = n;
}

// ------------------------------------------------------------ rebuild (c)
// grid: x = row tile, y = sequence, z = index into the changed-layer list.
struct RebuildArgs {
    dkv_drafter_t m;
    dkv_paged_t full;
    dkv_qcfg_t cfgs[64];
    int32_t layers[64];
    const int32_t* len;
    const int32_t* budget;
};

constexpr int RB_ROWS = 16;

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
    const int64_t crb = code_row_bytes(cfg.bits, D), mrb = meta_row_bytes(cfg.bits, D, cfg.group, cfg.meta_f16);
    int32_t* pos = m.pos + row_index(m, s, L);
    double* score = m.score + row_index(m, s, L);
    const int r0 = blockIdx.x * RB_ROWS;
    if (blockIdx.x == 0 && threadIdx.x == 0) m.n_rows[(int64_t)s * m.n_layers + L] = kept;
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    for (int item = w; item < RB_ROWS * H; item += NWAVES) {
        const int r = r0 + item / H, h = item % H;
        if (r >= kept) continue;
        const int p = r < sink ? r : n - (kept - sink) + (r - sink);
        const int32_t blk = paged_block(f, s, L, p);
        const int off = p % f.block_size;
        Seg sg = seg_of(m, s, L, h);
        quant_head_row([&](int j) { return load_elem(f.pool, paged_k_off(f, blk, off, h, j), f.dtype); }, D, cfg,
                       sg.kc + (int64_t)r * crb, sg.km + (int64_t)r * mrb, lane);
        quant_head_row([&](int j) { return load_elem(f.pool, paged_v_off(f, blk, off, h, j), f.dtype); }, D, cfg,
                       sg.vc + (int64_t)r * crb, sg.vm + (int64_t)r * mrb, lane);
        if (lane == 0 && h == 0) {
            pos[r] = p;
            score[r] = 0.0;
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
    const int64_t crb = code_row_bytes(cfg.bits, D), mrb = meta_row_bytes(cfg.bits, D, cfg.group, cfg.meta_f16);
    const int ng = cfg.bits >= 16 ? 0 : n_groups(D, cfg.group);
    if (threadIdx.x == 0 && pos_out) pos_out[r] = m.pos[row_index(m, s, L) + r];
    for (int i = threadIdx.x; i < 2 * H * D; i += blockDim.x) {
        const int kvsel = i / (H * D), h = (i / D) % H, j = i % D;
        Seg sg = seg_of(m, s, L, h);
        const uint8_t* crow = (kvsel ? sg.vc : sg.kc) + (int64_t)r * crb;
        const uint8_t* mrow = (kvsel ? sg.vm : sg.km) + (int64_t)r * mrb;
        const GatherOut& o = kvsel ? vo : ko;
        const int64_t oi = ((int64_t)r * H + h) * D + j;
        if (cfg.bits >= 16) {
            const float val = reinterpret_cast<const float*>(crow)[j];
            if (o.codes) o.codes[oi] = 0;
            if (o.deq) o.deq[oi] = val;
            continue;
        }
        const int g = j / cfg.group;
        const GroupMeta mt = get_meta(mrow, g, cfg.meta_f16);
        const int code = get_code(crow, j, cfg.bits);
        if (o.codes) o.codes[oi] = static_cast<uint8_t>(code);
        if (o.deq) o.deq[oi] = dequant(code, mt);
        if (j % cfg.group == 0) {
            const int64_t gi = ((int64_t)r * H + h) * ng + g;
            if (o.scale) o.scale[gi] = mt.scale;
            if (o.lo) o.lo[gi] = mt.lo;
        }
    }
}

// ------------------------------------------------------------ host checks
int check_mirror(const dkv_drafter_t* m, const char* fn) {
    DKV_REQUIRE(m != nullptr, std::string(fn) + ": mirror is NULL");
    DKV_REQUIRE(m->kc && m->vc && m->km && m->vm && m->pos && m->score && m->n_rows,
                std::string(fn) + ": mirror has a NULL buffer");
    DKV_REQUIRE(m->batch > 0 && m->n_layers > 0 && m->n_layers <= 64 && m->n_kv_heads > 0 && m->cap > 0,
                std::string(fn) + ": bad mirror shape (n_layers must be 1..64)");
    DKV_REQUIRE(m->head_dim > 0 && m->head_dim % 8 == 0, std::string(fn) + ": head_dim must be a multiple of 8");
    return DKV_OK;
}

int check_cfg(const dkv_drafter_t* m, const dkv_qcfg_t& c, const char* fn) {
    DKV_REQUIRE(c.bits == 2 || c.bits == 3 || c.bits == 4 || c.bits == 8 || c.bits == 16,
                std::string(fn) + ": bits must be 2, 3, 4, 8 or 16");
    DKV_REQUIRE(c.bits >= 16 || (c.group > 0 && (c.group % 2 == 0 || c.group >= m->head_dim)),
                std::string(fn) + ": group must be even");
    DKV_REQUIRE(c.sink >= 0 && c.recent >= 0, std::string(fn) + ": sink/recent must be >= 0");
    DKV_REQUIRE(code_row_bytes(c.bits, m->head_dim) <= m->code_stride,
                std::string(fn) + ": arm needs more code bytes per row than the mirror reserves");
    DKV_REQUIRE(meta_row_bytes(c.bits, m->head_dim, c.group, c.meta_f16) <= m->meta_stride,
                std::string(fn) + ": arm needs more meta bytes per row than the mirror reserves");
    return DKV_OK;
}

}  // namespace dkv

using namespace dkv;

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
    a.src_full = 0;
    a.do_trunc = 0;
    a.layer0 = layer;
    a.start = start;
    a.count = count;
    a.budget = budget;
    a.budget_per_layer = 0;
    hipLaunchKernelGGL(drafter_op_kernel, dim3(mirror->batch, 1), dim3(BLK), 0, as_stream(stream), a);
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
    a.src_full = 0;
    a.do_trunc = 1;
    a.T = 0;              // nothing appended, so no eviction and budget is never read
    a.start = start;
    a.budget = start;
    a.layer0 = 0;
    hipLaunchKernelGGL(drafter_op_kernel, dim3(mirror->batch, mirror->n_layers), dim3(BLK), 0, as_stream(stream), a);
    return check_launch("dkv_drafter_truncate");
}

extern "C" int dkv_drafter_sync(const dkv_drafter_t* mirror, const dkv_paged_t* full, const dkv_qcfg_t* cfgs,
                                const int32_t* start, const int32_t* end, const int32_t* budget,
                                dkv_stream_t stream) {
    int rc = check_mirror(mirror, "dkv_drafter_sync");
    if (rc) return rc;
    DKV_REQUIRE(full && cfgs && start && end && budget, "dkv_drafter_sync: NULL argument");
    DKV_REQUIRE(full->n_layers == mirror->n_layers && full->n_kv_heads == mirror->n_kv_heads &&
                    full->head_dim == mirror->head_dim && full->batch == mirror->batch,
                "dkv_drafter_sync: full cache and mirror shapes differ");
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
    a.layer0 = 0;
    hipLaunchKernelGGL(drafter_op_kernel, dim3(mirror->batch, mirror->n_layers), dim3(BLK), 0, as_stream(stream), a);
    return check_launch("dkv_drafter_sync");
}

extern "C" int dkv_drafter_rebuild(const dkv_drafter_t* mirror, const dkv_paged_t* full, const int32_t* layers,
                                   int32_t n_changed, const dkv_qcfg_t* cfgs, const int32_t* len,
                                   const int32_t* budget, dkv_stream_t stream) {
    int rc = check_mirror(mirror, "dkv_drafter_rebuild");
    if (rc) return rc;
    DKV_REQUIRE(full && layers && cfgs && len && budget, "dkv_drafter_rebuild: NULL argument");
    DKV_REQUIRE(full->n_layers == mirror->n_layers && full->n_kv_heads == mirror->n_kv_heads &&
                    full->head_dim == mirror->head_dim && full->batch == mirror->batch,
                "dkv_drafter_rebuild: full cache and mirror shapes differ");
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
    const int tiles = (mirror->cap + RB_ROWS - 1) / RB_ROWS;
    hipLaunchKernelGGL(drafter_rebuild_kernel, dim3(tiles, mirror->batch, n_changed), dim3(BLK), 0,
                       as_stream(stream), a);
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
