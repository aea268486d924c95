// Page format of the drafter mirror.
//
// A (sequence, layer, kv head) segment is a run of pages of 32 rows. A page
// holds, for its 32 rows:
//
//   K codes  32 rows x D codes, row-major (row i at i * D*cb/8 bytes). Inside
//            each 32-bit word the codes are interleaved so that one and/or
//            with a magic constant turns two codes into a packed f16 pair:
//              cb = 4: word holds 8 consecutive codes e0..e7 as nibbles
//                      e0 e2 e4 e6 | e1 e3 e5 e7   (bits 0..15 | 16..31)
//              cb = 8: word holds 4 consecutive codes as bytes e0 e2 e1 e3
//   K meta   [group][row] (scale, lo) pairs
//   V codes  transposed for the PV product: for d = 16*t + a and row
//            i -> (j, e) = ((i%16)/4, (i<16 ? 0 : 4) + i%4), the codes of the 8
//            rows (j, 0..7) of one d share a word (cb = 4) or two words
//            (cb = 8), in the same interleaved order; word index
//            ((a*4 + j) * NDT + t) [* 2 for cb = 8], NDT = ceil(D/16)
//   V meta   [group][j][e] (scale, lo) pairs
//
// cb (stored code bits) = 4 for bits <= 4, 8 for bits == 8, 32 for bits == 16
// (raw float32 values, K and V row-major, no meta). Meta pairs are float32
// or float16. The layout needs D % 16 == 0 or D == 8.
//
// 8-bit codes with D % 64 == 0 keep those words in the order the attention
// kernel's lanes load them, so that each 16-byte load instruction of a wave
// reads 1 KB of contiguous bytes (whole 64-byte segments, which lets the
// loads bypass the caches). In 16-row tile T of K, lane (c, g) = lane
// c + 16 g holds the D/16 words g D/16 .. (g + 1) D/16 - 1 of row 16 T + c,
// in pieces of 4 words, piece x at word 256 x + 4 lane of the tile (a tile
// is 4 D words). In V, lane L = 4 a + j holds the 2 NDT words of channel
// column a and row group j (word 2 t + half for d = 16 t + a), piece x at
// word 256 x + 4 L. The words are the ones above, at other places.
#pragma once

#include "dkv_common.h"

namespace dkv {

constexpr int PAGE = 32;

struct PageFmt {
    int cb, D, NG, group, meta_f16, metaB, NDT;
    int64_t kc, km, vc, vm, bytes;   // section offsets and page size in bytes
};

__host__ __device__ inline PageFmt page_fmt(int bits, int D, int group, int meta_f16) {
    PageFmt f;
    f.cb = bits >= 16 ? 32 : (bits == 8 ? 8 : 4);
    f.D = D;
    f.NG = bits >= 16 ? 0 : (D + group - 1) / group;
    f.group = group;
    f.meta_f16 = meta_f16;
    f.metaB = meta_f16 ? 4 : 8;
    f.NDT = (D + 15) / 16;
    const int64_t code = (int64_t)PAGE * D * f.cb / 8;
    const int64_t meta = (int64_t)PAGE * f.NG * f.metaB;
    f.kc = 0;
    f.km = code;
    f.vc = code + meta;
    f.vm = 2 * code + meta;
    f.bytes = 2 * (code + meta);
    return f;
}

__host__ __device__ inline PageFmt page_fmt(const dkv_qcfg_t& c, int D) {
    return page_fmt(c.bits, D, c.group, c.meta_f16);
}

// bit position of code e (0..7 for cb 4, 0..3 for cb 8) inside its word
__host__ __device__ inline int code_shift(int cb, int e) {
    if (cb == 4) return (e & 1) ? 16 + 4 * (e >> 1) : 4 * (e >> 1);
    return 8 * ((e & 1) * 2 + (e >> 1));
}

// 8-bit codes stored in lane load order (see the top of the file)
__host__ __device__ inline bool lane_order8(const PageFmt& f) { return f.cb == 8 && f.D % 64 == 0; }

// index in the K section of word w (0 .. D*cb/32 - 1) of row i
__host__ __device__ inline int64_t k_word(const PageFmt& f, int i, int w) {
    if (lane_order8(f)) {
        const int wpl = f.D / 16;           // words per lane group
        const int g = w / wpl, u = w % wpl;
        return (int64_t)(i / 16) * (4 * f.D) + (u / 4) * 256 + (i % 16 + 16 * g) * 4 + u % 4;
    }
    return (int64_t)i * (f.D * f.cb / 32) + w;
}

// (word index, shift) of K code (row i, channel d) relative to the K section
__host__ __device__ inline void k_code_loc(const PageFmt& f, int i, int d, int64_t* word, int* shift) {
    const int per = 32 / f.cb;                          // codes per word
    *word = k_word(f, i, d / per);
    *shift = code_shift(f.cb, d % per);
}

// index in the V section of 8-bit code word `half` of the (a*4 + j, t) group
// (channel d = 16 t + a, rows of group j; half 0: k-slots 0..3, 1: 4..7)
__host__ __device__ inline int64_t v8_word(const PageFmt& f, int aj, int t, int half) {
    if (lane_order8(f)) {
        const int u = 2 * t + half;         // the word's place in the lane's run
        return (int64_t)(u / 4) * 256 + aj * 4 + u % 4;
    }
    return ((int64_t)aj * f.NDT + t) * 2 + half;
}

// row i -> (lane group j, k-slot e) of the PV product
__host__ __device__ inline void v_slot(int i, int* j, int* e) {
    *j = (i % 16) / 4;
    *e = (i < 16 ? 0 : 4) + (i % 4);
}

__host__ __device__ inline void v_code_loc(const PageFmt& f, int i, int d, int64_t* word, int* shift) {
    int j, e;
    v_slot(i, &j, &e);
    const int a = d % 16, t = d / 16;
    if (f.cb == 4) {
        *word = ((int64_t)a * 4 + j) * f.NDT + t;
        *shift = code_shift(4, e);
    } else {
        *word = v8_word(f, a * 4 + j, t, e / 4);
        *shift = code_shift(8, e % 4);
    }
}

__host__ __device__ inline int64_t k_meta_off(const PageFmt& f, int i, int g) {
    return f.km + ((int64_t)g * PAGE + i) * f.metaB;
}
__host__ __device__ inline int64_t v_meta_off(const PageFmt& f, int i, int g) {
    int j, e;
    v_slot(i, &j, &e);
    return f.vm + ((int64_t)g * PAGE + j * 8 + e) * f.metaB;
}

// page p of segment (s, L, h). A layer's pages form one range in which the
// segments' pages are interleaved in chunks of PAGE_CHUNK: chunk c of every
// segment (segments in (seq, head) order), then chunk c + 1, ...; the last
// npg % PAGE_CHUNK pages of each segment follow the whole chunks. A drafter
// call's waves, walking their pages in step, then read from one moving
// window of the layer (Llama-3-8B mirror at b=32, int4 keep 0.25, 32
// layers: segment kernel 60.3 -> 56.9 us; the int8 drafter unchanged).
constexpr int PAGE_CHUNK = 8;
__host__ __device__ inline uint8_t* page_ptr(const dkv_drafter_t& m, int s, int L, int h, int p) {
    const int64_t nseg = (int64_t)m.batch * m.n_kv_heads, npg = m.cap / PAGE;
    const int64_t nf = npg / PAGE_CHUNK, rem = npg - nf * PAGE_CHUNK;
    const int64_t seg = (int64_t)s * m.n_kv_heads + h, base = (int64_t)L * npg * nseg;
    const int64_t slot = p < nf * PAGE_CHUNK
                             ? base + ((int64_t)(p / PAGE_CHUNK) * nseg + seg) * PAGE_CHUNK + p % PAGE_CHUNK
                             : base + nf * PAGE_CHUNK * nseg + seg * rem + (p - nf * PAGE_CHUNK);
    return static_cast<uint8_t*>(m.pages) + slot * m.page_stride;
}

// ---------------------------------------------------------------- device access
__device__ __forceinline__ GroupMeta read_meta(const uint8_t* p, int meta_f16) {
    if (meta_f16) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
        return {half_bits_to_f32(w & 0xffffu), half_bits_to_f32(w >> 16)};
    }
    const float2 v = *reinterpret_cast<const float2*>(p);
    return {v.x, v.y};
}
__device__ __forceinline__ void write_meta(uint8_t* p, GroupMeta m, int meta_f16) {
    if (meta_f16) {
        *reinterpret_cast<uint32_t*>(p) =
            (uint32_t)f32_to_half_bits_rne(m.scale) | ((uint32_t)f32_to_half_bits_rne(m.lo) << 16);
    } else {
        *reinterpret_cast<float2*>(p) = make_float2(m.scale, m.lo);
    }
}

__device__ __forceinline__ int read_code(const uint8_t* sec, int64_t word, int shift, int cb) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(sec)[word];
    return (w >> shift) & (cb == 4 ? 0xfu : 0xffu);
}

// Store one code. Words of 4-bit codes are shared with other rows (V) or other
// lanes (K), so the nibble is replaced with two atomics on disjoint bits; an
// 8-bit code is a plain byte store.
__device__ __forceinline__ void write_code(uint8_t* sec, int64_t word, int shift, int cb, int code) {
    if (cb == 8) {
        sec[word * 4 + shift / 8] = static_cast<uint8_t>(code);
        return;
    }
    unsigned* w = reinterpret_cast<unsigned*>(sec) + word;
    atomicAnd(w, ~(0xfu << shift));
    atomicOr(w, static_cast<unsigned>(code & 0xf) << shift);
}

}  // namespace dkv
