// Shared device/host helpers for the DRAFTKV gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <string>

#include "../../include/draftkv_hip.h"

namespace dkv {

// ------------------------------------------------------------ error state
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// Reserve `lds` bytes of dynamic LDS for kernel `fn` (needed above 64 KB).
// The attribute persists, so it is set once per kernel and device, at the
// largest size asked for so far: setting it on every launch can stall the
// host behind the work already queued. `done` is the caller's per-kernel
// record (one slot per device).
inline bool reserve_lds(const void* fn, size_t lds, size_t (&done)[16]) {
    if (lds <= 64 * 1024) return true;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) dev = 0;
    if (done[dev] >= lds) return true;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return false;
    done[dev] = lds;
    return true;
}

#define DKV_REQUIRE(cond, msg)                                   \
    do {                                                         \
        if (!(cond)) return ::dkv::fail(DKV_EINVAL, (msg));      \
    } while (0)

inline hipStream_t as_stream(dkv_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------ numerics
constexpr int WAVE = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);  // NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float half_bits_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t f32_to_half_bits_rne(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

// load element i of a row stored as f32 or bf16
__device__ __forceinline__ float load_elem(const void* base, int64_t i, int dtype) {
    return dtype == DKV_BF16 ? bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[i])
                             : reinterpret_cast<const float*>(base)[i];
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// ------------------------------------------------------------ quantizer
// Bit-exact restatement of the reference's float32 op order
// (draftkv/compress.py:38-43): lo/hi = group min/max (zero padding of a short
// last group takes part), scale = max((hi-lo)/levels, 1e-8), q = rint((x-lo)/
// scale) clipped to [0, levels], deq = q*scale + lo with two roundings.
// With fp16 meta the stored (rounded) lo/scale are used for the codes.
struct GroupMeta {
    float scale, lo;
};

__device__ __forceinline__ GroupMeta group_meta(float lo, float hi, int bits, int meta_f16) {
#pragma clang fp contract(off)
    const float levels = static_cast<float>((1 << bits) - 1);
    float scale = fmaxf(__fdiv_rn(__fsub_rn(hi, lo), levels), 1e-8f);
    if (meta_f16) {
        lo = half_bits_to_f32(f32_to_half_bits_rne(lo));
        scale = half_bits_to_f32(f32_to_half_bits_rne(scale));
        if (scale == 0.0f) scale = 5.9604644775390625e-08f;  // 2^-24, smallest half
    }
    return {scale, lo};
}

__device__ __forceinline__ int quant_code(float x, GroupMeta m, int bits) {
#pragma clang fp contract(off)
    const float levels = static_cast<float>((1 << bits) - 1);
    float q = rintf(__fdiv_rn(__fsub_rn(x, m.lo), m.scale));
    q = fminf(fmaxf(q, 0.0f), levels);
    return static_cast<int>(q);
}

// quant_code of 8 values of one group without a division on the common path.
// With inv = rcp(scale) (hardware reciprocal, within 1 ulp) the product
// q = RN(d * inv) lies within 2^-22 |Q| of the exact quotient Q = d / scale
// (d = RN(x - lo)), and RN(Q) within 2^-24 |Q| of Q. So when |q| <= levels + 1
// and q is farther than (levels + 1) 2^-20 from every half-integer,
// rint(q) == rint(RN(Q)); past levels + 1 (or below -1) the clamp to
// [0, levels] gives the same code whichever way either rounds. The values
// within that distance of a half-integer (rare) take the correctly rounded
// division, behind a wave-uniform branch. Same codes as quant_code for every
// input.
__device__ __forceinline__ void quant_codes8(const float (&v)[8], GroupMeta m, int bits, uint32_t (&code)[8]) {
#pragma clang fp contract(off)
    const float levels = static_cast<float>((1 << bits) - 1);
    const float tie = 0.5f - (levels + 1.0f) * 9.5367431640625e-07f;   // 0.5 - (levels + 1) 2^-20, exact
    const float inv = __builtin_amdgcn_rcpf(m.scale);
    const bool bad = !(inv >= 1.17549435e-38f && inv <= 3.0e38f);   // a reciprocal out of the normal range
    float r[8];
    bool near[8];
    bool any = bad;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float q = __fmul_rn(__fsub_rn(v[e], m.lo), inv);
        r[e] = rintf(q);
        near[e] = bad || fabsf(__fsub_rn(q, r[e])) >= tie;
        any = any || near[e];
    }
    if (__any(any)) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (near[e]) r[e] = rintf(__fdiv_rn(__fsub_rn(v[e], m.lo), m.scale));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) code[e] = static_cast<uint32_t>(__builtin_amdgcn_fmed3f(r[e], 0.0f, levels));
}

__device__ __forceinline__ float dequant(int code, GroupMeta m) {
    // the empty asm hides the product from the optimizer so it cannot be
    // contracted into an FMA: the reference rounds the product, then the sum
    float prod = __fmul_rn(static_cast<float>(code), m.scale);
    asm volatile("" : "+v"(prod));
    return __fadd_rn(prod, m.lo);
}

__host__ __device__ inline int n_groups(int d, int group) { return (d + group - 1) / group; }

// ------------------------------------------------------------ mirror addressing

__host__ __device__ inline int64_t row_index(const dkv_drafter_t& m, int s, int L) {
    return (int64_t)(s * m.n_layers + L) * m.cap;
}

// ------------------------------------------------------------ paged addressing
__host__ __device__ inline int64_t paged_esize(const dkv_paged_t& c) { return c.dtype == DKV_BF16 ? 2 : 4; }
__host__ __device__ inline int64_t paged_block_elems(const dkv_paged_t& c) {
    return 2LL * c.n_kv_heads * c.block_size * c.head_dim;
}

// element offsets (in elements) of K[pos][h][d] and V[pos][h][d] for (s, L)
__device__ __forceinline__ int32_t paged_block(const dkv_paged_t& c, int s, int L, int pos) {
    return c.block_table[((int64_t)s * c.n_layers + L) * c.max_blocks + pos / c.block_size];
}
__device__ __forceinline__ int64_t paged_k_off(const dkv_paged_t& c, int32_t blk, int off, int h, int d) {
    return (int64_t)blk * paged_block_elems(c) + ((int64_t)h * c.block_size + off) * c.head_dim + d;
}
__device__ __forceinline__ int64_t paged_v_off(const dkv_paged_t& c, int32_t blk, int off, int h, int d) {
    return (int64_t)blk * paged_block_elems(c) + (int64_t)c.n_kv_heads * c.block_size * c.head_dim +
           ((int64_t)h * c.head_dim + d) * c.block_size + off;
}

}  // namespace dkv
