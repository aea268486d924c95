// Group quantizer on contiguous rows -- reference draftkv/compress.py:21-46.
#include "dkv_common.h"

namespace dkv {

// One wave per row; the wave walks the row's groups. Lane l of a group covers
// elements l, l+64, ... of it; elements past d are the zero padding the
// reference appends (compress.py:32-35), which joins the last group's min/max.
__global__ void __launch_bounds__(256) quantize_rows_kernel(const float* __restrict__ x, int64_t rows, int d,
                                                            int bits, int group, int meta_f16,
                                                            uint8_t* codes, float* scale, float* lo,
                                                            float* deq) {
    const int lane = threadIdx.x % WAVE;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (row >= rows) return;
    const float* xr = x + row * d;
    const int ng = n_groups(d, group);
    for (int g = 0; g < ng; ++g) {
        float mn = INFINITY, mx = -INFINITY;
        for (int e = lane; e < group; e += WAVE) {
            const int j = g * group + e;
            const float v = j < d ? xr[j] : 0.0f;
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        mn = wave_min(mn);
        mx = wave_max(mx);
        const GroupMeta m = group_meta(mn, mx, bits, meta_f16);
        if (lane == 0) {
            if (scale) scale[row * ng + g] = m.scale;
            if (lo) lo[row * ng + g] = m.lo;
        }
        for (int e = lane; e < group; e += WAVE) {
            const int j = g * group + e;
            if (j >= d) break;
            const int c = quant_code(xr[j], m, bits);
            if (codes) codes[row * d + j] = static_cast<uint8_t>(c);
            if (deq) deq[row * d + j] = dequant(c, m);
        }
    }
}

}  // namespace dkv

extern "C" int dkv_quantize(const float* x, int64_t rows, int32_t d, int32_t bits, int32_t group,
                            int32_t meta_f16, uint8_t* codes, float* scale, float* lo, float* deq,
                            dkv_stream_t stream) {
    DKV_REQUIRE(x != nullptr, "dkv_quantize: x is NULL");
    DKV_REQUIRE(rows >= 0 && d > 0, "dkv_quantize: rows must be >= 0 and d > 0");
    DKV_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, "dkv_quantize: bits must be 2, 3, 4 or 8");
    DKV_REQUIRE(group > 0, "dkv_quantize: group must be > 0");
    if (rows == 0) return DKV_OK;
    const int waves = 4;
    const int64_t blocks = (rows + waves - 1) / waves;
    DKV_REQUIRE(blocks < (1LL << 31), "dkv_quantize: too many rows");
    hipLaunchKernelGGL(dkv::quantize_rows_kernel, dim3((unsigned)blocks), dim3(64 * waves), 0,
                       dkv::as_stream(stream), x, rows, d, bits, group, meta_f16, codes, scale, lo, deq);
    return dkv::check_launch("dkv_quantize");
}
