// Elementwise and normalisation kernels of the three model forwards, plus a
// batch-invariant float32 GEMM.
// Reference: draftkv/model.py:18-25,100-133 (RMSNorm, sinusoidal positions,
// ReLU MLP), draftkv/gpt2.py:114-127,182-213 (LayerNorm, GELU-tanh, learned
// positions), draftkv/llama.py:93-109,164-172,175-225 (RMSNorm, RoPE, SiLU).
//
// Activations are float32 rows; inputs that come out of a bf16 GEMM may be
// bf16, and outputs that feed a bf16 GEMM may be written as bf16 (RNE).
#include "dkv_common.h"

namespace dkv {

__device__ __forceinline__ void store_elem(void* base, int64_t i, float v, int dtype) {
    if (dtype == DKV_BF16)
        reinterpret_cast<uint16_t*>(base)[i] = f32_to_bf16_rne(v);
    else
        reinterpret_cast<float*>(base)[i] = v;
}

__device__ __forceinline__ float bias_at(const void* bias, int64_t i, int dtype) {
    return bias ? load_elem(bias, i, dtype) : 0.0f;
}

// An input row read either as stored (f32 or bf16 elements) or as the bf16
// GEMM's per-chunk float32 partials [np][rows][n] left for its consumer:
// then element i is their sum in chunk order rounded to bf16 to nearest even,
// the value the GEMM's reduce kernel would have stored.
struct XSrc {
    const void* x;
    int dt;
    const float* part;
    int np;
    int64_t ps;   // elements per partial (rows * n)
};
__device__ __forceinline__ float x_at(const XSrc& s, int64_t i) {
    if (s.np <= 0) return load_elem(s.x, i, s.dt);
    float t = s.part[i];
    for (int c = 1; c < s.np; ++c) t = t + s.part[(int64_t)c * s.ps + i];
    return (float)(__bf16)t;
}

// Sum over the block (up to 1024 threads = 16 waves); every thread gets the total.
__device__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, nw = blockDim.x / WAVE;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// h[r] = table[tok[r]] (+ pos_table[pos[r]]); grid (column tiles, rows)
__global__ void __launch_bounds__(256) embed_kernel(const void* __restrict__ table, int tdt,
                                                    const int32_t* __restrict__ tokens, int d,
                                                    const void* __restrict__ pos_table,
                                                    const int32_t* __restrict__ positions, float* __restrict__ out) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d) return;
    float v = load_elem(table, (int64_t)tokens[r] * d + i, tdt);
    if (pos_table) v += load_elem(pos_table, (int64_t)positions[r] * d + i, tdt);
    out[(int64_t)r * d + i] = v;
}

// One block per row, the row held in registers (NORM_EPT elements per
// thread): optionally h += x (+ bias) first, written back to h, then
//   RMSNorm:   out = h / sqrt(mean(h*h) + eps) * w
//   LayerNorm: out = (h - mean) / sqrt(mean((h-mean)^2) + eps) * w + b
constexpr int NORM_EPT = 8;
template <bool LN>
__global__ void __launch_bounds__(1024) norm_kernel(float* __restrict__ h, XSrc x,
                                                    const void* __restrict__ xb, int xbdt, const void* __restrict__ w,
                                                    const void* __restrict__ b, int wdt, int d, float eps, void* out,
                                                    int odt) {
    __shared__ float red[16];
    const int r = blockIdx.x;
    float* hr = h + (int64_t)r * d;
    float v[NORM_EPT];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NORM_EPT; ++j) {
        const int i = threadIdx.x + j * blockDim.x;
        float t = 0.0f;
        if (i < d) {
            t = hr[i];
            if (x.x || x.np > 0) {
                t += x_at(x, (int64_t)r * d + i) + bias_at(xb, i, xbdt);
                hr[i] = t;
            }
        }
        v[j] = t;
        s += LN ? t : t * t;
    }
    s = block_sum(s, red);
    float mu = 0.0f, inv;
    if (LN) {
        mu = s / d;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < NORM_EPT; ++j) {
            const int i = threadIdx.x + j * blockDim.x;
            if (i < d) q += (v[j] - mu) * (v[j] - mu);
        }
        inv = 1.0f / sqrtf(block_sum(q, red) / d + eps);
    } else {
        inv = 1.0f / sqrtf(s / d + eps);
    }
#pragma unroll
    for (int j = 0; j < NORM_EPT; ++j) {
        const int i = threadIdx.x + j * blockDim.x;
        if (i < d) {
            const float o = LN ? (v[j] - mu) * inv * load_elem(w, i, wdt) + load_elem(b, i, wdt)
                               : v[j] * inv * load_elem(w, i, wdt);
            store_elem(out, (int64_t)r * d + i, o, odt);
        }
    }
}

// The same row norm for d % 4 == 0, four consecutive elements per thread
// with 16-byte (f32) or 8-byte (bf16) accesses: fewer, wider loads per row,
// which matters when x is read as the GEMM's partials (np loads per element).
__device__ __forceinline__ float4 load4(const void* base, int64_t i, int dtype) {
    if (dtype == DKV_BF16) {
        const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + i);
        return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                           __uint_as_float(u.y & 0xffff0000u));
    }
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + i);
}
__device__ __forceinline__ float4 x_at4(const XSrc& s, int64_t i) {
    if (s.np <= 0) return load4(s.x, i, s.dt);
    float4 t = *reinterpret_cast<const float4*>(s.part + i);
    for (int c = 1; c < s.np; ++c) {
        const float4 u = *reinterpret_cast<const float4*>(s.part + (int64_t)c * s.ps + i);
        t.x = t.x + u.x;
        t.y = t.y + u.y;
        t.z = t.z + u.z;
        t.w = t.w + u.w;
    }
    return make_float4((float)(__bf16)t.x, (float)(__bf16)t.y, (float)(__bf16)t.z, (float)(__bf16)t.w);
}
__device__ __forceinline__ void store4(void* base, int64_t i, float4 v, int dtype) {
    if (dtype == DKV_BF16) {
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(base) + i) =
            make_uint2((uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16),
                       (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16));
    } else {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + i) = v;
    }
}
constexpr int NORM_EPT4 = 2;   // float4 groups per thread: d up to 8 * 1024
template <bool LN>
__global__ void __launch_bounds__(1024) norm4_kernel(float* __restrict__ h, XSrc x, const void* __restrict__ xb,
                                                     int xbdt, const void* __restrict__ w, const void* __restrict__ b,
                                                     int wdt, int d, float eps, void* out, int odt) {
    __shared__ float red[16];
    const int r = blockIdx.x;
    float* hr = h + (int64_t)r * d;
    const bool has_x = x.x || x.np > 0;
    float4 v[NORM_EPT4];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NORM_EPT4; ++j) {
        const int i = 4 * (threadIdx.x + j * blockDim.x);
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < d) {
            t = *reinterpret_cast<const float4*>(hr + i);
            if (has_x) {
                const float4 a = x_at4(x, (int64_t)r * d + i);
                const float4 bb = xb ? load4(xb, i, xbdt) : make_float4(0.f, 0.f, 0.f, 0.f);
                t.x += a.x + bb.x;
                t.y += a.y + bb.y;
                t.z += a.z + bb.z;
                t.w += a.w + bb.w;
                *reinterpret_cast<float4*>(hr + i) = t;
            }
        }
        v[j] = t;
        s += LN ? ((t.x + t.y) + t.z) + t.w : ((t.x * t.x + t.y * t.y) + t.z * t.z) + t.w * t.w;
    }
    s = block_sum(s, red);
    float mu = 0.0f, inv;
    if (LN) {
        mu = s / d;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < NORM_EPT4; ++j) {
            const int i = 4 * (threadIdx.x + j * blockDim.x);
            if (i < d) {
                const float4 t = v[j];
                q += (((t.x - mu) * (t.x - mu) + (t.y - mu) * (t.y - mu)) + (t.z - mu) * (t.z - mu)) +
                     (t.w - mu) * (t.w - mu);
            }
        }
        inv = 1.0f / sqrtf(block_sum(q, red) / d + eps);
    } else {
        inv = 1.0f / sqrtf(s / d + eps);
    }
#pragma unroll
    for (int j = 0; j < NORM_EPT4; ++j) {
        const int i = 4 * (threadIdx.x + j * blockDim.x);
        if (i < d) {
            const float4 t = v[j], wv = load4(w, i, wdt);
            float4 o;
            if (LN) {
                const float4 bv = load4(b, i, wdt);
                o = make_float4((t.x - mu) * inv * wv.x + bv.x, (t.y - mu) * inv * wv.y + bv.y,
                                (t.z - mu) * inv * wv.z + bv.z, (t.w - mu) * inv * wv.w + bv.w);
            } else {
                o = make_float4(t.x * inv * wv.x, t.y * inv * wv.y, t.z * inv * wv.z, t.w * inv * wv.w);
            }
            store4(out, (int64_t)r * d + i, o, odt);
        }
    }
}

// Split a fused projection row [q heads | k heads | v heads] (+ bias) into
// float32 q [r][hq][d], k [r][hkv][d], v [r][hkv][d], applying rotate-half
// RoPE to q and k when a cos/sin table is given: out[j] = x[j]c[j] - x[j+h]s[j],
// out[j+h] = x[j+h]c[j] + x[j]s[j] with h = d/2. Grid (item tiles, rows):
// with RoPE an item is a q/k rotation pair or a v element, else one element.
__global__ void __launch_bounds__(256) qkv_split_kernel(XSrc qkv,
                                                        const void* __restrict__ bias, int bdt, int hq, int hkv,
                                                        int d, const int32_t* __restrict__ positions,
                                                        const float* __restrict__ cs, int max_pos,
                                                        float* __restrict__ q, float* __restrict__ k,
                                                        float* __restrict__ v) {
    const int r = blockIdx.y;
    const int n = (hq + 2 * hkv) * d;
    const int64_t base = (int64_t)r * n;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (!cs) {
        if (i >= n) return;
        const float x = x_at(qkv, base + i) + bias_at(bias, i, bdt);
        const int head = i / d, c = i % d;
        if (head < hq)
            q[((int64_t)r * hq + head) * d + c] = x;
        else if (head < hq + hkv)
            k[((int64_t)r * hkv + head - hq) * d + c] = x;
        else
            v[((int64_t)r * hkv + head - hq - hkv) * d + c] = x;
        return;
    }
    const int half = d / 2;
    const int pairs = (hq + hkv) * half;
    if (i < pairs) {
        const int head = i / half, j = i % half;
        const int64_t p = positions[r];
        const float cj = cs[p * half + j];
        const float sj = cs[(int64_t)max_pos * half + p * half + j];
        const int c0 = head * d + j, c1 = c0 + half;
        const float a = x_at(qkv, base + c0) + bias_at(bias, c0, bdt);
        const float b = x_at(qkv, base + c1) + bias_at(bias, c1, bdt);
        float* dst = head < hq ? q + ((int64_t)r * hq + head) * d : k + ((int64_t)r * hkv + head - hq) * d;
        dst[j] = a * cj - b * sj;
        dst[j + half] = b * cj + a * sj;
    } else if (i < pairs + hkv * d) {
        const int e = i - pairs;
        const int c = (hq + hkv) * d + e;
        v[(int64_t)r * hkv * d + e] = x_at(qkv, base + c) + bias_at(bias, c, bdt);
    }
}

// Elementwise kernels: grid (column tiles of 256, rows).
// out = silu(gate) * up, gu = [rows][2*ff] (gate, then up)
__global__ void __launch_bounds__(256) silu_mul_kernel(const void* __restrict__ gu, int gdt, int ff, void* out,
                                                       int odt) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= ff) return;
    const float g = load_elem(gu, (int64_t)r * 2 * ff + i, gdt);
    const float u = load_elem(gu, (int64_t)r * 2 * ff + ff + i, gdt);
    store_elem(out, (int64_t)r * ff + i, g / (1.0f + __expf(-g)) * u, odt);
}

// out = gelu_tanh(x + bias)
__global__ void __launch_bounds__(256) bias_gelu_kernel(const void* __restrict__ x, int xdt,
                                                        const void* __restrict__ bias, int bdt, int n, void* out,
                                                        int odt) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = load_elem(x, (int64_t)r * n + i, xdt) + bias_at(bias, i, bdt);
    const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    store_elem(out, (int64_t)r * n + i, 0.5f * v * (1.0f + tanhf(u)), odt);
}

// out = max(x, 0)
__global__ void __launch_bounds__(256) relu_kernel(const void* __restrict__ x, int xdt, int n, void* out, int odt) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    store_elem(out, (int64_t)r * n + i, fmaxf(load_elem(x, (int64_t)r * n + i, xdt), 0.0f), odt);
}

// h += x (+ bias)
__global__ void __launch_bounds__(256) add_kernel(float* h, const void* __restrict__ x, int xdt,
                                                  const void* __restrict__ bias, int bdt, int n) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    h[(int64_t)r * n + i] += load_elem(x, (int64_t)r * n + i, xdt) + bias_at(bias, i, bdt);
}

// out[m][n] (+)= sum_k x[m][k] * w(k, n) (+ bias[n]), one thread per output,
// k in order, so a row's result never depends on how many rows share the
// launch. w_layout 0: w[k][n]; 1: w[n][k].
constexpr int GT = 16;
__global__ void __launch_bounds__(256) gemm_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       int wl, int M, int N, int K, const void* __restrict__ bias,
                                                       int bdt, float* out, int accumulate) {
    __shared__ float sx[GT][GT + 1];
    __shared__ float sw[GT][GT + 1];
    const int tm = threadIdx.x / GT, tn = threadIdx.x % GT;
    const int m = blockIdx.y * GT + tm, n = blockIdx.x * GT + tn;
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += GT) {
        const int kx = k0 + tn;
        sx[tm][tn] = (m < M && kx < K) ? x[(int64_t)m * K + kx] : 0.0f;
        // w tile sw[kk][nn]; for layout 1 consecutive threads walk k so the load is row-contiguous
        if (wl == 0) {
            const int kw = k0 + tm, nw = blockIdx.x * GT + tn;
            sw[tm][tn] = (kw < K && nw < N) ? w[(int64_t)kw * N + nw] : 0.0f;
        } else {
            const int kw = k0 + tn, nw = blockIdx.x * GT + tm;
            sw[tn][tm] = (kw < K && nw < N) ? w[(int64_t)nw * K + kw] : 0.0f;
        }
        __syncthreads();
        const int kmax = min(GT, K - k0);
        for (int kk = 0; kk < kmax; ++kk) acc = fmaf(sx[tm][kk], sw[kk][tn], acc);
        __syncthreads();
    }
    if (m < M && n < N) {
        const float b = bias_at(bias, n, bdt);
        const int64_t o = (int64_t)m * N + n;
        out[o] = accumulate ? out[o] + (acc + b) : acc + b;
    }
}

}  // namespace dkv

using namespace dkv;

// grid (ceil(cols / 256), rows), 256 threads
#define DKV_COLS_LAUNCH(kernel, rows, cols, ...)                                                              \
    do {                                                                                                      \
        if ((rows) <= 0 || (cols) <= 0) return DKV_OK;                                                        \
        DKV_REQUIRE((rows) <= 65535, #kernel ": more than 65535 rows in one launch");                         \
        hipLaunchKernelGGL(kernel, dim3(((cols) + 255) / 256, (rows)), dim3(256), 0, as_stream(stream),       \
                           __VA_ARGS__);                                                                      \
        return check_launch(#kernel);                                                                         \
    } while (0)

static bool dtype_ok(int32_t dt) { return dt == DKV_F32 || dt == DKV_BF16; }

static int norm_launch(bool ln, float* h, XSrc x, const void* xb, int32_t xb_dtype, const void* w, const void* b,
                       int32_t w_dtype, int32_t rows, int32_t d, float eps, void* out, int32_t out_dtype,
                       dkv_stream_t stream, const char* what) {
    DKV_REQUIRE(h && w && out && d > 0 && dtype_ok(w_dtype) && dtype_ok(out_dtype), std::string(what) + ": bad arguments");
    DKV_REQUIRE(x.np > 0 || !x.x || dtype_ok(x.dt), std::string(what) + ": bad residual dtype");
    DKV_REQUIRE(!xb || dtype_ok(xb_dtype), std::string(what) + ": bad bias dtype");
    DKV_REQUIRE(!ln || b, std::string(what) + ": LayerNorm needs a bias");
    DKV_REQUIRE(d <= NORM_EPT * 1024, std::string(what) + ": width above 8192");
    if (rows <= 0) return DKV_OK;
    auto al = [](const void* p, int n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
    const bool vec = d % 4 == 0 && al(h, 16) && al(out, 16) && al(w, 8) && (!b || al(b, 8)) && (!xb || al(xb, 16)) &&
                     (x.np > 0 ? al(x.part, 16) : (!x.x || al(x.x, 16)));
    if (vec) {   // one float4 group per thread where d allows (two above d = 4096)
        const int groups = d / 4;
        const int threads = groups >= 1024 ? 1024 : (groups + WAVE - 1) / WAVE * WAVE;
        if (groups > NORM_EPT4 * threads) return fail(DKV_EINVAL, std::string(what) + ": width too large");
        if (ln)
            hipLaunchKernelGGL(norm4_kernel<true>, dim3(rows), dim3(threads), 0, as_stream(stream), h, x, xb, xb_dtype,
                               w, b, w_dtype, d, eps, out, out_dtype);
        else
            hipLaunchKernelGGL(norm4_kernel<false>, dim3(rows), dim3(threads), 0, as_stream(stream), h, x, xb,
                               xb_dtype, w, b, w_dtype, d, eps, out, out_dtype);
        return check_launch(what);
    }
    const int threads = d > 2048 ? 1024 : d > 512 ? 256 : 64;
    if (d > NORM_EPT * threads) return fail(DKV_EINVAL, std::string(what) + ": width too large");
    if (ln)
        hipLaunchKernelGGL(norm_kernel<true>, dim3(rows), dim3(threads), 0, as_stream(stream), h, x, xb, xb_dtype, w,
                           b, w_dtype, d, eps, out, out_dtype);
    else
        hipLaunchKernelGGL(norm_kernel<false>, dim3(rows), dim3(threads), 0, as_stream(stream), h, x, xb, xb_dtype, w,
                           b, w_dtype, d, eps, out, out_dtype);
    return check_launch(what);
}

static XSrc xsrc(const void* x, int32_t dt) { return XSrc{x, dt, nullptr, 0, 0}; }

extern "C" int dkv_embed(const void* table, int32_t table_dtype, const int32_t* tokens, int32_t rows, int32_t d,
                         const void* pos_table, const int32_t* positions, float* out, dkv_stream_t stream) {
    DKV_REQUIRE(table && tokens && out && d > 0 && dtype_ok(table_dtype), "dkv_embed: bad arguments");
    DKV_REQUIRE(!pos_table || positions, "dkv_embed: positions needed with a position table");
    DKV_COLS_LAUNCH(embed_kernel, rows, d, table, table_dtype, tokens, d, pos_table, positions, out);
}

extern "C" int dkv_rmsnorm(const float* x, const void* w, int32_t w_dtype, int32_t rows, int32_t d, float eps,
                           void* out, int32_t out_dtype, dkv_stream_t stream) {
    return norm_launch(false, const_cast<float*>(x), xsrc(nullptr, 0), nullptr, 0, w, nullptr, w_dtype, rows, d, eps,
                       out, out_dtype, stream, "dkv_rmsnorm");
}

extern "C" int dkv_layernorm(const float* x, const void* w, const void* b, int32_t w_dtype, int32_t rows, int32_t d,
                             float eps, void* out, int32_t out_dtype, dkv_stream_t stream) {
    return norm_launch(true, const_cast<float*>(x), xsrc(nullptr, 0), nullptr, 0, w, b, w_dtype, rows, d, eps, out,
                       out_dtype, stream, "dkv_layernorm");
}

extern "C" int dkv_add_rmsnorm(float* h, const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype,
                               const void* w, int32_t w_dtype, int32_t rows, int32_t d, float eps, void* out,
                               int32_t out_dtype, dkv_stream_t stream) {
    DKV_REQUIRE(x, "dkv_add_rmsnorm: x is required");
    return norm_launch(false, h, xsrc(x, x_dtype), bias, bias_dtype, w, nullptr, w_dtype, rows, d, eps, out,
                       out_dtype, stream, "dkv_add_rmsnorm");
}

extern "C" int dkv_add_layernorm(float* h, const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype,
                                 const void* w, const void* b, int32_t w_dtype, int32_t rows, int32_t d, float eps,
                                 void* out, int32_t out_dtype, dkv_stream_t stream) {
    DKV_REQUIRE(x, "dkv_add_layernorm: x is required");
    return norm_launch(true, h, xsrc(x, x_dtype), bias, bias_dtype, w, b, w_dtype, rows, d, eps, out, out_dtype,
                       stream, "dkv_add_layernorm");
}

extern "C" int dkv_add_norm_partials(float* h, const float* part, int32_t n_part, const void* bias, int32_t bias_dtype,
                                     const void* w, const void* b, int32_t w_dtype, int32_t layer_norm, int32_t rows,
                                     int32_t d, float eps, void* out, int32_t out_dtype, dkv_stream_t stream) {
    DKV_REQUIRE(part && n_part > 0, "dkv_add_norm_partials: partials are required");
    return norm_launch(layer_norm != 0, h, XSrc{nullptr, 0, part, n_part, (int64_t)rows * d}, bias, bias_dtype, w,
                       layer_norm ? b : nullptr, w_dtype, rows, d, eps, out, out_dtype, stream,
                       "dkv_add_norm_partials");
}

extern "C" int dkv_qkv_split(const void* qkv, int32_t qkv_dtype, const void* bias, int32_t bias_dtype, int32_t rows,
                             int32_t n_q_heads, int32_t n_kv_heads, int32_t d, const int32_t* positions,
                             const float* cos_sin, int32_t max_pos, float* q, float* k, float* v,
                             dkv_stream_t stream) {
    DKV_REQUIRE(qkv && q && k && v && d > 0 && n_q_heads > 0 && n_kv_heads > 0 && dtype_ok(qkv_dtype),
                "dkv_qkv_split: bad arguments");
    DKV_REQUIRE(!bias || dtype_ok(bias_dtype), "dkv_qkv_split: bad bias dtype");
    DKV_REQUIRE(!cos_sin || (positions && d % 2 == 0 && max_pos > 0), "dkv_qkv_split: RoPE needs positions, even d");
    const int items = cos_sin ? (n_q_heads + n_kv_heads) * (d / 2) + n_kv_heads * d : (n_q_heads + 2 * n_kv_heads) * d;
    DKV_COLS_LAUNCH(qkv_split_kernel, rows, items, xsrc(qkv, qkv_dtype), bias, bias_dtype, n_q_heads, n_kv_heads, d,
                    positions, cos_sin, max_pos, q, k, v);
}

extern "C" int dkv_qkv_split_partials(const float* part, int32_t n_part, const void* bias, int32_t bias_dtype,
                                      int32_t rows, int32_t n_q_heads, int32_t n_kv_heads, int32_t d,
                                      const int32_t* positions, const float* cos_sin, int32_t max_pos, float* q,
                                      float* k, float* v, dkv_stream_t stream) {
    DKV_REQUIRE(part && n_part > 0 && q && k && v && d > 0 && n_q_heads > 0 && n_kv_heads > 0,
                "dkv_qkv_split_partials: bad arguments");
    DKV_REQUIRE(!bias || dtype_ok(bias_dtype), "dkv_qkv_split_partials: bad bias dtype");
    DKV_REQUIRE(!cos_sin || (positions && d % 2 == 0 && max_pos > 0),
                "dkv_qkv_split_partials: RoPE needs positions, even d");
    const int n = (n_q_heads + 2 * n_kv_heads) * d;
    const int items = cos_sin ? (n_q_heads + n_kv_heads) * (d / 2) + n_kv_heads * d : n;
    DKV_COLS_LAUNCH(qkv_split_kernel, rows, items, (XSrc{nullptr, 0, part, n_part, (int64_t)rows * n}), bias,
                    bias_dtype, n_q_heads, n_kv_heads, d, positions, cos_sin, max_pos, q, k, v);
}

extern "C" int dkv_silu_mul(const void* gate_up, int32_t gate_up_dtype, int32_t rows, int32_t ff, void* out,
                            int32_t out_dtype, dkv_stream_t stream) {
    DKV_REQUIRE(gate_up && out && ff > 0 && dtype_ok(gate_up_dtype) && dtype_ok(out_dtype),
                "dkv_silu_mul: bad arguments");
    DKV_COLS_LAUNCH(silu_mul_kernel, rows, ff, gate_up, gate_up_dtype, ff, out, out_dtype);
}

extern "C" int dkv_bias_gelu(const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype, int32_t rows,
                             int32_t n, void* out, int32_t out_dtype, dkv_stream_t stream) {
    DKV_REQUIRE(x && out && n > 0 && dtype_ok(x_dtype) && dtype_ok(out_dtype) && (!bias || dtype_ok(bias_dtype)),
                "dkv_bias_gelu: bad arguments");
    DKV_COLS_LAUNCH(bias_gelu_kernel, rows, n, x, x_dtype, bias, bias_dtype, n, out, out_dtype);
}

extern "C" int dkv_relu(const void* x, int32_t x_dtype, int32_t rows, int32_t n, void* out, int32_t out_dtype,
                        dkv_stream_t stream) {
    DKV_REQUIRE(x && out && n > 0 && dtype_ok(x_dtype) && dtype_ok(out_dtype), "dkv_relu: bad arguments");
    DKV_COLS_LAUNCH(relu_kernel, rows, n, x, x_dtype, n, out, out_dtype);
}

extern "C" int dkv_add(float* h, const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype, int32_t rows,
                       int32_t n, dkv_stream_t stream) {
    DKV_REQUIRE(h && x && n > 0 && dtype_ok(x_dtype) && (!bias || dtype_ok(bias_dtype)), "dkv_add: bad arguments");
    DKV_COLS_LAUNCH(add_kernel, rows, n, h, x, x_dtype, bias, bias_dtype, n);
}

extern "C" int dkv_gemm_f32(const float* x, const float* w, int32_t w_layout, int32_t M, int32_t N, int32_t K,
                            const void* bias, int32_t bias_dtype, float* out, int32_t accumulate,
                            dkv_stream_t stream) {
    DKV_REQUIRE(x && w && out && N > 0 && K > 0 && (w_layout == 0 || w_layout == 1), "dkv_gemm_f32: bad arguments");
    DKV_REQUIRE(!bias || dtype_ok(bias_dtype), "dkv_gemm_f32: bad bias dtype");
    DKV_REQUIRE(M <= 65535 * GT, "dkv_gemm_f32: too many rows for one launch");
    if (M <= 0) return DKV_OK;
    const dim3 grid((N + GT - 1) / GT, (M + GT - 1) / GT);
    hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(GT * GT), 0, as_stream(stream), x, w, w_layout, M, N, K, bias,
                       bias_dtype, out, accumulate);
    return check_launch("dkv_gemm_f32");
}
