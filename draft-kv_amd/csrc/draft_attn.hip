// (a5, a6) Drafter attention over the compressed mirror.
// Reference: the read + einsum + softmax + note_attention of the model
// forwards against CompressedKVCache (draftkv/compress.py:135-151,
// draftkv/llama.py:202-218, gpt2.py:197-206, model.py:117-127).
//
// One query position per sequence; the G query heads of a KV head share its
// rows. Grid: x = split of CH rows, y = KV head, z = sequence. Each block
// dequantizes its rows tile by tile into LDS and keeps an online softmax per
// query head; a combine kernel merges the splits. With want_mass the block
// also spills its scaled logits, and a third kernel turns them into each
// row's probability mass summed over query heads (added to the row's score).
#include "dkv_common.h"

namespace dkv {

constexpr int DQB = 16;     // max query heads per KV head
constexpr int DKT = 32;     // rows per tile
constexpr int DMAXD = 128;  // LDS tiles stay under 64 KB
constexpr int DCH = 512;    // rows per split

__global__ void __launch_bounds__(256) draft_attn_kernel(dkv_drafter_t m, int layer, dkv_qcfg_t cfg,
                                                         const float* __restrict__ q, int Hq, float scale,
                                                         int n_splits, float* __restrict__ part,
                                                         float* __restrict__ logits) {
    const int split = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
    const int D = m.head_dim, G = Hq / m.n_kv_heads;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int r_begin = split * DCH;
    const int r_end = min(r_begin + DCH, n);
    const int tid = threadIdx.x;

    extern __shared__ float smem[];
    float* sQ = smem;                   // [DQB][D]
    float* sK = sQ + DQB * D;           // [DKT][D+1]
    float* sV = sK + DKT * (D + 1);     // [DKT][D]
    float* sS = sV + DKT * D;           // [DQB][DKT]
    float* sM = sS + DQB * DKT;
    float* sL = sM + DQB;
    float* sA = sL + DQB;

    for (int i = tid; i < DQB * D; i += blockDim.x) {
        const int r = i / D, d = i % D;
        sQ[i] = r < G ? q[((int64_t)s * Hq + h * G + r) * D + d] : 0.0f;
    }
    if (tid < DQB) {
        sM[tid] = -INFINITY;
        sL[tid] = 0.0f;
    }
    constexpr int MAXACC = DQB * DMAXD / 256;
    float acc[MAXACC];
#pragma unroll
    for (int j = 0; j < MAXACC; ++j) acc[j] = 0.0f;
    const int n_out = DQB * D;

    const Seg sg = seg_of(m, s, layer, h);
    const int64_t crb = code_row_bytes(cfg.bits, D), mrb = meta_row_bytes(cfg.bits, D, cfg.group, cfg.meta_f16);

    for (int rt = r_begin; rt < r_end; rt += DKT) {
        __syncthreads();
        for (int i = tid; i < DKT * D; i += blockDim.x) {
            const int j = i / D, d = i % D;
            const int r = rt + j;
            float kv = 0.0f, vv = 0.0f;
            if (r < r_end) {
                if (cfg.bits >= 16) {
                    kv = reinterpret_cast<const float*>(sg.kc + (int64_t)r * crb)[d];
                    vv = reinterpret_cast<const float*>(sg.vc + (int64_t)r * crb)[d];
                } else {
                    const int g = d / cfg.group;
                    kv = dequant(get_code(sg.kc + (int64_t)r * crb, d, cfg.bits),
                                 get_meta(sg.km + (int64_t)r * mrb, g, cfg.meta_f16));
                    vv = dequant(get_code(sg.vc + (int64_t)r * crb, d, cfg.bits),
                                 get_meta(sg.vm + (int64_t)r * mrb, g, cfg.meta_f16));
                }
            }
            sK[j * (D + 1) + d] = kv;
            sV[j * D + d] = vv;
        }
        __syncthreads();
        for (int i = tid; i < DQB * DKT; i += blockDim.x) {
            const int r = i / DKT, j = i % DKT;
            float sc = -INFINITY;
            if (r < G && rt + j < r_end) {
                float dot = 0.0f;
                for (int d = 0; d < D; ++d) dot = fmaf(sQ[r * D + d], sK[j * (D + 1) + d], dot);
                sc = dot * scale;
                if (logits) logits[(((int64_t)s * Hq) + h * G + r) * m.cap + rt + j] = sc;
            }
            sS[i] = sc;
        }
        __syncthreads();
        {
            const int r = tid / 16, l16 = tid % 16;
            float mx = -INFINITY;
            for (int j = l16; j < DKT; j += 16) mx = fmaxf(mx, sS[r * DKT + j]);
            for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
            const float m_old = sM[r];
            const float m_new = fmaxf(m_old, mx);
            float sum = 0.0f;
            for (int j = l16; j < DKT; j += 16) {
                const float sc = sS[r * DKT + j];
                const float p = (sc == -INFINITY) ? 0.0f : __expf(sc - m_new);
                sS[r * DKT + j] = p;
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
#pragma unroll
        for (int jj = 0; jj < MAXACC; ++jj) {
            const int o = tid + 256 * jj;
            if (o < n_out) {
                const int r = o / D, d = o % D;
                float a = acc[jj] * sA[r];
                for (int j = 0; j < DKT; ++j) a = fmaf(sS[r * DKT + j], sV[j * D + d], a);
                acc[jj] = a;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < MAXACC; ++jj) {
        const int o = tid + 256 * jj;
        if (o < n_out) {
            const int r = o / D, d = o % D;
            if (r < G) {
                float* p = part + (((int64_t)s * Hq + h * G + r) * n_splits + split) * (D + 2);
                p[d] = acc[jj];
                if (d == 0) {
                    p[D] = sM[r];
                    p[D + 1] = sL[r];
                }
            }
        }
    }
}

// merge splits per (seq, query head); also records the final (max, sum)
__global__ void __launch_bounds__(128) draft_combine_kernel(dkv_drafter_t m, int layer, const float* __restrict__ part,
                                                            int Hq, int n_splits, float* __restrict__ out,
                                                            float* __restrict__ stats) {
    const int hq = blockIdx.x, s = blockIdx.y;
    const int D = m.head_dim;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int ns = min((n + DCH - 1) / DCH, n_splits);
    const float* p = part + ((int64_t)s * Hq + hq) * n_splits * (D + 2);
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float mm = -INFINITY, l = 0.0f, o = 0.0f;
        for (int c = 0; c < ns; ++c) {
            const float* pc = p + (int64_t)c * (D + 2);
            const float mc = pc[D], lc = pc[D + 1];
            const float mn = fmaxf(mm, mc);
            const float a = (mm == -INFINITY) ? 0.0f : __expf(mm - mn);
            const float b = (mc == -INFINITY) ? 0.0f : __expf(mc - mn);
            l = l * a + lc * b;
            o = o * a + pc[d] * b;
            mm = mn;
        }
        out[((int64_t)s * Hq + hq) * D + d] = (l > 0.0f) ? o / l : 0.0f;
        if (d == 0 && stats) {
            stats[((int64_t)s * Hq + hq) * 2] = mm;
            stats[((int64_t)s * Hq + hq) * 2 + 1] = l;
        }
    }
}

// score[row] += sum over query heads of exp(logit - max) / sum
__global__ void __launch_bounds__(256) draft_mass_kernel(dkv_drafter_t m, int layer, int Hq,
                                                         const float* __restrict__ logits,
                                                         const float* __restrict__ stats) {
    const int s = blockIdx.y;
    const int n = m.n_rows[(int64_t)s * m.n_layers + layer];
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    float mass = 0.0f;
    for (int hq = 0; hq < Hq; ++hq) {
        const float mm = stats[((int64_t)s * Hq + hq) * 2], l = stats[((int64_t)s * Hq + hq) * 2 + 1];
        mass += __expf(logits[((int64_t)s * Hq + hq) * m.cap + r] - mm) / l;
    }
    m.score[row_index(m, s, layer) + r] += static_cast<double>(mass);
}

static size_t smem_bytes(int D) {
    return sizeof(float) * (DQB * D + DKT * (D + 1) + DKT * D + DQB * DKT + 3 * DQB);
}

}  // namespace dkv

using namespace dkv;

static int n_splits_of(const dkv_drafter_t* m) { return (m->cap + DCH - 1) / DCH; }

extern "C" size_t dkv_drafter_attention_workspace(const dkv_drafter_t* mirror, int32_t n_q_heads,
                                                  int32_t want_mass) {
    if (!mirror || n_q_heads <= 0) return 0;
    const size_t b = mirror->batch, D = mirror->head_dim;
    size_t bytes = sizeof(float) * b * n_q_heads * n_splits_of(mirror) * (D + 2);   // partials
    bytes += sizeof(float) * b * n_q_heads * 2;                                      // stats
    if (want_mass) bytes += sizeof(float) * b * n_q_heads * (size_t)mirror->cap;     // logits
    return bytes;
}

extern "C" int dkv_drafter_attention(const dkv_drafter_t* mirror, int32_t layer, dkv_qcfg_t cfg, const float* q,
                                     int32_t n_q_heads, int32_t want_mass, float* out, void* work,
                                     size_t work_bytes, dkv_stream_t stream) {
    DKV_REQUIRE(mirror && q && out, "dkv_drafter_attention: NULL argument");
    const dkv_drafter_t m = *mirror;
    DKV_REQUIRE(layer >= 0 && layer < m.n_layers, "dkv_drafter_attention: layer out of range");
    DKV_REQUIRE(m.head_dim > 0 && m.head_dim <= DMAXD, "dkv_drafter_attention: head_dim must be 1..128");
    DKV_REQUIRE(n_q_heads > 0 && n_q_heads % m.n_kv_heads == 0 && n_q_heads / m.n_kv_heads <= DQB,
                "dkv_drafter_attention: query heads must be 1..16 per KV head");
    DKV_REQUIRE(cfg.bits >= 16 || cfg.group > 0, "dkv_drafter_attention: bad group");
    const size_t need = dkv_drafter_attention_workspace(mirror, n_q_heads, want_mass);
    if (!work || work_bytes < need)
        return fail(DKV_EWORKSPACE, "dkv_drafter_attention: workspace too small (need " + std::to_string(need) + ")");
    const int ns = n_splits_of(mirror);
    float* part = static_cast<float*>(work);
    float* stats = part + (size_t)m.batch * n_q_heads * ns * (m.head_dim + 2);
    float* logits = want_mass ? stats + (size_t)m.batch * n_q_heads * 2 : nullptr;
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(m.head_dim)));
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(draft_attn_kernel, dim3(ns, m.n_kv_heads, m.batch), dim3(256), smem_bytes(m.head_dim), st, m,
                       layer, cfg, q, n_q_heads, scale, ns, part, logits);
    int rc = check_launch("dkv_drafter_attention");
    if (rc) return rc;
    hipLaunchKernelGGL(draft_combine_kernel, dim3(n_q_heads, m.batch), dim3(128), 0, st, m, layer, part, n_q_heads, ns,
                       out, stats);
    if ((rc = check_launch("dkv_drafter_attention(combine)"))) return rc;
    if (want_mass) {
        hipLaunchKernelGGL(draft_mass_kernel, dim3((m.cap + 255) / 256, m.batch), dim3(256), 0, st, m, layer,
                           n_q_heads, logits, stats);
        rc = check_launch("dkv_drafter_attention(mass)");
    }
    return rc;
}
