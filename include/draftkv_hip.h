/*
 * draftkv_hip.h -- C ABI of the MI355X (gfx950) DRAFTKV decode-round library.
 *
 * The reference (aabhimittal/Draft-KV) is pure Python/numpy and has no FFI;
 * its drop-in boundary is the duck-typed cache protocol the models call
 * (append / read / note_attention / truncate, plus the mirror's sync_from /
 * rebuild_layers) and the engine's sampling/accept code. Each entry point
 * below replaces one piece of that protocol; the comment names the reference
 * file:line it stands in for. A Python host (draft-kv_amd/draftkv/_lib.py)
 * binds these with ctypes; INTEGRATION.md shows the binding.
 *
 * Conventions
 *   - All pointers are device pointers unless stated otherwise; the caller
 *     owns every buffer (the library allocates nothing).
 *   - Every function is stream-ordered on `stream` and returns 0 on success
 *     or a negative DKV_E* code; dkv_last_error() then describes the failure
 *     (thread-local). Sizes are validated on the host before any launch.
 *   - Positions are absolute token indices. A sequence's full cache always
 *     holds positions 0..len-1 (the engine never appends out of order).
 */
#ifndef DRAFTKV_HIP_H
#define DRAFTKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* dkv_stream_t; /* a hipStream_t; NULL = default stream */

enum { DKV_OK = 0, DKV_EINVAL = -1, DKV_ELAUNCH = -2, DKV_EWORKSPACE = -3, DKV_ECAPACITY = -4 };
enum { DKV_F32 = 0, DKV_BF16 = 1 };

/* Paged full (authoritative) cache -- reference draftkv/paged.py:76-176.
 * pool: n_blocks physical blocks; block b holds one layer's K and V for
 * block_size consecutive positions of one sequence:
 *     K part: [n_kv_heads][block_size][head_dim]
 *     V part: [n_kv_heads][head_dim][block_size]   (transposed)
 * elements DKV_F32 or DKV_BF16. block_table: int32 [batch][n_layers][max_blocks]
 * physical block ids (host-managed LIFO pools, paged.py:33-73). */
typedef struct {
    void* pool;
    const int32_t* block_table;
    int32_t batch, n_layers, n_kv_heads, head_dim, block_size, max_blocks, dtype;
} dkv_paged_t;

/* Compressed drafter mirror -- reference draftkv/compress.py:95-241.
 * Per (seq, layer, kv_head) a dense segment of `cap` row slots (cap a
 * multiple of 32) stored as cap/32 pages of 32 rows; rows 0..n_rows-1 are
 * live (eviction and truncation compact it). A layer's pages are one range
 * in which the segments interleave in chunks of 8 pages; with npg = cap/32,
 * nseg = batch*n_kv_heads, nf = npg/8, rem = npg - 8*nf and
 * seg = seq*n_kv_heads + head, page p of a segment is slot
 *     layer*npg*nseg + ((p/8)*nseg + seg)*8 + p%8          (p < 8*nf)
 *     layer*npg*nseg + 8*nf*nseg + seg*rem + (p - 8*nf)    (otherwise)
 * starting at pages + slot * page_stride
 * and holds K codes, K (scale, lo) pairs, V codes and V pairs of its rows in
 * the layout described in draft-kv_amd/csrc/mirror_layout.h (4-bit codes for
 * bits <= 4, bytes for 8 bits, raw float32 for 16 bits -- the reference
 * keeps an fp32 copy, compress.py:28-29; pairs in float32, or float16 when
 * meta_f16). pos/score/n_rows are per (seq, layer). */
typedef struct {
    void* pages;
    int32_t* pos;                /* [batch][n_layers][cap] absolute positions */
    double* score;               /* [batch][n_layers][cap] accumulated attention mass */
    int32_t* n_rows;             /* [batch][n_layers] live rows */
    int32_t batch, n_layers, n_kv_heads, head_dim, cap;
    int64_t page_stride;         /* bytes per page slot (>= the widest arm's page) */
} dkv_drafter_t;

/* Bytes of one 32-row page for an arm (bits, group, meta_f16) at head_dim d. */
int64_t dkv_page_bytes(int32_t bits, int32_t head_dim, int32_t group, int32_t meta_f16);

/* One layer's compression arm -- reference draftkv/config.py:9-33 plus the
 * `group` / fp16-meta extension. */
typedef struct {
    int32_t bits, group, meta_f16, sink, recent;
} dkv_qcfg_t;

/* ---------------------------------------------------------------- quantize */
/* Group quantizer on contiguous float32 rows x[rows][d] -- replaces
 * draftkv/compress.py:21-46 (`quantize`). Writes codes u8 [rows][d],
 * scale/lo f32 [rows][ceil(d/group)], deq f32 [rows][d] (any output may be
 * NULL). Bit-exact with the reference's float32 op order. */
int dkv_quantize(const float* x, int64_t rows, int32_t d, int32_t bits, int32_t group,
                 int32_t meta_f16, uint8_t* codes, float* scale, float* lo, float* deq,
                 dkv_stream_t stream);

/* ---------------------------------------------------------------- paged append */
/* Write K/V rows into the paged full cache -- replaces
 * draftkv/paged.py:120-128 (`PagedKVCache.append`). k, v: [batch][T][Hkv][D]
 * (in_dtype). Sequence s writes rows t < count[s] at positions start[s]+t;
 * blocks must already be in block_table (the host allocates them,
 * paged.py:112-117). count may be NULL (= T for all). */
int dkv_paged_append(const dkv_paged_t* cache, int32_t layer, const void* k, const void* v,
                     int32_t in_dtype, int32_t T, const int32_t* start, const int32_t* count,
                     dkv_stream_t stream);

/* ---------------------------------------------------------------- paged attention */
/* Causal attention of T query rows per sequence over the paged full cache
 * (verify pass, baseline decode, prefill) -- replaces the read + einsum +
 * softmax of draftkv/llama.py:202-218 / gpt2.py:197-206 / model.py:117-127
 * against FullKVCache/PagedKVCache. q: f32 [batch][T][Hq][D]; query t of
 * sequence s sits at position start[s]+t and sees positions <= its own.
 * count: NULL (every sequence appended all T rows) or int32 [batch], the
 * rows sequence s appended (dkv_paged_append's count); the cache of s then
 * ends at start[s]+count[s], positions past it are never read, and a
 * padding row t >= count[s] attends over the whole cache (zeros when it
 * is empty). out: f32 [batch][T][Hq][D]. Keys are split in fixed chunks of
 * chunk_keys absolute positions and merged in chunk order, so a query's
 * result does not depend on T or on the cache length (batch invariance).
 * work: dkv_paged_attention_workspace() bytes. */
size_t dkv_paged_attention_workspace(const dkv_paged_t* cache, int32_t T, int32_t n_q_heads,
                                     int32_t max_len, int32_t chunk_keys);
int dkv_paged_attention(const dkv_paged_t* cache, int32_t layer, const float* q, int32_t T,
                        int32_t n_q_heads, const int32_t* start, const int32_t* count,
                        int32_t max_len, int32_t chunk_keys, float* out, void* work,
                        size_t work_bytes, dkv_stream_t stream);

/* ------------------------------------------------------------ mirror append / evict */
/* Quantize and append T rows per sequence to one layer of the mirror, then
 * evict down to budget[s] -- replaces draftkv/compress.py:122-133 (`append`)
 * with :154-179 (`budget`, `_evict`). k, v: [batch][T][Hkv][D] (in_dtype);
 * row t < count[s] of sequence s has position start[s]+t. The victims are
 * the lowest (score, position) rows outside the `sink` lowest and `recent`
 * highest live positions (recent == 0 protects every row). count may be
 * NULL. */
int dkv_drafter_append(const dkv_drafter_t* mirror, int32_t layer, dkv_qcfg_t cfg,
                       const void* k, const void* v, int32_t in_dtype, int32_t T,
                       const int32_t* start, const int32_t* count, const int32_t* budget,
                       dkv_stream_t stream);

/* ---------------------------------------------------------------- mirror truncate / rebuild */
/* Drop every row at position >= start[s] in all layers -- replaces
 * draftkv/compress.py:181-188 (`truncate`). cfgs: host array of n_layers
 * arms (the row width of each layer). */
int dkv_drafter_truncate(const dkv_drafter_t* mirror, const dkv_qcfg_t* cfgs, const int32_t* start,
                         dkv_stream_t stream);

/* Per-round resync: truncate each layer to start[s], then quantize the full
 * cache's rows start[s]..end[s]-1 into it and evict to budget[layer*batch+s]
 * -- replaces draftkv/compress.py:190-207 (`sync_from`). cfgs: host array of
 * n_layers arms. */
int dkv_drafter_sync(const dkv_drafter_t* mirror, const dkv_paged_t* full, const dkv_qcfg_t* cfgs,
                     const int32_t* start, const int32_t* end, const int32_t* budget,
                     dkv_stream_t stream);

/* --------------------------------------------------------------- mirror requantize */
/* Requantize the listed layers from the full cache under new arms -- replaces
 * draftkv/compress.py:209-230 (`rebuild_layers`) and the first build
 * `sync_from(full, 0)`. All scores restart at 0, so the survivors are the
 * closed form [0, sink) u [n - (B - sink), n) (n = len[s], B = budget
 * [layer*batch+s]); only those rows are read and quantized, written densely
 * in position order. layers/cfgs are host arrays (cfgs indexed by layer). */
int dkv_drafter_rebuild(const dkv_drafter_t* mirror, const dkv_paged_t* full,
                        const int32_t* layers, int32_t n_changed, const dkv_qcfg_t* cfgs,
                        const int32_t* len, const int32_t* budget, dkv_stream_t stream);

/* ---------------------------------------------------------------- drafter attention */
/* Drafter attention: one query position per sequence over the live rows of
 * one mirror layer, dequantizing in registers -- replaces the read + einsum
 * + softmax + note_attention of the model forwards against CompressedKVCache
 * (compress.py:135-151; llama.py:202-218). q: f32 [batch][Hq][D] (GQA groups
 * of Hq/Hkv query heads share a KV head); out: f32 [batch][Hq][D]. When
 * want_mass, each live row's score gains the float32 sum over query heads of
 * its attention probability (compress.py:144-151; llama.py:213-214).
 * work: dkv_drafter_attention_workspace() bytes. */
size_t dkv_drafter_attention_workspace(const dkv_drafter_t* mirror, int32_t n_q_heads,
                                       int32_t want_mass);
int dkv_drafter_attention(const dkv_drafter_t* mirror, int32_t layer, dkv_qcfg_t cfg,
                          const float* q, int32_t n_q_heads, int32_t want_mass, float* out,
                          void* work, size_t work_bytes, dkv_stream_t stream);

/* Measurement hook (no counterpart in the reference; for benchmarks that
 * time the dominant kernel alone): when on, dkv_drafter_attention times
 * its split-K (or segment) kernel with a pair of HIP events carried by that
 * kernel's own launch (hipExtLaunchKernel) on its launch stream, one
 * pair per call for the first 1024 calls after switching on (later calls
 * reuse the last pair). dkv_drafter_kernel_last_ms waits for the last pair
 * and returns its elapsed milliseconds (-1 when there is none);
 * dkv_drafter_kernel_total_ms sums the recorded pairs (their number to
 * *n_pairs), so back-to-back calls can be timed with no host wait between
 * them. Not for concurrent callers. */
int dkv_drafter_kernel_timing(int32_t on);
float dkv_drafter_kernel_last_ms(void);
float dkv_drafter_kernel_total_ms(int32_t* n_pairs);

/* Unpack one layer of one sequence to plain arrays (debug/parity `read`,
 * compress.py:135-142): codes u8 [rows][Hkv][D], scale/lo f32
 * [rows][Hkv][groups], deq f32 [rows][Hkv][D] for K and V, pos int32 [rows].
 * Rows are in storage order; `rows` must equal the layer's live row count.
 * Any output may be NULL. */
int dkv_drafter_gather(const dkv_drafter_t* mirror, int32_t seq, int32_t layer, dkv_qcfg_t cfg,
                       int32_t rows, uint8_t* k_codes, float* k_scale, float* k_lo, float* k_deq,
                       uint8_t* v_codes, float* v_scale, float* v_lo, float* v_deq,
                       int32_t* pos, dkv_stream_t stream);

/* ---------------------------------------------------------------- sampling */
/* A row's normaliser under temperature T > 0, as dkv_sample computes it and
 * dkv_accept uses it: m = max(x)/T, s = the float64 sum over the row of
 * exp(x/T - m), inv_s = 1/s (arg: the first index of the max, greedy only).
 * The reference keeps the drafter's whole distribution q from each draft
 * step (draftkv/engine.py:176-179, `draft_probs`) for the verify decision;
 * these 32 bytes per row are what the decision needs of it besides the
 * logits. */
typedef struct {
    double m, s, inv_s;
    int32_t arg, reserved;
} dkv_row_stats_t;

/* One draw per row from softmax(logits/T) -- replaces draftkv/engine.py:36-41
 * (`_probs`) + :101-106 (`_sample`). logits f32 rows of length vocab at
 * row_stride; u: f64 uniforms [batch]. T <= 0: first argmax (u unused).
 * tokens: int32 [batch]. row_stats: NULL, or [batch] written with each
 * row's normaliser (for dkv_accept's draft_stats). work:
 * dkv_sample_workspace() bytes. */
size_t dkv_sample_workspace(int32_t batch, int32_t vocab);
int dkv_sample(const float* logits, int64_t row_stride, int32_t batch, int32_t vocab,
               float temperature, const double* u, int32_t* tokens, dkv_row_stats_t* row_stats,
               void* work, size_t work_bytes, dkv_stream_t stream);

/* ---------------------------------------------------------------- accept */
/* Verify decision of one round for every sequence -- replaces
 * draftkv/engine.py:188-213. target: f32 [batch][gamma+1][vocab];
 * draft: f32 [gamma][batch][vocab] (the drafter's logits, step-major as the
 * draft steps produce them; unused when T <= 0); draft_tokens int32
 * [batch][gamma]; u: f64 [batch][gamma+1]
 * uniforms in the order the reference draws them (one per tested position in
 * sampling mode, then one for the bonus/residual token). draft_stats: NULL,
 * or [gamma][batch] (step-major, as the draft steps produce them) the draft
 * rows' normalisers from dkv_sample on the same logits -- the draft rows'
 * statistics are then not recomputed (the decisions are the same either
 * way). Outputs int32 [batch]: accepted, next_token, and n_uniforms (draws
 * consumed). Any gamma up to 32767, vocab up to 1048576.
 * work: dkv_accept_workspace() bytes; calls that share a workspace must be in
 * stream order. */
size_t dkv_accept_workspace(int32_t batch, int32_t gamma, int32_t vocab);
int dkv_accept(const float* target, const float* draft, const int32_t* draft_tokens,
               int32_t batch, int32_t gamma, int32_t vocab, float temperature, const double* u,
               const dkv_row_stats_t* draft_stats, int32_t* accepted, int32_t* next_token,
               int32_t* n_uniforms, void* work, size_t work_bytes, dkv_stream_t stream);

/* dkv_accept with no workspace argument and no allocation: the workspace is a
 * static device array of DKV_ACCEPT_SCRATCH_BYTES inside the library (one per
 * GPU, held until the process ends). No counterpart in the reference; it is
 * for callers that cannot allocate device memory -- code under stream/graph
 * capture, serving loops that forbid hipMalloc. Returns DKV_ECAPACITY when
 * dkv_accept_workspace(batch, gamma, vocab) exceeds the scratch (at vocab
 * 128256 it holds batch 32 with gamma <= 112, batch 128 with gamma <= 15).
 * Calls that overlap on one GPU share the array and race; calls in stream
 * order do not. */
#define DKV_ACCEPT_SCRATCH_BYTES ((size_t)16 << 20)
int dkv_accept_noalloc(const float* target, const float* draft, const int32_t* draft_tokens,
                       int32_t batch, int32_t gamma, int32_t vocab, float temperature,
                       const double* u, const dkv_row_stats_t* draft_stats, int32_t* accepted,
                       int32_t* next_token, int32_t* n_uniforms, dkv_stream_t stream);

/* ------------------------------------------------------ model forward ops */
/* The non-attention pieces of the model forwards (reference
 * draftkv/model.py:100-133, draftkv/gpt2.py:182-213, draftkv/llama.py:175-225)
 * on float32 activations [rows][d]. Every `*_dtype` is DKV_F32 or DKV_BF16:
 * weight tables, inputs that come out of a bf16 GEMM, and outputs that feed
 * one. A NULL bias means none. */

/* out[r] = table[tokens[r]] (+ pos_table[positions[r]])  -- model.py:108, gpt2.py:186, llama.py:179 */
int dkv_embed(const void* table, int32_t table_dtype, const int32_t* tokens, int32_t rows, int32_t d,
              const void* pos_table, const int32_t* positions, float* out, dkv_stream_t stream);
/* out = x / sqrt(mean(x^2) + eps) * w  -- model.py:18-19, llama.py:93-94 */
int dkv_rmsnorm(const float* x, const void* w, int32_t w_dtype, int32_t rows, int32_t d, float eps, void* out,
                int32_t out_dtype, dkv_stream_t stream);
/* out = (x - mean) / sqrt(var + eps) * w + b  -- gpt2.py:120-123 */
int dkv_layernorm(const float* x, const void* w, const void* b, int32_t w_dtype, int32_t rows, int32_t d, float eps,
                  void* out, int32_t out_dtype, dkv_stream_t stream);
/* h += x (+ bias), written back to h, then out = RMSNorm(h) / LayerNorm(h): the residual add
 * of one block fused with the norm that opens the next  -- model.py:128-130, gpt2.py:207-209,
 * llama.py:219-221 (and the final norm, model.py:133, gpt2.py:212, llama.py:224) */
int dkv_add_rmsnorm(float* h, const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype, const void* w,
                    int32_t w_dtype, int32_t rows, int32_t d, float eps, void* out, int32_t out_dtype,
                    dkv_stream_t stream);
int dkv_add_layernorm(float* h, const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype, const void* w,
                      const void* b, int32_t w_dtype, int32_t rows, int32_t d, float eps, void* out,
                      int32_t out_dtype, dkv_stream_t stream);
/* dkv_add_rmsnorm / dkv_add_layernorm (layer_norm != 0) with x the bf16 GEMM's deferred
 * partials part [n_part][rows][d] (DKV_GEMM_DEFER): x[r][i] = bf16(sum over chunks, in chunk
 * order), the value dkv_gemm_bf16 would have stored, so the result is bit for bit that of the
 * GEMM followed by the add-norm; the GEMM's reduce launch is saved  -- the same reference lines */
int dkv_add_norm_partials(float* h, const float* part, int32_t n_part, const void* bias, int32_t bias_dtype,
                          const void* w, const void* b, int32_t w_dtype, int32_t layer_norm, int32_t rows, int32_t d,
                          float eps, void* out, int32_t out_dtype, dkv_stream_t stream);
/* Split fused projection rows [q heads | k heads | v heads] (+ bias) into f32 q [rows][Hq][d],
 * k and v [rows][Hkv][d]; with cos_sin (cos table [max_pos][d/2] then sin table) apply
 * rotate-half RoPE to q and k at positions[r]  -- model.py:118-120, gpt2.py:193-196,
 * llama.py:164-172,186-198 */
int dkv_qkv_split(const void* qkv, int32_t qkv_dtype, const void* bias, int32_t bias_dtype, int32_t rows,
                  int32_t n_q_heads, int32_t n_kv_heads, int32_t d, const int32_t* positions,
                  const float* cos_sin, int32_t max_pos, float* q, float* k, float* v, dkv_stream_t stream);
/* dkv_qkv_split with the projection rows as the bf16 GEMM's deferred partials
 * part [n_part][rows][(Hq + 2 Hkv) d] (DKV_GEMM_DEFER), summed and rounded as
 * dkv_add_norm_partials does  -- the same reference lines */
int dkv_qkv_split_partials(const float* part, int32_t n_part, const void* bias, int32_t bias_dtype, int32_t rows,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t d, const int32_t* positions,
                           const float* cos_sin, int32_t max_pos, float* q, float* k, float* v, dkv_stream_t stream);
/* out = silu(gate) * up with gate_up = [rows][2*ff]  -- llama.py:102-103,222 */
int dkv_silu_mul(const void* gate_up, int32_t gate_up_dtype, int32_t rows, int32_t ff, void* out, int32_t out_dtype,
                 dkv_stream_t stream);
/* out = gelu_tanh(x + bias)  -- gpt2.py:126-127,210 */
int dkv_bias_gelu(const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype, int32_t rows, int32_t n,
                  void* out, int32_t out_dtype, dkv_stream_t stream);
/* out = max(x, 0)  -- model.py:131 */
int dkv_relu(const void* x, int32_t x_dtype, int32_t rows, int32_t n, void* out, int32_t out_dtype,
             dkv_stream_t stream);
/* h += x (+ bias): residual adds  -- model.py:128,131, gpt2.py:207,210, llama.py:219,222 */
int dkv_add(float* h, const void* x, int32_t x_dtype, const void* bias, int32_t bias_dtype, int32_t rows, int32_t n,
            dkv_stream_t stream);
/* out (+)= x[M][K] . w (+ bias[N]), w[K][N] (w_layout 0) or w[N][K] (1), float32. Each output is
 * one in-order k reduction, so a row's result is the same for any M (the verify pass and the
 * one-token decode agree bit for bit)  -- the x @ W products of the model forwards */
int dkv_gemm_f32(const float* x, const float* w, int32_t w_layout, int32_t M, int32_t N, int32_t K,
                 const void* bias, int32_t bias_dtype, float* out, int32_t accumulate, dkv_stream_t stream);
/* y[M][N] = x[M][K] . w[N][K]^T (+ bias[N]), bf16 inputs, float32
 * accumulation, y bf16 (rounded once, to nearest even) or float32 (y_dtype
 * DKV_BF16 / DKV_F32); bias bf16 or NULL. x is bf16 or float32 (x_dtype);
 * a float32 x is rounded to bf16 (nearest even) as it is read, so the
 * result equals that of the converted x. N a multiple of 16, K of 32; x, w,
 * y 16-byte aligned, bias 8-byte aligned. K is cut into chunks fixed by
 * (N, K) alone; every output is one in-order chain of MFMA steps per chunk,
 * the chunk sums are added in chunk order and the bias last, so a row's
 * result is the same for any M and any launch shape (verify and one-token
 * decode agree bit for bit). work: dkv_gemm_bf16_workspace() bytes (0: none
 * needed)  -- the x @ W (+ b) products of the bf16 model forwards
 * (model.py:113-133, gpt2.py:191-213, llama.py:187-225) */
#define DKV_GEMM_SWIGLU 1  /* flags: W's rows interleave (gate_i, up_i); y is bf16 [M][N/2] with
                              y[m][i] = silu(g) * u of the two outputs, each first rounded to bf16
                              (the SwiGLU of llama.py:220-222 fused into the gate/up product; no bias) */
#define DKV_GEMM_DEFER 2   /* flags: when the launch plan for (M, N, K) makes per-chunk partials
                              (dkv_gemm_bf16_partials > 0), leave them, float32 [S][M][N], at the
                              start of work and skip the reduce: y is not written, and the consumer
                              sums them (dkv_add_norm_partials, dkv_qkv_split_partials); otherwise
                              y is written as usual. bf16 y only, no bias, no SwiGLU */
#define DKV_GEMM_WTILED 4  /* flags: w is stored in 16-row x 128-k tiles (K a multiple of 128): the
                              4 KB tile (fn, kb) at (fn * K/128 + kb) * 2048 elements, holding
                              element (16 fn + c, 128 kb + 32 j + 8 q + e) at j * 512 + (16 q + c) * 8 + e,
                              so every load of W is 1 KB contiguous; same arithmetic and results */
size_t dkv_gemm_bf16_workspace(int32_t M, int32_t N, int32_t K);
/* the chunk count S of the partials dkv_gemm_bf16 writes for (M, N, K), or 0 when its plan
 * writes y directly (a function of the launch plan, not of the arithmetic) */
int32_t dkv_gemm_bf16_partials(int32_t M, int32_t N, int32_t K);
int dkv_gemm_bf16(const void* x, int32_t x_dtype, const void* w, const void* bias, int32_t M, int32_t N,
                  int32_t K, void* y, int32_t y_dtype, int32_t flags, void* work, size_t work_bytes,
                  dkv_stream_t stream);

/* ---------------------------------------------------------------- misc */
const char* dkv_last_error(void);
int32_t dkv_version(void);

#ifdef __cplusplus
}
#endif
#endif /* DRAFTKV_HIP_H */
