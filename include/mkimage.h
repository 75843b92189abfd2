/* mkimage — MI355X (gfx950) denoising hot path of mako-image, as a C ABI.
 *
 * Two surfaces, both plain C (pointers, sizes, status codes; no HIP or C++ types):
 *  1. The engine: the sampler-facing API the reference's Engine subclasses expose,
 *       begin(prompt, h, w, slot) / step(latents, sigma, slot)   (src/image/engine.hpp:161-166)
 *     plus a batched classifier-free-guidance step that runs both slots as one batch of 2 and applies the guidance
 *     combine and the Euler update on the device (src/image/engine.cpp:471-503).
 *  2. The kernel-dispatch surface the step is built from: the runtime primitives the reference calls by name
 *     (proj, attention, heads_norm_half, heads_half, ln_modulate, gate_add, silu, gelu_tanh, swiglu_rows, geglu_rows,
 *     layer_norm, group_norm, norm; src/image/qwen_image.cpp:196-288, src/image/sdxl.cpp:425-457,742-796), taking
 *     device pointers and a stream.
 *
 * Conventions: every call returns MK_OK or an error code and never throws; mk_last_error() gives the message of the
 * calling thread's last failure. Device memory is the library's (mk_malloc) or the caller's; host buffers belong to
 * the caller and are copied in and out. Streams are opaque `void*` (a hipStream_t; NULL = the default stream).
 * An engine is not re-entrant: one thread drives it at a time (the reference serialises requests the same way,
 * src/server/image_server.cpp:583).
 */
#ifndef MKIMAGE_H
#define MKIMAGE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mk_status {
    MK_OK = 0,
    MK_ERR_ARG = 1,     /* a bad size, slot, null pointer or shape (the reference throws std::runtime_error) */
    MK_ERR_STATE = 2,   /* step before begin, missing weights */
    MK_ERR_DEVICE = 3,  /* a HIP runtime error */
    MK_ERR_NOMEM = 4,
    MK_ERR_UNSUPPORTED = 5
} mk_status;

const char* mk_last_error(void);
const char* mk_version(void);

/* ------------------------------------------------------------------------------------------------------------
 * Device plumbing (so callers need no other GPU runtime in the process).
 * ------------------------------------------------------------------------------------------------------------ */
mk_status mk_device_count(int* n);
mk_status mk_set_device(int dev);
/* name, compute units, max clock in kHz, gcn arch name ("gfx950...") */
mk_status mk_device_info(int dev, char* name, size_t name_len, int* cus, int* clock_khz, char* arch, size_t arch_len);
mk_status mk_malloc(void** p, size_t bytes);   /* zero-filled */
mk_status mk_free(void* p);
mk_status mk_memcpy_h2d(void* dst, const void* src, size_t bytes);
mk_status mk_memcpy_d2h(void* dst, const void* src, size_t bytes);
mk_status mk_memset(void* p, int v, size_t bytes);
mk_status mk_synchronize(void);
mk_status mk_stream_create(void** s);
mk_status mk_stream_destroy(void* s);
mk_status mk_stream_synchronize(void* s);
mk_status mk_event_create(void** e);
mk_status mk_event_destroy(void* e);
mk_status mk_event_record(void* e, void* stream);
mk_status mk_event_elapsed_ms(void* start, void* stop, float* ms);

/* ------------------------------------------------------------------------------------------------------------
 * Kernel-dispatch surface. Layouts: activations row-major [rows][cols]; weights row-major [out][in] (the
 * reference's Tensor with dims[0] = in features, qwen_image.cpp:79-111); bf16 = uint16 bit patterns; fp8 = OCP e4m3.
 * ------------------------------------------------------------------------------------------------------------ */

enum mk_dtype { MK_F32 = 0, MK_BF16 = 1, MK_FP8_E4M3 = 2, MK_F16 = 3, MK_DTYPE_OTHER = 255 /* a file dtype the
                                                                                          kernels do not take */ };

/* The GEMM's fused epilogue: what happens to acc = A W^T (* wscale[n]) + bias[n]. */
enum mk_epilogue {
    MK_EPI_STORE = 0,      /* C = acc (C dtype f32 or bf16) */
    MK_EPI_GELU_TANH = 1,  /* C = gelu_tanh(acc) */
    MK_EPI_GATE_ADD = 2,   /* X += gate[n] * acc, X fp32 (the dual-stream gated residual) */
    MK_EPI_GATE_TANH = 3,  /* X += tanh(gate[n]) * acc (gate_add, image.metal:55-65) */
    MK_EPI_SILU = 4,       /* C = silu(acc) */
    MK_EPI_ADD = 5,        /* X += acc (plain residual) */
    MK_EPI_HEADS = 6,      /* q|k|v columns scattered to heads with per-head RMSNorm + RoPE (see mk_heads_args) */
    /* Gated linear units fused into the projection: W holds N = 2F rows [first part; second part] (the fused
     * gate|up matrix as upload_rows stacks it), C is [M][F] (ldc >= F): */
    MK_EPI_SWIGLU = 7,     /* C[r][i] = silu(acc[r][i]) * acc[r][F + i] (swiglu_rows, qwen_image.cpp:275-280) */
    MK_EPI_GEGLU = 8,      /* C[r][i] = acc[r][i] * gelu_erf(acc[r][F + i]) (geglu_rows, image.metal:475-484) */
    MK_EPI_PAIR_SUM = 9    /* C[r][i] = acc[r][i] + acc[r][F + i]: an fp32 operand split into two halves (hi, lo)
                            * stacked as the weight's two row halves, summed (the VAE attention's F32 V^T) */
};

typedef struct mk_heads_args {
    /* Destination of the fused q/k/v epilogue: Q, K [batch][heads][n_pad][d] bf16 and V^T [batch][heads][d][k_pad]
     * bf16 (keys in the MK_VT_COL order), written at rows row0 + r (r the GEMM row within the batch). The GEMM's N
     * columns are q|k|v (N = 3 heads d), or Q alone when k and vt are NULL (N = heads d: a cross attention's query,
     * sdxl.cpp:778-779), or, for head_dim 64, K and V^T alone when q is NULL (N = 2 heads d: a cross attention's
     * context, sdxl.cpp:697-708). head_dim 128 (norm and RoPE optional) or 64 (the SDXL heads: no norm, no RoPE). */
    void* q;
    void* k;
    void* vt;
    uint32_t heads, head_dim, q_pad, k_pad;
    uint32_t row0;        /* sequence position of GEMM row 0: its RoPE table row and its K / V^T row */
    uint32_t q_row0;      /* Q row of GEMM row 0 (the 2.1 graph's later steps write Q from 0, K / V from S) */
    const float* norm_q;  /* [head_dim] or NULL (no norm) */
    const float* norm_k;
    const float* rope;    /* [rows][head_dim/2][2] (cos, sin) at row0 + r, or NULL */
    uint32_t rope_mode;   /* 0 none, 1 half-split pairs (i, i + d/2), 2 interleaved pairs (2i, 2i+1) */
    float eps;
    float k_scale;        /* K rows times this (0: 1), e.g. the softmax scale times log2(e) for mk_attention's scale 0 */
    uint32_t dtype;       /* element type of Q, K, V^T: 0 or MK_BF16 bf16; MK_F16 IEEE half (the reference's
                             heads_norm_half / heads_half, qwen_image.cpp:226-250) */
    int64_t rope_stride;  /* floats between the RoPE tables of consecutive batch items (0: one table for all): a
                             guidance batch whose prompts differ in length has one table per prompt */
} mk_heads_args;

typedef struct mk_gemm_args {
    const void* a;        /* [batch][M][lda] bf16 (f16 with f16 weights) */
    const void* w;        /* [N][K] bf16, fp8, or f16 (then A is f16 too: the products of F16 weights and half
                             activations, as the reference's VAE runs them) */
    const float* wscale;  /* [N] per-output-channel scale (fp8), or NULL */
    const float* bias;    /* [N] or NULL */
    void* c;              /* output [batch][M][ldc] (f32, bf16 or f16), or the fp32 residual X for GATE/ADD */
    const float* gate;    /* [N] gate row (GATE_ADD / GATE_TANH); rows r % seg_rows < split read gate + gate_alt */
    int64_t gate_alt;
    uint32_t split, seg_rows;
    uint32_t M, N, K;
    int64_t lda, ldc;
    int64_t stride_a, stride_c; /* between batches, in elements */
    uint32_t batch;
    uint32_t w_dtype;     /* MK_BF16, MK_FP8_E4M3 or MK_F16 (f16: epilogues STORE, ADD / GATE, PAIR_SUM) */
    uint32_t c_dtype;     /* MK_F32, MK_BF16 or MK_F16 */
    uint32_t epilogue;    /* mk_epilogue */
    const mk_heads_args* heads; /* MK_EPI_HEADS only */
} mk_gemm_args;

/* proj (the reference's GEMM, engine.cpp:768 / qwen_image.cpp:196-288): C = A W^T with the fused epilogue.
 * K % 64 == 0, N % 64 == 0. */
mk_status mk_gemm(const mk_gemm_args* a, void* stream);
/* count (1 or 2) GEMMs of equal N, K, weight dtype and epilogue kind in one launch: the dual-stream blocks' image and
 * text projections, whose separate launches would leave most of the chip idle on the text's few tiles. Each problem
 * keeps its own A, W, C, bias, gate, M, batch, strides and heads arguments. No counterpart in the reference (its 2.1
 * graph has one stream). */
mk_status mk_gemm_grouped(const mk_gemm_args* a, uint32_t count, void* stream);
/* Long GEMMs whose last wave of tiles would leave compute units idle split that wave's k steps over the chip
 * (stream-K); the tile's owner waits, bounded, for the other ranges' partials. A wait that gives up finishes the tile
 * from what is there and is reported as MK_ERR_DEVICE to its own stream: by that stream's next stream-K launch,
 * mk_stream_synchronize on it, or the engine call that launched it (mk_synchronize reports any stream's). This sets the bound in polls (an uncached load and a 128-cycle sleep each; default MK_GEMM_WAIT_LIMIT,
 * tens of seconds); a test hook: 0 gives up at once. Stream-K launches on different streams use different workspaces,
 * so they may run concurrently. No counterpart in the reference. */
#define MK_GEMM_WAIT_LIMIT (1u << 26)
mk_status mk_gemm_set_wait_limit(uint32_t polls);

/* 3x3 convolution, stride 1, zero padding 1 (the VAE decoder's conv, src/image/engine.cpp:732-746, 907-947), as one
 * GEMM over the padded pixel grid (implicit im2col on MFMA) in IEEE half operands with fp32 sums, as the reference
 * runs it (F16 weights, docs/performance.md:13). Layout "padded grid": an h x w image is stored as the
 * (h + 2) x (w + 2) grid with a zero ring, preceded and followed by w + 3 zero rows: row S + (y + 1)(w + 2) + x + 1
 * holds pixel (y, x), S = w + 3, each row c channels.
 *   x: f16 padded grid, c channels (ring and slack rows zero);
 *   w: f16 [n][9][c], tap = 3 dy + dx (the PyTorch weight [n][c][3][3] with its taps moved in front of c);
 *   y: (h + 2)(w + 2) rows of ldy values from its first grid row (a padded-grid buffer + S rows): the pixel rows are
 *      written; ring rows are left as they were or hold values the next layer must not read as pixels;
 *   epilogue MK_EPI_STORE (y = acc + bias, fp32 or f16) or MK_EPI_ADD (y += acc + bias, fp32).
 * c is a multiple of 64 (c <= 4096), n a multiple of 64 or 96; pad channels with zeros. */
typedef struct mk_conv_args {
    const void* x;
    const void* w;
    const float* bias; /* [n] or NULL */
    void* y;
    uint32_t h, width, c, n;
    int64_t ldy;
    uint32_t y_dtype;
    uint32_t epilogue;
} mk_conv_args;
mk_status mk_conv3x3(const mk_conv_args* a, void* stream);

/* GEMV for a few rows (the time embedding and modulation projections, rows <= 4):
 * y[r][n] = sum_k W[n][k] bf16(x'[r][k]) + b[n] with x' = silu(x) when silu_x (silu(temb) is the modulation
 * layers' input), else x; x fp32 [rows][K], W bf16 [N][K], y fp32. The activation is rounded to bf16 as every GEMM's
 * is. */
mk_status mk_gemv(const float* x, uint32_t rows, uint32_t K, const void* w, const float* bias, uint32_t N, float* y,
                  int silu_x, void* stream);

/* ln_modulate (image.metal:32-53): y = LN(x) (1 + scale) + shift, eps, no affine; x fp32 [rows][n], y bf16.
 * Row r takes the modulation at scale/shift + alt (floats) when r % seg_rows < split, else at scale/shift. */
mk_status mk_ln_modulate(const float* x, uint32_t rows, uint32_t n, const float* scale, const float* shift,
                         int64_t alt, uint32_t split, uint32_t seg_rows, float eps, void* y, void* stream);

/* gate_add (image.metal:55-65): x += g(gate) * y, g = tanh (tanh_gate = 1) or identity; x fp32, y fp32 or bf16
 * [rows][n]; row selection of the gate as in mk_ln_modulate. */
mk_status mk_gate_add(float* x, const void* y, uint32_t y_dtype, uint32_t rows, uint32_t n, const float* gate,
                      int64_t alt, uint32_t split, uint32_t seg_rows, int tanh_gate, void* stream);

/* heads_norm_half / heads_half (qwen_image.cpp:226-250, sdxl.cpp:439-448): per (row, head) of x bf16
 * [batch][rows][ld] at column col0 + head * d: optional RMSNorm * w, RoPE from table rows rope[row0 + r], written
 * to out [batch][heads][n_pad][d] at row0 + r (transpose = 0), or to out [batch][heads][d][n_pad] at column
 * MK_VT_COL(row0 + r) (transpose = 1: the V^T layout the attention reads), as out_dtype: MK_BF16 or MK_F16 (the
 * reference's half; rounded to nearest even). */
mk_status mk_heads(const void* x, uint32_t batch, uint32_t rows, int64_t ld, int64_t stride_x, uint32_t col0,
                   uint32_t heads, uint32_t d, const float* w, float eps, const float* rope, uint32_t rope_mode,
                   void* out, uint32_t n_pad, uint32_t row0, int transpose, uint32_t out_dtype, void* stream);

/* V^T key order: within each group of 16 keys, key k sits at column k with bits 2 and 3 swapped (the order in which
 * a lane of the P V matrix product reads 8 keys as one 16-byte load). */
#define MK_VT_COL(k) (((k) & ~12u) | (((k) & 4u) << 1) | (((k) & 8u) >> 1))

/* attention (qwen_image.cpp:271 and the AttnArgs it fills, sdxl.cpp:24-27, 450-457): softmax(Q K^T scale) V, fp32
 * online softmax on MFMA in the inputs' type `dtype`: MK_BF16, or MK_F16 (the reference's half heads; the
 * probabilities then enter P V as half too). q [batch][heads][q_pad][d], k [batch][kv_heads][k_pad][d], vt
 * [batch][kv_heads][d][k_pad] with keys in the MK_VT_COL order (padding keys zero); query head h reads key /
 * value head h / (heads / kv_heads) (grouped-query attention; kv_heads == heads for every graph here).
 * out bf16 [batch][n_q][ldo] at column head * d. Query row i (absolute q_pos0 + i) sees key c < n_k iff
 * q_pos0 + i >= block or c <= q_pos0 + i (block 0: no mask; UINT32_MAX: causal; S: causal text prefix), and c lies
 * outside its batch item's masked range: key_hole NULL, or a host array of batch pairs (lo, hi) (batch <= 8): keys
 * [lo, hi) of item b are masked (a classifier-free-guidance batch whose shorter prompt is padded to the longer one's
 * rows; lo >= 1). d in {64, 128}; kv_heads divides heads; q_pad % 128 == 0; k_pad % 64 == 0. */
mk_status mk_attention(const void* q, const void* k, const void* vt, void* out, uint32_t dtype, uint32_t batch,
                       uint32_t heads, uint32_t kv_heads, uint32_t d, uint32_t n_q, uint32_t q_pad, uint32_t n_k,
                       uint32_t k_pad, int64_t ldo, int64_t stride_o, uint32_t q_pos0, uint32_t block, float scale,
                       const uint32_t* key_hole, void* stream);

/* Elementwise and norms (fp32 unless stated). */
mk_status mk_silu(float* x, size_t n, void* stream);
mk_status mk_gelu_tanh(float* x, size_t n, void* stream);
/* m[r][i] = silu(gu[r][i]) * gu[r][F + i] (swiglu_rows); m bf16 */
mk_status mk_swiglu(const void* gu, uint32_t gu_dtype, uint32_t rows, uint32_t F, void* m, void* stream);
/* m[r][i] = hg[r][i] * gelu_erf(hg[r][F + i]) (geglu_rows, image.metal:475-484); m bf16 */
mk_status mk_geglu(const void* hg, uint32_t hg_dtype, uint32_t rows, uint32_t F, void* m, void* stream);
/* y = x * rsqrt(mean(x^2) + eps) * w (+ w_offset), x fp32, y bf16 (norm) */
mk_status mk_rms_norm(const float* x, uint32_t rows, uint32_t n, const float* w, float w_offset, float eps, void* y,
                      void* stream);
/* layer_norm with gamma, beta (sdxl.cpp:425-437): x fp32, y bf16 */
mk_status mk_layer_norm(const float* x, uint32_t rows, uint32_t n, const float* g, const float* b, float eps, void* y,
                        void* stream);
/* group_norm over channels-last [batch][rows][c], `groups` groups, affine; y bf16 */
mk_status mk_group_norm(const float* x, uint32_t batch, uint32_t rows, uint32_t c, uint32_t groups, const float* g,
                        const float* b, float eps, void* y, void* stream);
/* mk_group_norm without allocating: no counterpart in the reference; for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments and results
 * (bit-identical); the partial sums live in a fixed 4 MiB array of the library on each device instead of a per-call
 * allocation: 16 bytes for each of batch x ceil(rows / 16) x groups partials plus 8 for each of batch x groups
 * statistics must fit (e.g. batch 2, 4096 rows, 32 groups: 264 KiB), else MK_ERR_ARG. Every call on a device shares
 * that device's array: calls that overlap on one device (different streams, or threads) race and must not be made. */
mk_status mk_group_norm_noalloc(const float* x, uint32_t batch, uint32_t rows, uint32_t c, uint32_t groups,
                                const float* g, const float* b, float eps, void* y, void* stream);
/* x_out = x + dt * (neg + guidance * (pos - neg)) over n floats (engine.cpp:476-502); guidance 1 / neg NULL:
 * x + dt * pos. */
mk_status mk_cfg_euler(const float* x, const float* pos, const float* neg, size_t n, float guidance, float dt,
                       float* x_out, void* stream);
/* The RoPE table mk_begin builds for a prompt of S rows and an h x w token grid (QwenImage::begin with rope3,
 * src/image/qwen_image.cpp:33-45, 113-142): out [S + h * w][64][2] fp32 (cos, sin) of the 64 rotation pairs, axes of
 * 16 / 56 / 56 dims (theta 10000); text row t at position (t, t, t), image row S + y * w + x at (S, y - (h - h / 2),
 * x - (w - w / 2)). Host arithmetic only: the engine uploads exactly this table. */
mk_status mk_rope_table(uint32_t S, uint32_t h, uint32_t w, float* out);
/* 2x2 patchify: lat [batch][C][2h][2w] -> tokens [batch][h*w][4C] (feature c*4 + py*2 + px), and back. */
mk_status mk_patchify(const float* lat, uint32_t batch, uint32_t C, uint32_t h, uint32_t w, float* tokens,
                      void* stream);
mk_status mk_unpatchify(const float* tokens, uint32_t batch, uint32_t C, uint32_t h, uint32_t w, float* lat,
                        void* stream);
/* Counter RNG fill (synthetic weights and inputs): value i = mean + std * N(0,1)[key, i], stored as dtype
 * (MK_F32, or MK_BF16 / MK_F16 rounded to nearest even). */
mk_status mk_fill_normal(void* p, size_t n, uint32_t dtype, uint64_t key, double mean, double std, void* stream);
uint64_t mk_tensor_key(uint64_t seed, const char* name);
/* Per-output-row fp8 quantisation: scale[r] = max|W[r]| / 448 (1 for a zero row), dst[r][c] = e4m3(W[r][c] /
 * scale[r]) rounded to nearest even, saturating; src bf16 [rows][cols]. */
mk_status mk_quantize_fp8_rows(const void* src, uint64_t rows, uint64_t cols, void* dst, float* scale, void* stream);
/* fp32 <-> bf16 conversions on the device */
mk_status mk_f32_to_bf16(const float* x, size_t n, void* y, void* stream);
mk_status mk_bf16_to_f32(const void* x, size_t n, float* y, void* stream);

/* LoRA merge into a weight matrix on the device: W[r][c] += factor * sum_j B[r][j] A[j][c] for rows x cols, A fp32
 * [rank][cols], B fp32 [rows][rank] (rank <= 1024), the sum in fp32 in ascending j, the result rounded to W's dtype:
 * bf16 or IEEE half (nearest even), or e4m3 with W's per-row scale recomputed from the merged row (max / 448, cols <= 32768), the
 * rule mk_quantize_fp8_rows applies. The merge of a LoRA added for good (TransformerRuntime::add_lora, called from
 * src/image/h3_image.cpp:136; targets from QwenImage::lora_target, src/image/qwen_image.cpp:295-331). */
mk_status mk_lora_merge(void* w, uint32_t w_dtype, float* w_scale, uint64_t rows, uint64_t cols, const float* a,
                        const float* b, uint32_t rank, float factor, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * VAE decoder: the step after the loop (Engine::decode, src/image/engine.cpp:862-954; weights as load_vae reads
 * them, :589-628): Qwen-Image's Wan-2.1-layout decoder for one frame. Channels base x {4, 4, 4, 2, 1} per level
 * (base 96 for Qwen-Image), z latent channels (16), tokens [h][w][4 z] (a 2x2 patch each) -> RGBA [16 h][16 w][4]
 * fp32 in [-1, 1] with alpha 1. Every 3x3 conv is an mk_conv3x3 launch; the mid block's one-head attention runs as
 * GEMMs and a row softmax.
 * ------------------------------------------------------------------------------------------------------------ */
typedef struct mk_vae mk_vae;
typedef struct mk_vae_config {
    uint32_t base;      /* 96 */
    uint32_t z;         /* 16 */
    const float* mean;  /* [z]: latents_mean of the VAE's config (copied) */
    const float* std;   /* [z]: latents_std */
} mk_vae_config;
mk_status mk_vae_create(const mk_vae_config* cfg, mk_vae** out);
mk_status mk_vae_destroy(mk_vae* v);
/* Weights by checkpoint name (Diffusers AutoencoderKLQwenImage layout: "decoder.up_blocks.0.resnets.0.conv1.weight",
 * "decoder.mid_block.attentions.0.to_qkv.weight", ...), fp32 in PyTorch layout: conv weights [out][in][k][k], or the
 * causal 3-D form [out][in][kt][k][k] of which the last time tap is used (a single frame sees only it); vectors
 * [n] (or [n, 1, 1 ...]). */
mk_status mk_vae_load(mk_vae* v, const char* name, const float* data, const int64_t* dims, uint32_t ndim);
mk_status mk_vae_load_safetensors(mk_vae* v, const char* path, uint64_t* loaded);
/* Counter-RNG weights keyed by (seed, name): convs N(0, 1 / fan_in) as bf16, biases N(0, 0.02), gammas 1 + N(0, 0.1). */
mk_status mk_vae_init_random(mk_vae* v, uint64_t seed);
/* tokens [h * w][4 z] host fp32 (n values) -> rgba [16 h][16 w][4] host fp32; h, w <= 256 (images up to 4096^2) */
mk_status mk_vae_decode(mk_vae* v, const float* tokens, size_t n, uint32_t h, uint32_t w, float* rgba);
/* the same on device buffers, queued on the VAE's stream (mk_vae_stream) */
mk_status mk_vae_decode_device(mk_vae* v, const float* tokens, uint32_t h, uint32_t w, float* rgba);
mk_status mk_vae_stream(mk_vae* v, void** stream);

/* ------------------------------------------------------------------------------------------------------------
 * Checkpoint files: safetensors (the reference's safetensors::Files, tests/safetensors_test.cpp:36-98). Host code
 * only: no device is needed to open, list or read.
 * ------------------------------------------------------------------------------------------------------------ */

typedef struct mk_st mk_st;
#define MK_ST_MAX_DIMS 8
typedef struct mk_st_tensor {
    const char* name;         /* valid until mk_st_close */
    const char* dtype_name;   /* the header's dtype string: "BF16", "F32", "F8_E4M3", ... */
    uint32_t dtype;           /* mk_dtype (MK_DTYPE_OTHER for the rest) */
    uint32_t ndim;
    uint64_t dims[MK_ST_MAX_DIMS]; /* GGUF order: dims[0] is the contiguous axis (the header's shape reversed) */
    uint32_t file;            /* index of the file that holds it (mk_st_file_path) */
    uint64_t offset;          /* absolute byte offset of its data in that file */
    uint64_t bytes;
} mk_st_tensor;

/* path: one .safetensors file, or a directory whose *.safetensors files (sorted by name) form one checkpoint. The
 * headers are validated against the files (offsets, sizes, dtypes, duplicate names): MK_ERR_ARG names the problem. */
mk_status mk_st_open(const char* path, mk_st** out);
mk_status mk_st_close(mk_st* st);
mk_status mk_st_count(const mk_st* st, size_t* tensors, uint32_t* files);
const char* mk_st_file_path(const mk_st* st, uint32_t file); /* NULL when out of range */
mk_status mk_st_at(const mk_st* st, size_t i, mk_st_tensor* t);          /* in file order, then header order */
mk_status mk_st_find(const mk_st* st, const char* name, mk_st_tensor* t); /* MK_ERR_ARG when absent */
/* The tensor's raw bytes; `bytes` must equal its size. */
mk_status mk_st_read(const mk_st* st, const char* name, void* dst, size_t bytes);

/* ------------------------------------------------------------------------------------------------------------
 * Engine: the denoiser of one model family, weights resident on the device.
 * ------------------------------------------------------------------------------------------------------------ */

enum mk_family {
    MK_FAMILY_DUAL = 0,  /* Qwen-Image (v1)-shaped dual-stream MMDiT (text and image weight sets, shift/scale/gate
                            adaLN, GELU-tanh FFN, non-causal joint attention) */
    MK_FAMILY_Q21 = 1,   /* Qwen-Image 2.1 as the reference runs it (qwen_image.cpp): one weight set, scale + tanh
                            gate, SwiGLU, causal text prefix, text K/V cached after the first step */
    MK_FAMILY_SDXL = 2   /* SDXL spatial transformer (sdxl.cpp:742-796) */
};

typedef struct mk_config {
    uint32_t family;     /* mk_family */
    uint32_t blocks;
    uint32_t dim;        /* hidden width (SDXL: channels) */
    uint32_t heads;
    uint32_t head_dim;   /* 128 (SDXL: 64) */
    uint32_t ffn;        /* FFN inner width (SwiGLU / GEGLU inner) */
    uint32_t text_dim;   /* prompt embedding width */
    uint32_t latent;     /* token latent width (64) */
    uint32_t weight_dtype; /* MK_BF16 or MK_FP8_E4M3 for the block linears; MK_SDXL also MK_F16: the matrices
                              Sdxl::load_trans reads through Engine::matrix (proj_in, proj_out, to_out, attn2.to_q, ff)
                              are kept half, as that keeps an F16 checkpoint's (engine.cpp:292-302, sdxl.cpp:267-306),
                              and their GEMMs take half inputs; q|k|v and the context's k|v stay bf16 */
    uint32_t max_batch;  /* 1 or 2 (CFG) */
} mk_config;

typedef struct mk_engine mk_engine;

mk_status mk_engine_create(const mk_config* cfg, mk_engine** out);
mk_status mk_engine_destroy(mk_engine* e);
/* Upload one named weight (the reference's upload / upload_rows, qwen_image.cpp:79-111): `data` holds rows x cols
 * values of `dtype` (fp32 vectors, bf16 matrices, e4m3 matrices; an fp8 matrix's scale is the fp32 tensor
 * name + ".scale"). Names are the checkpoint's (Diffusers layout). */
mk_status mk_engine_load(mk_engine* e, const char* name, const void* data, uint32_t dtype, uint64_t rows,
                         uint64_t cols);
/* Every weight of the engine from a safetensors checkpoint (file or shard directory; QwenImage::load_transformer,
 * src/image/qwen_image.cpp:79-111): each tensor by its checkpoint name (Diffusers layout, also found under a
 * "model.diffusion_model." or "transformer." prefix), streamed from the file through pinned host buffers into its
 * place in the fused device tensors (upload_rows). Matrices are [out][in] (dims {in, out} in GGUF order), vectors
 * [n]. Conversions: F32 / F16 / BF16 to what the engine stores (nearest even); into fp8 weights by the per-row rule
 * of mk_quantize_fp8_rows after rounding to bf16, or F8_E4M3 as stored with its per-row fp32 scale named
 * name + ".scale". A missing tensor, a wrong shape or a checkpoint with more blocks than the engine is MK_ERR_ARG
 * (the reference throws); other tensors in the files are ignored. `loaded` (may be NULL): tensors read. */
mk_status mk_engine_load_safetensors(mk_engine* e, const char* path, uint64_t* loaded);
/* mk_engine_load_safetensors with each name looked up under `prefix` first (NULL or "": none), then under the default
 * prefixes: an SDXL spatial transformer inside a whole UNet checkpoint, as Sdxl::load_trans reads it under
 * kUnet + its path (sdxl.cpp:264-306), e.g. prefix "model.diffusion_model.input_blocks.4.1." finds
 * "...input_blocks.4.1.transformer_blocks.0.attn1.to_q.weight"; the block-count check then counts the blocks under
 * the prefix only. */
mk_status mk_engine_load_safetensors_at(mk_engine* e, const char* path, const char* prefix, uint64_t* loaded);
/* Merge a LoRA file into the weights for good (the reference's add_lora with merging, engine.hpp:195-197; targets as
 * QwenImage::lora_target gives them, qwen_image.cpp:295-331: a module's rows inside the fused tensor that holds it).
 * Pairs <module>.lora_A.weight / .lora_B.weight or .lora_down.weight / .lora_up.weight, with an optional scalar
 * <module>.alpha: W += scale * (alpha / rank) * B A (alpha absent: scale * B A). Module names are checkpoint names,
 * optionally prefixed "transformer.", "diffusion_model.", "base_model.model." or written Kohya-style
 * ("lora_unet_transformer_blocks_0_attn_to_q": '_' and '.' alike). A pair whose shapes do not match its module is
 * MK_ERR_ARG and nothing is merged; a module with parts beyond the pair and alpha (DoRA magnitudes, bias diffs) is
 * MK_ERR_UNSUPPORTED; modules that name no weight of the engine (text encoders, full-weight diffs) are skipped.
 * `merged` / `skipped` (may be NULL): module counts. */
mk_status mk_engine_add_lora(mk_engine* e, const char* path, float scale, uint64_t* merged, uint64_t* skipped);
/* The engine's weights in name order: checkpoint name, stored dtype, rows and cols (vectors: cols = 1). The name
 * stays valid while the engine lives. */
mk_status mk_engine_tensor_count(const mk_engine* e, size_t* n);
mk_status mk_engine_tensor_at(const mk_engine* e, size_t i, const char** name, uint32_t* dtype, uint64_t* rows,
                              uint64_t* cols);
/* Copy one named weight back to the host as stored: bytes = rows x cols x element size (name + ".scale": the fp32
 * per-row scales of an fp8 matrix). */
mk_status mk_engine_fetch(const mk_engine* e, const char* name, void* data, size_t bytes);
/* Every weight from the counter RNG on the device: matrices N(0, 0.02), biases N(0, 0.02), norm scales 1 + N(0, 0.02),
 * keyed by (seed, name) exactly as the CPU reference keys them. */
mk_status mk_engine_init_random(mk_engine* e, uint64_t seed);
/* Bytes of device memory the weights hold. */
mk_status mk_engine_weight_bytes(const mk_engine* e, uint64_t* bytes);

/* begin (engine.hpp:165): prompt [rows][text_dim] fp32 for a grid of h x w tokens; slot 0 or 1. */
mk_status mk_begin(mk_engine* e, const float* prompt, size_t rows, uint32_t h, uint32_t w, uint32_t slot);
/* step (engine.hpp:166): latents [h*w][latent] fp32 -> velocity [h*w][latent] fp32. */
mk_status mk_step(mk_engine* e, const float* latents, size_t n, float sigma, uint32_t slot, float* out);
/* Classifier-free guidance as one batch of 2 (slot 0 positive, slot 1 negative, both begun), then the Euler update:
 * latents_out = latents + (sigma_next - sigma) (neg + guidance (pos - neg)). Host buffers. */
mk_status mk_step_cfg(mk_engine* e, const float* latents, size_t n, float sigma, float sigma_next, float guidance,
                      float* latents_out);
/* The same on device buffers already resident (no host copies): lat and lat_out [h*w][latent] fp32 device pointers
 * (may alias). The bench times this. */
mk_status mk_step_cfg_device(mk_engine* e, const float* lat, float sigma, float sigma_next, float guidance,
                             float* lat_out, void* stream);
/* The step's stream (kernels are launched on it). */
mk_status mk_engine_stream(mk_engine* e, void** stream);

/* The noise schedule of Engine::sigmas (engine.cpp:335-365; Schedule defaults engine.hpp:251-254): mu = the fixed
 * shift when has_mu, else linear in the token count from (base_seq, base_shift) to (max_seq, max_shift). */
typedef struct mk_schedule {
    double base_seq, max_seq, base_shift, max_shift, terminal;
    int has_mu;
    double mu;
} mk_schedule;
/* sigmas of `steps` steps for an image of `tokens` tokens, then 0: out[steps + 1]. t = linspace(1, 1/steps) in float,
 * sigma = e^mu / (e^mu + 1/t - 1) in double rounded to float, stretched so the last is `terminal` when terminal > 0.
 * sched NULL: the defaults (256, 4096, 0.5, 1.15, terminal 0, no fixed mu). Host arithmetic only. */
mk_status mk_sigmas(uint32_t steps, uint32_t tokens, const mk_schedule* sched, float* out);
/* The Euler flow-matching loop of Engine::generate (engine.cpp:459-506) with the latents resident on the device:
 * x = noise [h*w][latent] fp32 (host); for i < steps: v = step(x, sigmas[i]) guided as neg + guidance (pos - neg)
 * (slot 1 the negative prompt; no negative pass when guidance == 1), x += (sigmas[i+1] - sigmas[i]) v; the final
 * latents are copied to latents_out (host). Slot 0 (and slot 1 when guidance != 1) must have been begun. */
mk_status mk_generate(mk_engine* e, const float* noise, size_t n, const float* sigmas, uint32_t steps, float guidance,
                      float* latents_out);
/* The start noise Engine::generate draws when a request brings none (engine.cpp:398-408): out[i] =
 * std::normal_distribution<float>{}(rng) in order over std::mt19937_64 rng(seed). Host arithmetic only. The engine
 * is fixed by the C++ standard; the normal distribution's algorithm is the C++ library's, so the values equal the
 * reference's where both are built against the same standard library (this build: libstdc++). */
mk_status mk_noise(uint64_t seed, float* out, size_t n);

/* Probe of intermediates (the reference's set_probe, tests/image_ref_test.cpp:133-136): called synchronously on the
 * host after a stage with its name ("temb", "modulation", "txt_in", "img_in", "block", "norm_out"), its layer
 * (-1 none), the data copied to host fp32 and its length. NULL turns it off. Slows the step (synchronises). */
typedef void (*mk_probe_fn)(void* user, const char* name, int layer, const float* data, size_t n);
mk_status mk_engine_set_probe(mk_engine* e, mk_probe_fn fn, void* user);
/* VAE probes: "vae_conv_in", "vae_mid", "vae_up" (layer = up block), "vae_out" (before the clamp), [pixels][channels] */
mk_status mk_vae_set_probe(mk_vae* v, mk_probe_fn fn, void* user);

/* Per-kernel timing of the last step with events on the step's stream (enable before the step): names and total
 * milliseconds per kernel class ("gemm", "attention", ...). */
mk_status mk_engine_set_timing(mk_engine* e, int on);
mk_status mk_engine_timing(mk_engine* e, uint32_t i, const char** name, float* ms, uint32_t* launches, double* flops);

/* SDXL spatial transformer (config: MK_FAMILY_SDXL): x [batch][n][c] fp32 device -> y [batch][n][c] fp32 device,
 * cross-attending to the context of mk_begin (slot 0 for batch row 0, slot 1 for row 1). */
mk_status mk_sdxl_forward(mk_engine* e, const float* x, uint32_t batch, uint32_t n, float* y, void* stream);

#ifdef __cplusplus
}
#endif
#endif
