/* mkref — CPU restatement of mako-image's denoising hot path.
 *
 * TEST INFRASTRUCTURE ONLY. The HIP path's results are compared against this library: tests/, the smoke() of
 * __graft_entry__.py and bench.py's cpu_baseline leg load it, nothing else. The product library
 * (mako-image_amd/libmkimage.so) never links, loads or calls it.
 *
 * Arithmetic model (mirrors the reference: bf16 storage, fp32 accumulation, fp32 residual stream):
 *  - matrix weights hold bf16 values (or OCP fp8-e4m3 values with a per-output-channel fp32 scale; or, for the SDXL
 *    matrices Engine::matrix keeps F16 when the checkpoint's are, engine.cpp:292-302 and sdxl.cpp:267-306, half);
 *  - every GEMM rounds its activation operand to bf16 (half for half weights: both matrix-core operands take one
 *    type) with round-to-nearest-even, accumulates in fp32;
 *  - attention operands Q, K, V are rounded to bf16 in the dual-stream graph, and to IEEE half in the reference's own
 *    graphs (Qwen-Image 2.1 and SDXL, whose heads kernels write `half`: qwen_image.cpp:165-167, 226-250,
 *    sdxl.cpp:439-448), the 2.1 graph's cached text keys / values with them; the softmax is fp32;
 *  - norms reduce in double (more exact than any kernel), elementwise math is fp32.
 *
 * Parity unpinned: the reference's GEMM / attention / heads kernels live in an un-vendored submodule
 * (external/mako-common, no source or pinned commit in the tree) and the reference holds no vectors for this path,
 * so these choices are inferred, not pinned to the reference: the GEMM's bf16 rounding of its activation operand;
 * RoPE mode 2 as interleaved pairs (2i, 2i+1); the causal-prefix rule of attention(block = S); the textbook
 * gelu_tanh and swiglu forms; the precision of P in P V (fp32 here; a kernel may round it to the operands' type
 * within the tolerance). Everything else is pinned by tests/test_oracle.py and
 * tests/test_oracle_graph.py (library routines in float64, closed forms, invariants).
 *
 * Reference files restated (see each function in mkref.cpp for its file:line):
 *   src/image/qwen_image.cpp, src/kernels/image.metal:9-65,450-484, src/image/engine.cpp:335-365,459-506,
 *   src/image/sdxl.cpp:68-87,425-457,672-796; the VAE decoder src/image/engine.cpp:589-628,722-777,862-954 (pinned
 *   by tests/test_oracle_graph.py against torch's conv2d / interpolate / softmax).
 */
#ifndef MKREF_H
#define MKREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---- */
uint16_t mkref_f32_to_bf16(float x);
float mkref_bf16_to_f32(uint16_t b);
void mkref_round_bf16(float* x, size_t n);
void mkref_round_f16(float* x, size_t n); /* IEEE half, nearest even */
uint8_t mkref_f32_to_e4m3(float x);
float mkref_e4m3_to_f32(uint8_t b);

/* ---- counter RNG: value i of the tensor `name` under `seed`, N(mean, std) ---- */
uint64_t mkref_tensor_key(uint64_t seed, const char* name);
void mkref_fill_normal(float* out, size_t n, uint64_t key, double mean, double std, int round_bf16);

/* ---- primitives ---- */
/* C[m][n] = (sum_k bf16(A[m][k]) * W[n][k]) * (wscale ? wscale[n] : 1) + (bias ? bias[n] : 0) */
void mkref_gemm(const float* A, int64_t lda, int64_t M, int64_t K, const float* W, int64_t N, const float* wscale,
                const float* bias, float* C, int64_t ldc);
/* y = LN(x) * (1 + scale) + shift, no affine (shift may be NULL) */
void mkref_ln_modulate(const float* x, int64_t rows, int64_t n, const float* shift, const float* scale, float eps,
                       float* y);
/* y = LN(x) * g + b */
void mkref_layer_norm(const float* x, int64_t rows, int64_t n, const float* g, const float* b, float eps, float* y);
/* y = x * rsqrt(mean(x^2) + eps) * w */
void mkref_rms_norm(const float* x, int64_t rows, int64_t n, const float* w, float eps, float* y);
/* channels-last group norm over [rows][c], `groups` groups of c / groups channels, affine g, b */
void mkref_group_norm(const float* x, int64_t rows, int64_t c, int64_t groups, const float* g, const float* b,
                      float eps, float* y);
/* rope3 table (qwen_image.cpp:31-45,132-141): cs[(S + h*w)][64][2] */
void mkref_rope_table(float* cs, uint32_t S, uint32_t h, uint32_t w);
/* per (row, head) RMSNorm * w (w may be NULL: no norm), then RoPE (mode 0 none, 1 half-split, 2 interleaved pairs)
 * from cs rows [rows][d/2][2]; out[head][out_row0 + row][d] with out_rows rows per head */
void mkref_heads_norm_rope(const float* x, int64_t rows, int64_t ld, int64_t col0, int64_t heads, int64_t d,
                           const float* w, float eps, const float* cs, int rope, float* out, int64_t out_rows,
                           int64_t out_row0);
/* softmax(q k^T * scale) v for q [B][H][Tq][d], k, v [B][H][Tk][d]; out [B][Tq][H*d].
 * Query row r (absolute q_pos0 + i) sees key c iff r >= block or c <= r. */
void mkref_attention(const float* q, const float* k, const float* v, int64_t B, int64_t H, int64_t Tq, int64_t Tk,
                     int64_t d, float scale, uint32_t q_pos0, uint32_t block, float* out);
void mkref_gelu_tanh(float* x, size_t n);
void mkref_silu(float* x, size_t n);
/* m[r][i] = silu(gu[r][i]) * gu[r][F + i] (gate rows first, qwen_image.cpp:315) */
void mkref_swiglu(const float* gu, int64_t rows, int64_t F, float* m);
/* m[r][i] = hg[r][i] * gelu_erf(hg[r][F + i]) (image.metal:475-484) */
void mkref_geglu(const float* hg, int64_t rows, int64_t F, float* m);
/* 2.1's sinusoid: cos half first, arg = v * exp(-ln(1e4) i / half) (qwen_image.cpp:179-187) */
void mkref_sinusoid(float v, uint32_t dim, float* out);
/* Engine::sigmas (engine.cpp:335-365): steps + 1 values */
void mkref_sigmas(uint32_t steps, uint32_t tokens, double base_seq, double max_seq, double base_shift,
                  double max_shift, double terminal, float* out);
/* 2x2 patchify of a [C][2h][2w] latent into tokens [h*w][C*4] (token feature c*4 + py*2 + px) and back */
void mkref_patchify(const float* lat, uint32_t C, uint32_t h, uint32_t w, float* tokens);
void mkref_unpatchify(const float* tokens, uint32_t C, uint32_t h, uint32_t w, float* lat);

/* ---- models: synthetic weights by name, and their steps ---- */
enum { MKREF_DUAL = 0, MKREF_Q21 = 1, MKREF_SDXL = 2 };
typedef struct mkref_dims {
    uint32_t kind;       /* MKREF_* */
    uint32_t blocks;
    uint32_t dim;        /* hidden width (SDXL: channels) */
    uint32_t heads;
    uint32_t head_dim;   /* 128 (SDXL 64) */
    uint32_t ffn;        /* FFN inner width (SDXL: GEGLU inner) */
    uint32_t text_dim;   /* prompt width */
    uint32_t latent;     /* 64 */
    uint32_t fp8;        /* block linears stored fp8-e4m3 with per-row scales */
    uint32_t f16;        /* SDXL: the matrices Engine::matrix keeps F16 are half, their GEMMs take half inputs */
} mkref_dims;
typedef struct mkref_model mkref_model;
/* weights N(0, wstd) (biases too), norm scales 1 + N(0, wstd); wstd 0.02 is the synthetic checkpoint's */
mkref_model* mkref_model_create(const mkref_dims* dims, uint64_t seed, double wstd);
void mkref_model_destroy(mkref_model* m);
size_t mkref_model_count(const mkref_model* m);
/* tensor i: its name, its fp32 values (bf16-, e4m3- or half-exact for matrices), rows x cols, and kind
 * (0 fp32 vector, 1 bf16 matrix, 2 fp8 matrix whose scale is the tensor named name + ".scale", 3 half matrix) */
const char* mkref_model_name(const mkref_model* m, size_t i);
const float* mkref_model_tensor(const mkref_model* m, size_t i, int64_t* rows, int64_t* cols, int* kind);
int64_t mkref_model_find(const mkref_model* m, const char* name);

/* Probe: called with a stage name ("temb", "modulation", "txt_in", "img_in", "block", "norm_out"), a layer (-1 none),
 * the data and its element count. */
typedef void (*mkref_probe_fn)(void* user, const char* name, int layer, const float* data, size_t n);

/* Dual-stream step for B samples sharing sigma: prompt [B][S][text_dim], latents [B][N][latent], out [B][N][latent].
 * The grid is h x w tokens (N = h*w). */
int mkref_dual_step(const mkref_model* m, int64_t B, const float* prompt, int64_t S, const float* latents, uint32_t h,
                    uint32_t w, float sigma, float* out, mkref_probe_fn probe, void* user);
/* Qwen-Image 2.1 step (qwen_image.cpp:144-293) over the whole sequence [text; image], one sample. */
int mkref_q21_step(const mkref_model* m, const float* prompt, int64_t S, const float* latents, uint32_t h, uint32_t w,
                   float sigma, float* out, mkref_probe_fn probe, void* user);
/* SDXL spatial transformer (sdxl.cpp:742-796) for one sample: x [n][c] -> y [n][c], context [S][text_dim]. */
int mkref_sdxl_trans(const mkref_model* m, const float* x, int64_t n, const float* ctx, int64_t S, float* y);
/* One block of the dual-stream step for one sample with inputs given (for timing a bounded sample):
 * img [N][D], txt [S][D] updated in place; mod rows img/txt [6][D]; cs [S+N][64][2]. */
int mkref_dual_block(const mkref_model* m, int block, float* img, int64_t N, float* txt, int64_t S,
                     const float* mod_img, const float* mod_txt, const float* cs);

/* ---- VAE decoder (Qwen-Image's Wan-2.1-layout decoder as src/image/engine.cpp:589-628, 722-760, 862-954 runs it, one
 * frame): tokens [h][w][4 z] -> RGBA [16 h][16 w][4] in [-1, 1], alpha 1. Channels base x {4, 4, 4, 2, 1} per level
 * (decoder dims 4b, then up blocks 4b -> 4b, 2b -> 4b, 2b -> 2b, b -> b, each 3 residual blocks, the first three
 * followed by a nearest 2x upsample and a 3x3 conv to half the channels), RMS norms over channels, one-head attention
 * in the middle block. Weights by checkpoint name from the counter RNG (PyTorch layout [out][in][k][k]): convs
 * N(0, 1 / fan_in) as bf16, biases N(0, 0.02), norm gammas 1 + N(0, 0.1). ---- */
typedef struct mkref_vae mkref_vae;
mkref_vae* mkref_vae_create(uint32_t base, uint32_t z, uint64_t seed, const float* mean, const float* std);
void mkref_vae_destroy(mkref_vae* v);
size_t mkref_vae_count(const mkref_vae* v);
const char* mkref_vae_name(const mkref_vae* v, size_t i);
/* tensor i's values and dims (PyTorch order: [out][in][k][k] for convs, [n] otherwise) */
const float* mkref_vae_tensor(const mkref_vae* v, size_t i, uint32_t* ndim, int64_t* dims);
/* probes: "vae_conv_in", "vae_mid", "vae_up" (layer = up block) as [pixels][channels], "vae_out" before the clamp */
int mkref_vae_decode(const mkref_vae* v, const float* tokens, uint32_t h, uint32_t w, float* rgba,
                     mkref_probe_fn probe, void* user);

int mkref_threads(void);

#ifdef __cplusplus
}
#endif
#endif
