// mkref — CPU restatement of mako-image's denoising hot path. TEST INFRASTRUCTURE ONLY (the tests compare the HIP
// path against it; the product library never links or calls it). Arithmetic model and scope: mkref.h.
#include "mkref.h"

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

// ---------------------------------------------------------------------------------------------------------------
// Number formats
// ---------------------------------------------------------------------------------------------------------------

inline uint32_t bits(float x)
{
    uint32_t u;
    std::memcpy(&u, &x, 4);
    return u;
}
inline float from_bits(uint32_t u)
{
    float x;
    std::memcpy(&x, &u, 4);
    return x;
}

// Round-to-nearest-even to bfloat16 (NaN kept quiet).
inline uint16_t to_bf16(float x)
{
    uint32_t u = bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return uint16_t((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}
inline float bf16(float x) { return from_bits(uint32_t(to_bf16(x)) << 16); }

// Round-to-nearest-even to IEEE binary16 (`half`, the reference's heads and attention precision: heads_norm_half /
// heads_half, qwen_image.cpp:165-167, 226-250, sdxl.cpp:439-448), as the float it stands for: 11 significant bits,
// subnormals below 2^-14 on the grid of 2^-24, overflow (at or past the midpoint 65520) to infinity, NaN kept.
inline float f16(float x)
{
    if (std::isnan(x))
        return x;
    const float a = std::fabs(x);
    if (a >= 65520.0f)
        return std::copysign(INFINITY, x);
    int e;
    std::frexp(a, &e);                       // a = f 2^e, f in [0.5, 1): binade 2^(e - 1)
    const int b = std::max(e - 1, -14);      // subnormals share the step of binade -14
    const float step = std::ldexp(1.0f, b - 10);
    return std::copysign(std::nearbyint(a / step) * step, x); // exact scaling; ties to even in the default mode
}

// OCP fp8 e4m3 ("fn"): bias 7, no infinities, 0x7f / 0xff NaN, max 448; saturating round-to-nearest-even.
inline float e4m3_decode(uint8_t b)
{
    const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7)
        v = NAN;
    else if (e == 0)
        v = std::ldexp(float(m), -9); // subnormal: m / 8 * 2^-6
    else
        v = std::ldexp(1.0f + float(m) / 8.0f, e - 7);
    return s ? -v : v;
}
uint8_t e4m3_encode(float x)
{
    if (std::isnan(x))
        return 0x7f;
    const uint8_t sign = std::signbit(x) ? 0x80 : 0;
    float a = std::fabs(x);
    if (a >= 448.0f)
        return sign | 0x7e;
    // Exhaustive nearest among the 127 finite magnitudes, ties to the even code: exact and simple.
    int best = 0;
    float bd = INFINITY;
    for (int c = 0; c <= 0x7e; ++c) {
        const float d = std::fabs(e4m3_decode(uint8_t(c)) - a);
        if (d < bd || (d == bd && (c & 1) == 0 && (best & 1))) {
            bd = d;
            best = c;
        }
    }
    return sign | uint8_t(best);
}

// ---------------------------------------------------------------------------------------------------------------
// Counter RNG: splitmix64 of (key + counter); Box-Muller in double.
// ---------------------------------------------------------------------------------------------------------------

inline uint64_t splitmix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

inline double normal_at(uint64_t key, uint64_t i)
{
    const uint64_t a = splitmix64(key + 2 * i), b = splitmix64(key + 2 * i + 1);
    const double u1 = (double((a >> 11) + 1)) * 0x1.0p-53; // (0, 1]
    const double u2 = double(b >> 11) * 0x1.0p-53;         // [0, 1)
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// ---------------------------------------------------------------------------------------------------------------
// GEMM: C = r(A) W^T (* scale) + bias with r = bf16 rounding (half rounding for half weights), blocked for the
// cache, OpenMP over 64x64 tiles.
// ---------------------------------------------------------------------------------------------------------------

typedef float v8 __attribute__((vector_size(32)));

void gemm(const float* A, int64_t lda, int64_t M, int64_t K, const float* W, int64_t N, const float* wscale,
          const float* bias, float* C, int64_t ldc, bool half_a = false)
{
    if (M <= 0 || N <= 0)
        return;
    const int64_t NS = (N + 15) / 16;
    // W packed into strips of 16 output columns, [strip][K][16], zero past N.
    std::vector<float> Wp(size_t(NS) * K * 16, 0.0f);
#pragma omp parallel for schedule(static)
    for (int64_t s = 0; s < NS; ++s)
        for (int64_t c = 0; c < 16; ++c) {
            const int64_t n = s * 16 + c;
            if (n >= N)
                continue;
            for (int64_t k = 0; k < K; ++k)
                Wp[(size_t(s) * K + k) * 16 + c] = W[size_t(n) * K + k];
        }
    // A rounded to bf16 (the GEMM's activation operand; half for half weights: the matrix-core operands share a
    // type), rows padded to a multiple of 4.
    const int64_t Mp = (M + 3) / 4 * 4;
    std::vector<float> Ap(size_t(Mp) * K, 0.0f);
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k)
            Ap[size_t(m) * K + k] = half_a ? f16(A[size_t(m) * lda + k]) : bf16(A[size_t(m) * lda + k]);
    const int64_t TM = 64, TS = 4, KC = 512; // 64 rows x 4 strips (64 columns) per task, K in chunks
    const int64_t mt = (Mp + TM - 1) / TM, st = (NS + TS - 1) / TS;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int64_t bm = 0; bm < mt; ++bm)
        for (int64_t bs = 0; bs < st; ++bs) {
            const int64_t m0 = bm * TM, m1 = std::min(Mp, m0 + TM);
            const int64_t s0 = bs * TS, s1 = std::min(NS, s0 + TS);
            float acc[64][64];
            std::memset(acc, 0, sizeof(acc));
            for (int64_t k0 = 0; k0 < K; k0 += KC) {
                const int64_t k1 = std::min(K, k0 + KC);
                for (int64_t s = s0; s < s1; ++s) {
                    const float* ws = Wp.data() + size_t(s) * K * 16;
                    for (int64_t m = m0; m < m1; m += 4) {
                        v8 c00 = {}, c01 = {}, c10 = {}, c11 = {}, c20 = {}, c21 = {}, c30 = {}, c31 = {};
                        const float* a0 = Ap.data() + size_t(m) * K;
                        const float* a1 = a0 + K;
                        const float* a2 = a1 + K;
                        const float* a3 = a2 + K;
                        for (int64_t k = k0; k < k1; ++k) {
                            v8 w0, w1;
                            std::memcpy(&w0, ws + k * 16, 32);
                            std::memcpy(&w1, ws + k * 16 + 8, 32);
                            const float x0 = a0[k], x1 = a1[k], x2 = a2[k], x3 = a3[k];
                            c00 += x0 * w0;
                            c01 += x0 * w1;
                            c10 += x1 * w0;
                            c11 += x1 * w1;
                            c20 += x2 * w0;
                            c21 += x2 * w1;
                            c30 += x3 * w0;
                            c31 += x3 * w1;
                        }
                        float* r = &acc[m - m0][(s - s0) * 16];
                        for (int j = 0; j < 8; ++j) {
                            r[j] += c00[j];
                            r[8 + j] += c01[j];
                            r[64 + j] += c10[j];
                            r[72 + j] += c11[j];
                            r[128 + j] += c20[j];
                            r[136 + j] += c21[j];
                            r[192 + j] += c30[j];
                            r[200 + j] += c31[j];
                        }
                    }
                }
            }
            for (int64_t m = m0; m < std::min(M, m1); ++m)
                for (int64_t s = s0; s < s1; ++s)
                    for (int64_t c = 0; c < 16; ++c) {
                        const int64_t n = s * 16 + c;
                        if (n >= N)
                            continue;
                        float v = acc[m - m0][(s - s0) * 16 + c];
                        if (wscale)
                            v *= wscale[n];
                        if (bias)
                            v += bias[n];
                        C[size_t(m) * ldc + n] = v;
                    }
        }
}

// ---------------------------------------------------------------------------------------------------------------
// Norms and elementwise
// ---------------------------------------------------------------------------------------------------------------

// image.metal:32-53 (ln_modulate), with the dual-stream shift: y = (x - mean) * rsqrt(var + eps) * (1 + scale) + shift.
void ln_modulate(const float* x, int64_t rows, int64_t n, const float* shift, const float* scale, float eps, float* y)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + size_t(r) * n;
        float* yr = y + size_t(r) * n;
        double s = 0;
        for (int64_t i = 0; i < n; ++i)
            s += xr[i];
        const double mean = s / double(n);
        double v = 0;
        for (int64_t i = 0; i < n; ++i)
            v += (xr[i] - mean) * (xr[i] - mean);
        const float inv = float(1.0 / std::sqrt(v / double(n) + double(eps)));
        const float mf = float(mean);
        for (int64_t i = 0; i < n; ++i)
            yr[i] = (xr[i] - mf) * inv * (1.0f + scale[i]) + (shift ? shift[i] : 0.0f);
    }
}

void layer_norm(const float* x, int64_t rows, int64_t n, const float* g, const float* b, float eps, float* y)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + size_t(r) * n;
        float* yr = y + size_t(r) * n;
        double s = 0;
        for (int64_t i = 0; i < n; ++i)
            s += xr[i];
        const double mean = s / double(n);
        double v = 0;
        for (int64_t i = 0; i < n; ++i)
            v += (xr[i] - mean) * (xr[i] - mean);
        const float inv = float(1.0 / std::sqrt(v / double(n) + double(eps)));
        const float mf = float(mean);
        for (int64_t i = 0; i < n; ++i)
            yr[i] = (xr[i] - mf) * inv * g[i] + b[i];
    }
}

void rms_norm(const float* x, int64_t rows, int64_t n, const float* w, float eps, float* y)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + size_t(r) * n;
        float* yr = y + size_t(r) * n;
        double s = 0;
        for (int64_t i = 0; i < n; ++i)
            s += double(xr[i]) * xr[i];
        const float inv = float(1.0 / std::sqrt(s / double(n) + double(eps)));
        for (int64_t i = 0; i < n; ++i)
            yr[i] = xr[i] * inv * (w ? w[i] : 1.0f);
    }
}

void group_norm(const float* x, int64_t rows, int64_t c, int64_t groups, const float* g, const float* b, float eps,
                float* y)
{
    const int64_t cg = c / groups;
#pragma omp parallel for schedule(static)
    for (int64_t gi = 0; gi < groups; ++gi) {
        double s = 0;
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t i = 0; i < cg; ++i)
                s += x[size_t(r) * c + gi * cg + i];
        const double cnt = double(rows) * double(cg), mean = s / cnt;
        double v = 0;
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t i = 0; i < cg; ++i) {
                const double d = x[size_t(r) * c + gi * cg + i] - mean;
                v += d * d;
            }
        const float inv = float(1.0 / std::sqrt(v / cnt + double(eps))), mf = float(mean);
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t i = 0; i < cg; ++i) {
                const int64_t ch = gi * cg + i;
                y[size_t(r) * c + ch] = (x[size_t(r) * c + ch] - mf) * inv * g[ch] + b[ch];
            }
    }
}

// qwen_image.cpp:31-45: pairs of the (frame, height, width) axes, 8 / 28 / 28 of the 64, theta 10000.
void rope3(float* cs, int64_t f, int64_t hpos, int64_t wpos)
{
    const int dims[3] = {16, 56, 56};
    const int64_t pos[3] = {f, hpos, wpos};
    int i = 0;
    for (int a = 0; a < 3; ++a)
        for (int j = 0; j < dims[a] / 2; ++j, ++i) {
            const float inv = 1.0f / std::pow(10000.0f, float(2 * j) / float(dims[a]));
            const float ang = float(pos[a]) * inv;
            cs[2 * i] = std::cos(ang);
            cs[2 * i + 1] = std::sin(ang);
        }
}

// qwen_image.cpp:132-141: the text along all three axes at (t, t, t), the image at frame S with a height / width
// grid centred on zero.
void rope_table(float* cs, uint32_t S, uint32_t h, uint32_t w)
{
    for (uint32_t t = 0; t < S; ++t)
        rope3(cs + size_t(t) * 128, t, t, t);
    for (uint32_t y = 0; y < h; ++y)
        for (uint32_t x = 0; x < w; ++x)
            rope3(cs + size_t(S + y * w + x) * 128, S, int64_t(y) - int64_t(h - h / 2), int64_t(x) - int64_t(w - w / 2));
}

// The heads' norm and rotation (heads_norm_half, called at qwen_image.cpp:226-242): per (row, head) RMSNorm * w, then
// the pairs rotated by the table row's angle: mode 2 pairs (2p, 2p+1), mode 1 pairs (p, p + d/2).
void heads_norm_rope(const float* x, int64_t rows, int64_t ld, int64_t col0, int64_t heads, int64_t d, const float* w,
                     float eps, const float* cs, int rope, float* out, int64_t out_rows, int64_t out_row0)
{
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t hd = 0; hd < heads; ++hd) {
            float v[256];
            const float* xr = x + size_t(r) * ld + col0 + hd * d;
            for (int64_t i = 0; i < d; ++i)
                v[i] = xr[i];
            if (w) {
                double s = 0;
                for (int64_t i = 0; i < d; ++i)
                    s += double(v[i]) * v[i];
                const float inv = float(1.0 / std::sqrt(s / double(d) + double(eps)));
                for (int64_t i = 0; i < d; ++i)
                    v[i] = v[i] * inv * w[i];
            }
            if (rope) {
                const float* c = cs + size_t(r) * d; // d/2 pairs of (cos, sin)
                for (int64_t p = 0; p < d / 2; ++p) {
                    const int64_t i0 = rope == 2 ? 2 * p : p, i1 = rope == 2 ? 2 * p + 1 : p + d / 2;
                    const float a = v[i0], b = v[i1], co = c[2 * p], si = c[2 * p + 1];
                    v[i0] = a * co - b * si;
                    v[i1] = a * si + b * co;
                }
            }
            float* o = out + (size_t(hd) * out_rows + out_row0 + r) * d;
            for (int64_t i = 0; i < d; ++i)
                o[i] = v[i];
        }
}

// Joint attention: softmax(q k^T scale) v, fp32 softmax, with the causal prefix of `block` rows.
void attention(const float* q, const float* k, const float* v, int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t d,
               float scale, uint32_t q_pos0, uint32_t block, float* out)
{
#pragma omp parallel for collapse(3) schedule(dynamic, 16)
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t i = 0; i < Tq; ++i) {
                const float* qi = q + ((size_t(b) * H + h) * Tq + i) * d;
                const float* kb = k + (size_t(b) * H + h) * Tk * d;
                const float* vb = v + (size_t(b) * H + h) * Tk * d;
                const int64_t r = int64_t(q_pos0) + i;
                const int64_t nk = r >= int64_t(block) ? Tk : std::min(Tk, r + 1);
                std::vector<float> s(size_t(std::max<int64_t>(nk, 1)));
                float mx = -INFINITY;
                for (int64_t j = 0; j < nk; ++j) {
                    float a = 0;
                    for (int64_t t = 0; t < d; ++t)
                        a += qi[t] * kb[size_t(j) * d + t];
                    s[j] = a * scale;
                    mx = std::max(mx, s[j]);
                }
                float sum = 0;
                for (int64_t j = 0; j < nk; ++j) {
                    s[j] = std::exp(s[j] - mx);
                    sum += s[j];
                }
                float acc[256] = {};
                for (int64_t j = 0; j < nk; ++j)
                    for (int64_t t = 0; t < d; ++t)
                        acc[t] += s[j] * vb[size_t(j) * d + t];
                float* o = out + (size_t(b) * Tq + i) * H * d + h * d;
                for (int64_t t = 0; t < d; ++t)
                    o[t] = nk ? acc[t] / sum : 0.0f;
            }
}

inline float gelu_tanh1(float x)
{
    return 0.5f * x * (1.0f + std::tanh(0.7978845608028654f * (x + 0.044715f * x * x * x)));
}
inline float silu1(float x) { return x / (1.0f + std::exp(-x)); }

void sinusoid(float v, uint32_t dim, float* out)
{
    const uint32_t half = dim / 2;
    for (uint32_t i = 0; i < half; ++i) {
        const float f = std::exp(-std::log(10000.0f) * float(i) / float(half));
        out[i] = std::cos(v * f);
        out[half + i] = std::sin(v * f);
    }
}

} // namespace

// ---------------------------------------------------------------------------------------------------------------
// C API: formats, RNG, primitives
// ---------------------------------------------------------------------------------------------------------------

extern "C" {

uint16_t mkref_f32_to_bf16(float x) { return to_bf16(x); }
float mkref_bf16_to_f32(uint16_t b) { return from_bits(uint32_t(b) << 16); }
void mkref_round_bf16(float* x, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        x[i] = bf16(x[i]);
}
void mkref_round_f16(float* x, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        x[i] = f16(x[i]);
}
uint8_t mkref_f32_to_e4m3(float x) { return e4m3_encode(x); }
float mkref_e4m3_to_f32(uint8_t b) { return e4m3_decode(b); }

// FNV-1a of the name, mixed with the seed.
uint64_t mkref_tensor_key(uint64_t seed, const char* name)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (const char* p = name; *p; ++p)
        h = (h ^ uint8_t(*p)) * 0x100000001b3ull;
    return splitmix64(h ^ splitmix64(seed));
}

void mkref_fill_normal(float* out, size_t n, uint64_t key, double mean, double std, int round_bf16)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(n); ++i) {
        const float v = float(mean + std * normal_at(key, uint64_t(i)));
        out[i] = round_bf16 ? bf16(v) : v;
    }
}

void mkref_gemm(const float* A, int64_t lda, int64_t M, int64_t K, const float* W, int64_t N, const float* wscale,
                const float* bias, float* C, int64_t ldc)
{
    gemm(A, lda, M, K, W, N, wscale, bias, C, ldc);
}
void mkref_ln_modulate(const float* x, int64_t rows, int64_t n, const float* shift, const float* scale, float eps,
                       float* y)
{
    ln_modulate(x, rows, n, shift, scale, eps, y);
}
void mkref_layer_norm(const float* x, int64_t rows, int64_t n, const float* g, const float* b, float eps, float* y)
{
    layer_norm(x, rows, n, g, b, eps, y);
}
void mkref_rms_norm(const float* x, int64_t rows, int64_t n, const float* w, float eps, float* y)
{
    rms_norm(x, rows, n, w, eps, y);
}
void mkref_group_norm(const float* x, int64_t rows, int64_t c, int64_t groups, const float* g, const float* b,
                      float eps, float* y)
{
    group_norm(x, rows, c, groups, g, b, eps, y);
}
void mkref_rope_table(float* cs, uint32_t S, uint32_t h, uint32_t w) { rope_table(cs, S, h, w); }
void mkref_heads_norm_rope(const float* x, int64_t rows, int64_t ld, int64_t col0, int64_t heads, int64_t d,
                           const float* w, float eps, const float* cs, int rope, float* out, int64_t out_rows,
                           int64_t out_row0)
{
    heads_norm_rope(x, rows, ld, col0, heads, d, w, eps, cs, rope, out, out_rows, out_row0);
}
void mkref_attention(const float* q, const float* k, const float* v, int64_t B, int64_t H, int64_t Tq, int64_t Tk,
                     int64_t d, float scale, uint32_t q_pos0, uint32_t block, float* out)
{
    attention(q, k, v, B, H, Tq, Tk, d, scale, q_pos0, block, out);
}
void mkref_gelu_tanh(float* x, size_t n)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(n); ++i)
        x[i] = gelu_tanh1(x[i]);
}
void mkref_silu(float* x, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        x[i] = silu1(x[i]);
}
void mkref_swiglu(const float* gu, int64_t rows, int64_t F, float* m)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < F; ++i)
            m[size_t(r) * F + i] = silu1(gu[size_t(r) * 2 * F + i]) * gu[size_t(r) * 2 * F + F + i];
}
void mkref_geglu(const float* hg, int64_t rows, int64_t F, float* m)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < F; ++i) {
            const float g = hg[size_t(r) * 2 * F + F + i];
            m[size_t(r) * F + i] = hg[size_t(r) * 2 * F + i] * 0.5f * g * (1.0f + std::erf(g * 0.70710678f));
        }
}
void mkref_sinusoid(float v, uint32_t dim, float* out) { sinusoid(v, dim, out); }

// engine.cpp:335-339 (shift_mu) and :347-365 (sigmas).
void mkref_sigmas(uint32_t steps, uint32_t tokens, double base_seq, double max_seq, double base_shift,
                  double max_shift, double terminal, float* out)
{
    const double m = (max_shift - base_shift) / (max_seq - base_seq);
    const double mu = double(tokens) * m + (base_shift - m * base_seq);
    for (uint32_t i = 0; i < steps; ++i) {
        const float t = steps == 1 ? 1.0f : float(1.0 + (1.0 / steps - 1.0) * double(i) / double(steps - 1));
        out[i] = float(std::exp(mu) / (std::exp(mu) + (1.0 / double(t) - 1.0)));
    }
    if (terminal > 0 && steps > 0 && out[steps - 1] < 1.0f) {
        const float scale = (1.0f - out[steps - 1]) / (1.0f - float(terminal));
        for (uint32_t i = 0; i < steps; ++i)
            out[i] = 1.0f - (1.0f - out[i]) / scale;
    }
    out[steps] = 0.0f;
}

// The token layout of sdxl.cpp:79-87 (channel, row, column of the 2x2 patch), for C channels.
void mkref_patchify(const float* lat, uint32_t C, uint32_t h, uint32_t w, float* tokens)
{
    for (uint32_t y = 0; y < 2 * h; ++y)
        for (uint32_t x = 0; x < 2 * w; ++x)
            for (uint32_t c = 0; c < C; ++c)
                tokens[(size_t(y / 2) * w + x / 2) * C * 4 + c * 4 + (y % 2) * 2 + x % 2] =
                    lat[(size_t(c) * 2 * h + y) * 2 * w + x];
}
void mkref_unpatchify(const float* tokens, uint32_t C, uint32_t h, uint32_t w, float* lat)
{
    for (uint32_t y = 0; y < 2 * h; ++y)
        for (uint32_t x = 0; x < 2 * w; ++x)
            for (uint32_t c = 0; c < C; ++c)
                lat[(size_t(c) * 2 * h + y) * 2 * w + x] =
                    tokens[(size_t(y / 2) * w + x / 2) * C * 4 + c * 4 + (y % 2) * 2 + x % 2];
}

int mkref_threads(void) { return omp_get_max_threads(); }

} // extern "C"

// ---------------------------------------------------------------------------------------------------------------
// Models
// ---------------------------------------------------------------------------------------------------------------

struct mkref_model {
    mkref_dims dims;
    struct T {
        std::string name;
        std::vector<float> v;
        int64_t rows, cols;
        int kind; // 0 vector, 1 bf16 matrix, 2 fp8 matrix, 3 half matrix
    };
    std::vector<T> ts;
    std::map<std::string, size_t> index;
    uint64_t seed;
    double wstd = 0.02;

    const T& get(const std::string& n) const
    {
        auto it = index.find(n);
        if (it == index.end())
            throw std::runtime_error("mkref: no tensor " + n);
        return ts[it->second];
    }
    const float* vec(const std::string& n) const { return get(n).v.data(); }
    const float* opt(const std::string& n) const
    {
        auto it = index.find(n);
        return it == index.end() ? nullptr : ts[it->second].v.data();
    }
    void add(const std::string& n, int64_t rows, int64_t cols, int kind, double mean, double std)
    {
        T t{n, std::vector<float>(size_t(rows) * cols), rows, cols, kind};
        mkref_fill_normal(t.v.data(), t.v.size(), mkref_tensor_key(seed, n.c_str()), mean, std, kind == 1);
        if (kind == 3)
            mkref_round_f16(t.v.data(), t.v.size());
        index[n] = ts.size();
        ts.push_back(std::move(t));
    }
    // A matrix [rows][cols] of N(0, 0.02); in fp8 mode (block linears only) stored e4m3 with a per-row scale
    // max|W_row| / 448.
    // half: a matrix Engine::matrix keeps F16 (SDXL with dims.f16), N(0, wstd) rounded to half, not bf16.
    void mat(const std::string& n, int64_t rows, int64_t cols, bool quant = false, bool half = false)
    {
        add(n, rows, cols, half ? 3 : 1, 0.0, wstd);
        if (half)
            return;
        if (quant && dims.fp8) {
            T& t = ts[index[n]];
            t.kind = 2;
            T s{n + ".scale", std::vector<float>(size_t(rows)), rows, 1, 0};
            for (int64_t r = 0; r < rows; ++r) {
                float mx = 0;
                for (int64_t c = 0; c < cols; ++c)
                    mx = std::max(mx, std::fabs(t.v[size_t(r) * cols + c]));
                const float sc = mx > 0 ? mx / 448.0f : 1.0f;
                s.v[r] = sc;
                for (int64_t c = 0; c < cols; ++c) {
                    float& x = t.v[size_t(r) * cols + c];
                    x = e4m3_decode(e4m3_encode(x / sc));
                }
            }
            index[s.name] = ts.size();
            ts.push_back(std::move(s));
        }
    }
    void bias(const std::string& n, int64_t len) { add(n, len, 1, 0, 0.0, wstd); }
    void normw(const std::string& n, int64_t len) { add(n, len, 1, 0, 1.0, wstd); }

    // Linear layer y = x W^T + b over rows of x (W bf16 or fp8 with scale).
    void linear(const std::string& n, const float* x, int64_t lda, int64_t M, float* y, int64_t ldy,
                bool has_bias = true) const
    {
        const T& W = get(n + ".weight");
        const float* sc = W.kind == 2 ? vec(n + ".weight.scale") : nullptr;
        gemm(x, lda, M, W.cols, W.v.data(), W.rows, sc, has_bias ? opt(n + ".bias") : nullptr, y, ldy, W.kind == 3);
    }
    int64_t out_dim(const std::string& n) const { return get(n + ".weight").rows; }
};

extern "C" {

mkref_model* mkref_model_create(const mkref_dims* d, uint64_t seed, double wstd)
{
    auto* m = new mkref_model();
    m->dims = *d;
    m->seed = seed;
    m->wstd = wstd;
    const int64_t D = d->dim, F = d->ffn, L = d->latent, E = d->text_dim, hd = d->head_dim;
    if (d->kind == MKREF_DUAL) {
        // Names follow the public Qwen-Image (v1) transformer.
        m->mat("img_in.weight", D, L);
        m->bias("img_in.bias", D);
        m->normw("txt_norm.weight", E);
        m->mat("txt_in.weight", D, E);
        m->bias("txt_in.bias", D);
        m->mat("time_text_embed.timestep_embedder.linear_1.weight", D, 256);
        m->bias("time_text_embed.timestep_embedder.linear_1.bias", D);
        m->mat("time_text_embed.timestep_embedder.linear_2.weight", D, D);
        m->bias("time_text_embed.timestep_embedder.linear_2.bias", D);
        m->mat("norm_out.linear.weight", 2 * D, D);
        m->bias("norm_out.linear.bias", 2 * D);
        m->mat("proj_out.weight", L, D);
        m->bias("proj_out.bias", L);
        for (uint32_t i = 0; i < d->blocks; ++i) {
            const std::string b = "transformer_blocks." + std::to_string(i) + ".";
            for (const char* s : {"img_mod.1", "txt_mod.1"}) {
                m->mat(b + s + ".weight", 6 * D, D);
                m->bias(b + s + ".bias", 6 * D);
            }
            for (const char* s : {"attn.to_q", "attn.to_k", "attn.to_v", "attn.add_q_proj", "attn.add_k_proj",
                                  "attn.add_v_proj", "attn.to_out.0", "attn.to_add_out"}) {
                m->mat(b + s + ".weight", D, D, true);
                m->bias(b + s + ".bias", D);
            }
            for (const char* s : {"attn.norm_q", "attn.norm_k", "attn.norm_added_q", "attn.norm_added_k"})
                m->normw(b + s + ".weight", hd);
            for (const char* s : {"img_mlp", "txt_mlp"}) {
                m->mat(b + s + ".net.0.proj.weight", F, D, true);
                m->bias(b + s + ".net.0.proj.bias", F);
                m->mat(b + s + ".net.2.weight", D, F, true);
                m->bias(b + s + ".net.2.bias", D);
            }
        }
    } else if (d->kind == MKREF_Q21) {
        // Names and the zero-centred text norm of qwen_image.cpp:79-111; no biases.
        m->mat("img_in.weight", D, L);
        m->add("txt_in.text_norm.weight", E, 1, 0, 0.0, m->wstd);
        m->mat("txt_in.in_layer.weight", D, E);
        m->mat("txt_in.out_layer.weight", D, D);
        m->mat("time_text_embed.timestep_embedder.linear_1.weight", D, 256);
        m->mat("time_text_embed.timestep_embedder.linear_2.weight", D, D);
        m->mat("modulation.1.weight", 4 * D, D);
        m->mat("norm_out.linear.weight", D, D);
        m->mat("proj_out.weight", L, D);
        for (uint32_t i = 0; i < d->blocks; ++i) {
            const std::string b = "transformer_blocks." + std::to_string(i) + ".";
            for (const char* s : {"attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0"})
                m->mat(b + s + ".weight", D, D, true);
            m->normw(b + "attn.norm_q.weight", hd);
            m->normw(b + "attn.norm_k.weight", hd);
            m->mat(b + "img_mlp.gate_layer.weight", F, D, true);
            m->mat(b + "img_mlp.proj.weight", F, D, true);
            m->mat(b + "img_mlp.out.weight", D, F, true);
        }
    } else if (d->kind == MKREF_SDXL) {
        // One spatial transformer (sdxl.cpp:264-310): C channels, GEGLU inner F, context E. With dims.f16 the
        // matrices Sdxl::load_trans reads through Engine::matrix (proj_in, proj_out, to_out, attn2.to_q, ff;
        // sdxl.cpp:267-306) are half, as that keeps an F16 checkpoint's (engine.cpp:292-302); q|k|v and the
        // context's k|v go through upload_rows and stay bf16.
        const bool h = d->f16 != 0;
        m->normw("norm.weight", D);
        m->bias("norm.bias", D);
        m->mat("proj_in.weight", D, D, false, h);
        m->bias("proj_in.bias", D);
        m->mat("proj_out.weight", D, D, false, h);
        m->bias("proj_out.bias", D);
        for (uint32_t i = 0; i < d->blocks; ++i) {
            const std::string b = "transformer_blocks." + std::to_string(i) + ".";
            for (const char* s : {"norm1", "norm2", "norm3"}) {
                m->normw(b + s + ".weight", D);
                m->bias(b + s + ".bias", D);
            }
            for (const char* s : {"attn1.to_q", "attn1.to_k", "attn1.to_v"})
                m->mat(b + s + ".weight", D, D, true);
            m->mat(b + "attn2.to_q.weight", D, D, true, h);
            m->mat(b + "attn2.to_k.weight", D, E, true);
            m->mat(b + "attn2.to_v.weight", D, E, true);
            for (const char* s : {"attn1.to_out.0", "attn2.to_out.0"}) {
                m->mat(b + s + ".weight", D, D, true, h);
                m->bias(b + s + ".bias", D);
            }
            m->mat(b + "ff.net.0.proj.weight", 2 * F, D, true, h);
            m->bias(b + "ff.net.0.proj.bias", 2 * F);
            m->mat(b + "ff.net.2.weight", D, F, true, h);
            m->bias(b + "ff.net.2.bias", D);
        }
    } else {
        delete m;
        return nullptr;
    }
    return m;
}

void mkref_model_destroy(mkref_model* m) { delete m; }
size_t mkref_model_count(const mkref_model* m) { return m->ts.size(); }
const char* mkref_model_name(const mkref_model* m, size_t i) { return m->ts[i].name.c_str(); }
const float* mkref_model_tensor(const mkref_model* m, size_t i, int64_t* rows, int64_t* cols, int* kind)
{
    const auto& t = m->ts[i];
    *rows = t.rows;
    *cols = t.cols;
    *kind = t.kind;
    return t.v.data();
}
int64_t mkref_model_find(const mkref_model* m, const char* name)
{
    auto it = m->index.find(name);
    return it == m->index.end() ? -1 : int64_t(it->second);
}

} // extern "C"

namespace {

// One dual-stream block for one sample: img [N][D] and txt [S][D] updated in place.
// The block follows the public Qwen-Image (v1) block: per stream LN -> (1 + scale), + shift -> q, k, v with per-head
// RMSNorm and RoPE -> joint attention over [text; image] -> o -> x += gate * o; LN -> modulate -> GELU-tanh FFN ->
// x += gate * f. The modulation rows are [shift1, scale1, gate1, shift2, scale2, gate2].
void dual_block(const mkref_model& m, int i, float* img, int64_t N, float* txt, int64_t S, const float* mi,
                const float* mt, const float* cs)
{
    const int64_t D = m.dims.dim, H = m.dims.heads, hd = m.dims.head_dim, F = m.dims.ffn, T = S + N;
    const float eps = 1e-6f;
    const std::string b = "transformer_blocks." + std::to_string(i) + ".";
    std::vector<float> xn(size_t(std::max(N, S)) * D), q(size_t(N) * D), k(size_t(N) * D), v(size_t(N) * D);
    std::vector<float> Q(size_t(H) * T * hd), K(size_t(H) * T * hd), V(size_t(H) * T * hd), att(size_t(T) * D);
    std::vector<float> o(size_t(std::max(N, S)) * D), f(size_t(std::max(N, S)) * F);
    struct Stream {
        float* x;
        int64_t rows, row0;
        const float* mod;
        const char *q, *k, *v, *nq, *nk, *out, *mlp;
    };
    const Stream st[2] = {
        {txt, S, 0, mt, "attn.add_q_proj", "attn.add_k_proj", "attn.add_v_proj", "attn.norm_added_q",
         "attn.norm_added_k", "attn.to_add_out", "txt_mlp"},
        {img, N, S, mi, "attn.to_q", "attn.to_k", "attn.to_v", "attn.norm_q", "attn.norm_k", "attn.to_out.0",
         "img_mlp"}};
    for (const Stream& s : st) {
        if (!s.rows)
            continue;
        ln_modulate(s.x, s.rows, D, s.mod, s.mod + D, eps, xn.data());
        m.linear(b + s.q, xn.data(), D, s.rows, q.data(), D);
        m.linear(b + s.k, xn.data(), D, s.rows, k.data(), D);
        m.linear(b + s.v, xn.data(), D, s.rows, v.data(), D);
        const float* tab = cs + size_t(s.row0) * hd;
        heads_norm_rope(q.data(), s.rows, D, 0, H, hd, m.vec(b + s.nq + ".weight"), eps, tab, 2, Q.data(), T, s.row0);
        heads_norm_rope(k.data(), s.rows, D, 0, H, hd, m.vec(b + s.nk + ".weight"), eps, tab, 2, K.data(), T, s.row0);
        heads_norm_rope(v.data(), s.rows, D, 0, H, hd, nullptr, eps, nullptr, 0, V.data(), T, s.row0);
    }
    mkref_round_bf16(Q.data(), Q.size());
    mkref_round_bf16(K.data(), K.size());
    mkref_round_bf16(V.data(), V.size());
    attention(Q.data(), K.data(), V.data(), 1, H, T, T, hd, 1.0f / std::sqrt(float(hd)), 0, 0, att.data());
    for (const Stream& s : st) {
        if (!s.rows)
            continue;
        m.linear(b + s.out, att.data() + size_t(s.row0) * D, D, s.rows, o.data(), D);
        const float* g1 = s.mod + 2 * D;
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < s.rows; ++r)
            for (int64_t c = 0; c < D; ++c)
                s.x[size_t(r) * D + c] += g1[c] * o[size_t(r) * D + c];
        ln_modulate(s.x, s.rows, D, s.mod + 3 * D, s.mod + 4 * D, eps, xn.data());
        const std::string mlp = b + s.mlp;
        m.linear(mlp + ".net.0.proj", xn.data(), D, s.rows, f.data(), F);
        mkref_gelu_tanh(f.data(), size_t(s.rows) * F);
        m.linear(mlp + ".net.2", f.data(), F, s.rows, o.data(), D);
        const float* g2 = s.mod + 5 * D;
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < s.rows; ++r)
            for (int64_t c = 0; c < D; ++c)
                s.x[size_t(r) * D + c] += g2[c] * o[size_t(r) * D + c];
    }
}

// Time embedding of the public Qwen-Image: sinusoid(1000 sigma) (cos half first) -> linear_1 -> SiLU -> linear_2;
// returns silu(temb), the input of every modulation layer.
std::vector<float> time_silu(const mkref_model& m, float sigma, std::vector<float>* temb_out)
{
    const int64_t D = m.dims.dim;
    float tp[256];
    sinusoid(1000.0f * sigma, 256, tp);
    std::vector<float> h(D), t(D);
    m.linear("time_text_embed.timestep_embedder.linear_1", tp, 256, 1, h.data(), D);
    mkref_silu(h.data(), D);
    m.linear("time_text_embed.timestep_embedder.linear_2", h.data(), D, 1, t.data(), D);
    if (temb_out)
        *temb_out = t;
    mkref_silu(t.data(), D);
    return t;
}

} // namespace

extern "C" {

int mkref_dual_block(const mkref_model* m, int block, float* img, int64_t N, float* txt, int64_t S,
                     const float* mod_img, const float* mod_txt, const float* cs)
{
    try {
        dual_block(*m, block, img, N, txt, S, mod_img, mod_txt, cs);
        return 0;
    } catch (...) {
        return -1;
    }
}

int mkref_dual_step(const mkref_model* mp, int64_t B, const float* prompt, int64_t S, const float* latents, uint32_t h,
                    uint32_t w, float sigma, float* out, mkref_probe_fn probe, void* user)
{
    try {
        const mkref_model& m = *mp;
        const int64_t D = m.dims.dim, E = m.dims.text_dim, L = m.dims.latent, N = int64_t(h) * w;
        std::vector<float> temb;
        const std::vector<float> ts = time_silu(m, sigma, &temb);
        if (probe)
            probe(user, "temb", -1, temb.data(), temb.size());
        // Every block's modulation rows for both streams: [blocks][2][6D] (image first).
        const int nb = int(m.dims.blocks);
        std::vector<float> mod(size_t(nb) * 2 * 6 * D);
        for (int i = 0; i < nb; ++i) {
            const std::string b = "transformer_blocks." + std::to_string(i) + ".";
            m.linear(b + "img_mod.1", ts.data(), D, 1, mod.data() + size_t(i) * 12 * D, 6 * D);
            m.linear(b + "txt_mod.1", ts.data(), D, 1, mod.data() + size_t(i) * 12 * D + 6 * D, 6 * D);
        }
        if (probe)
            probe(user, "modulation", -1, mod.data(), mod.size());
        std::vector<float> omod(2 * D);
        m.linear("norm_out.linear", ts.data(), D, 1, omod.data(), 2 * D); // [scale | shift]
        std::vector<float> cs(size_t(S + N) * 128);
        rope_table(cs.data(), uint32_t(S), h, w);
        for (int64_t bi = 0; bi < B; ++bi) {
            std::vector<float> txt(size_t(S) * D), img(size_t(N) * D), tn(size_t(S) * E);
            rms_norm(prompt + size_t(bi) * S * E, S, E, m.vec("txt_norm.weight"), 1e-6f, tn.data());
            m.linear("txt_in", tn.data(), E, S, txt.data(), D);
            m.linear("img_in", latents + size_t(bi) * N * L, L, N, img.data(), D);
            if (probe) {
                probe(user, "txt_in", int(bi), txt.data(), txt.size());
                probe(user, "img_in", int(bi), img.data(), img.size());
            }
            for (int i = 0; i < nb; ++i) {
                dual_block(m, i, img.data(), N, txt.data(), S, mod.data() + size_t(i) * 12 * D,
                           mod.data() + size_t(i) * 12 * D + 6 * D, cs.data());
                if (probe)
                    probe(user, "block", i * int(B) + int(bi), img.data(), img.size());
            }
            std::vector<float> xn(size_t(N) * D);
            ln_modulate(img.data(), N, D, omod.data() + D, omod.data(), 1e-6f, xn.data());
            if (probe)
                probe(user, "norm_out", int(bi), xn.data(), xn.size());
            m.linear("proj_out", xn.data(), D, N, out + size_t(bi) * N * L, L);
        }
        return 0;
    } catch (...) {
        return -1;
    }
}

// qwen_image.cpp:144-293 over the whole sequence each step (the first step's graph; later steps' image rows equal
// it because the text rows see only text keys and take the t = 0 modulation).
int mkref_q21_step(const mkref_model* mp, const float* prompt, int64_t S, const float* latents, uint32_t h, uint32_t w,
                   float sigma, float* out, mkref_probe_fn probe, void* user)
{
    try {
        const mkref_model& m = *mp;
        const int64_t D = m.dims.dim, E = m.dims.text_dim, L = m.dims.latent, N = int64_t(h) * w, T = S + N;
        const int64_t H = m.dims.heads, hd = m.dims.head_dim, F = m.dims.ffn;
        const float eps = 1e-6f;
        // qwen_image.cpp:179-205: rows [sigma, 0]; t_lin1 -> silu -> t_lin2 -> silu -> mod / out_lin.
        std::vector<float> tp(2 * 256), t1(2 * D), t2(2 * D), mod(2 * 4 * D), omod(2 * D);
        sinusoid(1000.0f * sigma, 256, tp.data());
        sinusoid(0.0f, 256, tp.data() + 256);
        m.linear("time_text_embed.timestep_embedder.linear_1", tp.data(), 256, 2, t1.data(), D, false);
        mkref_silu(t1.data(), t1.size());
        m.linear("time_text_embed.timestep_embedder.linear_2", t1.data(), D, 2, t2.data(), D, false);
        if (probe)
            probe(user, "temb", -1, t2.data(), t2.size());
        mkref_silu(t2.data(), t2.size());
        m.linear("modulation.1", t2.data(), D, 2, mod.data(), 4 * D, false);
        if (probe)
            probe(user, "modulation", -1, mod.data(), mod.size());
        m.linear("norm_out.linear", t2.data(), D, 2, omod.data(), D, false);
        // Text in: RMSNorm with the zero-centred weight + 1 (qwen_image.cpp:82-86,206-214).
        std::vector<float> tw(E), x(size_t(T) * D), tn(size_t(S) * E), t3(size_t(S) * D);
        const float* tz = m.vec("txt_in.text_norm.weight");
        for (int64_t i = 0; i < E; ++i)
            tw[i] = tz[i] + 1.0f;
        rms_norm(prompt, S, E, tw.data(), eps, tn.data());
        m.linear("txt_in.in_layer", tn.data(), E, S, t3.data(), D, false);
        mkref_gelu_tanh(t3.data(), t3.size());
        m.linear("txt_in.out_layer", t3.data(), D, S, x.data(), D, false);
        m.linear("img_in", latents, L, N, x.data() + size_t(S) * D, D, false);
        if (probe) {
            probe(user, "txt_in", -1, x.data(), size_t(S) * D);
            probe(user, "img_in", -1, x.data() + size_t(S) * D, size_t(N) * D);
        }
        std::vector<float> cs(size_t(T) * 128);
        rope_table(cs.data(), uint32_t(S), h, w);
        std::vector<float> xn(size_t(T) * D), q(size_t(T) * D), k(size_t(T) * D), v(size_t(T) * D), o(size_t(T) * D);
        std::vector<float> Q(size_t(H) * T * hd), K(Q.size()), V(Q.size()), att(size_t(T) * D);
        std::vector<float> g(size_t(T) * F), u(size_t(T) * F), mm(size_t(T) * F);
        // ln_modulate / gate_add with rows before `split` = S taking modulation row 1 (image.metal:32-65).
        auto lnmod = [&](const float* sc_rows, int64_t stride) {
            ln_modulate(x.data(), S, D, nullptr, sc_rows + stride, eps, xn.data());
            ln_modulate(x.data() + size_t(S) * D, N, D, nullptr, sc_rows, eps, xn.data() + size_t(S) * D);
        };
        auto gate_add = [&](const float* g_rows, int64_t stride) {
#pragma omp parallel for schedule(static)
            for (int64_t r = 0; r < T; ++r) {
                const float* gg = g_rows + (r < S ? stride : 0);
                for (int64_t c = 0; c < D; ++c)
                    x[size_t(r) * D + c] += std::tanh(gg[c]) * o[size_t(r) * D + c];
            }
        };
        for (uint32_t i = 0; i < m.dims.blocks; ++i) {
            const std::string b = "transformer_blocks." + std::to_string(i) + ".";
            lnmod(mod.data(), 4 * D);
            m.linear(b + "attn.to_q", xn.data(), D, T, q.data(), D, false);
            m.linear(b + "attn.to_k", xn.data(), D, T, k.data(), D, false);
            m.linear(b + "attn.to_v", xn.data(), D, T, v.data(), D, false);
            heads_norm_rope(q.data(), T, D, 0, H, hd, m.vec(b + "attn.norm_q.weight"), eps, cs.data(), 2, Q.data(), T, 0);
            heads_norm_rope(k.data(), T, D, 0, H, hd, m.vec(b + "attn.norm_k.weight"), eps, cs.data(), 2, K.data(), T, 0);
            heads_norm_rope(v.data(), T, D, 0, H, hd, nullptr, eps, nullptr, 0, V.data(), T, 0);
            // q, k, v (and the text's cached keys / values) are half (heads_norm_half / heads_half)
            mkref_round_f16(Q.data(), Q.size());
            mkref_round_f16(K.data(), K.size());
            mkref_round_f16(V.data(), V.size());
            attention(Q.data(), K.data(), V.data(), 1, H, T, T, hd, 1.0f / std::sqrt(float(hd)), 0, uint32_t(S),
                      att.data());
            m.linear(b + "attn.to_out.0", att.data(), D, T, o.data(), D, false);
            gate_add(mod.data() + D, 4 * D);
            lnmod(mod.data() + 2 * D, 4 * D);
            m.linear(b + "img_mlp.gate_layer", xn.data(), D, T, g.data(), F, false);
            m.linear(b + "img_mlp.proj", xn.data(), D, T, u.data(), F, false);
#pragma omp parallel for schedule(static)
            for (int64_t j = 0; j < T * F; ++j)
                mm[j] = silu1(g[j]) * u[j];
            m.linear(b + "img_mlp.out", mm.data(), F, T, o.data(), D, false);
            gate_add(mod.data() + 3 * D, 4 * D);
            if (probe)
                probe(user, "block", int(i), x.data(), x.size());
        }
        // Tail: ln_modulate(omod) with the same split (qwen_image.cpp:285-288), image rows out.
        ln_modulate(x.data(), S, D, nullptr, omod.data() + D, eps, xn.data());
        ln_modulate(x.data() + size_t(S) * D, N, D, nullptr, omod.data(), eps, xn.data() + size_t(S) * D);
        if (probe)
            probe(user, "norm_out", -1, xn.data(), xn.size());
        m.linear("proj_out", xn.data() + size_t(S) * D, D, N, out, L, false);
        return 0;
    } catch (...) {
        return -1;
    }
}

// sdxl.cpp:742-796 for one sample, with the cross-attention keys / values of sdxl.cpp:693-719.
int mkref_sdxl_trans(const mkref_model* mp, const float* x, int64_t n, const float* ctx, int64_t S, float* y)
{
    try {
        const mkref_model& m = *mp;
        const int64_t c = m.dims.dim, H = c / 64, F = m.dims.ffn, E = m.dims.text_dim;
        const float scale = 1.0f / 8.0f;
        std::vector<float> xn(size_t(n) * c), hs(size_t(n) * c), hn(size_t(n) * c), q(size_t(n) * c), k(size_t(n) * c),
            v(size_t(n) * c), o(size_t(n) * c), att(size_t(n) * c), ff(size_t(n) * 2 * F), mm(size_t(n) * F);
        std::vector<float> Q(size_t(H) * n * 64), K(Q.size()), V(Q.size());
        std::vector<float> ck(size_t(S) * c), cv(size_t(S) * c), CK(size_t(H) * S * 64), CV(CK.size());
        group_norm(x, n, c, 32, m.vec("norm.weight"), m.vec("norm.bias"), 1e-6f, xn.data());
        m.linear("proj_in", xn.data(), c, n, hs.data(), c);
        auto add = [&](std::vector<float>& a, const std::vector<float>& b) {
            for (size_t i = 0; i < size_t(n) * c; ++i)
                a[i] += b[i];
        };
        for (uint32_t i = 0; i < m.dims.blocks; ++i) {
            const std::string b = "transformer_blocks." + std::to_string(i) + ".";
            layer_norm(hs.data(), n, c, m.vec(b + "norm1.weight"), m.vec(b + "norm1.bias"), 1e-5f, hn.data());
            m.linear(b + "attn1.to_q", hn.data(), c, n, q.data(), c, false);
            m.linear(b + "attn1.to_k", hn.data(), c, n, k.data(), c, false);
            m.linear(b + "attn1.to_v", hn.data(), c, n, v.data(), c, false);
            heads_norm_rope(q.data(), n, c, 0, H, 64, nullptr, 0, nullptr, 0, Q.data(), n, 0);
            heads_norm_rope(k.data(), n, c, 0, H, 64, nullptr, 0, nullptr, 0, K.data(), n, 0);
            heads_norm_rope(v.data(), n, c, 0, H, 64, nullptr, 0, nullptr, 0, V.data(), n, 0);
            // half heads (heads64 -> heads_half, sdxl.cpp:439-448)
            mkref_round_f16(Q.data(), Q.size());
            mkref_round_f16(K.data(), K.size());
            mkref_round_f16(V.data(), V.size());
            attention(Q.data(), K.data(), V.data(), 1, H, n, n, 64, scale, 0, 0, att.data());
            m.linear(b + "attn1.to_out.0", att.data(), c, n, o.data(), c);
            add(hs, o);
            layer_norm(hs.data(), n, c, m.vec(b + "norm2.weight"), m.vec(b + "norm2.bias"), 1e-5f, hn.data());
            m.linear(b + "attn2.to_q", hn.data(), c, n, q.data(), c, false);
            heads_norm_rope(q.data(), n, c, 0, H, 64, nullptr, 0, nullptr, 0, Q.data(), n, 0);
            m.linear(b + "attn2.to_k", ctx, E, S, ck.data(), c, false);
            m.linear(b + "attn2.to_v", ctx, E, S, cv.data(), c, false);
            heads_norm_rope(ck.data(), S, c, 0, H, 64, nullptr, 0, nullptr, 0, CK.data(), S, 0);
            heads_norm_rope(cv.data(), S, c, 0, H, 64, nullptr, 0, nullptr, 0, CV.data(), S, 0);
            mkref_round_f16(Q.data(), Q.size());
            mkref_round_f16(CK.data(), CK.size());
            mkref_round_f16(CV.data(), CV.size());
            attention(Q.data(), CK.data(), CV.data(), 1, H, n, S, 64, scale, 0, 0, att.data());
            m.linear(b + "attn2.to_out.0", att.data(), c, n, o.data(), c);
            add(hs, o);
            layer_norm(hs.data(), n, c, m.vec(b + "norm3.weight"), m.vec(b + "norm3.bias"), 1e-5f, hn.data());
            m.linear(b + "ff.net.0.proj", hn.data(), c, n, ff.data(), 2 * F);
            mkref_geglu(ff.data(), n, F, mm.data());
            m.linear(b + "ff.net.2", mm.data(), F, n, o.data(), c);
            add(hs, o);
        }
        m.linear("proj_out", hs.data(), c, n, y, c);
        for (size_t i = 0; i < size_t(n) * c; ++i)
            y[i] += x[i];
        return 0;
    } catch (...) {
        return -1;
    }
}

} // extern "C"

// =====================================================================================================================
// VAE decoder: src/image/engine.cpp:589-628 (the weights it loads), 722-746 (norm_silu, res_block), 748-777
// (vae_attention), 862-954 (decode: latent denormalisation over 2x2 patches, post_quant_conv, conv_in, mid block,
// up blocks with nearest 2x upsampling, norm_out + SiLU, conv_out, clamp to [-1, 1], alpha 1). Images are
// [pixels][channels] fp32. Precision points as the reference runs them: every convolution multiplies F16 weights with
// its input rounded to half (docs/performance.md:13: "the VAE's convolution weights in F16 on that GEMM"; its GEMM
// takes half activations), sums in double here; the mid block's attention multiplies half queries with fp32 keys and
// half probabilities with fp32 values (engine.cpp:764-773: gemm_->encode with F32 kc / vt and halves() of Q and P).
// The RMS norm is x / sqrt(sum x^2 + 1e-24) * sqrt(c) * gamma (engine.cpp:725-727).
// =====================================================================================================================

struct mkref_vae {
    uint32_t base = 0, z = 0;
    std::vector<float> mean, std_;
    std::vector<std::string> names;
    std::map<std::string, std::pair<std::vector<float>, std::vector<int64_t>>> t;
    const std::vector<float>& w(const std::string& n) const { return t.at(n).first; }
    int64_t dim(const std::string& n, int i) const { return t.at(n).second[size_t(i)]; }
};

namespace {

struct Img {
    uint32_t h = 0, w = 0, c = 0;
    std::vector<float> v;
    Img() = default;
    Img(uint32_t h_, uint32_t w_, uint32_t c_) : h(h_), w(w_), c(c_), v(size_t(h_) * w_ * c_) {}
};

void vae_add(mkref_vae* m, const std::string& name, std::vector<int64_t> dims, uint64_t seed)
{
    size_t n = 1;
    for (int64_t d : dims)
        n *= size_t(d);
    std::vector<float> v(n);
    const uint64_t key = mkref_tensor_key(seed, name.c_str());
    const bool conv = dims.size() == 4, gamma = name.size() > 6 && name.compare(name.size() - 6, 6, ".gamma") == 0;
    if (conv)
        mkref_fill_normal(v.data(), n, key, 0.0, 1.0 / std::sqrt(double(dims[1] * dims[2] * dims[3])), 1);
    else
        mkref_fill_normal(v.data(), n, key, gamma ? 1.0 : 0.0, gamma ? 0.1 : 0.02, 0);
    m->names.push_back(name);
    m->t[name] = {std::move(v), std::move(dims)};
}

// y = conv(half(x)) with half(W) + bias, k = 1 or 3, zero padding; or y += that (accumulate).
void vae_conv(const mkref_vae* m, const std::string& p, const Img& x, Img& y, bool accumulate)
{
    std::vector<float> W(m->w(p + ".weight"));
    mkref_round_f16(W.data(), W.size());
    const std::vector<float>& b = m->w(p + ".bias");
    const int64_t co = m->dim(p + ".weight", 0), ci = m->dim(p + ".weight", 1), k = m->dim(p + ".weight", 2);
    if (ci != x.c)
        throw std::runtime_error("vae_conv: channels");
    std::vector<float> xb(x.v);
    mkref_round_f16(xb.data(), xb.size());
    if (!accumulate)
        y = Img(x.h, x.w, uint32_t(co));
    const int H = int(x.h), Wd = int(x.w), r = int(k / 2);
#pragma omp parallel for schedule(static)
    for (int yy = 0; yy < H; ++yy)
        for (int xx = 0; xx < Wd; ++xx)
            for (int64_t o = 0; o < co; ++o) {
                double acc = 0.0;
                for (int dy = 0; dy < k; ++dy) {
                    const int sy = yy + dy - r;
                    if (sy < 0 || sy >= H)
                        continue;
                    for (int dx = 0; dx < k; ++dx) {
                        const int sx = xx + dx - r;
                        if (sx < 0 || sx >= Wd)
                            continue;
                        const float* xp = &xb[(size_t(sy) * Wd + sx) * size_t(ci)];
                        const float* wp = &W[size_t(o) * ci * k * k + size_t(dy) * k + dx];
                        for (int64_t c = 0; c < ci; ++c)
                            acc += double(xp[c]) * wp[size_t(c) * k * k];
                    }
                }
                float& out = y.v[(size_t(yy) * Wd + xx) * size_t(co) + o];
                const float v = float(acc) + b[size_t(o)];
                out = accumulate ? out + v : v;
            }
}

// RMS norm over each pixel's channels with gamma, then SiLU (silu = true); the result as half values (the next
// convolution's input).
Img vae_norm(const Img& x, const std::vector<float>& g, bool silu)
{
    Img y(x.h, x.w, x.c);
    const size_t px = size_t(x.h) * x.w;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < px; ++i) {
        const float* a = &x.v[i * x.c];
        double ss = 0.0;
        for (uint32_t c = 0; c < x.c; ++c)
            ss += double(a[c]) * a[c];
        const float r = float(1.0 / std::sqrt(ss / x.c + 1e-24 / x.c));
        for (uint32_t c = 0; c < x.c; ++c) {
            float v = a[c] * r * g[c];
            if (silu)
                v = v / (1.0f + std::exp(-v));
            y.v[i * x.c + c] = f16(v);
        }
    }
    return y;
}

void vae_res(const mkref_vae* m, const std::string& p, Img& x)
{
    Img h1, h2;
    vae_conv(m, p + ".conv1", vae_norm(x, m->w(p + ".norm1.gamma"), true), h1, false);
    Img y;
    if (m->t.count(p + ".conv_shortcut.weight"))
        vae_conv(m, p + ".conv_shortcut", x, y, false);
    else
        y = x;
    vae_conv(m, p + ".conv2", vae_norm(h1, m->w(p + ".norm2.gamma"), true), y, true);
    x = std::move(y);
}

// One-head attention over the pixels (engine.cpp:748-777): q, k, v (with their biases) from the 1x1 to_qkv conv of
// the normed image, softmax(q k^T / sqrt(c)) v with q and P rounded to half and k, v in fp32, then proj and the
// residual.
void vae_attn(const mkref_vae* m, Img& x)
{
    const std::string a = "decoder.mid_block.attentions.0.";
    const uint32_t n = x.h * x.w, c = x.c;
    Img xn = vae_norm(x, m->w(a + "norm.gamma"), false);
    Img qkv;
    vae_conv(m, a + "to_qkv", xn, qkv, false);
    // q -> half; k, v stay fp32
    for (uint32_t i = 0; i < n; ++i)
        for (uint32_t k = 0; k < c; ++k)
            qkv.v[size_t(i) * 3 * c + k] = f16(qkv.v[size_t(i) * 3 * c + k]);
    Img o(x.h, x.w, c);
    const double scale = 1.0 / std::sqrt(double(c));
#pragma omp parallel for schedule(dynamic)
    for (uint32_t i = 0; i < n; ++i) {
        std::vector<double> s(n);
        double mx = -1e300;
        for (uint32_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (uint32_t k = 0; k < c; ++k)
                acc += double(qkv.v[size_t(i) * 3 * c + k]) * qkv.v[size_t(j) * 3 * c + c + k];
            s[j] = float(acc);
            mx = std::max(mx, s[j]);
        }
        double sum = 0.0;
        for (uint32_t j = 0; j < n; ++j)
            sum += (s[j] = std::exp((s[j] - mx) * scale));
        for (uint32_t k = 0; k < c; ++k) {
            double acc = 0.0;
            for (uint32_t j = 0; j < n; ++j)
                acc += double(f16(float(s[j] / sum))) * qkv.v[size_t(j) * 3 * c + 2 * c + k];
            o.v[size_t(i) * c + k] = float(acc);
        }
    }
    vae_conv(m, a + "proj", o, x, true);
}

Img vae_up2(const Img& x)
{
    Img y(2 * x.h, 2 * x.w, x.c);
    for (uint32_t yy = 0; yy < y.h; ++yy)
        for (uint32_t xx = 0; xx < y.w; ++xx)
            std::memcpy(&y.v[(size_t(yy) * y.w + xx) * x.c], &x.v[(size_t(yy / 2) * x.w + xx / 2) * x.c],
                        x.c * sizeof(float));
    return y;
}

} // namespace

mkref_vae* mkref_vae_create(uint32_t base, uint32_t z, uint64_t seed, const float* mean, const float* std)
{
    if (!base || !z || !mean || !std)
        return nullptr;
    auto m = new mkref_vae;
    m->base = base;
    m->z = z;
    m->mean.assign(mean, mean + z);
    m->std_.assign(std, std + z);
    const int64_t b = base, d0 = 4 * b;
    auto conv = [&](const std::string& p, int64_t co, int64_t ci, int64_t k) {
        vae_add(m, p + ".weight", {co, ci, k, k}, seed);
        vae_add(m, p + ".bias", {co}, seed);
    };
    auto res = [&](const std::string& p, int64_t ci, int64_t co) {
        vae_add(m, p + ".norm1.gamma", {ci}, seed);
        conv(p + ".conv1", co, ci, 3);
        vae_add(m, p + ".norm2.gamma", {co}, seed);
        conv(p + ".conv2", co, co, 3);
        if (ci != co)
            conv(p + ".conv_shortcut", co, ci, 1);
    };
    conv("post_quant_conv", z, z, 1);
    conv("decoder.conv_in", d0, z, 3);
    res("decoder.mid_block.resnets.0", d0, d0);
    vae_add(m, "decoder.mid_block.attentions.0.norm.gamma", {d0}, seed);
    conv("decoder.mid_block.attentions.0.to_qkv", 3 * d0, d0, 1);
    conv("decoder.mid_block.attentions.0.proj", d0, d0, 1);
    res("decoder.mid_block.resnets.1", d0, d0);
    const int64_t ins[4] = {4 * b, 2 * b, 2 * b, b}, outs[4] = {4 * b, 4 * b, 2 * b, b};
    for (int i = 0; i < 4; ++i) {
        const std::string p = "decoder.up_blocks." + std::to_string(i);
        for (int j = 0; j < 3; ++j)
            res(p + ".resnets." + std::to_string(j), j ? outs[i] : ins[i], outs[i]);
        if (i < 3)
            conv(p + ".upsamplers.0.resample.1", outs[i] / 2, outs[i], 3);
    }
    vae_add(m, "decoder.norm_out.gamma", {b}, seed);
    conv("decoder.conv_out", 3, b, 3);
    return m;
}

void mkref_vae_destroy(mkref_vae* v) { delete v; }
size_t mkref_vae_count(const mkref_vae* v) { return v->names.size(); }
const char* mkref_vae_name(const mkref_vae* v, size_t i) { return v->names[i].c_str(); }

const float* mkref_vae_tensor(const mkref_vae* v, size_t i, uint32_t* ndim, int64_t* dims)
{
    const auto& e = v->t.at(v->names[i]);
    *ndim = uint32_t(e.second.size());
    for (size_t k = 0; k < e.second.size(); ++k)
        dims[k] = e.second[k];
    return e.first.data();
}

int mkref_vae_decode(const mkref_vae* m, const float* tokens, uint32_t h, uint32_t w, float* rgba,
                     mkref_probe_fn probe, void* user)
{
    try {
        const uint32_t z = m->z, L = 4 * z;
        auto pr = [&](const char* n, int layer, const Img& x) {
            if (probe)
                probe(user, n, layer, x.v.data(), x.v.size());
        };
        // tokens -> the latent image (2h x 2w x z): value (c * 2 + py) * 2 + px of token (y, x) is channel c of
        // pixel (2y + py, 2x + px), denormalised by the channel's mean and deviation (engine.cpp:887-898)
        Img lat(2 * h, 2 * w, z);
        for (uint32_t y = 0; y < h; ++y)
            for (uint32_t x = 0; x < w; ++x)
                for (uint32_t c = 0; c < z; ++c)
                    for (uint32_t py = 0; py < 2; ++py)
                        for (uint32_t px = 0; px < 2; ++px)
                            lat.v[((size_t(2 * y + py)) * 2 * w + 2 * x + px) * z + c] =
                                tokens[(size_t(y) * w + x) * L + (c * 2 + py) * 2 + px] * m->std_[c] + m->mean[c];
        // post_quant_conv (a 1x1 convolution: half inputs, half weights), then conv_in
        Img pq;
        vae_conv(m, "post_quant_conv", lat, pq, false);
        Img x;
        vae_conv(m, "decoder.conv_in", pq, x, false);
        pr("vae_conv_in", -1, x);
        vae_res(m, "decoder.mid_block.resnets.0", x);
        vae_attn(m, x);
        vae_res(m, "decoder.mid_block.resnets.1", x);
        pr("vae_mid", -1, x);
        for (int i = 0; i < 4; ++i) {
            const std::string p = "decoder.up_blocks." + std::to_string(i);
            for (int j = 0; j < 3; ++j)
                vae_res(m, p + ".resnets." + std::to_string(j), x);
            if (i < 3) {
                Img y;
                vae_conv(m, p + ".upsamplers.0.resample.1", vae_up2(x), y, false);
                x = std::move(y);
            }
            pr("vae_up", i, x);
        }
        Img o;
        vae_conv(m, "decoder.conv_out", vae_norm(x, m->w("decoder.norm_out.gamma"), true), o, false);
        pr("vae_out", -1, o);
        for (size_t i = 0; i < size_t(o.h) * o.w; ++i)
            for (uint32_t c = 0; c < 4; ++c)
                rgba[i * 4 + c] = c < 3 ? std::min(1.0f, std::max(-1.0f, o.v[i * 3 + c])) : 1.0f;
        return 0;
    } catch (...) {
        return 1;
    }
}
