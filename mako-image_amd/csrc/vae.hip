// The VAE decoder after the denoise loop (src/image/engine.cpp:862-954; weights as load_vae reads them, :589-628): the
// Wan-2.1-layout decoder Qwen-Image uses, one frame. Every 3 x 3 convolution is one implicit-GEMM launch on the matrix
// cores (mk_conv3x3 over the padded pixel grid), 1 x 1 convolutions are plain GEMMs over the same rows, and the kernels
// here do the rest: token unpacking with the latent denormalisation and post_quant_conv, RMS norms (+ SiLU) that write
// the next convolution's input with its zero ring, nearest 2x upsampling into the next grid, the mid block's softmax,
// and the clamp to RGBA. Every convolution multiplies IEEE half weights with half activations in fp32 sums, as the
// reference does (its convolution weights F16, docs/performance.md:13): the 16-bit grids here hold half values.
//
// Image layout "padded grid" (h x w, c channels, row stride cs): (h + 2)(w + 2) grid rows with a one-pixel ring, and
// S = w + 3 slack rows before and after; pixel (y, x) is row S + (y + 1)(w + 2) + x + 1. fp32 activations use it as
// written by the convolutions (ring rows hold values nobody reads as pixels); half convolution inputs keep ring and
// slack rows zero, and channels past c zero.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace mk {
namespace {

struct GridDims {
    uint32_t h, w;
    __host__ __device__ uint32_t pw() const { return w + 2; }
    __host__ __device__ uint32_t slack() const { return w + 3; }
    __host__ __device__ uint64_t grid_rows() const { return uint64_t(h + 2) * (w + 2); }
    __host__ __device__ uint64_t rows() const { return grid_rows() + 2ull * slack(); }
    __host__ __device__ uint64_t row_of(uint32_t y, uint32_t x) const { return slack() + uint64_t(y + 1) * pw() + x + 1; }
    // the pixel of buffer row r (r < 2^32), or false for ring and slack rows: 32-bit arithmetic
    __device__ bool pixel32(uint32_t r, uint32_t& y, uint32_t& x) const
    {
        const uint32_t g = r - slack();
        if (r < slack() || g >= uint32_t(grid_rows()))
            return false;
        const uint32_t gy = g / pw(), gx = g - gy * pw();
        if (gy == 0 || gy > h || gx == 0 || gx > w)
            return false;
        y = gy - 1;
        x = gx - 1;
        return true;
    }
    // the pixel of buffer row r, or false for ring and slack rows
    __host__ __device__ bool pixel(uint64_t r, uint32_t& y, uint32_t& x) const
    {
        if (r < slack() || r >= slack() + grid_rows())
            return false;
        const uint64_t g = r - slack();
        const uint32_t gy = uint32_t(g / pw()), gx = uint32_t(g % pw());
        if (gy == 0 || gy > h || gx == 0 || gx > w)
            return false;
        y = gy - 1;
        x = gx - 1;
        return true;
    }
};

inline uint32_t cpad(uint32_t c) { return (c + 63) / 64 * 64; }
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// tokens [th][tw][4 z] -> the latent image (2 th x 2 tw, z channels: value (c * 2 + py) * 2 + px of a token is channel
// c of pixel (2 y + py, 2 x + px)), denormalised (v * std + mean, engine.cpp:887-898), then post_quant_conv as the
// reference's 1 x 1 conv computes it: half inputs times half weights (w [z][z] holds half values as floats, b [z]) in
// fp32, written as the half padded grid with cp channels (conv_in's input). One thread a (buffer row, channel).
__global__ __launch_bounds__(256) void vae_in_kernel(const float* __restrict__ tok, uint32_t tw, GridDims g, uint32_t z,
                                                     uint32_t cp, const float* __restrict__ mean,
                                                     const float* __restrict__ sd, const float* __restrict__ w,
                                                     const float* __restrict__ b, uint16_t* __restrict__ out)
{
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= g.rows() * cp)
        return;
    const uint64_t r = i / cp;
    const uint32_t c = uint32_t(i % cp);
    uint32_t y, x;
    float v = 0.0f;
    if (c < z && g.pixel(r, y, x)) {
        const float* t = tok + (uint64_t(y / 2) * tw + x / 2) * 4 * z + (y % 2) * 2 + (x % 2);
        float acc = b[c];
        for (uint32_t ch = 0; ch < z; ++ch)
            acc = fmaf(w[c * z + ch], h2f_bits(f2h_bits(t[4 * ch] * sd[ch] + mean[ch])), acc);
        v = acc;
    }
    out[i] = f2h_bits(v);
}

// RMS norm over a pixel's c channels (x / sqrt(mean(x^2) + 1e-24 / c) * gamma, engine.cpp:725-727), then SiLU (mode
// 0), or not (mode 1), or a plain half copy (mode 2). 16 lanes a row, J = cp / 64 chunks of 4 channels a lane; x fp32
// rows of stride cs (c a multiple of 4); y half rows of stride cp. Grid output (compact = 0): every buffer row of y,
// ring and slack rows and channels past c zero. Compact output: y row p = pixel p (y * w + x), p < rows.
template <int J>
__global__ __launch_bounds__(256) void vae_norm_kernel(const float* __restrict__ xg, uint32_t cs, GridDims g,
                                                       uint32_t c, const float* __restrict__ gamma, int mode,
                                                       int compact, uint32_t rows, uint16_t* __restrict__ y)
{
    constexpr uint32_t cp = 64 * J;
    const uint32_t r = (blockIdx.x * 256 + threadIdx.x) >> 4;
    const uint32_t l = threadIdx.x & 15;
    if (r >= rows) // whole 16-lane groups leave together
        return;
    uint16_t* yr = y + uint64_t(r) * cp;
    uint32_t py, px;
    bool on;
    if (compact) {
        py = r / g.w;
        px = r - py * g.w;
        on = true;
    } else {
        on = g.pixel32(r, py, px);
    }
    if (!on) {
#pragma unroll
        for (int j = 0; j < J; ++j)
            *reinterpret_cast<u32x2*>(yr + 4 * (l + 16 * j)) = u32x2{0, 0};
        return;
    }
    const float* xr = xg + g.row_of(py, px) * cs;
    f32x4 v[J];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t k = 4 * (l + 16 * j);
        v[j] = k < c ? *reinterpret_cast<const f32x4*>(xr + k) : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            ss = fmaf(v[j][e], v[j][e], ss);
    }
    float sc = 1.0f;
    if (mode != 2) {
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1)
            ss += __shfl_xor(ss, m, 16);
        sc = rsqrtf(ss / float(c) + 1e-24f / float(c));
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t k = 4 * (l + 16 * j);
        float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (k < c) {
            const f32x4 gm = mode == 2 ? f32x4{1, 1, 1, 1} : *reinterpret_cast<const f32x4*>(gamma + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float t = mode == 2 ? v[j][e] : v[j][e] * sc * gm[e];
                if (mode == 0)
                    t = t / (1.0f + __expf(-t));
                o[e] = t;
            }
        }
        *reinterpret_cast<u32x2*>(yr + k) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
    }
}

// Zeroes the rows of a 16-bit padded grid (ld channels a row, a multiple of 8) that hold no pixel: the slack rows, the
// top and bottom ring rows and each image row's two ring pixels, 2 (w + 3) + 2 (w + 2) + 2 h rows in all. One thread a
// (row, 8 channels).
__global__ __launch_bounds__(256) void vae_ring_zero_kernel(uint16_t* __restrict__ y, GridDims g, uint32_t ld)
{
    const uint32_t q = ld / 8, i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t edge = g.slack() + g.pw(), n = 2 * edge + 2 * g.h; // rows
    if (i >= n * q)
        return;
    const uint32_t k = i / q, j = i - k * q;
    uint64_t r;
    if (k < edge) // slack before, top ring row
        r = k;
    else if (k < 2 * edge) // bottom ring row, slack after
        r = g.rows() - 2 * edge + k;
    else { // image row y's left or right ring pixel
        const uint32_t y = (k - 2 * edge) / 2, right = (k - 2 * edge) % 2;
        r = g.slack() + uint64_t(y + 1) * g.pw() + (right ? g.pw() - 1 : 0);
    }
    *reinterpret_cast<u32x4*>(y + r * ld + 8 * j) = u32x4{0, 0, 0, 0};
}

// Nearest 2x: the half padded grid of the 2h x 2w image (cp channels) from the fp32 grid of the h x w one (c
// channels, a multiple of 4, stride cs). One thread a (output row, 4 channels); 32-bit indexing.
__global__ __launch_bounds__(256) void vae_up_kernel(const float* __restrict__ x, uint32_t cs, GridDims gi,
                                                     uint32_t c, GridDims go, uint32_t cp, uint16_t* __restrict__ y)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x, q = cp / 4;
    if (i >= uint32_t(go.rows()) * q)
        return;
    const uint32_t r = i / q, k = 4 * (i - r * q);
    uint32_t py, px;
    f32x4 v{0, 0, 0, 0};
    if (k < c && go.pixel32(r, py, px))
        v = *reinterpret_cast<const f32x4*>(x + gi.row_of(py / 2, px / 2) * cs + k);
    *reinterpret_cast<u32x2*>(y + uint64_t(i) * 4) = u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
}

// Row softmax for the mid block's attention: p[j] = exp(scale (s[j] - max)) / sum over the n real columns, as half
// (the reference's halves() of P, engine.cpp:773), 0
// for the padding columns up to ld. One block a row: one read for the max and the sum together (each thread keeps a
// running max and a sum rescaled to it; pairs merge the same way), one more to write P.
__device__ inline void ms_merge(float& m, float& s, float m2, float s2)
{
    const float mm = fmaxf(m, m2);
    s = (m == -INFINITY ? 0.0f : s * __expf(m - mm)) + (m2 == -INFINITY ? 0.0f : s2 * __expf(m2 - mm));
    m = mm;
}

// The same softmax with the row held in registers (NV float4 a thread, rows up to 1024 NV): one read of the scores
// instead of two. Out-of-row columns (n .. ld) get probability 0.
template <int NV>
__global__ __launch_bounds__(256) void vae_softmax1_kernel(const float* __restrict__ s, uint32_t n, uint32_t ld,
                                                           float scale, uint16_t* __restrict__ p)
{
    __shared__ float red[2][4];
    const float* sr = s + uint64_t(blockIdx.x) * ld;
    uint16_t* pr = p + uint64_t(blockIdx.x) * ld;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    f32x4 v[NV];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t j = 4 * (tid + 256 * i);
        v[i] = j < ld ? *reinterpret_cast<const f32x4*>(sr + j) : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[i][e] = j + e < n ? scale * v[i][e] : -INFINITY;
            m = fmaxf(m, v[i][e]);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0)
        red[0][wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[i][e] = __expf(v[i][e] - m);
            sum += v[i][e];
        }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        sum += __shfl_xor(sum, o);
    if (lane == 0)
        red[1][wave] = sum;
    __syncthreads();
    const float inv = 1.0f / (red[1][0] + red[1][1] + red[1][2] + red[1][3]);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t j = 4 * (tid + 256 * i);
        if (j < ld)
            *reinterpret_cast<u32x2*>(pr + j) = u32x2{pack_f16x2(v[i][0] * inv, v[i][1] * inv),
                                                      pack_f16x2(v[i][2] * inv, v[i][3] * inv)};
    }
}

__global__ __launch_bounds__(256) void vae_softmax_kernel(const float* __restrict__ s, uint32_t n, uint32_t ld,
                                                          float scale, uint16_t* __restrict__ p)
{
    __shared__ float rm[4], rs[4];
    const float* sr = s + uint64_t(blockIdx.x) * ld;
    uint16_t* pr = p + uint64_t(blockIdx.x) * ld;
    float m = -INFINITY, sum = 0.0f; // in units of scale * s
    for (uint32_t j = 4 * threadIdx.x; j < n; j += 1024) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(sr + j); // n is a multiple of 4 here or the tail is masked
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (j + e < n)
                ms_merge(m, sum, scale * v[e], 1.0f);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(sum, o);
        ms_merge(m, sum, m2, s2);
    }
    if ((threadIdx.x & 63) == 0) {
        rm[threadIdx.x >> 6] = m;
        rs[threadIdx.x >> 6] = sum;
    }
    __syncthreads();
    m = rm[0];
    sum = rs[0];
    for (int i = 1; i < 4; ++i)
        ms_merge(m, sum, rm[i], rs[i]);
    const float inv = 1.0f / sum;
    for (uint32_t j = 4 * threadIdx.x; j < ld; j += 1024) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(sr + j);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = j + e < n ? __expf(scale * v[e] - m) * inv : 0.0f;
        *reinterpret_cast<u32x2*>(pr + j) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
    }
}

// x (fp32 grid, stride cs) += y (compact [pixels][cs]) over c channels. One thread a (pixel, channel).
__global__ __launch_bounds__(256) void vae_add_kernel(float* __restrict__ x, uint32_t cs, GridDims g, uint32_t c,
                                                      const float* __restrict__ y)
{
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= uint64_t(g.h) * g.w * c)
        return;
    const uint64_t p = i / c;
    const uint32_t k = uint32_t(i % c);
    x[g.row_of(uint32_t(p / g.w), uint32_t(p % g.w)) * cs + k] += y[p * cs + k];
}

// fp32 grid (stride cs, c channels) -> compact [pixels][c] (probes).
__global__ __launch_bounds__(256) void vae_compact_kernel(const float* __restrict__ x, uint32_t cs, GridDims g,
                                                          uint32_t c, float* __restrict__ y)
{
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= uint64_t(g.h) * g.w * c)
        return;
    const uint64_t p = i / c;
    y[i] = x[g.row_of(uint32_t(p / g.w), uint32_t(p % g.w)) * cs + i % c];
}

// conv_out (3 x 3, c -> 3 channels, engine.cpp:940-946) fused with the clamp to RGBA (engine.cpp:948-953). Three
// output channels are too few for the matrix cores (a 64-channel tile computes 61 zero channels), so: a workgroup
// takes a 16 x 16 pixel tile, stages its 18 x 18 input neighbourhood (c channels, rows padded by 8 so the 16 lanes of a
// pixel row read distinct banks) and the 3 x 9 x c weights in LDS with whole-row loads, then each thread sums its
// pixel's 9 taps from LDS (weights: broadcasts), half pairs by v_dot2_f32_f16 with fp32 accumulation. x: the half
// grid (rows of stride xs, zero ring and zero channels past the input's); c: the input's channels rounded up to 8
// (<= xs, cs <= 128); w: the packed weight rows [3][9][cs]; pre (may be NULL): the unclamped values into the fp32 grid
// rows (stride ps), for probes.
constexpr int kCoTile = 16;
struct alignas(16) HalfQuad { // 4 half pairs: one 16-byte LDS access
    f16x2cv v[4];
};
__global__ __launch_bounds__(256) void vae_conv_out_kernel(const uint16_t* __restrict__ x, uint32_t xs, uint32_t cs,
                                                           uint32_t c,
                                                           GridDims g, const uint16_t* __restrict__ w,
                                                           const float* __restrict__ bias, float* __restrict__ rgba,
                                                           float* __restrict__ pre, uint32_t ps)
{
    // (operands are read as half pairs: no bit casts of vector elements, which this compiler gets wrong)
    constexpr int NB = kCoTile + 2;
    __shared__ HalfQuad sw[3][9][16];
    extern __shared__ __attribute__((aligned(16))) uint16_t sx[]; // NB x NB pixels x (c + 8): the launch's size
    const uint32_t pst = c + 8; // LDS pixel stride (elements)
    const uint32_t tid = threadIdx.x, cq = c / 8;
    const uint32_t ty0 = blockIdx.y * kCoTile, tx0 = blockIdx.x * kCoTile;
    for (uint32_t i = tid; i < 3 * 9 * cq; i += 256) {
        const uint32_t o = i / (9 * cq), r = i - o * 9 * cq, tap = r / cq, j = r - tap * cq;
        sw[o][tap][j] = *reinterpret_cast<const HalfQuad*>(w + (uint64_t(o) * 9 + tap) * cs + 8 * j);
    }
    // neighbourhood pixel (qy, qx) is grid pixel (ty0 + qy - 1, tx0 + qx - 1): grid row slack + (ty0 + qy) (w + 2) +
    // tx0 + qx, inside the grid while ty0 + qy <= h + 1 and tx0 + qx <= w + 1
    for (uint32_t i = tid; i < NB * NB * cq; i += 256) {
        const uint32_t q = i / cq, k = i - q * cq, qy = q / NB, qx = q - qy * NB;
        u32x4 v = u32x4{0, 0, 0, 0};
        if (ty0 + qy <= g.h + 1 && tx0 + qx <= g.w + 1)
            v = *reinterpret_cast<const u32x4*>(x + (g.slack() + uint64_t(ty0 + qy) * g.pw() + tx0 + qx) * xs + 8 * k);
        *reinterpret_cast<u32x4*>(sx + q * pst + 8 * k) = v;
    }
    __syncthreads();
    const uint32_t ly = tid / kCoTile, lx = tid - ly * kCoTile, py = ty0 + ly, px = tx0 + lx;
    if (py >= g.h || px >= g.w)
        return;
    float acc[3] = {bias[0], bias[1], bias[2]};
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
        const int dy = tap / 3, dx = tap - 3 * dy;
        const HalfQuad* xq = reinterpret_cast<const HalfQuad*>(sx + ((ly + dy) * NB + lx + dx) * pst);
        for (uint32_t j = 0; j < cq; ++j) {
            const HalfQuad a = xq[j];
#pragma unroll
            for (int o = 0; o < 3; ++o) {
                const HalfQuad wq = sw[o][tap][j];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[o] = __builtin_amdgcn_fdot2(a.v[e], wq.v[e], acc[o], false);
            }
        }
    }
    if (pre)
#pragma unroll
        for (int o = 0; o < 3; ++o)
            pre[g.row_of(py, px) * ps + o] = acc[o];
    const uint64_t p = uint64_t(py) * g.w + px;
    *reinterpret_cast<f32x4*>(rgba + 4 * p) = f32x4{fminf(1.0f, fmaxf(-1.0f, acc[0])), fminf(1.0f, fmaxf(-1.0f, acc[1])),
                                                    fminf(1.0f, fmaxf(-1.0f, acc[2])), 1.0f};
}

// conv_out over 96 input channels on the matrix cores (v_mfma_f32_16x16x32_f16). The weights are the A operand: its
// 16 rows are the 3 output channels and 13 zero rows, and a tap's 96 channels are three 32-deep k chunks, so the 27
// fragments stay in registers. 16 pixels of one tile row are the B operand, one 16-byte LDS read a lane from the
// neighbourhood (pixel stride 208 B: the 16 pixels of a read fall on distinct bank groups). A lane of the product
// holds outputs 4 g4 .. 4 g4 + 3 of pixel r16, so the lanes with g4 = 0 hold each pixel's (r, g, b) for one
// 16-byte RGBA store. Wave w takes tile rows 4 w .. 4 w + 3: four independent accumulator chains of 27 products.
__global__ __launch_bounds__(256) void vae_conv_out96_kernel(const uint16_t* __restrict__ x, uint32_t xs, uint32_t cs,
                                                             GridDims g, const uint16_t* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             float* __restrict__ rgba, float* __restrict__ pre,
                                                             uint32_t ps)
{
    constexpr uint32_t NB = kCoTile + 2, C = 96, PST = C + 8, CQ = C / 8;
    static_assert(kCoTile == 16, "a tile row is one 16-pixel B operand, four rows a wave");
    __shared__ __attribute__((aligned(16))) uint16_t sx[NB * NB * PST];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
    const uint32_t ty0 = blockIdx.y * kCoTile, tx0 = blockIdx.x * kCoTile;
    // the weight fragments (rows past the 3 outputs zero), loaded while the neighbourhood comes in
    bf16x8 wf[9][3];
#pragma unroll
    for (int tap = 0; tap < 9; ++tap)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            wf[tap][j] = r16 < 3
                             ? *reinterpret_cast<const bf16x8*>(w + (uint64_t(r16) * 9 + tap) * cs + 32 * j + 8 * g4)
                             : bf16x8{};
    // neighbourhood pixel (qy, qx) is grid pixel (ty0 + qy - 1, tx0 + qx - 1): grid row slack + (ty0 + qy) (w + 2) +
    // tx0 + qx, inside the grid while ty0 + qy <= h + 1 and tx0 + qx <= w + 1 (zeros beyond). All of a thread's
    // loads go out before its LDS stores (a load-store loop would wait for each load in turn).
    constexpr uint32_t NF = NB * NB * CQ, NL = (NF + 255) / 256;
    u32x4 v[NL];
#pragma unroll
    for (uint32_t n = 0; n < NL; ++n) {
        const uint32_t i = tid + 256 * n, q = i / CQ, k = i - q * CQ, qy = q / NB, qx = q - qy * NB;
        v[n] = u32x4{0, 0, 0, 0};
        if (i < NF && ty0 + qy <= g.h + 1 && tx0 + qx <= g.w + 1)
            v[n] = *reinterpret_cast<const u32x4*>(x + (g.slack() + uint64_t(ty0 + qy) * g.pw() + tx0 + qx) * xs +
                                                   8 * k);
    }
#pragma unroll
    for (uint32_t n = 0; n < NL; ++n) {
        const uint32_t i = tid + 256 * n;
        if (i < NF)
            *reinterpret_cast<u32x4*>(sx + i / CQ * PST + 8 * (i % CQ)) = v[n];
    }
    __syncthreads();
    f32x4 acc[4] = {};
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
        const uint32_t dy = tap / 3, dx = tap - 3 * dy;
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bf16x8 b = *reinterpret_cast<const bf16x8*>(
                    sx + ((4 * wave + r + dy) * NB + r16 + dx) * PST + 32 * j + 8 * g4);
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, wf[tap][j]),
                                                                 __builtin_bit_cast(f16x8, b), acc[r], 0, 0, 0);
            }
    }
    if (g4 != 0)
        return;
    const uint32_t px = tx0 + r16;
    const float b0 = bias[0], b1 = bias[1], b2 = bias[2];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t py = ty0 + 4 * wave + r;
        if (py < g.h && px < g.w) {
            const float o0 = acc[r][0] + b0, o1 = acc[r][1] + b1, o2 = acc[r][2] + b2;
            if (pre) {
                float* q = pre + g.row_of(py, px) * ps;
                q[0] = o0;
                q[1] = o1;
                q[2] = o2;
            }
            *reinterpret_cast<f32x4*>(rgba + 4 * (uint64_t(py) * g.w + px)) =
                f32x4{fminf(1.0f, fmaxf(-1.0f, o0)), fminf(1.0f, fmaxf(-1.0f, o1)), fminf(1.0f, fmaxf(-1.0f, o2)), 1.0f};
        }
    }
}

// A weight's 16-bit source value as IEEE half: bf16 rounded to the nearest half, or a half as it is.
__device__ inline uint16_t w_half(uint16_t v, bool src_f16) { return src_f16 ? v : f2h_bits(bf2f_bits(v)); }

// A PyTorch conv weight [parts * co][ci][kt][k][k] (bf16 or half; kt time taps of a causal 3-D conv, the last one
// used: a single frame sees only it) -> [parts][cop][k * k][cip] half, tap-major, zero-padded. One thread an output
// value.
__global__ __launch_bounds__(256) void vae_pack_kernel(const uint16_t* __restrict__ src, int src_f16, uint32_t parts,
                                                       uint32_t co, uint32_t ci, uint32_t kt, uint32_t kk,
                                                       uint32_t cop, uint32_t cip, uint16_t* __restrict__ dst)
{
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    const uint64_t n = uint64_t(parts) * cop * kk * cip;
    if (i >= n)
        return;
    const uint32_t c = uint32_t(i % cip);
    const uint64_t q = i / cip;
    const uint32_t tap = uint32_t(q % kk);
    const uint64_t po = q / kk;
    const uint32_t o = uint32_t(po % cop), part = uint32_t(po / cop);
    uint16_t v = 0;
    if (o < co && c < ci)
        v = w_half(src[((uint64_t(part * co + o) * ci + c) * kt + (kt - 1)) * kk + tap], src_f16);
    dst[i] = v;
}

// A 3 x 3 conv weight packed dense for conv3x3_dense: dst [cop][kp], k = tap ci + c for k < 9 ci, zero beyond and
// for rows past co (source as vae_pack_kernel's, one part).
__global__ __launch_bounds__(256) void vae_pack_dense_kernel(const uint16_t* __restrict__ src, int src_f16,
                                                             uint32_t co, uint32_t ci, uint32_t kt, uint32_t cop,
                                                             uint32_t kp, uint16_t* __restrict__ dst)
{
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= uint64_t(cop) * kp)
        return;
    const uint32_t o = uint32_t(i / kp), k = uint32_t(i - uint64_t(o) * kp);
    uint16_t v = 0;
    if (o < co && k < 9 * ci) {
        const uint32_t tap = k / ci, c = k - tap * ci;
        v = w_half(src[((uint64_t(o) * ci + c) * kt + (kt - 1)) * 9 + tap], src_f16);
    }
    dst[i] = v;
}

// fp32 vector [parts * n] -> [parts][np] zero-padded.
__global__ __launch_bounds__(256) void vae_pack_vec_kernel(const float* __restrict__ src, uint32_t parts, uint32_t n,
                                                           uint32_t np, float* __restrict__ dst)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= parts * np)
        return;
    const uint32_t k = i % np, part = i / np;
    dst[i] = k < n ? src[part * n + k] : 0.0f;
}

// post_quant_conv's weight [z][z] from its 16-bit source to the half values it multiplies with, held as floats.
__global__ __launch_bounds__(256) void vae_w16_to_f32_kernel(const uint16_t* __restrict__ src, int src_f16, uint32_t n,
                                                             float* __restrict__ dst)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n)
        dst[i] = h2f_bits(w_half(src[i], src_f16));
}

// An fp32 operand of the attention's products as two half planes, hi = half(v) and lo = half(v - hi) (the sum holds
// v to about 22 bits: the reference keeps K and V^T in fp32, engine.cpp:764-773): rows [rows][cols] (stride ld) plus
// an optional per-row bias (V^T's value bias) -> hi at dst + r * dld + c, lo at that + lo_off. One thread a value.
__global__ __launch_bounds__(256) void vae_split_kernel(const float* __restrict__ x, uint32_t rows, uint32_t cols,
                                                        uint32_t ld, const float* __restrict__ bias,
                                                        uint16_t* __restrict__ dst, uint32_t dld, uint64_t lo_off)
{
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= uint64_t(rows) * cols)
        return;
    const uint32_t r = uint32_t(i / cols), c = uint32_t(i - uint64_t(r) * cols);
    const float v = x[uint64_t(r) * ld + c] + (bias ? bias[r] : 0.0f);
    const uint16_t hi = f2h_bits(v);
    uint16_t* d = dst + uint64_t(r) * dld + c;
    d[0] = hi;
    d[lo_off] = f2h_bits(v - h2f_bits(hi));
}

inline uint32_t blocks_for(uint64_t n) { return uint32_t((n + 255) / 256); }

// MK_OK, or the HIP error as a status (hip_check records a failure; it is only called on one)
inline mk_status hip_ok(hipError_t e, const char* what) { return e == hipSuccess ? MK_OK : hip_check(e, what); }

} // namespace
} // namespace mk

using namespace mk;

// A norm + SiLU that a 96- or 192-channel conv's epilogue applies to its rows: gain g, into the half grid buf (rows of
// the conv's channels; its slack and ring rows zeroed by mk_vae::conv3)
struct NormTo {
    const float* g = nullptr;
    uint16_t* buf = nullptr;
    bool only = false; // the conv's own fp32 rows are not needed (the decode's last residual, without probes)
};

struct mk_vae {
    // A convolution's packed weight [parts][cop][k * k][cip] and bias [parts][cop] (fp32).
    struct Conv {
        uint16_t* w = nullptr;
        float* b = nullptr;
        uint32_t co = 0, ci = 0, k = 0, parts = 1;
        bool dense = false; // 3 x 3 weights packed [cop][kp] for conv3x3_dense (ci not a multiple of 64)
        bool narrow = false; // a 3 x 3 conv whose output channels, an odd multiple of 96, stay unpadded (128 x 96 tiles)
        uint32_t cop() const { return narrow ? co : cpad(co); }
        uint32_t cip() const { return cpad(ci); }
        uint32_t kp() const { return (9 * ci + 63) / 64 * 64; }
    };
    struct Res {
        float *g1 = nullptr, *g2 = nullptr;
        Conv c1, c2, sc;
        bool shortcut = false;
    };
    // a checkpoint tensor: where it goes and how
    struct Slot {
        enum Kind { CONV_W, CONV_B, VEC, PQ_W } kind;
        Conv* conv = nullptr;
        float* vec = nullptr;
        uint32_t n = 0; // VEC: values
        std::vector<int64_t> dims; // PyTorch shape of the synthetic tensor
    };

    uint32_t base = 0, z = 0;
    std::vector<float> mean, sd;
    hipStream_t stream = nullptr;
    std::vector<void*> allocs;
    std::map<std::string, Slot> slots;
    std::vector<std::unique_ptr<Conv>> convs;

    float *pq_w = nullptr, *pq_b = nullptr, *d_mean = nullptr, *d_sd = nullptr;
    Conv conv_in, qkv, proj, conv_out;
    Res mid0, mid1;
    float* attn_g = nullptr;
    struct Up {
        Res res[3];
        bool up = false;
        Conv conv;
        uint32_t cin = 0, cout = 0;
    } ups[4];
    float* out_g = nullptr;

    // scratch
    struct Buf {
        void* p = nullptr;
        size_t bytes = 0;
    };
    Buf x, y, t, a, sc, qb, kb, vtb, kf, sb, pb, ob, pj, tok, rgba, probe_buf;
    mk_probe_fn probe = nullptr;
    void* probe_user = nullptr;

    ~mk_vae()
    {
        if (stream)
            (void)hipStreamSynchronize(stream);
        for (void* p : allocs)
            (void)hipFree(p);
        for (Buf* b : {&x, &y, &t, &a, &sc, &qb, &kb, &vtb, &kf, &sb, &pb, &ob, &pj, &tok, &rgba, &probe_buf})
            if (b->p)
                (void)hipFree(b->p);
        if (stream)
            (void)hipStreamDestroy(stream);
    }

    mk_status alloc(size_t bytes, void** p)
    {
        MK_HIP(hipMalloc(p, bytes));
        MK_HIP(hipMemsetAsync(*p, 0, bytes, stream)); // ordered before the stream's packing kernels
        allocs.push_back(*p);
        return MK_OK;
    }
    mk_status ensure(Buf& b, size_t bytes)
    {
        if (b.bytes >= bytes)
            return MK_OK;
        MK_HIP(hipStreamSynchronize(stream));
        if (b.p)
            MK_HIP(hipFree(b.p));
        b.p = nullptr;
        b.bytes = 0;
        MK_HIP(hipMalloc(&b.p, bytes));
        MK_HIP(hipMemsetAsync(b.p, 0, bytes, stream)); // ordered before the stream's kernels
        b.bytes = bytes;
        return MK_OK;
    }

    // dense_ok: a 3 x 3 conv run by conv3 may take dense weights (not conv_out, whose kernel reads [3][9][cip]);
    // narrow_ok: its output may keep 96 channels unpadded (not where a 1 x 1 shortcut, padded to 64, writes the same
    // rows)
    mk_status conv(Conv& c, const std::string& name, uint32_t co, uint32_t ci, uint32_t k, uint32_t parts = 1,
                   bool dense_ok = true, bool narrow_ok = true)
    {
        c.co = co;
        c.ci = ci;
        c.k = k;
        c.parts = parts;
        c.dense = dense_ok && k == 3 && parts == 1 && ci % 64 && ci % 8 == 0 && ci <= 512;
        c.narrow = narrow_ok && dense_ok && k == 3 && parts == 1 && co % 64 && co % 96 == 0;
        MK_TRY(alloc(size_t(parts) * c.cop() * k * k * c.cip() * 2, reinterpret_cast<void**>(&c.w)));
        MK_TRY(alloc(size_t(parts) * c.cop() * 4, reinterpret_cast<void**>(&c.b)));
        Slot w{Slot::CONV_W, &c, nullptr, 0, {int64_t(parts) * co, ci, k, k}};
        Slot b{Slot::CONV_B, &c, nullptr, 0, {int64_t(parts) * co}};
        slots[name + ".weight"] = w;
        slots[name + ".bias"] = b;
        return MK_OK;
    }
    mk_status vec(float** p, const std::string& name, uint32_t n)
    {
        MK_TRY(alloc(size_t(n) * 4, reinterpret_cast<void**>(p)));
        slots[name] = Slot{Slot::VEC, nullptr, *p, n, {int64_t(n)}};
        return MK_OK;
    }
    mk_status res(Res& r, const std::string& p, uint32_t ci, uint32_t co)
    {
        MK_TRY(vec(&r.g1, p + ".norm1.gamma", ci));
        MK_TRY(conv(r.c1, p + ".conv1", co, ci, 3));
        MK_TRY(vec(&r.g2, p + ".norm2.gamma", co));
        r.shortcut = ci != co;
        MK_TRY(conv(r.c2, p + ".conv2", co, co, 3, 1, true, !r.shortcut));
        if (r.shortcut)
            MK_TRY(conv(r.sc, p + ".conv_shortcut", co, ci, 1));
        return MK_OK;
    }

    mk_status build()
    {
        const uint32_t b = base, d0 = 4 * b;
        MK_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        MK_TRY(alloc(size_t(z) * z * 4, reinterpret_cast<void**>(&pq_w)));
        MK_TRY(alloc(size_t(z) * 4, reinterpret_cast<void**>(&pq_b)));
        slots["post_quant_conv.weight"] = Slot{Slot::PQ_W, nullptr, pq_w, z * z, {z, z, 1, 1}};
        slots["post_quant_conv.bias"] = Slot{Slot::VEC, nullptr, pq_b, z, {z}};
        MK_TRY(alloc(size_t(z) * 4, reinterpret_cast<void**>(&d_mean)));
        MK_TRY(alloc(size_t(z) * 4, reinterpret_cast<void**>(&d_sd)));
        MK_HIP(hipMemcpy(d_mean, mean.data(), z * 4, hipMemcpyHostToDevice));
        MK_HIP(hipMemcpy(d_sd, sd.data(), z * 4, hipMemcpyHostToDevice));
        MK_TRY(conv(conv_in, "decoder.conv_in", d0, z, 3));
        MK_TRY(res(mid0, "decoder.mid_block.resnets.0", d0, d0));
        MK_TRY(vec(&attn_g, "decoder.mid_block.attentions.0.norm.gamma", d0));
        MK_TRY(conv(qkv, "decoder.mid_block.attentions.0.to_qkv", d0, d0, 1, 3));
        MK_TRY(conv(proj, "decoder.mid_block.attentions.0.proj", d0, d0, 1));
        MK_TRY(res(mid1, "decoder.mid_block.resnets.1", d0, d0));
        const uint32_t ins[4] = {4 * b, 2 * b, 2 * b, b}, outs[4] = {4 * b, 4 * b, 2 * b, b};
        for (int i = 0; i < 4; ++i) {
            const std::string p = "decoder.up_blocks." + std::to_string(i);
            Up& u = ups[i];
            u.cin = ins[i];
            u.cout = outs[i];
            for (int j = 0; j < 3; ++j)
                MK_TRY(res(u.res[j], p + ".resnets." + std::to_string(j), j ? outs[i] : ins[i], outs[i]));
            u.up = i < 3;
            if (u.up)
                MK_TRY(conv(u.conv, p + ".upsamplers.0.resample.1", outs[i] / 2, outs[i], 3));
        }
        MK_TRY(vec(&out_g, "decoder.norm_out.gamma", b));
        MK_TRY(conv(conv_out, "decoder.conv_out", 3, b, 3, 1, false));
        return MK_OK;
    }

    // One tensor from device memory in PyTorch layout: conv weights 16-bit [parts * co][ci][kt][k][k] (kt >= 1; half,
    // or bf16 when src_f16 is false), everything else fp32. Convolution weights are stored as half.
    mk_status put(const Slot& s, const void* src, uint32_t kt, bool src_f16)
    {
        switch (s.kind) {
        case Slot::CONV_W: {
            const Conv& c = *s.conv;
            if (c.dense) {
                const uint64_t n = uint64_t(c.cop()) * c.kp();
                vae_pack_dense_kernel<<<blocks_for(n), 256, 0, stream>>>(static_cast<const uint16_t*>(src), src_f16,
                                                                         c.co, c.ci, kt, c.cop(), c.kp(), c.w);
                break;
            }
            const uint64_t n = uint64_t(c.parts) * c.cop() * c.k * c.k * c.cip();
            vae_pack_kernel<<<blocks_for(n), 256, 0, stream>>>(static_cast<const uint16_t*>(src), src_f16, c.parts,
                                                              c.co, c.ci, kt, c.k * c.k, c.cop(), c.cip(), c.w);
            break;
        }
        case Slot::CONV_B: {
            const Conv& c = *s.conv;
            vae_pack_vec_kernel<<<blocks_for(c.parts * c.cop()), 256, 0, stream>>>(
                static_cast<const float*>(src), c.parts, c.co, c.cop(), c.b);
            break;
        }
        case Slot::PQ_W: // 16-bit [z][z] -> its half values as fp32
            vae_w16_to_f32_kernel<<<blocks_for(s.n), 256, 0, stream>>>(static_cast<const uint16_t*>(src), src_f16,
                                                                       s.n, s.vec);
            break;
        case Slot::VEC:
            MK_HIP(hipMemcpyAsync(s.vec, src, size_t(s.n) * 4, hipMemcpyDeviceToDevice, stream));
            return MK_OK;
        }
        MK_LAUNCH_CHECK("vae weight pack");
        return MK_OK;
    }

    // ---- the decoder ----
    // the rows of a half grid that hold no pixel (a conv whose tiles cover pixels only leaves them unwritten)
    mk_status zero_ring(uint16_t* buf, GridDims g, uint32_t ld)
    {
        const uint64_t n = (2ull * (g.slack() + g.pw()) + 2ull * g.h) * (ld / 8);
        vae_ring_zero_kernel<<<blocks_for(n), 256, 0, stream>>>(buf, g, ld);
        MK_LAUNCH_CHECK("vae_ring_zero");
        return MK_OK;
    }
    // Whether conv c's epilogue can norm its rows: 96 output channels unpadded (one 128 x 96 tile spans a row) or 192
    // (a 256 x 192 tile). The normed grid has rows of c.co channels.
    static bool norm_fusable(const Conv& c)
    {
        return c.k == 3 && c.parts == 1 && ((c.narrow && c.co == 96) || (c.co == 192 && c.cop() == 192));
    }
    // Whether a conv reads a normed grid of rows of C channels as its input: dense K over 96, or 192 channels.
    static bool reads_normed(const Conv& c, uint32_t C) { return c.ci == C && (c.dense || c.cip() == C); }
    // lda: the input rows' stride (0: c.cip()). only: the output is only the normed rows (half grid out, ldo = c.co);
    // else, with nt.g set, out gets the conv's fp32 rows (store or add) and nt.buf their norm.
    // up: the sums go to the nearest-2x grid up->out instead of back into out (an ADD; see conv3x3_up)
    mk_status conv3(const Conv& c, const void* in, GridDims g, void* out, uint32_t ldo, bool add, uint32_t lda = 0,
                    NormTo nt = {}, bool only = false, const ConvUp* up = nullptr)
    {
        mk_conv_args a{};
        a.x = in;
        a.w = c.w;
        a.bias = c.b;
        a.y = only ? static_cast<void*>(static_cast<uint16_t*>(out) + uint64_t(g.slack()) * ldo)
                   : static_cast<void*>(static_cast<float*>(out) + uint64_t(g.slack()) * ldo);
        a.h = g.h;
        a.width = g.w;
        a.c = c.cip();
        a.n = c.cop();
        a.ldy = ldo;
        a.y_dtype = only ? MK_F16 : MK_F32;
        a.epilogue = add ? MK_EPI_ADD : MK_EPI_STORE;
        ConvNorm nm;
        if (nt.g) {
            if (!norm_fusable(c))
                return fail(MK_ERR_ARG, "vae: a fused norm needs a conv with 96 or 192 unpadded output channels");
            MK_TRY(zero_ring(only ? static_cast<uint16_t*>(out) : nt.buf, g, c.co));
            nm.g = nt.g;
            if (!only) {
                nm.out = nt.buf + uint64_t(g.slack()) * c.co;
                nm.ld = c.co;
                nm.skip_y = nt.only;
            }
        }
        if (c.dense) {
            a.c = c.ci;
            return conv3x3_dense(&a, lda ? lda : c.cip(), stream, nt.g ? &nm : nullptr);
        }
        if (lda)
            return fail(MK_ERR_ARG, "vae: an input stride needs a dense conv");
        if (up)
            return nt.g ? fail(MK_ERR_ARG, "vae: a 2x-grid output has no norm") : conv3x3_up(&a, *up, stream);
        return nt.g ? conv3x3_fused(&a, nm, stream) : mk_conv3x3(&a, stream);
    }
    // 1 x 1 conv over rows (grid or compact), half operands: y[rows][ldo] (fp32 or half) = a[rows][cip] W^T + b (or +=)
    mk_status conv1(const Conv& c, uint32_t part, const void* a, uint64_t rows, void* out, uint32_t ldo,
                    uint32_t out_dtype, uint32_t epi)
    {
        mk_gemm_args g{};
        g.a = a;
        g.w = c.w + size_t(part) * c.cop() * c.cip();
        g.bias = c.b + size_t(part) * c.cop();
        g.c = out;
        g.M = uint32_t(rows);
        g.N = c.cop();
        g.K = c.cip();
        g.lda = c.cip();
        g.ldc = ldo;
        g.batch = 1;
        g.w_dtype = MK_F16;
        g.c_dtype = out_dtype;
        g.epilogue = epi;
        return mk_gemm(&g, stream);
    }
    mk_status norm(const void* xg, uint32_t cs, GridDims g, uint32_t c, const float* gamma, int mode, void* out,
                   uint32_t cp, int compact = 0, uint64_t rows = 0)
    {
        if (!compact)
            rows = g.rows();
        const dim3 grid(blocks_for(rows * 16));
        const float* x = static_cast<const float*>(xg);
        uint16_t* y = static_cast<uint16_t*>(out);
        switch (cp / 64) {
#define MK_VAE_NORM(J)                                                                                             \
    case J:                                                                                                        \
        vae_norm_kernel<J><<<grid, 256, 0, stream>>>(x, cs, g, c, gamma, mode, compact, uint32_t(rows), y);        \
        break;
            MK_VAE_NORM(1)
            MK_VAE_NORM(2)
            MK_VAE_NORM(3)
            MK_VAE_NORM(4)
            MK_VAE_NORM(5)
            MK_VAE_NORM(6)
            MK_VAE_NORM(7)
            MK_VAE_NORM(8)
#undef MK_VAE_NORM
        default:
            return fail(MK_ERR_ARG, "vae norm: more than 512 channels");
        }
        MK_LAUNCH_CHECK("vae_norm");
        return MK_OK;
    }
    mk_status probe_grid(const char* name, int layer, const void* xg, uint32_t cs, GridDims g, uint32_t c)
    {
        if (!probe)
            return MK_OK;
        const uint64_t n = uint64_t(g.h) * g.w * c;
        MK_TRY(ensure(probe_buf, n * 4));
        vae_compact_kernel<<<blocks_for(n), 256, 0, stream>>>(static_cast<const float*>(xg), cs, g, c,
                                                              static_cast<float*>(probe_buf.p));
        MK_LAUNCH_CHECK("vae_compact");
        std::vector<float> h(n);
        MK_HIP(hipMemcpyAsync(h.data(), probe_buf.p, n * 4, hipMemcpyDeviceToHost, stream));
        MK_HIP(hipStreamSynchronize(stream));
        probe(probe_user, name, layer, h.data(), n);
        return MK_OK;
    }

    // res_block (engine.cpp:732-746): x (fp32 grid, stride cs = c2.cop() after) <- conv2(silu(norm2(conv1(
    // silu(norm1(x)))))) + shortcut(x). x and the result may differ in channels; xs is x's stride. At 96 and 192
    // channels the norms come from the convs' epilogues: normed_in (rows of the channels) already holds silu(norm1(x)),
    // conv1 writes silu(norm2(.)) straight into t as conv2's half input, and with next.g conv2 also writes the norm the
    // next layer takes of the result into next.buf (which conv2 does not read).
    // With up, conv2's sums go to the nearest-2x grid (see conv3x3_up) and x is left as it was.
    mk_status res_block(const Res& r, GridDims g, float*& xp, uint32_t xs, float*& yp, const uint16_t* normed_in = nullptr,
                        NormTo next = {}, const ConvUp* up = nullptr)
    {
        const Conv &c1 = r.c1, &c2 = r.c2;
        const void* c1_in = a.p;
        uint32_t c1_lda = 0;
        if (normed_in) {
            c1_in = normed_in;
            c1_lda = c1.dense ? c1.ci : 0;
        } else {
            MK_TRY(norm(xp, xs, g, c1.ci, r.g1, 0, a.p, c1.cip()));
        }
        const void* c2_in = a.p;
        uint32_t c2_lda = 0;
        if (norm_fusable(c1) && reads_normed(c2, c1.co)) {
            uint16_t* tn = static_cast<uint16_t*>(t.p);
            MK_TRY(conv3(c1, c1_in, g, tn, c1.co, false, c1_lda, NormTo{r.g2, nullptr}, true));
            c2_in = tn;
            c2_lda = c2.dense ? c2.ci : 0;
        } else {
            MK_TRY(conv3(c1, c1_in, g, t.p, c1.cop(), false, c1_lda));
            MK_TRY(norm(t.p, c1.cop(), g, c1.co, r.g2, 0, a.p, c2.cip()));
        }
        if (r.shortcut) {
            // y = shortcut(x) over the grid rows, then y += conv2
            MK_TRY(norm(xp, xs, g, r.sc.ci, nullptr, 2, sc.p, r.sc.cip()));
            MK_TRY(conv1(r.sc, 0, static_cast<uint16_t*>(sc.p) + uint64_t(g.slack()) * r.sc.cip(), g.grid_rows(),
                         yp + uint64_t(g.slack()) * r.sc.cop(), r.sc.cop(), MK_F32, MK_EPI_STORE));
            if (up)
                return fail(MK_ERR_ARG, "vae: a 2x-grid output after a shortcut");
            MK_TRY(conv3(c2, c2_in, g, yp, c2.cop(), true, c2_lda, next));
            std::swap(xp, yp);
        } else {
            MK_TRY(conv3(c2, c2_in, g, xp, c2.cop(), true, c2_lda, next, false, up));
        }
        return MK_OK;
    }

    // vae_attention (engine.cpp:748-777): one head over the n pixels, d = c, in the reference's precision: the scores
    // are half queries times fp32 keys, the output half probabilities times fp32 values (its gemm_->encode with F32
    // K / V^T and halves() of Q and P, engine.cpp:764-773). The matrix cores multiply halves, so each fp32 operand
    // goes in as two half planes hi + lo (vae_split_kernel): scores = [Q | Q] [K_hi | K_lo]^T (a GEMM over 2 c), the
    // output = P [V^T_hi ; V^T_lo]^T with the two c-wide halves summed in the epilogue (MK_EPI_PAIR_SUM).
    mk_status attention(GridDims g, float* xp)
    {
        const uint32_t c = qkv.co, cp = qkv.cip();
        const uint64_t n = uint64_t(g.h) * g.w, np = (n + 63) / 64 * 64;
        // q2 [np][2 cp] = [Q | Q], k2 [np][2 cp] = [K_hi | K_lo], vt2 [2 cp][np] = [V^T_hi ; V^T_lo] (halves); kf the
        // fp32 projections (K [np][cp], then V^T [cp][np]); the normed pixels [np][cp] (rows past n zero)
        MK_TRY(ensure(qb, np * cp * 4));
        MK_TRY(ensure(kb, np * cp * 4));
        MK_TRY(ensure(vtb, np * cp * 4));
        MK_TRY(ensure(kf, np * cp * 4));
        MK_TRY(ensure(ob, np * cp * 2));
        MK_TRY(ensure(pj, np * cp * 4));
        MK_TRY(ensure(sc, np * cp * 2));
        MK_HIP(hipMemsetAsync(sc.p, 0, np * cp * 2, stream));
        uint16_t* xn = static_cast<uint16_t*>(sc.p);
        MK_TRY(norm(xp, cp, g, c, attn_g, 1, xn, cp, 1, n));
        // Q (with its bias) rounded to half, twice side by side; K (with its bias) in fp32, split
        uint16_t* q2 = static_cast<uint16_t*>(qb.p);
        MK_TRY(conv1(qkv, 0, xn, np, q2, 2 * cp, MK_F16, MK_EPI_STORE));
        MK_TRY(conv1(qkv, 0, xn, np, q2 + cp, 2 * cp, MK_F16, MK_EPI_STORE));
        float* kfp = static_cast<float*>(kf.p);
        MK_TRY(conv1(qkv, 1, xn, np, kfp, cp, MK_F32, MK_EPI_STORE));
        vae_split_kernel<<<blocks_for(np * cp), 256, 0, stream>>>(kfp, uint32_t(np), cp, cp, nullptr,
                                                                  static_cast<uint16_t*>(kb.p), 2 * cp, cp);
        MK_LAUNCH_CHECK("vae_split k");
        {
            // V^T [cp][np] = W_v xn^T in fp32, then + the value bias and split into rows [0, cp) and [cp, 2 cp)
            mk_gemm_args v{};
            v.a = qkv.w + size_t(2) * cp * cp;
            v.w = xn;
            v.c = kfp;
            v.M = cp;
            v.N = uint32_t(np);
            v.K = cp;
            v.lda = cp;
            v.ldc = int64_t(np);
            v.batch = 1;
            v.w_dtype = MK_F16;
            v.c_dtype = MK_F32;
            v.epilogue = MK_EPI_STORE;
            MK_TRY(mk_gemm(&v, stream));
            vae_split_kernel<<<blocks_for(np * cp), 256, 0, stream>>>(kfp, cp, uint32_t(np), uint32_t(np),
                                                                      qkv.b + size_t(2) * cp,
                                                                      static_cast<uint16_t*>(vtb.p), uint32_t(np),
                                                                      uint64_t(cp) * np);
            MK_LAUNCH_CHECK("vae_split vt");
        }
        // Queries in groups whose half P stays within 512 MB (one P V product each), and within a group in chunks
        // whose fp32 scores (near 128 MB) stay in the memory-side cache between the score GEMM that writes them and
        // the softmax that reads them. (At 128 x 128 pixels: one group, 8 chunks of 2048 queries.)
        const uint64_t qg = std::min<uint64_t>(n, std::max<uint64_t>(256, (uint64_t(1) << 28) / np / 256 * 256));
        const uint64_t qc = std::min<uint64_t>(qg, std::max<uint64_t>(256, (uint64_t(1) << 25) / np / 256 * 256));
        MK_TRY(ensure(sb, qc * np * 4));
        MK_TRY(ensure(pb, qg * np * 2));
        const float scale = 1.0f / std::sqrt(float(c));
        for (uint64_t g0 = 0; g0 < n; g0 += qg) {
            const uint64_t gm = std::min(qg, n - g0);
            for (uint64_t q0 = g0; q0 < g0 + gm; q0 += qc) {
                const uint64_t m = std::min(qc, g0 + gm - q0);
                mk_gemm_args s{};
                s.a = q2 + q0 * 2 * cp;
                s.w = kb.p;
                s.c = sb.p;
                s.M = uint32_t(m);
                s.N = uint32_t(np);
                s.K = 2 * cp;
                s.lda = 2 * cp;
                s.ldc = int64_t(np);
                s.batch = 1;
                s.w_dtype = MK_F16;
                s.c_dtype = MK_F32;
                s.epilogue = MK_EPI_STORE;
                MK_TRY(mk_gemm(&s, stream));
                float* sp = static_cast<float*>(sb.p);
                uint16_t* pp = static_cast<uint16_t*>(pb.p) + (q0 - g0) * np;
                // rows that fit the registers (up to 16384 columns) in one read, longer ones in two
                if (np <= 1024)
                    vae_softmax1_kernel<1><<<uint32_t(m), 256, 0, stream>>>(sp, uint32_t(n), uint32_t(np), scale, pp);
                else if (np <= 4096)
                    vae_softmax1_kernel<4><<<uint32_t(m), 256, 0, stream>>>(sp, uint32_t(n), uint32_t(np), scale, pp);
                else if (np <= 16384)
                    vae_softmax1_kernel<16><<<uint32_t(m), 256, 0, stream>>>(sp, uint32_t(n), uint32_t(np), scale, pp);
                else
                    vae_softmax_kernel<<<uint32_t(m), 256, 0, stream>>>(sp, uint32_t(n), uint32_t(np), scale, pp);
                MK_LAUNCH_CHECK("vae_softmax");
            }
            mk_gemm_args o{};
            o.a = pb.p;
            o.w = vtb.p;
            o.c = static_cast<uint16_t*>(ob.p) + g0 * cp;
            o.M = uint32_t(gm);
            o.N = 2 * cp;
            o.K = uint32_t(np);
            o.lda = int64_t(np);
            o.ldc = cp;
            o.batch = 1;
            o.w_dtype = MK_F16;
            o.c_dtype = MK_F16;
            o.epilogue = MK_EPI_PAIR_SUM;
            MK_TRY(mk_gemm(&o, stream));
        }
        MK_TRY(conv1(proj, 0, ob.p, n, pj.p, cp, MK_F32, MK_EPI_STORE));
        vae_add_kernel<<<blocks_for(n * c), 256, 0, stream>>>(xp, cp, g, c, static_cast<float*>(pj.p));
        MK_LAUNCH_CHECK("vae_add");
        return MK_OK;
    }

    // tokens (device) [th][tw][4 z] -> rgba (device) [16 th][16 tw][4]
    mk_status decode(const float* tokens, uint32_t th, uint32_t tw, float* out)
    {
        const uint32_t b = base, d0 = 4 * b;
        // the largest level's buffers: rows x the widest channels (padded) any buffer holds at that level; an upsample
        // conv's input has the previous level's channels (4b at levels 1 and 2, 2b at level 3)
        uint64_t most = 0;
        {
            GridDims g{2 * th, 2 * tw};
            const uint32_t ch[4] = {cpad(d0), cpad(4 * b), cpad(4 * b), cpad(2 * b)};
            for (int l = 0; l < 4; ++l) {
                most = std::max(most, g.rows() * std::max<uint64_t>(ch[l], 64));
                g = GridDims{2 * g.h, 2 * g.w};
            }
        }
        MK_TRY(ensure(x, most * 4));
        MK_TRY(ensure(y, most * 4));
        MK_TRY(ensure(t, most * 4));
        MK_TRY(ensure(a, most * 2));
        MK_TRY(ensure(sc, most * 2));
        GridDims g{2 * th, 2 * tw};
        vae_in_kernel<<<blocks_for(g.rows() * conv_in.cip()), 256, 0, stream>>>(
            tokens, tw, g, z, conv_in.cip(), d_mean, d_sd, pq_w, pq_b, static_cast<uint16_t*>(a.p));
        MK_LAUNCH_CHECK("vae_in");
        float* xp = static_cast<float*>(x.p);
        float* yp = static_cast<float*>(y.p);
        MK_TRY(conv3(conv_in, a.p, g, xp, conv_in.cop(), false));
        MK_TRY(probe_grid("vae_conv_in", -1, xp, conv_in.cop(), g, d0));
        MK_TRY(res_block(mid0, g, xp, cpad(d0), yp));
        MK_TRY(attention(g, xp));
        MK_TRY(res_block(mid1, g, xp, cpad(d0), yp));
        MK_TRY(probe_grid("vae_mid", -1, xp, cpad(d0), g, d0));
        uint32_t cs = cpad(d0);
        // At 96 channels each conv that produces x also writes the norm + SiLU its consumer takes of x (the next res
        // block's norm1, or norm_out before conv_out): `normed` is that grid (rows of 96) when the last conv wrote it.
        // A res block's conv2 writes it into a (conv2 reads t), the upsampling conv into sc (it reads a).
        auto takes_normed = [](const Res& r, const Conv& from) { return reads_normed(r.c1, from.co); };
        uint16_t* const na = static_cast<uint16_t*>(a.p);
        uint16_t* const ns = static_cast<uint16_t*>(sc.p);
        const uint16_t* normed = nullptr;
        for (int i = 0; i < 4; ++i) {
            Up& u = ups[i];
            // the last res block's conv2 can write the nearest-2x grid the upsampling conv reads (into sc, since its
            // input may be a): whole 192-channel tiles over the pixels of one image row each
            const Res& rl = u.res[2];
            const bool up_fused = u.up && !rl.shortcut && !rl.c2.dense && rl.c2.co % 192 == 0 &&
                                  rl.c2.cop() == rl.c2.co && u.cout == rl.c2.co && u.conv.cip() == rl.c2.co &&
                                  g.w % 256 == 0;
            uint16_t* const upbuf = up_fused ? ns : na;
            for (int j = 0; j < 3; ++j) {
                const Res& r = u.res[j];
                NormTo next{};
                if (norm_fusable(r.c2) && !r.shortcut) {
                    if (j < 2 && takes_normed(u.res[j + 1], r.c2))
                        next = NormTo{u.res[j + 1].g1, na};
                    else if (j == 2 && i == 3 && r.c2.co == 96 && conv_out.ci == 96)
                        next = NormTo{out_g, na, !probe}; // x itself is read only by the probe
                }
                ConvUp cu;
                if (j == 2 && up_fused) {
                    const GridDims g2{2 * g.h, 2 * g.w};
                    MK_TRY(zero_ring(ns, g2, u.conv.cip()));
                    cu = ConvUp{ns, u.conv.cip()};
                }
                MK_TRY(res_block(r, g, xp, cs, yp, normed, next, cu.out ? &cu : nullptr));
                normed = next.g ? next.buf : nullptr;
                cs = r.c2.cop();
            }
            if (u.up) {
                const GridDims g2{2 * g.h, 2 * g.w};
                if (!up_fused) {
                    vae_up_kernel<<<blocks_for(g2.rows() * u.conv.cip() / 4), 256, 0, stream>>>(
                        xp, cs, g, u.cout, g2, u.conv.cip(), na);
                    MK_LAUNCH_CHECK("vae_up");
                }
                // the conv's norm output goes to whichever of a and sc it does not read
                NormTo next{};
                if (norm_fusable(u.conv) && i + 1 < 4 && takes_normed(ups[i + 1].res[0], u.conv))
                    next = NormTo{ups[i + 1].res[0].g1, upbuf == na ? ns : na};
                MK_TRY(conv3(u.conv, upbuf, g2, yp, u.conv.cop(), false, 0, next));
                normed = next.g ? next.buf : nullptr;
                std::swap(xp, yp);
                g = g2;
                cs = u.conv.cop();
            }
            MK_TRY(probe_grid("vae_up", i, xp, cs, g, u.up ? u.conv.co : u.cout));
        }
        if (!normed)
            MK_TRY(norm(xp, cs, g, b, out_g, 0, na, conv_out.cip()));
        // (base <= 128: conv_out's input takes at most 128 padded channels)
        const dim3 cog((g.w + kCoTile - 1) / kCoTile, (g.h + kCoTile - 1) / kCoTile);
        const uint32_t c8 = (conv_out.ci + 7) / 8 * 8;
        const size_t lds = size_t(kCoTile + 2) * (kCoTile + 2) * (c8 + 8) * 2;
        if (c8 == 96)
            vae_conv_out96_kernel<<<cog, 256, 0, stream>>>(normed ? normed : na, normed ? 96 : conv_out.cip(),
                                                           conv_out.cip(), g, conv_out.w, conv_out.b, out,
                                                           probe ? yp : nullptr, conv_out.cop());
        else
            vae_conv_out_kernel<<<cog, 256, lds, stream>>>(normed ? normed : na, normed ? 96 : conv_out.cip(),
                                                           conv_out.cip(), c8, g, conv_out.w, conv_out.b, out,
                                                           probe ? yp : nullptr, conv_out.cop());
        MK_LAUNCH_CHECK("vae_conv_out");
        MK_TRY(probe_grid("vae_out", -1, yp, conv_out.cop(), g, 3));
        return MK_OK;
    }
};

namespace {

// conv weight kt (time taps) from a PyTorch shape: 4-D [o][i][k][k] -> 1, 5-D [o][i][kt][k][k] -> kt
bool shape_fits(const mk_vae::Slot& s, const int64_t* dims, uint32_t ndim, uint32_t* kt)
{
    *kt = 1;
    uint64_t n = 1;
    for (uint32_t i = 0; i < ndim; ++i)
        n *= uint64_t(dims[i]);
    if (s.kind == mk_vae::Slot::CONV_W || s.kind == mk_vae::Slot::PQ_W) {
        const auto& d = s.dims;
        if (ndim == 4)
            return dims[0] == d[0] && dims[1] == d[1] && dims[2] == d[2] && dims[3] == d[3];
        if (ndim == 5 && dims[0] == d[0] && dims[1] == d[1] && dims[3] == d[2] && dims[4] == d[3] && dims[2] >= 1 &&
            (s.kind == mk_vae::Slot::CONV_W || dims[2] == 1)) {
            *kt = uint32_t(dims[2]);
            return true;
        }
        return false;
    }
    return n == uint64_t(s.dims[0]); // vectors: [n] or [n, 1, 1(, 1)]
}

} // namespace

extern "C" {

mk_status mk_vae_create(const mk_vae_config* cfg, mk_vae** out)
{
    if (!cfg || !out || !cfg->mean || !cfg->std)
        return fail(MK_ERR_ARG, "vae_create: null");
    *out = nullptr;
    if (!cfg->base || cfg->base > 128 || cfg->base % 4 || !cfg->z || cfg->z > 64)
        return fail(MK_ERR_ARG, "vae_create: base channels a multiple of 4 up to 128 (levels 4 base <= 512), latent "
                                "channels 1..64");
    auto v = std::make_unique<mk_vae>();
    v->base = cfg->base;
    v->z = cfg->z;
    v->mean.assign(cfg->mean, cfg->mean + cfg->z);
    v->sd.assign(cfg->std, cfg->std + cfg->z);
    MK_TRY(v->build());
    *out = v.release();
    return MK_OK;
}

mk_status mk_vae_destroy(mk_vae* v)
{
    delete v;
    return MK_OK;
}

mk_status mk_vae_load(mk_vae* v, const char* name, const float* data, const int64_t* dims, uint32_t ndim)
{
    if (!v || !name || !data || (!dims && ndim))
        return fail(MK_ERR_ARG, "vae_load: null");
    auto it = v->slots.find(name);
    if (it == v->slots.end())
        return fail(MK_ERR_ARG, std::string("vae_load: no tensor named ") + name);
    uint32_t kt = 1;
    if (!shape_fits(it->second, dims, ndim, &kt))
        return fail(MK_ERR_ARG, std::string("vae_load: ") + name + " has the wrong shape");
    uint64_t n = 1;
    for (uint32_t i = 0; i < ndim; ++i)
        n *= uint64_t(dims[i]);
    const bool mat = it->second.kind == mk_vae::Slot::CONV_W || it->second.kind == mk_vae::Slot::PQ_W;
    // convolution weights go in as half (rounded to nearest even: an F16 checkpoint's values exactly)
    std::vector<uint16_t> hb;
    const void* host = data;
    if (mat) {
        hb.resize(n);
        for (uint64_t i = 0; i < n; ++i)
            hb[i] = f2h_bits(data[i]);
        host = hb.data();
    }
    void* tmp = nullptr;
    MK_HIP(hipMalloc(&tmp, n * (mat ? 2 : 4)));
    mk_status st = hip_ok(hipMemcpy(tmp, host, n * (mat ? 2 : 4), hipMemcpyHostToDevice), "vae_load copy");
    if (st == MK_OK)
        st = v->put(it->second, tmp, kt, true);
    if (st == MK_OK)
        st = hip_ok(hipStreamSynchronize(v->stream), "vae_load sync");
    (void)hipFree(tmp);
    return st;
}

mk_status mk_vae_init_random(mk_vae* v, uint64_t seed)
{
    if (!v)
        return fail(MK_ERR_ARG, "vae_init_random: null");
    for (const auto& [name, s] : v->slots) {
        uint64_t n = 1;
        for (int64_t d : s.dims)
            n *= uint64_t(d);
        const bool mat = s.kind == mk_vae::Slot::CONV_W || s.kind == mk_vae::Slot::PQ_W;
        const bool gamma = name.size() > 6 && name.compare(name.size() - 6, 6, ".gamma") == 0;
        const double sd = mat ? 1.0 / std::sqrt(double(s.dims[1] * s.dims[2] * s.dims[3])) : gamma ? 0.1 : 0.02;
        void* tmp = nullptr;
        MK_HIP(hipMalloc(&tmp, n * (mat ? 2 : 4)));
        mk_status st = mk_fill_normal(tmp, n, mat ? MK_BF16 : MK_F32, tensor_key(seed, name.c_str()),
                                      gamma ? 1.0 : 0.0, sd, v->stream);
        if (st == MK_OK)
            st = v->put(s, tmp, 1, false); // bf16 draws, stored as the nearest halves
        if (st == MK_OK)
            st = hip_ok(hipStreamSynchronize(v->stream), "vae_init_random sync");
        (void)hipFree(tmp);
        if (st != MK_OK)
            return st;
    }
    return MK_OK;
}

mk_status mk_vae_load_safetensors(mk_vae* v, const char* path, uint64_t* loaded)
{
    if (!v || !path)
        return fail(MK_ERR_ARG, "vae_load_safetensors: null");
    mk_st* st = nullptr;
    MK_TRY(mk_st_open(path, &st));
    std::unique_ptr<mk_st, mk_status (*)(mk_st*)> hold(st, mk_st_close);
    uint64_t count = 0;
    for (const auto& [name, s] : v->slots) {
        mk_st_tensor t;
        if (mk_st_find(st, name.c_str(), &t) != MK_OK)
            return fail(MK_ERR_ARG, "vae_load_safetensors: the checkpoint has no tensor " + name);
        if (t.dtype != MK_F32 && t.dtype != MK_BF16 && t.dtype != MK_F16)
            return fail(MK_ERR_ARG, "vae_load_safetensors: " + name + " has dtype " + t.dtype_name);
        std::vector<uint8_t> raw(t.bytes);
        if (!st_read(st, t, raw.data(), t.bytes, 0))
            return fail(MK_ERR_ARG, "vae_load_safetensors: cannot read " + name);
        const uint64_t n = t.bytes / (t.dtype == MK_F32 ? 4 : 2);
        std::vector<float> f(n);
        for (uint64_t i = 0; i < n; ++i) {
            if (t.dtype == MK_F32) {
                std::memcpy(&f[i], &raw[4 * i], 4);
            } else {
                uint16_t h;
                std::memcpy(&h, &raw[2 * i], 2);
                if (t.dtype == MK_BF16) {
                    f[i] = bf2f_bits(h);
                } else {
                    const int e = (h >> 10) & 31, m = h & 1023;
                    const float a = e == 0 ? std::ldexp(float(m), -24)
                                    : e == 31 ? (m ? NAN : INFINITY)
                                              : std::ldexp(float(1024 + m), e - 25);
                    f[i] = h & 0x8000 ? -a : a;
                }
            }
        }
        int64_t dims[MK_ST_MAX_DIMS];
        for (uint32_t i = 0; i < t.ndim; ++i)
            dims[i] = int64_t(t.dims[t.ndim - 1 - i]); // back to PyTorch order
        MK_TRY(mk_vae_load(v, name.c_str(), f.data(), dims, t.ndim));
        ++count;
    }
    if (loaded)
        *loaded = count;
    return MK_OK;
}

mk_status mk_vae_decode_device(mk_vae* v, const float* tokens, uint32_t h, uint32_t w, float* rgba)
{
    if (!v || !tokens || !rgba)
        return fail(MK_ERR_ARG, "vae_decode: null");
    if (!h || !w || h > 256 || w > 256)
        return fail(MK_ERR_ARG, "vae_decode: a grid of 1 .. 256 tokens a side (32-bit indexing of the 4096^2 level)");
    return v->decode(tokens, h, w, rgba);
}

mk_status mk_vae_decode(mk_vae* v, const float* tokens, size_t n, uint32_t h, uint32_t w, float* rgba)
{
    if (!v || !tokens || !rgba)
        return fail(MK_ERR_ARG, "vae_decode: null");
    if (n != uint64_t(h) * w * 4 * v->z)
        return fail(MK_ERR_ARG, "vae_decode: latents must be [h * w][" + std::to_string(4 * v->z) + "]");
    if (!h || !w || h > 256 || w > 256)
        return fail(MK_ERR_ARG, "vae_decode: a grid of 1 .. 256 tokens a side (32-bit indexing of the 4096^2 level)");
    const uint64_t out_n = uint64_t(16) * h * 16 * w * 4;
    MK_TRY(v->ensure(v->tok, n * 4));
    MK_TRY(v->ensure(v->rgba, out_n * 4));
    MK_HIP(hipMemcpyAsync(v->tok.p, tokens, n * 4, hipMemcpyHostToDevice, v->stream));
    MK_TRY(v->decode(static_cast<float*>(v->tok.p), h, w, static_cast<float*>(v->rgba.p)));
    MK_HIP(hipMemcpyAsync(rgba, v->rgba.p, out_n * 4, hipMemcpyDeviceToHost, v->stream));
    MK_HIP(hipStreamSynchronize(v->stream));
    return MK_OK;
}

mk_status mk_vae_set_probe(mk_vae* v, mk_probe_fn fn, void* user)
{
    if (!v)
        return fail(MK_ERR_ARG, "vae_set_probe: null");
    v->probe = fn;
    v->probe_user = user;
    return MK_OK;
}

mk_status mk_vae_stream(mk_vae* v, void** stream)
{
    if (!v || !stream)
        return fail(MK_ERR_ARG, "vae_stream: null");
    *stream = v->stream;
    return MK_OK;
}

} // extern "C"
