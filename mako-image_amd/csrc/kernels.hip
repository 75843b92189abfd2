// Bandwidth-bound kernels of the step: modulated layer norm, gated residual, heads pack with per-head RMSNorm and
// RoPE, the V^T transpose, GEMV for the time / modulation projections, activations, norms, guidance + Euler,
// patchify, and the counter-RNG fill. Each is a wave64 kernel with 16-byte coalesced accesses where the row allows.
#include "common.hpp"

#include <cmath>
#include <algorithm>
#include <mutex>
#include <vector>

namespace mk {

namespace {

constexpr int kMaxVec = 16; // float4s per lane a row-resident norm keeps in registers (rows up to 4096 floats)

// ------------------------------------------------------------------------------------------------------------
// ln_modulate (image.metal:32-53): one wave per row, the row held in registers; two-pass mean / variance in fp32.
// y = (x - mean) rsqrt(var + eps) (1 + scale) + shift, bf16 out.
// ------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ln_modulate_kernel(const float* __restrict__ x, uint32_t rows, uint32_t n,
                                                          const float* __restrict__ scale,
                                                          const float* __restrict__ shift, int64_t alt, uint32_t split,
                                                          uint32_t seg_rows, float eps, uint16_t* __restrict__ y)
{
    const uint32_t lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + uint64_t(row) * n);
    const uint32_t nv = n / 4;
    f32x4 v[kMaxVec];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const uint32_t c = lane + 64u * i;
        v[i] = c < nv ? xr[c] : f32x4{0, 0, 0, 0};
        s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
    }
    const float mean = wave_sum(s) / float(n);
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const uint32_t c = lane + 64u * i;
        if (c < nv)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float d = v[i][j] - mean;
                q += d * d;
            }
    }
    const float inv = rsqrtf(wave_sum(q) / float(n) + eps);
    const int64_t off = (row % seg_rows) < split ? alt : 0;
    const f32x4* sc = reinterpret_cast<const f32x4*>(scale + off);
    const f32x4* sh = shift ? reinterpret_cast<const f32x4*>(shift + off) : nullptr;
    u32x2* yr = reinterpret_cast<u32x2*>(y + uint64_t(row) * n);
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const uint32_t c = lane + 64u * i;
        if (c < nv) {
            const f32x4 a = sc[c];
            const f32x4 b = sh ? sh[c] : f32x4{0, 0, 0, 0};
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = (v[i][j] - mean) * inv * (1.0f + a[j]) + b[j];
            yr[c] = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        }
    }
}

// ln_modulate for rows of exactly 256 NV floats: the lane's NV float4s of scale and shift are loaded before the row's
// statistics are reduced (their L2 latency overlaps the row's HBM read), and the register arrays are sized to the row.
// Up to two ln_modulate problems in one launch (the image and text streams of a block): blocks [0, blocks0) take
// problem 0, the rest problem 1, four rows a block.
struct LnP {
    const float* x;
    const float* scale;
    const float* shift;
    int64_t alt;
    uint32_t rows, split, seg_rows;
    uint16_t* y;
};
struct LnG {
    LnP p[2];
    uint32_t blocks0;
};

template <int NV>
__global__ __launch_bounds__(256) void ln_modulate_nv_kernel(LnG g, float eps)
{
    constexpr uint32_t n = 256 * NV;
    const bool second = blockIdx.x >= g.blocks0;
    const LnP& P = g.p[second];
    const uint32_t lane = threadIdx.x & 63, row = (blockIdx.x - (second ? g.blocks0 : 0)) * 4 + (threadIdx.x >> 6);
    if (row >= P.rows)
        return;
    const int64_t off = (row % P.seg_rows) < P.split ? P.alt : 0;
    const f32x4* sc = reinterpret_cast<const f32x4*>(P.scale + off);
    const f32x4* sh = P.shift ? reinterpret_cast<const f32x4*>(P.shift + off) : nullptr;
    const f32x4* xr = reinterpret_cast<const f32x4*>(P.x + uint64_t(row) * n);
    f32x4 a[NV], b[NV], v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        a[i] = sc[lane + 64 * i];
        b[i] = sh ? sh[lane + 64 * i] : f32x4{0, 0, 0, 0};
        v[i] = xr[lane + 64 * i];
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        s += v[i][0] + v[i][1] + v[i][2] + v[i][3];
    const float mean = wave_sum(s) / float(n);
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float d = v[i][j] - mean;
            q += d * d;
        }
    const float inv = rsqrtf(wave_sum(q) / float(n) + eps);
    u32x2* yr = reinterpret_cast<u32x2*>(P.y + uint64_t(row) * n);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            o[j] = (v[i][j] - mean) * inv * (1.0f + a[i][j]) + b[i][j];
        yr[lane + 64 * i] = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    }
}

// Layer norm with gamma / beta (sdxl.cpp:425-437), or RMSNorm * (w + w_offset) (rms = 1): bf16 or half out (f16: the
// input of a GEMM over half weights). One row a wave,
// NV float4s a lane (the row's n floats, rounded up to 256): the row, gamma and beta are all requested before the
// first reduction, so the launch waits on memory once.
template <bool kRms, int NV>
__global__ __launch_bounds__(256) void norm_kernel(const float* __restrict__ x, uint32_t rows, uint32_t n,
                                                   const float* __restrict__ g, const float* __restrict__ b,
                                                   float w_offset, float eps, uint16_t* __restrict__ y, bool f16)
{
    const uint32_t lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + uint64_t(row) * n);
    const uint32_t nv = n / 4;
    f32x4 v[NV], gg[NV], bb[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t c = lane + 64u * i;
        v[i] = c < nv ? xr[c] : f32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t c = lane + 64u * i;
        gg[i] = c < nv ? reinterpret_cast<const f32x4*>(g)[c] : f32x4{0, 0, 0, 0};
        bb[i] = !kRms && c < nv ? reinterpret_cast<const f32x4*>(b)[c] : f32x4{0, 0, 0, 0};
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        s += kRms ? v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3]
                  : v[i][0] + v[i][1] + v[i][2] + v[i][3];
    float mean = 0.0f, inv;
    if (kRms) {
        inv = rsqrtf(wave_sum(s) / float(n) + eps);
    } else {
        mean = wave_sum(s) / float(n);
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (lane + 64u * i < nv)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q += (v[i][j] - mean) * (v[i][j] - mean);
        inv = rsqrtf(wave_sum(q) / float(n) + eps);
    }
    u32x2* yr = reinterpret_cast<u32x2*>(y + uint64_t(row) * n);
    // one branch on the output type around stores specialised for each (a test at every pair becomes a branch each)
    auto store = [&](auto h_c) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = lane + 64u * i;
            if (c < nv) {
                float o[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[j] = kRms ? v[i][j] * inv * (gg[i][j] + w_offset) : (v[i][j] - mean) * inv * gg[i][j] + bb[i][j];
                yr[c] = u32x2{pack_x2(o[0], o[1], decltype(h_c)::value), pack_x2(o[2], o[3], decltype(h_c)::value)};
            }
        }
    };
    if (f16)
        store(std::true_type{});
    else
        store(std::false_type{});
}

// norm_kernel with the smallest NV >= nvec (1 .. kMaxVec float4s a lane)
template <bool kRms, int NV = 1>
void launch_norm(uint32_t nvec, const float* x, uint32_t rows, uint32_t n, const float* g, const float* b,
                 float w_offset, float eps, uint16_t* y, bool f16, hipStream_t stream)
{
    if constexpr (NV < kMaxVec) {
        if (nvec > uint32_t(NV))
            return launch_norm<kRms, NV + 1>(nvec, x, rows, n, g, b, w_offset, eps, y, f16, stream);
    }
    norm_kernel<kRms, NV><<<cdiv(rows, 4), 256, 0, stream>>>(x, rows, n, g, b, w_offset, eps, y, f16);
}

// Group norm statistics (sdxl.cpp:425-437), two kernels: 16-row chunks of a sample, one workgroup each, sum x and
// x^2 per channel in double over coalesced rows and reduce them per group through LDS (partials [batch][chunk][group]);
// then one wave a (sample, group) adds its chunks and writes (mean, 1 / sqrt(var + eps)). (One workgroup a
// (sample, group) walking the group's columns was a 181 us launch for 2 x 4096 x 640.)
constexpr uint32_t kGnRows = 16;
__global__ __launch_bounds__(256) void group_partial_kernel(const float* __restrict__ x, uint32_t rows, uint32_t c,
                                                            uint32_t groups, double2* __restrict__ part)
{
    __shared__ double ls[4096], lq[4096];
    const uint32_t chunk = blockIdx.x, bi = blockIdx.y, r0 = chunk * kGnRows, r1 = min(rows, r0 + kGnRows);
    const float* xb = x + uint64_t(bi) * rows * c;
    for (uint32_t ch = threadIdx.x; ch < c; ch += 256) {
        // the chunk's rows all requested before the first add (one memory wait, not one a row), summed in row order
        float v[kGnRows];
#pragma unroll
        for (uint32_t i = 0; i < kGnRows; ++i)
            v[i] = r0 + i < r1 ? xb[uint64_t(r0 + i) * c + ch] : 0.0f;
        double s = 0.0, q = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < kGnRows; ++i)
            if (r0 + i < r1) {
                const double d = v[i];
                s += d;
                q += d * d;
            }
        ls[ch] = s;
        lq[ch] = q;
    }
    __syncthreads();
    const uint32_t cg = c / groups;
    for (uint32_t g = threadIdx.x; g < groups; g += 256) {
        double s = 0.0, q = 0.0;
        for (uint32_t i = 0; i < cg; ++i) {
            s += ls[g * cg + i];
            q += lq[g * cg + i];
        }
        part[(uint64_t(bi) * gridDim.x + chunk) * groups + g] = double2{s, q};
    }
}

// one wave a (sample, group): lanes stride over the chunks, then a tree in LDS
__global__ __launch_bounds__(64) void group_final_kernel(const double2* __restrict__ part, uint32_t chunks,
                                                         uint32_t groups, double count, float eps,
                                                         float2* __restrict__ stats)
{
    __shared__ double rs[64], rq[64];
    const uint32_t g = blockIdx.x, bi = blockIdx.y, lane = threadIdx.x;
    double s = 0.0, q = 0.0;
    for (uint32_t k = lane; k < chunks; k += 64) {
        const double2 v = part[(uint64_t(bi) * chunks + k) * groups + g];
        s += v.x;
        q += v.y;
    }
    rs[lane] = s;
    rq[lane] = q;
    __syncthreads();
    for (uint32_t h = 32; h > 0; h >>= 1) {
        if (lane < h) {
            rs[lane] += rs[lane + h];
            rq[lane] += rq[lane + h];
        }
        __syncthreads();
    }
    if (lane == 0) {
        const double mean = rs[0] / count, var = rq[0] / count - mean * mean;
        stats[bi * groups + g] = float2{float(mean), float(1.0 / sqrt((var > 0.0 ? var : 0.0) + double(eps)))};
    }
}

__global__ __launch_bounds__(256) void group_apply_kernel(const float* __restrict__ x, uint32_t rows, uint32_t c,
                                                          uint32_t groups, const float2* __restrict__ stats,
                                                          const float* __restrict__ g, const float* __restrict__ b,
                                                          uint16_t* __restrict__ y, bool f16)
{
    const uint64_t n = uint64_t(rows) * c;
    const uint32_t bi = blockIdx.y;
    auto run = [&](auto h_c) { // the loop for one output type (no test of it per element)
        for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) {
            const uint32_t ch = uint32_t(i % c);
            const float2 st = stats[bi * groups + ch / (c / groups)];
            const float v = (x[uint64_t(bi) * n + i] - st.x) * st.y * g[ch] + b[ch];
            y[uint64_t(bi) * n + i] = decltype(h_c)::value ? f2h_bits(v) : f2bf_bits(v);
        }
    };
    if (f16)
        run(std::true_type{});
    else
        run(std::false_type{});
}

// group_apply_kernel four channels a thread (c a multiple of 4; x, g, b 16-byte and y 8-byte aligned): float4 loads,
// 32-bit indexing, the same arithmetic per element
__global__ __launch_bounds__(256) void group_apply4_kernel(const float* __restrict__ x, uint32_t rows, uint32_t c,
                                                           uint32_t groups, const float2* __restrict__ stats,
                                                           const float* __restrict__ g, const float* __restrict__ b,
                                                           uint16_t* __restrict__ y, bool f16)
{
    const uint32_t c4 = c / 4, n4 = rows * c4, cg = c / groups, bi = blockIdx.y;
    const f32x4* xb = reinterpret_cast<const f32x4*>(x + uint64_t(bi) * rows * c);
    u32x2* yb = reinterpret_cast<u32x2*>(y + uint64_t(bi) * rows * c);
    const float2* sb = stats + bi * groups;
    auto run = [&](auto h_c) { // the loop for one output type (no test of it per element)
        for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n4; i += gridDim.x * 256) {
            const uint32_t ch = (i % c4) * 4;
            const f32x4 v = xb[i], gg = *reinterpret_cast<const f32x4*>(g + ch),
                        bb = *reinterpret_cast<const f32x4*>(b + ch);
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float2 st = sb[(ch + j) / cg];
                o[j] = (v[j] - st.x) * st.y * gg[j] + bb[j];
            }
            yb[i] = u32x2{pack_x2(o[0], o[1], decltype(h_c)::value), pack_x2(o[2], o[3], decltype(h_c)::value)};
        }
    };
    if (f16)
        run(std::true_type{});
    else
        run(std::false_type{});
}

// gate_add (image.metal:55-65) with an identity or tanh gate; y fp32 or bf16.
template <typename Y, bool kTanh>
__global__ __launch_bounds__(256) void gate_add_kernel(float* __restrict__ x, const Y* __restrict__ y, uint32_t rows,
                                                       uint32_t n, const float* __restrict__ gate, int64_t alt,
                                                       uint32_t split, uint32_t seg_rows)
{
    const uint64_t total = uint64_t(rows) * n;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < total; i += uint64_t(gridDim.x) * 256) {
        const uint32_t row = uint32_t(i / n), c = uint32_t(i % n);
        float g = gate[((row % seg_rows) < split ? alt : 0) + c];
        if (kTanh)
            g = tanh_f(g);
        float v;
        if constexpr (sizeof(Y) == 2)
            v = bf2f_bits(y[i]);
        else
            v = y[i];
        x[i] += g * v;
    }
}

// heads_norm_half / heads_half (qwen_image.cpp:226-250): one wave per (row, head); lane l holds the pair it rotates:
// (2l, 2l+1) in mode 2 (interleaved, also used with no rope), (l, l + d/2) in mode 1.
__global__ __launch_bounds__(256) void heads_kernel(const uint16_t* __restrict__ x, uint32_t rows, int64_t ld,
                                                    int64_t stride_x, uint32_t col0, uint32_t heads, uint32_t d,
                                                    const float* __restrict__ w, float eps,
                                                    const float* __restrict__ rope, uint32_t mode,
                                                    uint16_t* __restrict__ out, uint32_t n_pad, uint32_t row0,
                                                    bool f16)
{
    const uint32_t lane = threadIdx.x & 63, bi = blockIdx.y;
    const uint64_t idx = uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (idx >= uint64_t(rows) * heads)
        return;
    const uint32_t r = uint32_t(idx / heads), h = uint32_t(idx % heads);
    const uint16_t* xr = x + uint64_t(bi) * stride_x + uint64_t(r) * ld + col0 + uint64_t(h) * d;
    const bool act = lane < d / 2;
    const uint32_t i0 = mode == 1 ? lane : 2 * lane, i1 = mode == 1 ? lane + d / 2 : 2 * lane + 1;
    float a = act ? bf2f_bits(xr[i0]) : 0.0f, b = act ? bf2f_bits(xr[i1]) : 0.0f;
    if (w) {
        const float inv = rsqrtf(wave_sum(a * a + b * b) / float(d) + eps);
        if (act) {
            a = a * inv * w[i0];
            b = b * inv * w[i1];
        }
    }
    if (rope && mode && act) {
        const float* cs = rope + (uint64_t(row0) + r) * d + 2 * lane; // pair `lane` of the row's d/2 (cos, sin)
        const float co = cs[0], si = cs[1];
        const float na = a * co - b * si, nb = a * si + b * co;
        a = na;
        b = nb;
    }
    if (act) {
        uint16_t* o = out + ((uint64_t(bi) * heads + h) * n_pad + row0 + r) * d;
        o[i0] = f16 ? f2h_bits(a) : f2bf_bits(a);
        o[i1] = f16 ? f2h_bits(b) : f2bf_bits(b);
    }
}

// The layout alone (no norm, no rope): 16 bytes a thread, 32-bit indexing (rows * heads * d / 8 < 2^31; ld, col0,
// stride_x multiples of 8; 16-byte aligned buffers). out [batch][heads][n_pad][d] row row0 + r = x's row r (as half
// when f16).
__global__ __launch_bounds__(256) void heads_copy_kernel(const uint16_t* __restrict__ x, uint32_t rows, int64_t ld,
                                                         int64_t stride_x, uint32_t col0, uint32_t heads, uint32_t d,
                                                         uint16_t* __restrict__ out, uint32_t n_pad, uint32_t row0,
                                                         bool f16)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x, q = d / 8, bi = blockIdx.y;
    if (i >= rows * heads * q)
        return;
    const uint32_t c = (i % q) * 8, p = i / q, r = p / heads, h = p - r * heads;
    u32x4 v =
        *reinterpret_cast<const u32x4*>(x + uint64_t(bi) * stride_x + uint64_t(r) * ld + col0 + uint64_t(h) * d + c);
    if (f16)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = bf16x2_to_f16x2(v[j]);
    *reinterpret_cast<u32x4*>(out + ((uint64_t(bi) * heads + h) * n_pad + row0 + r) * d + c) = v;
}

// V^T pack: x bf16 [batch][rows][ld] columns col0 + h*d .. -> out [batch][heads][d][n_pad] at column
// vt_col(row0 + r).
// One block per (64 rows, head, batch), transposed through LDS so both sides are coalesced.
template <int kD>
__global__ __launch_bounds__(256) void heads_t_kernel(const uint16_t* __restrict__ x, uint32_t rows, int64_t ld,
                                                      int64_t stride_x, uint32_t col0, uint32_t heads,
                                                      uint16_t* __restrict__ out, uint32_t n_pad, uint32_t row0,
                                                      bool f16)
{
    __shared__ uint16_t t[64][kD + 2];
    const uint32_t r0 = blockIdx.x * 64, h = blockIdx.y, bi = blockIdx.z, tid = threadIdx.x;
    // load: 64 rows x kD values, 2 per thread-step (u32)
    for (uint32_t i = tid; i < 64 * kD / 2; i += 256) {
        const uint32_t r = i / (kD / 2), c = (i % (kD / 2)) * 2;
        uint32_t v = 0;
        if (r0 + r < rows)
            v = *reinterpret_cast<const uint32_t*>(x + uint64_t(bi) * stride_x + uint64_t(r0 + r) * ld + col0 +
                                                   uint64_t(h) * kD + c);
        if (f16)
            v = bf16x2_to_f16x2(v);
        t[r][c] = uint16_t(v);
        t[r][c + 1] = uint16_t(v >> 16);
    }
    __syncthreads();
    // store: kD rows of 64 columns, 2 per thread-step
    for (uint32_t i = tid; i < kD * 32; i += 256) {
        const uint32_t dd = i / 32, c = (i % 32) * 2;
        if (r0 + c >= rows)
            continue;
        // keys in the vt_col order; an even key and the next share bits 2 and 3, so they stay adjacent
        uint16_t* o = out + ((uint64_t(bi) * heads + h) * kD + dd) * n_pad;
        const uint32_t key = row0 + r0 + c;
        if (r0 + c + 1 < rows && (key & 1) == 0) {
            *reinterpret_cast<uint32_t*>(o + vt_col(key)) = uint32_t(t[c][dd]) | (uint32_t(t[c + 1][dd]) << 16);
        } else {
            o[vt_col(key)] = t[c][dd];
            if (r0 + c + 1 < rows)
                o[vt_col(key + 1)] = t[c + 1][dd];
        }
    }
}

// GEMV for rows <= 4: y[r][n] = sum_k W[n][k] bf16(x'[r][k]) + b[n], x' = silu(x) if asked; x' staged in LDS.
// Each wave computes 4 outputs at a time, 16-byte weight loads.
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, uint32_t rows, uint32_t K,
                                                   const uint16_t* __restrict__ w, const float* __restrict__ bias,
                                                   uint32_t N, float* __restrict__ y, int silu_x)
{
    extern __shared__ float xs[];
    for (uint32_t i = threadIdx.x; i < rows * K; i += 256) {
        const float v = x[i];
        xs[i] = bf2f_bits(f2bf_bits(silu_x ? v / (1.0f + __expf(-v)) : v)); // the GEMMs' bf16 activation operand
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n0 = (blockIdx.x * 4 + wave) * 4;
    if (n0 >= N)
        return;
    float acc[4][4] = {};
    for (uint32_t k = lane * 8; k < K; k += 512) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 wv = *reinterpret_cast<const u32x4*>(w + uint64_t(min(n0 + j, N - 1)) * K + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float w0 = bf2f_bits(uint16_t(wv[e])), w1 = bf2f_bits(uint16_t(wv[e] >> 16));
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (uint32_t(r) < rows)
                        acc[j][r] += w0 * xs[r * K + k + 2 * e] + w1 * xs[r * K + k + 2 * e + 1];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[j][r] = wave_sum(acc[j][r]);
    if (lane < 16) {
        const uint32_t j = lane / 4, r = lane % 4;
        float v = 0.0f;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                if (uint32_t(jj) == j && uint32_t(rr) == r)
                    v = acc[jj][rr];
        if (n0 + j < N && r < rows)
            y[uint64_t(r) * N + n0 + j] = v + (bias ? bias[n0 + j] : 0.0f);
    }
}

// GEMV for one row with K = 512 * KI: each wave computes 4 outputs with all 4 * KI of its 16-byte weight loads
// issued first; while they are in flight the workgroup (8 waves, 32 outputs) converts x' to bf16 in LDS once (each
// wave converting the whole row itself cost more VALU time than the dot products), and the dot products take the
// bf16 pairs as they are (v_dot2_f32_bf16).
template <int KI>
__global__ __launch_bounds__(512) void gemv1_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                    const float* __restrict__ bias, uint32_t N, float* __restrict__ y,
                                                    int silu_x)
{
    constexpr uint32_t K = 512 * KI;
    __shared__ __attribute__((aligned(16))) uint16_t xs[K];
    const uint32_t lane = threadIdx.x & 63, n0 = (blockIdx.x * 8 + (threadIdx.x >> 6)) * 4;
    // the wave's 4 weight rows first (16-byte chunks, all in flight; rows past N read the last row), as nontemporal
    // loads: the stacked modulation matrix streams through once a step and is not kept in the caches
    u32x4 wv[4][KI];
    if (n0 < N)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < KI; ++i)
                wv[j][i] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(w + uint64_t(min(n0 + j, N - 1)) * K + lane * 8 + 512 * i));
    // meanwhile the input row, once a workgroup, as the GEMMs' bf16 activation operand (silu first when asked)
    for (uint32_t k = threadIdx.x; k < K / 2; k += 512) {
        float a = x[2 * k], b = x[2 * k + 1];
        if (silu_x) {
            a = a / (1.0f + __expf(-a));
            b = b / (1.0f + __expf(-b));
        }
        *reinterpret_cast<uint32_t*>(&xs[2 * k]) = pack_bf16x2(a, b);
    }
    __syncthreads();
    if (n0 >= N)
        return;
    // bf16 pairs straight into v_dot2_f32_bf16 (exact products, fp32 sums)
    typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < KI; ++i) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(&xs[lane * 8 + 512 * i]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t wu = wv[j][i][e], xu = xv[e];
                acc[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wu),
                                                         __builtin_bit_cast(bf16x2, xu), acc[j], false);
            }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        acc[j] = wave_sum(acc[j]);
    if (lane < 4) {
        const float v = lane == 0 ? acc[0] : lane == 1 ? acc[1] : lane == 2 ? acc[2] : acc[3];
        if (n0 + lane < N)
            y[n0 + lane] = v + (bias ? bias[n0 + lane] : 0.0f);
    }
}

template <int kOp>
__global__ __launch_bounds__(256) void unary_kernel(float* __restrict__ x, uint64_t n)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256)
        x[i] = kOp == 0 ? silu_f(x[i]) : gelu_tanh_f(x[i]);
}

// swiglu_rows (gate rows first) and geglu_rows (h first, then g): m bf16 [rows][F].
template <typename In, bool kGeglu>
__global__ __launch_bounds__(256) void glu_kernel(const In* __restrict__ in, uint32_t rows, uint32_t F,
                                                  uint16_t* __restrict__ m)
{
    const uint64_t n = uint64_t(rows) * F;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) {
        const uint64_t r = i / F, c = i % F;
        float a, b;
        if constexpr (sizeof(In) == 2) {
            a = bf2f_bits(in[r * 2 * F + c]);
            b = bf2f_bits(in[r * 2 * F + F + c]);
        } else {
            a = in[r * 2 * F + c];
            b = in[r * 2 * F + F + c];
        }
        m[i] = f2bf_bits(kGeglu ? a * 0.5f * b * (1.0f + erf_fit(b * 0.70710678f)) : silu_f(a) * b);
    }
}

// The same for bf16 input 8 values a thread: 16-byte loads and stores, 32-bit indexing (rows * F / 8 < 2^32, F a
// multiple of 8, rows 16-byte aligned); each value's arithmetic and rounding are glu_kernel's.
template <bool kGeglu>
__global__ __launch_bounds__(256) void glu8_kernel(const uint16_t* __restrict__ in, uint32_t rows, uint32_t F,
                                                   uint16_t* __restrict__ m)
{
    const uint32_t F8 = F / 8, n8 = rows * F8;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n8; i += gridDim.x * 256) {
        const uint32_t r = i / F8, c = (i - r * F8) * 8;
        const uint16_t* row = in + uint64_t(r) * 2 * F + c;
        const u32x4 av = *reinterpret_cast<const u32x4*>(row), bv = *reinterpret_cast<const u32x4*>(row + F);
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float y[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float a = bf2f_bits(uint16_t(av[k] >> (16 * h))), b = bf2f_bits(uint16_t(bv[k] >> (16 * h)));
                y[h] = kGeglu ? a * 0.5f * b * (1.0f + erf_fit(b * 0.70710678f)) : silu_f(a) * b;
            }
            o[k] = pack_bf16x2(y[0], y[1]);
        }
        *reinterpret_cast<u32x4*>(m + uint64_t(r) * F + c) = o;
    }
}

__global__ __launch_bounds__(256) void cfg_euler_kernel(const float* __restrict__ x, const float* __restrict__ pos,
                                                        const float* __restrict__ neg, uint64_t n, float guidance,
                                                        float dt, float* __restrict__ out)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) {
        const float v = neg ? neg[i] + guidance * (pos[i] - neg[i]) : pos[i];
        out[i] = x[i] + dt * v;
    }
}

template <bool kPack>
__global__ __launch_bounds__(256) void patch_kernel(const float* __restrict__ src, uint32_t C, uint32_t h, uint32_t w,
                                                    float* __restrict__ dst)
{
    const uint64_t n = uint64_t(C) * 4 * h * w, bi = blockIdx.y;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) {
        // i indexes the latent [C][2h][2w]
        const uint32_t xx = uint32_t(i % (2 * w)), yy = uint32_t((i / (2 * w)) % (2 * h)), c = uint32_t(i / (4ull * h * w));
        const uint64_t t = (uint64_t(yy / 2) * w + xx / 2) * C * 4 + c * 4 + (yy % 2) * 2 + xx % 2;
        if (kPack)
            dst[bi * n + t] = src[bi * n + i];
        else
            dst[bi * n + i] = src[bi * n + t];
    }
}

__global__ __launch_bounds__(256) void fill_normal_kernel(void* __restrict__ p, uint64_t n, uint32_t dtype,
                                                          uint64_t key, double mean, double std)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256) {
        const uint64_t a = splitmix64(key + 2 * i), b = splitmix64(key + 2 * i + 1);
        const double u1 = double((a >> 11) + 1) * 0x1.0p-53, u2 = double(b >> 11) * 0x1.0p-53;
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        const float v = float(mean + std * z);
        if (dtype == MK_F32)
            static_cast<float*>(p)[i] = v;
        else
            static_cast<uint16_t*>(p)[i] = dtype == MK_F16 ? f2h_bits(v) : f2bf_bits(v);
    }
}

__global__ __launch_bounds__(256) void f2bf_kernel(const float* __restrict__ x, uint64_t n, uint16_t* __restrict__ y)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256)
        y[i] = f2bf_bits(x[i]);
}
__global__ __launch_bounds__(256) void f2h_kernel(const float* __restrict__ x, uint64_t n, uint16_t* __restrict__ y)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256)
        y[i] = f2h_bits(x[i]);
}
__global__ __launch_bounds__(256) void bf2f_kernel(const uint16_t* __restrict__ x, uint64_t n, float* __restrict__ y)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256)
        y[i] = bf2f_bits(x[i]);
}


// e4m3 encode of a finite float, nearest with ties to the even code, saturating at 448 (the CPU reference's rule).
__device__ inline uint8_t e4m3_encode(float x)
{
    const uint8_t sign = __builtin_bit_cast(uint32_t, x) >> 31 ? 0x80 : 0;
    const float a = fabsf(x);
    if (!(a < 448.0f))
        return sign | 0x7e;
    // the binade 2^b of a: subnormals (and zero, for which frexpf reports exponent 0) share the step of binade -6
    int b = -6;
    if (a >= 0x1p-6f) {
        int e;
        frexpf(a, &e); // a = f * 2^e, f in [0.5, 1)
        b = e - 1;
    }
    const float step = ldexpf(1.0f, b - 3);
    const float q = rintf(a / step); // exact scaling by a power of two, then round half to even
    int code;
    if (b == -6 && q < 8.0f)
        code = int(q); // subnormal (or zero)
    else {
        int m = int(q);
        if (m == 16) {
            m = 8;
            ++b;
        }
        code = ((b + 7) << 3) | (m - 8);
    }
    return sign | uint8_t(min(code, 0x7e));
}

// One block per row: the row's max |w| -> scale = max / 448 (1 for a zero row), then the e4m3 codes.
__global__ __launch_bounds__(256) void quant_fp8_kernel(const uint16_t* __restrict__ src, uint64_t cols,
                                                        uint8_t* __restrict__ dst, float* __restrict__ scale)
{
    __shared__ float red[4];
    const uint64_t r = blockIdx.x;
    const uint16_t* s = src + r * cols;
    float mx = 0.0f;
    for (uint64_t c = threadIdx.x; c < cols; c += 256)
        mx = fmaxf(mx, fabsf(bf2f_bits(s[c])));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = mx > 0.0f ? mx / 448.0f : 1.0f;
    if (threadIdx.x == 0)
        scale[r] = sc;
    for (uint64_t c = threadIdx.x; c < cols; c += 256)
        dst[r * cols + c] = e4m3_encode(bf2f_bits(s[c]) / sc);
}

// e4m3 code -> float: 2^(e-7) (1 + m/8) for e > 0, m 2^-9 for the subnormals (no code above 0x7e is ever written).
__device__ inline float e4m3_decode(uint8_t v)
{
    const int e = (v >> 3) & 15, m = v & 7;
    const float a = e ? ldexpf(float(8 + m), e - 10) : ldexpf(float(m), -9);
    return v & 0x80 ? -a : a;
}

// LoRA merge into bf16 (or half: f16) rows: RB rows a block share each A value they load; B's RB rows sit in LDS.
template <int RB>
__global__ __launch_bounds__(256) void lora_bf16_kernel(uint16_t* __restrict__ w, uint64_t rows, uint64_t cols,
                                                        const float* __restrict__ a, const float* __restrict__ b,
                                                        uint32_t rank, float factor, bool f16)
{
    extern __shared__ float bs[]; // [RB][rank]
    const uint64_t r0 = uint64_t(blockIdx.x) * RB;
    for (uint32_t i = threadIdx.x; i < RB * rank; i += 256) {
        const uint64_t r = r0 + i / rank;
        bs[i] = r < rows ? b[r * rank + i % rank] : 0.0f;
    }
    __syncthreads();
    const uint64_t c = uint64_t(blockIdx.y) * 256 + threadIdx.x;
    if (c >= cols)
        return;
    float acc[RB];
    for (int t = 0; t < RB; ++t)
        acc[t] = 0.0f;
    for (uint32_t j = 0; j < rank; ++j) {
        const float av = a[uint64_t(j) * cols + c];
        for (int t = 0; t < RB; ++t)
            acc[t] = fmaf(bs[t * rank + j], av, acc[t]);
    }
    for (int t = 0; t < RB; ++t)
        if (r0 + t < rows) {
            uint16_t* x = w + (r0 + t) * cols + c;
            *x = f16 ? f2h_bits(h2f_bits(*x) + factor * acc[t]) : f2bf_bits(bf2f_bits(*x) + factor * acc[t]);
        }
}

// LoRA merge into e4m3 rows, one row a block: the merged row's max |w| gives the new scale (max / 448, 1 for a zero
// row), then the codes. Both passes compute each merged value by the same operations, so they agree bit for bit.
__global__ __launch_bounds__(256) void lora_fp8_kernel(uint8_t* __restrict__ w, float* __restrict__ scale,
                                                       uint64_t cols, const float* __restrict__ a,
                                                       const float* __restrict__ b, uint32_t rank, float factor)
{
    extern __shared__ float bs[]; // [rank]
    __shared__ float red[4];
    const uint64_t r = blockIdx.x;
    for (uint32_t i = threadIdx.x; i < rank; i += 256)
        bs[i] = b[r * rank + i];
    const float sc0 = scale[r];
    __syncthreads();
    auto merged = [&](uint64_t c) {
        float acc = 0.0f;
        for (uint32_t j = 0; j < rank; ++j)
            acc = fmaf(bs[j], a[uint64_t(j) * cols + c], acc);
        return e4m3_decode(w[r * cols + c]) * sc0 + factor * acc;
    };
    float mx = 0.0f;
    for (uint64_t c = threadIdx.x; c < cols; c += 256)
        mx = fmaxf(mx, fabsf(merged(c)));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = mx > 0.0f ? mx / 448.0f : 1.0f;
    // each thread rewrites only the columns it read in the first pass
    for (uint64_t c = threadIdx.x; c < cols; c += 256) {
        const float v = merged(c);
        w[r * cols + c] = e4m3_encode(v / sc);
    }
    if (threadIdx.x == 0)
        scale[r] = sc;
}

inline uint32_t grid_for(uint64_t n)
{
    const uint64_t b = (n + 255) / 256;
    return uint32_t(b < 65536 ? (b ? b : 1) : 65536);
}
inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

} // namespace

__global__ __launch_bounds__(256) void zero_kernel(uint32_t* __restrict__ p, uint64_t n)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256)
        p[i] = 0;
}

mk_status fill_zero(void* p, size_t bytes, void* stream)
{
    if (bytes % 4 || (reinterpret_cast<uintptr_t>(p) & 3))
        return fail(MK_ERR_ARG, "fill_zero: bytes and address must be multiples of 4");
    if (!bytes)
        return MK_OK;
    zero_kernel<<<grid_for(bytes / 4), 256, 0, S(stream)>>>(static_cast<uint32_t*>(p), bytes / 4);
    MK_LAUNCH_CHECK("fill_zero");
    return MK_OK;
}

mk_status ln_modulate_group(const LnArgs* a, int count, uint32_t n, float eps, void* stream)
{
    if (count < 1 || count > 2 || n % 4 || n > 4u * 64 * kMaxVec)
        return fail(MK_ERR_ARG, "ln_modulate: 1 or 2 problems, n a multiple of 4 up to 4096");
    LnG g{};
    uint32_t blocks = 0;
    int m = 0;
    for (int i = 0; i < count; ++i) {
        if (!a[i].x || !a[i].scale || !a[i].y || !a[i].seg_rows)
            return fail(MK_ERR_ARG, "ln_modulate: null pointer or seg_rows 0");
        if (!a[i].rows)
            continue;
        g.p[m] = LnP{a[i].x, a[i].scale, a[i].shift, a[i].alt, a[i].rows, a[i].split, a[i].seg_rows,
                     static_cast<uint16_t*>(a[i].y)};
        if (m == 0)
            g.blocks0 = cdiv(a[i].rows, 4);
        blocks += cdiv(a[i].rows, 4);
        ++m;
    }
    if (!m)
        return MK_OK;
    if (m == 1)
        g.blocks0 = blocks;
    const dim3 grid(blocks);
    if (n == 3072)
        ln_modulate_nv_kernel<12><<<grid, 256, 0, S(stream)>>>(g, eps);
    else if (n == 4096)
        ln_modulate_nv_kernel<16><<<grid, 256, 0, S(stream)>>>(g, eps);
    else if (n == 2048)
        ln_modulate_nv_kernel<8><<<grid, 256, 0, S(stream)>>>(g, eps);
    else
        for (int i = 0; i < m; ++i) {
            const LnP& P = g.p[i];
            ln_modulate_kernel<<<cdiv(P.rows, 4), 256, 0, S(stream)>>>(P.x, P.rows, n, P.scale, P.shift, P.alt,
                                                                       P.split, P.seg_rows, eps, P.y);
        }
    MK_LAUNCH_CHECK("ln_modulate");
    return MK_OK;
}
} // namespace mk

using namespace mk;

// Scratch of mk_group_norm_noalloc, the entry point that allocates nothing: the per-chunk partial sums and the
// per-(sample, group) statistics of one call, 4 MiB a device for the life of the process. Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not the device address): it takes each device's address once
// with hipGetSymbolAddress and uses that.
static __device__ __align__(256) double2 scratch[1 << 18];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch[kScratchDevices] = {};

// The current device's copy of `scratch`, its address looked up on the device's first call.
mk_status scratch_of_device(char** out)
{
    int dev = 0;
    MK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kScratchDevices)
        return fail(MK_ERR_DEVICE, "scratch: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        MK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch[dev] = static_cast<char*>(p);
    }
    *out = g_scratch[dev];
    return MK_OK;
}
} // namespace

extern "C" {

mk_status mk_ln_modulate(const float* x, uint32_t rows, uint32_t n, const float* scale, const float* shift,
                         int64_t alt, uint32_t split, uint32_t seg_rows, float eps, void* y, void* stream)
{
    const LnArgs a{x, scale, shift, alt, rows, split, seg_rows, y};
    return ln_modulate_group(&a, 1, n, eps, stream);
}

mk_status mk_rms_norm(const float* x, uint32_t rows, uint32_t n, const float* w, float w_offset, float eps, void* y,
                      void* stream)
{
    if (!x || !w || !y || n % 4 || n > 4u * 64 * kMaxVec)
        return fail(MK_ERR_ARG, "rms_norm: null pointer, or n not a multiple of 4 up to 4096");
    if (!rows)
        return MK_OK;
    launch_norm<true>(cdiv(n / 4, 64), x, rows, n, w, nullptr, w_offset, eps, static_cast<uint16_t*>(y), false,
                      S(stream));
    MK_LAUNCH_CHECK("rms_norm");
    return MK_OK;
}

mk_status mk_layer_norm(const float* x, uint32_t rows, uint32_t n, const float* g, const float* b, float eps, void* y,
                        void* stream)
{
    return mk::layer_norm_to(x, rows, n, g, b, eps, y, MK_BF16, stream);
}

// Both group norm entry points: arguments checked, then the three kernels over the scratch `ws` (the per-chunk
// partials, then the (mean, 1 / std) pairs; group_norm_scratch bytes).
static mk_status group_norm_check(const float* x, uint32_t batch, uint32_t c, uint32_t groups, const float* g,
                                  const float* b, void* y)
{
    if (!x || !g || !b || !y || !groups || c % groups || !batch)
        return fail(MK_ERR_ARG, "group_norm: null pointer or channels not a multiple of groups");
    if (c > 4096 || groups > 1024)
        return fail(MK_ERR_ARG, "group_norm: at most 4096 channels and 1024 groups");
    return MK_OK;
}
static size_t group_norm_part_bytes(uint32_t batch, uint32_t rows, uint32_t groups)
{
    return sizeof(double2) * batch * cdiv(rows, kGnRows) * groups;
}
static size_t group_norm_scratch(uint32_t batch, uint32_t rows, uint32_t groups)
{
    return group_norm_part_bytes(batch, rows, groups) + sizeof(float2) * batch * groups;
}
static mk_status group_norm_run(const float* x, uint32_t batch, uint32_t rows, uint32_t c, uint32_t groups,
                                const float* g, const float* b, float eps, void* y, char* ws, hipStream_t s,
                                bool f16 = false)
{
    const uint32_t chunks = cdiv(rows, kGnRows);
    double2* part = reinterpret_cast<double2*>(ws);
    float2* stats = reinterpret_cast<float2*>(ws + group_norm_part_bytes(batch, rows, groups));
    group_partial_kernel<<<dim3(chunks, batch), 256, 0, s>>>(x, rows, c, groups, part);
    group_final_kernel<<<dim3(groups, batch), 64, 0, s>>>(part, chunks, groups, double(rows) * double(c / groups), eps,
                                                          stats);
    const bool vec = c % 4 == 0 && uint64_t(rows) * c < (uint64_t(1) << 32) &&
                     !((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(g) |
                        reinterpret_cast<uintptr_t>(b)) & 15) && !(reinterpret_cast<uintptr_t>(y) & 7);
    if (vec)
        group_apply4_kernel<<<dim3(std::min<uint32_t>(cdiv(uint64_t(rows) * c / 4, 256), 4096), batch), 256, 0, s>>>(
            x, rows, c, groups, stats, g, b, static_cast<uint16_t*>(y), f16);
    else
        group_apply_kernel<<<dim3(std::min<uint32_t>(cdiv(uint64_t(rows) * c, 256), 4096), batch), 256, 0, s>>>(
            x, rows, c, groups, stats, g, b, static_cast<uint16_t*>(y), f16);
    MK_LAUNCH_CHECK("group_norm");
    return MK_OK;
}

// mk_group_norm's partial sums: one buffer a device, grown (stream-ordered) when a call needs more and kept, so a
// steady-state call allocates nothing. A call's stream first waits for the event of the buffer's previous user (any
// stream), and records it after its own kernels: calls on different streams take turns on the buffer.
struct GnScratch {
    int dev = -1;
    char* p = nullptr;
    size_t bytes = 0;
    hipEvent_t last = nullptr;
};
static std::mutex g_gn_mutex;
static std::vector<GnScratch> g_gn;

mk_status mk_group_norm(const float* x, uint32_t batch, uint32_t rows, uint32_t c, uint32_t groups, const float* g,
                        const float* b, float eps, void* y, void* stream)
{
    return mk::group_norm_to(x, batch, rows, c, groups, g, b, eps, y, MK_BF16, stream);
}
} // extern "C"

namespace mk {
mk_status group_norm_to(const float* x, uint32_t batch, uint32_t rows, uint32_t c, uint32_t groups, const float* g,
                        const float* b, float eps, void* y, uint32_t y_dtype, void* stream)
{
    MK_TRY(group_norm_check(x, batch, c, groups, g, b, y));
    if (y_dtype != MK_BF16 && y_dtype != MK_F16)
        return fail(MK_ERR_ARG, "group_norm: output bf16 or f16");
    if (!rows)
        return MK_OK;
    int dev = 0;
    MK_HIP(hipGetDevice(&dev));
    const hipStream_t s = S(stream);
    std::lock_guard<std::mutex> lock(g_gn_mutex);
    GnScratch* w = nullptr;
    for (GnScratch& e : g_gn)
        if (e.dev == dev)
            w = &e;
    if (!w) {
        g_gn.push_back(GnScratch{});
        w = &g_gn.back();
        w->dev = dev;
        MK_HIP(hipEventCreateWithFlags(&w->last, hipEventDisableTiming));
        MK_HIP(hipEventRecord(w->last, s));
    }
    MK_HIP(hipStreamWaitEvent(s, w->last, 0));
    const size_t need = group_norm_scratch(batch, rows, groups);
    if (need > w->bytes) {
        if (w->p)
            MK_HIP(hipFreeAsync(w->p, s));
        w->p = nullptr;
        w->bytes = 0;
        const size_t bytes = std::max(need, size_t(1) << 20);
        MK_HIP(hipMallocAsync(reinterpret_cast<void**>(&w->p), bytes, s));
        w->bytes = bytes;
    }
    const mk_status st = group_norm_run(x, batch, rows, c, groups, g, b, eps, y, w->p, s, y_dtype == MK_F16);
    MK_HIP(hipEventRecord(w->last, s));
    return st;
}

mk_status layer_norm_to(const float* x, uint32_t rows, uint32_t n, const float* g, const float* b, float eps, void* y,
                        uint32_t y_dtype, void* stream)
{
    if (!x || !g || !b || !y || n % 4 || n > 4u * 64 * kMaxVec || (y_dtype != MK_BF16 && y_dtype != MK_F16))
        return fail(MK_ERR_ARG, "layer_norm: null pointer, n not a multiple of 4 up to 4096, or output not bf16 / f16");
    if (!rows)
        return MK_OK;
    launch_norm<false>(cdiv(n / 4, 64), x, rows, n, g, b, 0.0f, eps, static_cast<uint16_t*>(y), y_dtype == MK_F16,
                       S(stream));
    MK_LAUNCH_CHECK("layer_norm");
    return MK_OK;
}

mk_status f32_to_f16(const float* x, size_t n, void* y, void* stream)
{
    if (!x || !y)
        return fail(MK_ERR_ARG, "f32_to_f16: null pointer");
    if (!n)
        return MK_OK;
    f2h_kernel<<<grid_for(n), 256, 0, S(stream)>>>(x, n, static_cast<uint16_t*>(y));
    MK_LAUNCH_CHECK("f32_to_f16");
    return MK_OK;
}
} // namespace mk

extern "C" {

mk_status mk_group_norm_noalloc(const float* x, uint32_t batch, uint32_t rows, uint32_t c, uint32_t groups,
                                const float* g, const float* b, float eps, void* y, void* stream)
{
    MK_TRY(group_norm_check(x, batch, c, groups, g, b, y));
    if (!rows)
        return MK_OK;
    const size_t need = group_norm_scratch(batch, rows, groups);
    if (need > sizeof(scratch))
        return fail(MK_ERR_ARG, "group_norm_noalloc: needs " + std::to_string(need) + " bytes of scratch, more than its " +
                                    std::to_string(sizeof(scratch)) + " (16 bytes for each of batch x ceil(rows / 16) "
                                    "x groups partials, 8 for each of batch x groups statistics)");
    char* ws = nullptr;
    MK_TRY(scratch_of_device(&ws));
    return group_norm_run(x, batch, rows, c, groups, g, b, eps, y, ws, S(stream));
}

mk_status mk_gate_add(float* x, const void* y, uint32_t y_dtype, uint32_t rows, uint32_t n, const float* gate,
                      int64_t alt, uint32_t split, uint32_t seg_rows, int tanh_gate, void* stream)
{
    if (!x || !y || !gate || !seg_rows || (y_dtype != MK_F32 && y_dtype != MK_BF16))
        return fail(MK_ERR_ARG, "gate_add: null pointer, seg_rows 0 or bad y dtype");
    const uint32_t g = grid_for(uint64_t(rows) * n);
    if (y_dtype == MK_F32) {
        if (tanh_gate)
            gate_add_kernel<float, true><<<g, 256, 0, S(stream)>>>(x, static_cast<const float*>(y), rows, n, gate, alt,
                                                                  split, seg_rows);
        else
            gate_add_kernel<float, false><<<g, 256, 0, S(stream)>>>(x, static_cast<const float*>(y), rows, n, gate,
                                                                   alt, split, seg_rows);
    } else {
        if (tanh_gate)
            gate_add_kernel<uint16_t, true><<<g, 256, 0, S(stream)>>>(x, static_cast<const uint16_t*>(y), rows, n,
                                                                     gate, alt, split, seg_rows);
        else
            gate_add_kernel<uint16_t, false><<<g, 256, 0, S(stream)>>>(x, static_cast<const uint16_t*>(y), rows, n,
                                                                      gate, alt, split, seg_rows);
    }
    MK_LAUNCH_CHECK("gate_add");
    return MK_OK;
}

mk_status mk_heads(const void* x, uint32_t batch, uint32_t rows, int64_t ld, int64_t stride_x, uint32_t col0,
                   uint32_t heads, uint32_t d, const float* w, float eps, const float* rope, uint32_t rope_mode,
                   void* out, uint32_t n_pad, uint32_t row0, int transpose, uint32_t out_dtype, void* stream)
{
    if (!x || !out || !batch || (d != 64 && d != 128) || rope_mode > 2 || (rope_mode && !rope) ||
        uint64_t(row0) + rows > n_pad || (out_dtype != MK_BF16 && out_dtype != MK_F16))
        return fail(MK_ERR_ARG, "heads: null pointer, d not 64 / 128, bad rope mode, rows past n_pad, or an output "
                                "dtype other than bf16 / f16");
    const bool f16 = out_dtype == MK_F16;
    if (!rows)
        return MK_OK;
    if (transpose) {
        if (w || rope_mode)
            return fail(MK_ERR_UNSUPPORTED, "heads: the transposed (V) layout takes no norm or rope");
        if (n_pad % 16)
            return fail(MK_ERR_ARG, "heads: the transposed (V) layout needs n_pad a multiple of 16");
        const dim3 grid(cdiv(rows, 64), heads, batch);
        if (d == 128)
            heads_t_kernel<128><<<grid, 256, 0, S(stream)>>>(static_cast<const uint16_t*>(x), rows, ld, stride_x, col0,
                                                             heads, static_cast<uint16_t*>(out), n_pad, row0, f16);
        else
            heads_t_kernel<64><<<grid, 256, 0, S(stream)>>>(static_cast<const uint16_t*>(x), rows, ld, stride_x, col0,
                                                            heads, static_cast<uint16_t*>(out), n_pad, row0, f16);
    } else if (!w && !(rope && rope_mode) && ld % 8 == 0 && col0 % 8 == 0 && stride_x % 8 == 0 &&
               !(reinterpret_cast<uintptr_t>(x) & 15) && !(reinterpret_cast<uintptr_t>(out) & 15) &&
               uint64_t(rows) * heads * d / 8 < (uint64_t(1) << 31)) {
        heads_copy_kernel<<<dim3(cdiv(uint64_t(rows) * heads * d / 8, 256), batch), 256, 0, S(stream)>>>(
            static_cast<const uint16_t*>(x), rows, ld, stride_x, col0, heads, d, static_cast<uint16_t*>(out), n_pad,
            row0, f16);
    } else {
        heads_kernel<<<dim3(cdiv(uint64_t(rows) * heads, 4), batch), 256, 0, S(stream)>>>(
            static_cast<const uint16_t*>(x), rows, ld, stride_x, col0, heads, d, w, eps, rope, rope_mode,
            static_cast<uint16_t*>(out), n_pad, row0, f16);
    }
    MK_LAUNCH_CHECK("heads");
    return MK_OK;
}

mk_status mk_gemv(const float* x, uint32_t rows, uint32_t K, const void* w, const float* bias, uint32_t N, float* y,
                  int silu_x, void* stream)
{
    if (!x || !w || !y || rows == 0 || rows > 4 || K % 8 || uint64_t(rows) * K * 4 > 64 * 1024)
        return fail(MK_ERR_ARG, "gemv: null pointer, rows not 1..4, K not a multiple of 8 or rows*K over 16384");
    const uint16_t* wb = static_cast<const uint16_t*>(w);
    const dim3 grid(cdiv(N, 16)), grid1(cdiv(N, 32));
    if (rows == 1 && K == 3072)
        gemv1_kernel<6><<<grid1, 512, 0, S(stream)>>>(x, wb, bias, N, y, silu_x);
    else if (rows == 1 && K == 4096)
        gemv1_kernel<8><<<grid1, 512, 0, S(stream)>>>(x, wb, bias, N, y, silu_x);
    else if (rows == 1 && K == 2048)
        gemv1_kernel<4><<<grid1, 512, 0, S(stream)>>>(x, wb, bias, N, y, silu_x);
    else
        gemv_kernel<<<grid, 256, rows * K * 4, S(stream)>>>(x, rows, K, wb, bias, N, y, silu_x);
    MK_LAUNCH_CHECK("gemv");
    return MK_OK;
}

mk_status mk_silu(float* x, size_t n, void* stream)
{
    if (!x)
        return fail(MK_ERR_ARG, "silu: null pointer");
    unary_kernel<0><<<grid_for(n), 256, 0, S(stream)>>>(x, n);
    MK_LAUNCH_CHECK("silu");
    return MK_OK;
}

mk_status mk_gelu_tanh(float* x, size_t n, void* stream)
{
    if (!x)
        return fail(MK_ERR_ARG, "gelu_tanh: null pointer");
    unary_kernel<1><<<grid_for(n), 256, 0, S(stream)>>>(x, n);
    MK_LAUNCH_CHECK("gelu_tanh");
    return MK_OK;
}

mk_status mk_swiglu(const void* gu, uint32_t gu_dtype, uint32_t rows, uint32_t F, void* m, void* stream)
{
    if (!gu || !m || (gu_dtype != MK_F32 && gu_dtype != MK_BF16))
        return fail(MK_ERR_ARG, "swiglu: null pointer or bad dtype");
    if (gu_dtype == MK_BF16 && F % 8 == 0 && uint64_t(rows) * F / 8 < (uint64_t(1) << 31) &&
        !(reinterpret_cast<uintptr_t>(gu) & 15) && !(reinterpret_cast<uintptr_t>(m) & 15)) {
        glu8_kernel<false><<<grid_for(uint64_t(rows) * F / 8), 256, 0, S(stream)>>>(
            static_cast<const uint16_t*>(gu), rows, F, static_cast<uint16_t*>(m));
        MK_LAUNCH_CHECK("swiglu");
        return MK_OK;
    }
    const uint32_t g = grid_for(uint64_t(rows) * F);
    if (gu_dtype == MK_F32)
        glu_kernel<float, false><<<g, 256, 0, S(stream)>>>(static_cast<const float*>(gu), rows, F,
                                                           static_cast<uint16_t*>(m));
    else
        glu_kernel<uint16_t, false><<<g, 256, 0, S(stream)>>>(static_cast<const uint16_t*>(gu), rows, F,
                                                              static_cast<uint16_t*>(m));
    MK_LAUNCH_CHECK("swiglu");
    return MK_OK;
}

mk_status mk_geglu(const void* hg, uint32_t hg_dtype, uint32_t rows, uint32_t F, void* m, void* stream)
{
    if (!hg || !m || (hg_dtype != MK_F32 && hg_dtype != MK_BF16))
        return fail(MK_ERR_ARG, "geglu: null pointer or bad dtype");
    if (hg_dtype == MK_BF16 && F % 8 == 0 && uint64_t(rows) * F / 8 < (uint64_t(1) << 31) &&
        !(reinterpret_cast<uintptr_t>(hg) & 15) && !(reinterpret_cast<uintptr_t>(m) & 15)) {
        glu8_kernel<true><<<grid_for(uint64_t(rows) * F / 8), 256, 0, S(stream)>>>(
            static_cast<const uint16_t*>(hg), rows, F, static_cast<uint16_t*>(m));
        MK_LAUNCH_CHECK("geglu");
        return MK_OK;
    }
    const uint32_t g = grid_for(uint64_t(rows) * F);
    if (hg_dtype == MK_F32)
        glu_kernel<float, true><<<g, 256, 0, S(stream)>>>(static_cast<const float*>(hg), rows, F,
                                                          static_cast<uint16_t*>(m));
    else
        glu_kernel<uint16_t, true><<<g, 256, 0, S(stream)>>>(static_cast<const uint16_t*>(hg), rows, F,
                                                             static_cast<uint16_t*>(m));
    MK_LAUNCH_CHECK("geglu");
    return MK_OK;
}

mk_status mk_cfg_euler(const float* x, const float* pos, const float* neg, size_t n, float guidance, float dt,
                       float* x_out, void* stream)
{
    if (!x || !pos || !x_out)
        return fail(MK_ERR_ARG, "cfg_euler: null pointer");
    cfg_euler_kernel<<<grid_for(n), 256, 0, S(stream)>>>(x, pos, neg, n, guidance, dt, x_out);
    MK_LAUNCH_CHECK("cfg_euler");
    return MK_OK;
}

mk_status mk_patchify(const float* lat, uint32_t batch, uint32_t C, uint32_t h, uint32_t w, float* tokens,
                      void* stream)
{
    if (!lat || !tokens || !batch)
        return fail(MK_ERR_ARG, "patchify: null pointer");
    patch_kernel<true><<<dim3(grid_for(uint64_t(C) * 4 * h * w), batch), 256, 0, S(stream)>>>(lat, C, h, w, tokens);
    MK_LAUNCH_CHECK("patchify");
    return MK_OK;
}

mk_status mk_unpatchify(const float* tokens, uint32_t batch, uint32_t C, uint32_t h, uint32_t w, float* lat,
                        void* stream)
{
    if (!lat || !tokens || !batch)
        return fail(MK_ERR_ARG, "unpatchify: null pointer");
    patch_kernel<false><<<dim3(grid_for(uint64_t(C) * 4 * h * w), batch), 256, 0, S(stream)>>>(tokens, C, h, w, lat);
    MK_LAUNCH_CHECK("unpatchify");
    return MK_OK;
}

mk_status mk_fill_normal(void* p, size_t n, uint32_t dtype, uint64_t key, double mean, double std, void* stream)
{
    if (!p || (dtype != MK_F32 && dtype != MK_BF16 && dtype != MK_F16))
        return fail(MK_ERR_ARG, "fill_normal: null pointer or dtype not f32 / bf16 / f16");
    fill_normal_kernel<<<grid_for(n), 256, 0, S(stream)>>>(p, n, dtype, key, mean, std);
    MK_LAUNCH_CHECK("fill_normal");
    return MK_OK;
}

mk_status mk_quantize_fp8_rows(const void* src, uint64_t rows, uint64_t cols, void* dst, float* scale, void* stream)
{
    if (!src || !dst || !scale || rows > 0x7fffffffu)
        return fail(MK_ERR_ARG, "quantize_fp8_rows: null pointer or too many rows");
    if (!rows)
        return MK_OK;
    quant_fp8_kernel<<<uint32_t(rows), 256, 0, S(stream)>>>(static_cast<const uint16_t*>(src), cols,
                                                            static_cast<uint8_t*>(dst), scale);
    MK_LAUNCH_CHECK("quantize_fp8_rows");
    return MK_OK;
}

mk_status mk_lora_merge(void* w, uint32_t w_dtype, float* w_scale, uint64_t rows, uint64_t cols, const float* a,
                        const float* b, uint32_t rank, float factor, void* stream)
{
    if (!w || !a || !b || (w_dtype == MK_FP8_E4M3 && !w_scale))
        return fail(MK_ERR_ARG, "lora_merge: null pointer");
    if (w_dtype != MK_BF16 && w_dtype != MK_F16 && w_dtype != MK_FP8_E4M3)
        return fail(MK_ERR_ARG, "lora_merge: weights bf16, f16 or fp8-e4m3");
    if (!rank || rank > 1024)
        return fail(MK_ERR_ARG, "lora_merge: rank " + std::to_string(rank) + " not in 1..1024");
    if (!rows || !cols)
        return MK_OK;
    if (w_dtype != MK_FP8_E4M3) {
        constexpr int RB = 8;
        const uint64_t gx = (rows + RB - 1) / RB, gy = (cols + 255) / 256;
        if (gx > 0x7fffffffu || gy > 65535)
            return fail(MK_ERR_ARG, "lora_merge: matrix too large");
        lora_bf16_kernel<RB><<<dim3(uint32_t(gx), uint32_t(gy)), 256, RB * rank * 4, S(stream)>>>(
            static_cast<uint16_t*>(w), rows, cols, a, b, rank, factor, w_dtype == MK_F16);
    } else {
        if (rows > 0x7fffffffu)
            return fail(MK_ERR_ARG, "lora_merge: too many rows");
        lora_fp8_kernel<<<uint32_t(rows), 256, rank * 4, S(stream)>>>(static_cast<uint8_t*>(w), w_scale, cols, a, b,
                                                                       rank, factor);
    }
    MK_LAUNCH_CHECK("lora_merge");
    return MK_OK;
}

mk_status mk_f32_to_bf16(const float* x, size_t n, void* y, void* stream)
{
    if (!x || !y)
        return fail(MK_ERR_ARG, "f32_to_bf16: null pointer");
    f2bf_kernel<<<grid_for(n), 256, 0, S(stream)>>>(x, n, static_cast<uint16_t*>(y));
    MK_LAUNCH_CHECK("f32_to_bf16");
    return MK_OK;
}

mk_status mk_bf16_to_f32(const void* x, size_t n, float* y, void* stream)
{
    if (!x || !y)
        return fail(MK_ERR_ARG, "bf16_to_f32: null pointer");
    bf2f_kernel<<<grid_for(n), 256, 0, S(stream)>>>(static_cast<const uint16_t*>(x), n, y);
    MK_LAUNCH_CHECK("bf16_to_f32");
    return MK_OK;
}

} // extern "C"
