// Shared device helpers for the gfx950 kernels: bf16 / fp8 conversions, wave64 reductions, vector types, the
// counter RNG, and the thread-local error state of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "../../include/mkimage.h"

namespace mk {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;

constexpr int kWave = 64;

typedef __attribute__((address_space(3))) void lds_void;

// Buffer resource (raw, dword format) over `bytes` bytes from `base`, and a 16-byte load through it into LDS at
// byte offset voff + soff: the buffer form of the direct-to-LDS load. Unlike the global form it does not count as
// an LDS access, so the LDS reads around it keep precise (partial) waits.
#if defined(__HIP_DEVICE_COMPILE__)
typedef __amdgpu_buffer_rsrc_t BufRes;
__device__ inline BufRes buf_res(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}
__device__ inline void buf_load_lds16(BufRes r, lds_void* lds, uint32_t voff, uint32_t soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, soff, 0, 0);
}
// the same 16 bytes into registers (buffer_load_dwordx4)
__device__ inline u32x4 buf_load16(BufRes r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), 0);
}
#else
typedef int BufRes; // host pass: never called
__device__ inline BufRes buf_res(const void*, uint32_t) { return 0; }
__device__ inline void buf_load_lds16(BufRes, lds_void*, uint32_t, uint32_t) {}
__device__ inline u32x4 buf_load16(BufRes, uint32_t, uint32_t) { return u32x4{}; }
#endif

// ---- GEMM dispatch plan (gemm.hip), shared with the engine's launch-grouping cost model ----
struct GemmPlan {
    int bm;          // tile height in tokens (256, or 128 for launches of few tiles)
    int bn;          // tile width in channels (256, 192 (convolutions), 128 or 64)
    uint64_t tiles;  // tiles of the launch
    bool sk;         // stream-K: whole waves round robin, the last partial wave split by k steps
    uint64_t dp;     // tiles done whole (stream-K)
    double cost;     // estimated duration in units of one k step of a 256 x 256 tile
};
// The plan of a launch of n grouped problems (equal N, K, weight type, epilogue kind) on `cus` compute units;
// `conv`: a 3 x 3 convolution (256-token tiles only).
GemmPlan gemm_plan(const mk_gemm_args* a, uint32_t n, uint32_t cus, bool conv = false);
// Its estimated duration in units of one 256-channel k step.
double gemm_cost(const mk_gemm_args* a, uint32_t n, uint32_t cus);
// MK_ERR_DEVICE when a stream-K launch on `stream` (all: on any stream of any device) gave up waiting for a partial
// tile since the last check (the check clears it); called after synchronisations of that stream (all: of the device).
mk_status gemm_take_error(const void* stream, bool all = false);

// ---- ln_modulate over one or two problems in one launch (kernels.hip; the engine groups the two streams) ----
struct LnArgs {
    const float* x;
    const float* scale;
    const float* shift;
    int64_t alt;
    uint32_t rows, split, seg_rows;
    void* y;
};
// count 1 or 2 problems of width n (the mk_ln_modulate arguments each); one launch when n is 2048, 3072 or 4096
mk_status ln_modulate_group(const LnArgs* a, int count, uint32_t n, float eps, void* stream);

// mk_layer_norm / mk_group_norm with the output in y_dtype (MK_BF16, or MK_F16: the input of a GEMM over half
// weights), and fp32 -> IEEE half (nearest even) (kernels.hip)
mk_status layer_norm_to(const float* x, uint32_t rows, uint32_t n, const float* g, const float* b, float eps, void* y,
                        uint32_t y_dtype, void* stream);
mk_status group_norm_to(const float* x, uint32_t batch, uint32_t rows, uint32_t c, uint32_t groups, const float* g,
                        const float* b, float eps, void* y, uint32_t y_dtype, void* stream);
mk_status f32_to_f16(const float* x, size_t n, void* y, void* stream);
// mk_attention with the output in out_dtype (MK_BF16, or MK_F16: the input of a GEMM over half weights) (attention.hip)
mk_status attention_to(const void* q, const void* k, const void* vt, void* out, uint32_t dtype, uint32_t batch,
                       uint32_t heads, uint32_t kv_heads, uint32_t d, uint32_t n_q, uint32_t q_pad, uint32_t n_k,
                       uint32_t k_pad, int64_t ldo, int64_t stride_o, uint32_t q_pos0, uint32_t block, float scale,
                       const uint32_t* key_hole, uint32_t out_dtype, void* stream);

// Zero `bytes` (a multiple of 4, 4-byte aligned) of device memory on a stream with a kernel (kernels.hip): a fill node
// a caller's graph capture can replay, unlike a memset node.
mk_status fill_zero(void* p, size_t bytes, void* stream);
// A 96- or 192-output-channel conv's rows RMS-normed (mean of squares over the C channels, + 1e-24 / C), times the gain g,
// then SiLU (the VAE's norm_silu): with out NULL they are the conv's output (y bf16, STORE); otherwise y takes the
// conv's fp32 rows (STORE or ADD) and out (bf16 rows of stride ld, from its first grid row) the normed ones. Ring rows
// of the normed output are written as zeros, so it is the next conv's input grid (its slack rows are the caller's).
struct ConvNorm {
    const float* g = nullptr;
    uint16_t* out = nullptr;
    uint32_t ld = 0;
    bool skip_y = false; // with out: the fp32 rows are not stored (nothing reads them after the norm)
};
// mk_conv3x3 for c (a multiple of 8, not of 64, <= 512) input channels in rows of stride lda, with dense weights
// [n][K], K = 9 c rounded up to 64 (k = tap c + channel, zero past 9 c); optionally a norm epilogue (gemm.hip).
mk_status conv3x3_dense(const mk_conv_args* a, uint32_t lda, void* stream, const ConvNorm* nm = nullptr);
// mk_conv3x3 with a norm epilogue
mk_status conv3x3_fused(const mk_conv_args* a, const ConvNorm& nm, void* stream);
// mk_conv3x3 (ADD, output channels a multiple of 192, width a multiple of 256) whose sums y + conv go, as bf16, to the
// four pixels each becomes in the nearest-2x padded grid at out (its first buffer row, rows of ld channels), instead
// of back into y; the 2x grid's ring and slack rows are the caller's.
struct ConvUp {
    uint16_t* out = nullptr;
    uint32_t ld = 0;
};
mk_status conv3x3_up(const mk_conv_args* a, const ConvUp& up, void* stream);

// ---- error state (thread-local, read by mk_last_error) ----
void set_error(const std::string& msg);
mk_status fail(mk_status s, const std::string& msg);
mk_status hip_check(hipError_t e, const char* what);

// Chunked read of a safetensors tensor's bytes [off, off + bytes) (safetensors.cpp).
bool st_read(const mk_st* st, const mk_st_tensor& t, void* dst, uint64_t bytes, uint64_t off);

#define MK_HIP(call)                                                                                               \
    do {                                                                                                           \
        hipError_t e_ = (call);                                                                                    \
        if (e_ != hipSuccess)                                                                                      \
            return ::mk::hip_check(e_, #call);                                                                     \
    } while (0)

#define MK_TRY(x)                                                                                                  \
    do {                                                                                                           \
        mk_status s_ = (x);                                                                                        \
        if (s_ != MK_OK)                                                                                           \
            return s_;                                                                                             \
    } while (0)

#define MK_LAUNCH_CHECK(what)                                                                                      \
    do {                                                                                                           \
        hipError_t e_ = hipGetLastError();                                                                         \
        if (e_ != hipSuccess)                                                                                      \
            return ::mk::hip_check(e_, what);                                                                      \
    } while (0)

// ---- bf16: round-to-nearest-even, bit-exact with the CPU reference's rule ----
// On the device gfx950's conversion instruction (v_cvt_pk_bf16_f32) does it: it matches the integer rule below on
// every one of the 2^32 float bit patterns (NaNs quieted the same way), checked exhaustively on the GPU.
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2cv __attribute__((ext_vector_type(2)));
__host__ __device__ inline uint16_t f2bf_bits(float x)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{x, 0.0f}, bf16x2cv));
    return uint16_t(p);
#else
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return uint16_t((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
#endif
}
__host__ __device__ inline float bf2f_bits(uint16_t b) { return __builtin_bit_cast(float, uint32_t(b) << 16); }
// Two floats to a packed pair of bf16 (low half = a), one conversion instruction.
__device__ inline uint32_t pack_bf16x2(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, bf16x2cv));
}

// ---- IEEE half (the reference's heads and attention precision, `half` in image.metal): round to nearest even,
// subnormals kept, overflow to infinity. On the device gfx950's v_cvt_pk_f16_f32. ----
typedef _Float16 f16x2cv __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pack_f16x2(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, f16x2cv));
}
__host__ __device__ inline uint16_t f2h_bits(float x) { return __builtin_bit_cast(uint16_t, _Float16(x)); }
__host__ __device__ inline float h2f_bits(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }
// A pair in the heads' element type: bf16 or half.
__device__ inline uint32_t pack_x2(float a, float b, bool f16) { return f16 ? pack_f16x2(a, b) : pack_bf16x2(a, b); }
// bf16 pair -> half pair (exact scaling aside, rounded to nearest even)
__device__ inline uint32_t bf16x2_to_f16x2(uint32_t v)
{
    return pack_f16x2(__builtin_bit_cast(float, v << 16), __builtin_bit_cast(float, v & 0xffff0000u));
}

// ---- wave64 reductions, every lane gets the result ----
// On the device on the VALU only: two quad permutations, the half-row and row mirrors (DPP operands), then
// gfx950's v_permlane16_swap (rows 2k <-> 2k + 1) and v_permlane32_swap (halves); each step adds the partner's value.
// (A shfl_xor ladder is six ds_bpermute round trips through the LDS unit, the latency that bounds one-wave-a-row
// kernels.) Patterns stay inside a row, so no lane reads out of range.
#if defined(__HIP_DEVICE_COMPILE__)
template <int CTRL> __device__ inline float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <class Op> __device__ inline float wave_reduce(float v, Op op)
{
    v = op(v, dpp_f<0xB1>(v));  // quad_perm [1,0,3,2]
    v = op(v, dpp_f<0x4E>(v));  // quad_perm [2,3,0,1]
    v = op(v, dpp_f<0x141>(v)); // row_half_mirror: lane i <-> 7 - i within each 8
    v = op(v, dpp_f<0x140>(v)); // row_mirror: lane i <-> 15 - i within each row
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t a16 = r16[0], b16 = r16[1];
    v = op(__builtin_bit_cast(float, a16), __builtin_bit_cast(float, b16));
    u = __builtin_bit_cast(uint32_t, v);
    const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t a32 = r32[0], b32 = r32[1];
    return op(__builtin_bit_cast(float, a32), __builtin_bit_cast(float, b32));
}
__device__ inline float wave_sum(float v)
{
    return wave_reduce(v, [](float a, float b) { return a + b; });
}
// sum over the 32 lanes of each half wave (lanes 0-31, 32-63): the same steps without the final 32-lane swap
__device__ inline float half_sum(float v)
{
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t a = r[0], b = r[1];
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ inline float wave_max(float v)
{
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
// sum over each 8 consecutive lanes: the two quad permutations, then the half-row mirror (lane i <-> 7 - i)
__device__ inline float oct_sum(float v)
{
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0x141>(v);
}
#else
__device__ inline float oct_sum(float v) { return v; }
__device__ inline float wave_sum(float v) { return v; }
__device__ inline float half_sum(float v) { return v; }
__device__ inline float wave_max(float v) { return v; }
#endif

// Combine lane i with lane i ^ 32 through v_permlane32_swap (a VALU op: swaps the upper 32 lanes of one register
// with the lower 32 of the other), not a ds_bpermute round trip through the LDS unit. Swapping a value with itself
// leaves lane i holding its own value in one half of the result and the partner's in the other.
#if defined(__HIP_DEVICE_COMPILE__)
__device__ inline float max_xor32(float v)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t a = r[0], b = r[1];
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ inline float add_xor32(float v)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t a = r[0], b = r[1];
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
#else
__device__ inline float max_xor32(float v) { return v; }
__device__ inline float add_xor32(float v) { return v; }
#endif
// max of 16 values as a depth-4 tree (a running fmaxf chain is 16 dependent VALU ops on the softmax's critical path)
template <class V16> __device__ inline float max16(const V16& s)
{
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        a[i] = fmaxf(s[2 * i], s[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        a[i] = fmaxf(a[2 * i], a[2 * i + 1]);
    return fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
}

// ---- activations (fp32) ----
// The per-element activations divide by the hardware reciprocal (v_rcp_f32, within 1 ulp) rather than an IEEE
// division (a dozen instructions): in the step their outputs are rounded to bf16 or feed a bf16 operand.
__device__ inline float silu_f(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
// tanh(u) = 2 sigmoid(2u) - 1 (one exp, one divide; saturates cleanly at both ends)
__device__ inline float tanh_f(float u) { return 2.0f / (1.0f + __expf(-2.0f * u)) - 1.0f; }
// GELU with the tanh approximation: 0.5 x (1 + tanh(u)) = x sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3)
__device__ inline float gelu_tanh_f(float x)
{
    // 0.5 x (1 + tanh u) = x / (1 + e^(-2u)), u = sqrt(2/pi) (x + 0.044715 x^3); e^(-2u) = 2^(x (c1 + c2 x^2)) with
    // c1 = -2 sqrt(2/pi) log2(e), c2 = 0.044715 c1 folded: three multiply-adds, v_exp_f32 (2^y), v_rcp_f32, one add
    constexpr float c1 = -2.3022082f, c2 = -0.10294324f;
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * fmaf(x * x, c2, c1)));
}
// erf by the Numerical Recipes erfc Chebyshev fit (max error ~1.2e-7), the form the reference's geglu uses
// (image.metal:450-463).
__device__ inline float erf_fit(float x)
{
    const float z = fabsf(x), t = 1.0f / (1.0f + 0.5f * z);
    const float r =
        t * __expf(-z * z - 1.26551223f +
                   t * (1.00002368f +
                        t * (0.37409196f +
                             t * (0.09678418f +
                                  t * (-0.18628806f +
                                       t * (0.27886807f +
                                            t * (-1.13520398f + t * (1.48851587f + t * (-0.82215223f + t * 0.17087277f)))))))));
    return x >= 0.0f ? 1.0f - r : r - 1.0f;
}

// ---- counter RNG: splitmix64, Box-Muller in double (the same sequence as the CPU reference's) ----
__host__ __device__ inline uint64_t splitmix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
uint64_t tensor_key(uint64_t seed, const char* name);

// V^T column of key k: within each group of 16 keys, k with its bits 2 and 3 swapped. The P V MFMA's A operand lane
// reads keys 4h .. 4h + 3 and 8 + 4h .. 8 + 4h + 3 of a 16-key step (h its half-wave); in this order they are 8
// contiguous bf16, one 16-byte LDS read.
__host__ __device__ inline uint32_t vt_col(uint32_t k) { return (k & ~12u) | ((k & 4u) << 1) | ((k & 8u) >> 1); }

inline uint32_t cdiv(uint64_t a, uint64_t b) { return uint32_t((a + b - 1) / b); }
inline uint64_t round_up(uint64_t a, uint64_t b) { return (a + b - 1) / b * b; }

} // namespace mk
