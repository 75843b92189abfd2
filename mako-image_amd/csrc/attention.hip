// attention: joint softmax(Q K^T scale) V on gfx950 MFMA (v_mfma_f32_32x32x16_bf16, or _f16 for half inputs),
// online softmax in fp32.
//
// Each wave owns 32 queries and computes S^T = K Q^T: the MFMA's A operand is a K tile (rows = keys), its B operand
// the wave's Q held in registers for the whole pass (cols = queries). A lane then holds 16 scores of one query per
// 32-key block, so the row max is lane-local plus one swap with lane ^ 32, and the probabilities convert in registers
// to the B operand of O^T = V^T P^T: the A operand is read from a V^T tile (rows = head dims, keys contiguous). The
// P^T slots permute keys (slot 8h + 4ii + j <-> key 16s + 8ii + 4h + j); the V^T fragment reads use the same
// permutation, so the dot products are unchanged.
//
// A workgroup of 4 waves (128 queries) shares each 64-key K and V^T tile, staged in LDS by direct global->LDS loads
// into two buffers (64 KB), with XOR swizzles chosen so every fragment read is bank-conflict free: K [key][d] chunk c
// at c ^ (key & 15), V^T [d][key] chunk c at c ^ ((d >> 1) & 7). V^T holds its keys in the vt_col order, so a lane's
// 8 P V keys are one 16-byte read. Two workgroups run on a CU (two waves a SIMD, <= 256 registers each): while one
// wave of a SIMD runs its softmax on the VALUs, the other's MFMAs keep the matrix core busy.
// built with -fno-honor-nans (the max needs no canonicalization); the shared header's fp8 decoder names a NaN
// constant, unused here
#pragma clang diagnostic ignored "-Wnan-infinity-disabled"
#include "common.hpp"

#include <type_traits>

namespace mk {

namespace {

constexpr int kMaxHoleBatch = 8; // batch items that can carry a masked key range

struct AttnP {
    const uint16_t *q, *k, *vt;
    uint16_t* out;
    uint32_t heads, group, batch, n_q, q_pad, n_k, k_pad, q_pos0, block; // group: query heads a key / value head
    int64_t ldo, so;
    float c; // scale * log2(e)
    // keys [hole[b][0], hole[b][1]) of batch item b are masked (a shorter prompt's padding rows); empty: none
    uint32_t hole[kMaxHoleBatch][2];
    uint32_t out_f16; // the output as IEEE half (the input of a GEMM over half weights), else bf16
};

constexpr int kKT = 64; // keys per tile
// Lazy rescaling: the running max m the exponentials use moves only when a score exceeds it by more than kLazy (log2
// units; the unit-scale path notices it as a row-sum part above 2^kLazy), so P stays near or below 256 (exact enough
// in bf16, far from fp32 overflow) and the output is rescaled on few tiles.
constexpr float kLazy = 8.0f, kLazyP = 256.0f; // kLazyP = 2^kLazy

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__device__ inline uint32_t cvt_bf16x2(float a, float b)
{
    const bf16x2 v = {(__bf16)a, (__bf16)b}; // v_cvt_pk_bf16_f32: round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

// The element type of Q, K, V^T and the probabilities: bf16, or IEEE half (the reference's half heads). The same
// kernel over either: the 32 x 32 x 16 MFMA, the packed conversion (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32, both
// round to nearest even), the two-deep dot product the row sums use, and the rounding that keeps the running max
// exactly representable.
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;
template <bool F16> struct Elem;
template <> struct Elem<false> {
    typedef bf16x8 v8;
    typedef __bf16 e;
    static __device__ f32x16 mfma(v8 a, v8 b, f32x16 c, int, int, int)
    {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ uint32_t pack(float a, float b) { return cvt_bf16x2(a, b); }
    // acc + the two values of p (a packed pair) times 1
    static __device__ float sum2(uint32_t p, float acc)
    {
        const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), ones, acc, false);
    }
};
template <> struct Elem<true> {
    typedef f16x8 v8;
    typedef _Float16 e;
    static __device__ f32x16 mfma(v8 a, v8 b, f32x16 c, int, int, int)
    {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ uint32_t pack(float a, float b) { return pack_f16x2(a, b); }
    static __device__ float sum2(uint32_t p, float acc)
    {
        const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p), ones, acc, false);
    }
};

// U: K carries the softmax scale in log2 units (scale 0 at the API). The running max then enters the S^T MFMAs as
// one more 16-deep product, a constant fragment of ones (K side, dim 0) times a fragment holding -m (Q side), so
// S - m comes out of the matrix core: the softmax needs no per-score multiply-add, and the row sums are taken on the
// bf16 probabilities the P V product uses (v_dot2 against ones), which halves those adds too. m is kept
// bf16-representable so the product subtracts it exactly.
// NW waves a workgroup (32 queries each): 4, or 2 for launches of few query blocks (64-dim heads), whose 64-query
// workgroups then spread over every CU, four a CU.
template <int D, bool U, bool F16, bool HOLE, int NW = 4>
__global__ __launch_bounds__(64 * NW, 2) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn2_kernel(AttnP p)
{
    typedef Elem<F16> X;
    typedef typename X::v8 V8;
    typedef typename X::e E;
    constexpr int DS = D / 16, DT = D / 32, KC = D / 8, QB = 32 * NW; // QB: queries a workgroup
    constexpr int RK = kKT * KC / (64 * NW), RV = D * 8 / (64 * NW);
    static_assert(NW == 4 || NW == 2, "4 or 2 waves a workgroup");
    // the two buffers are separate objects, so the compiler can tell a direct load into one from the fragment reads
    // of the other (with one array indexed by the buffer it waits for the loads before each read)
    __shared__ __attribute__((aligned(16))) uint16_t sK0[kKT * D], sK1[kKT * D];
    __shared__ __attribute__((aligned(16))) uint16_t sV0[D * kKT], sV1[D * kKT];
    auto sK = [&](int b) { return b ? sK1 : sK0; };
    auto sV = [&](int b) { return b ? sV1 : sV0; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r32 = lane & 31, hk = lane >> 5;
    // (the direct loads' LDS bases from a uniform copy of the wave index: scalar, no v_readfirstlane before a load)
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    auto kswz = [](int key, int c) { return KC == 16 ? c ^ (key & 15) : c ^ ((key >> 1) & 7); };
    // XCD-aware order: workgroup i runs on XCD i % 8 (round-robin dispatch), so give each XCD a contiguous run of
    // (batch, head, query block) items: the query blocks of one head then share its K / V in that XCD's L2, instead
    // of every XCD streaming every head's K / V.
    const uint32_t nqb = (p.n_q + QB - 1) / QB, total = nqb * p.heads * p.batch;
    uint32_t item = blockIdx.x;
    if (total % 8 == 0)
        item = (item % 8) * (total / 8) + item / 8;
    const uint32_t qb = item % nqb, head = (item / nqb) % p.heads, bi = item / (nqb * p.heads);
    // HOLE: the batch item's masked key range (a shorter prompt padded to the batch's text rows); a variant of its
    // own, so the launches without one carry none of its registers
    int hole_lo = 0, hole_hi = 0;
    if constexpr (HOLE) {
        hole_lo = bi < uint32_t(kMaxHoleBatch) ? int(p.hole[bi][0]) : 0;
        hole_hi = bi < uint32_t(kMaxHoleBatch) ? int(p.hole[bi][1]) : 0;
    }
    auto in_hole = [&](int key) { return HOLE && key >= hole_lo && key < hole_hi; };
    // keys [k0, k0 + n) reach into the hole (the general path masks them score by score; the scale-0 path through
    // the matrix core, below)
    auto hits_hole = [&](int k0, int n) {
        return HOLE && !U && hole_lo < hole_hi && k0 < hole_hi && k0 + n > hole_lo;
    };
    const int64_t bh = int64_t(bi) * p.heads + head, bkv = int64_t(bi) * (p.heads / p.group) + head / p.group;
    const uint16_t* Q = p.q + bh * p.q_pad * D;
    const uint16_t* K = p.k + bkv * p.k_pad * D;
    const uint16_t* VT = p.vt + bkv * int64_t(D) * p.k_pad;
    const int q0 = int(qb) * QB + wave * 32;

    V8 qf[DS];
    {
        const int qi = min(q0 + r32, int(p.n_q) - 1);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
            qf[ds] = *reinterpret_cast<const V8*>(Q + int64_t(qi) * D + ds * 16 + hk * 8);
    }
    // K / V^T tiles go to LDS by buffer loads (resources over the head's rows; lane byte offsets select key / dim and
    // chunk, the tile's key offset is a scalar): unlike the global form they leave the LDS counter alone.
    const BufRes rsK = buf_res(K, uint32_t(p.k_pad) * D * 2), rsV = buf_res(VT, uint32_t(p.k_pad) * D * 2);
    uint32_t ok[RK], ov[RV];
#pragma unroll
    for (int i = 0; i < RK; ++i) {
        const int P = (i * NW + wave) * 64 + lane, key = P / KC, c = kswz(key, P % KC);
        ok[i] = uint32_t(key * D + c * 8) * 2;
    }
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        const int P = (i * NW + wave) * 64 + lane, d = P >> 3, c = (P & 7) ^ ((d >> 1) & 7);
        ov[i] = uint32_t(d * int(p.k_pad) + c * 8) * 2;
    }
    const int ntiles = int((p.n_k + kKT - 1) / kKT);
    // direct load i of tile t into buffer buf: K rounds first, then V^T rounds
    auto dma1 = [&](int t, int buf, int i) {
        const uint32_t k0 = uint32_t(min(t, ntiles - 1) * kKT);
        if (i < RK)
            buf_load_lds16(rsK, (lds_void*)&sK(buf)[(i * NW + wave_s) * 512], ok[i], k0 * D * 2);
        else if (i < RK + RV)
            buf_load_lds16(rsV, (lds_void*)&sV(buf)[((i - RK) * NW + wave_s) * 512], ov[i - RK], k0 * 2);
    };
    auto issue = [&](int t, int buf) {
        const uint32_t k0 = uint32_t(min(t, ntiles - 1) * kKT);
#pragma unroll
        for (int i = 0; i < RK; ++i)
            buf_load_lds16(rsK, (lds_void*)&sK(buf)[(i * NW + wave_s) * 512], ok[i], k0 * D * 2);
#pragma unroll
        for (int i = 0; i < RV; ++i)
            buf_load_lds16(rsV, (lds_void*)&sV(buf)[(i * NW + wave_s) * 512], ov[i], k0 * 2);
    };
    // S^T of a 32-key half of a tile: value r <-> key 8(r/4) + 4hk + r%4 of the half
    V8 kone = {}, qm = {}; // U: ones at dim 0 (K side); -m at dim 0 (Q side), lanes of the first k half
    if (hk == 0)
        kone[0] = (E)1.0f;
    // U with a masked key range: the same product also adds bias(key) x 1 at dim 1, bias -inf for the masked keys
    // (0 otherwise), so their scores leave the matrix core as -inf (lanes of the first k half hold dims 0 .. 7)
    if (HOLE && U && hk == 0)
        qm[1] = (E)1.0f;
    auto kbias = [&](int key) {
        V8 kb = kone;
        if (hk == 0 && key >= hole_lo && key < hole_hi)
            kb[1] = (E)(-__builtin_inff());
        return kb;
    };
    f32x16 oacc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
        oacc[dt] = f32x16{};
    float m = U ? 0.0f : -1e30f, l = 0.0f;
    const int qpos = int(p.q_pos0) + q0 + r32;
    const bool wave_causal = uint32_t(int(p.q_pos0) + q0) < p.block;
    auto softmax = [&](f32x16& sacc, int k0, u32x4 (&pb)[2]) {
        if (k0 + 32 > int(p.n_k) || (wave_causal && k0 + 31 > int(p.q_pos0) + q0) || hits_hole(k0, 32)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r / 4) + 4 * hk + (r % 4);
                if (key >= int(p.n_k) || (uint32_t(qpos) < p.block && key > qpos) || in_hole(key))
                    sacc[r] = -__builtin_inff();
            }
        }
        const float mx = max_xor32(max16(sacc)) * p.c;
        if (__any(mx > m + kLazy)) {
            const float mn = fmaxf(m, mx);
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    oacc[dt][r] *= alpha;
        }
        float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float e = __builtin_amdgcn_exp2f(fmaf(sacc[r], p.c, -m));
            sacc[r] = e;
            sum[r % 4] += e;
        }
        l += (sum[0] + sum[1]) + (sum[2] + sum[3]);
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int o = 8 * st;
            pb[st] = u32x4{X::pack(sacc[o], sacc[o + 1]), X::pack(sacc[o + 2], sacc[o + 3]),
                           X::pack(sacc[o + 4], sacc[o + 5]), X::pack(sacc[o + 6], sacc[o + 7])};
        }
    };
    issue(0, 0);
    f32x16 s_a, s_b;
    // General scale: one 64-key tile from buffer `buf` (a constant: the loop is unrolled by two, so the LDS reads and
    // the next tile's loads provably touch different buffers and the reads wait for nothing but themselves). The
    // tile's 32 fragment reads (K of both 32-key halves interleaved, then V of each half) stream four ahead of the
    // MFMAs that use them, in a fixed order (fenced); the two halves' S^T products alternate so neither accumulator
    // chain waits on its previous MFMA.
    constexpr int LA = 4; // fragment reads in flight ahead of their MFMA
    auto tile = [&](int t, auto buf_c) {
        constexpr int buf = decltype(buf_c)::value;
        __builtin_amdgcn_s_waitcnt(0); // tile t resident
        __syncthreads();               // ... for every wave, and every wave done with tile t - 1's buffer
        issue(t + 1, buf ^ 1);         // past the end: the last tile again (discarded)
        V8 fk[2 * DS], fv[4 * DT];
        // read g: K fragments g < 2 DS as (ds, half) pairs, then V fragments of half 0, then half 1
        auto rd = [&](int g) {
            if (g < 2 * DS) {
                const int ds = g / 2, kt = g % 2, key = kt * 32 + r32, c = kswz(key, ds * 2 + hk);
                fk[g] = *reinterpret_cast<const V8*>(&sK(buf)[key * D + c * 8]);
            } else if (g < 2 * DS + 4 * DT) {
                const int j = g - 2 * DS, kt = j / (2 * DT), dt = (j % (2 * DT)) % DT, st = (j % (2 * DT)) / DT;
                const int d = dt * 32 + r32, s2 = 2 * kt + st;
                fv[j] = *reinterpret_cast<const V8*>(&sV(buf)[d * kKT + (((2 * s2 + hk) ^ ((d >> 1) & 7)) << 3)]);
            }
        };
#pragma unroll
        for (int g = 0; g < LA; ++g)
            rd(g);
        __builtin_amdgcn_sched_barrier(0);
        s_a = f32x16{};
        s_b = f32x16{};
#pragma unroll
        for (int g = 0; g < 2 * DS; ++g) {
            f32x16& acc = g % 2 ? s_b : s_a;
            acc = X::mfma(fk[g], qf[g / 2], acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            rd(g + LA);
            __builtin_amdgcn_sched_barrier(0);
        }
        u32x4 pb[2];
        auto pv = [&](int kt) {
#pragma unroll
            for (int j = 0; j < 2 * DT; ++j) {
                const int dt = j % DT, st = j / DT;
                oacc[dt] = X::mfma(fv[kt * 2 * DT + j], __builtin_bit_cast(V8, pb[st]),
                                                                   oacc[dt], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                rd(2 * DS + kt * 2 * DT + j + LA);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        softmax(s_a, t * kKT, pb);
        pv(0);
        softmax(s_b, t * kKT + 32, pb);
        pv(1);
    };
    // U: one 64-key tile with the softmax work in the matrix core's shadow. The scores arrive as S - m, so each
    // half's probabilities are computed speculatively, before its row max is known: P = 2^(S - m) is what the tile
    // needs whenever no score exceeds m by more than kLazy. The exponentials, conversions and row sums of half a then
    // run in chunks between the S^T MFMAs of half b, those of half b between the P V MFMAs of half a, and the lane's
    // part of the row sum only decides afterwards whether a half is redone against a new m (the first half of the
    // pass, and the rare tiles whose max jumps: a score more than kLazy above m puts that sum above 2^kLazy). EDGE
    // tiles (ragged key end, causal diagonal, a masked key range) mask scores in the chunks.
    constexpr int CH = 16 / DS;                  // scores per chunk: DS S^T MFMAs (= 2 DT P V MFMAs) per half
    auto tile_u = [&](int t, auto buf_c, auto edge_c) {
        constexpr int buf = decltype(buf_c)::value;
        constexpr bool EDGE = decltype(edge_c)::value;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        V8 fk[2 * DS], fv[4 * DT];
        // read g: K fragments of half a, of half b, then V fragments of half a, of half b
        auto rd = [&](int g) {
            if (g < 2 * DS) {
                const int kt = g / DS, ds = g % DS, key = kt * 32 + r32, c = kswz(key, ds * 2 + hk);
                fk[g] = *reinterpret_cast<const V8*>(&sK(buf)[key * D + c * 8]);
            } else if (g < 2 * DS + 4 * DT) {
                const int j = g - 2 * DS, kt = j / (2 * DT), dt = (j % (2 * DT)) % DT, st = (j % (2 * DT)) / DT;
                const int d = dt * 32 + r32, s2 = 2 * kt + st;
                fv[j] = *reinterpret_cast<const V8*>(&sV(buf)[d * kKT + (((2 * s2 + hk) ^ ((d >> 1) & 7)) << 3)]);
            }
        };
        // chunk c of a half: scores 2j, 2j + 1 for pairs j of the chunk -> a packed pair pw[j], added to the lane's
        // row-sum part ls (one chain: its links sit an MFMA apart, and one accumulator needs no zeroing or final adds)
        auto chunk = [&](f32x16& sc, int k0, uint32_t (&pw)[8], float& ls, int c) {
#pragma unroll
            for (int i = 0; i < CH / 2; ++i) {
                const int j = c * (CH / 2) + i;
                float x0 = sc[2 * j], x1 = sc[2 * j + 1];
                if constexpr (EDGE) {
                    const int key = k0 + 8 * (2 * j / 4) + 4 * hk + (2 * j % 4);
                    const bool causal = uint32_t(qpos) < p.block;
                    if (key >= int(p.n_k) || (causal && key > qpos))
                        x0 = -__builtin_inff();
                    if (key + 1 >= int(p.n_k) || (causal && key + 1 > qpos))
                        x1 = -__builtin_inff();
                    sc[2 * j] = x0;
                    sc[2 * j + 1] = x1;
                }
                pw[j] = X::pack(__builtin_amdgcn_exp2f(x0), __builtin_amdgcn_exp2f(x1));
                ls = X::sum2(pw[j], ls);
                // pinned here: the redo path overwrites them, so the compiler would otherwise sink the
                // speculative work out of the MFMA shadow into the path that keeps it
                asm volatile("" : "+v"(pw[j]), "+v"(ls));
            }
        };
        // moves m to cover the half's max (the pass's first half: to its max), rescales what was accumulated against
        // the old m, and redoes the half's probabilities and row sum
        auto redo = [&](f32x16& sc, uint32_t (&pw)[8], float& lh, bool first, f32x16* other) {
            const float mx = max_xor32(max16(sc));
            const float mn = float((E)(m + (first ? mx : fmaxf(mx, 0.0f))));
            const float dm = mn - m;
            const float alpha = first ? 1.0f : __builtin_amdgcn_exp2f(-dm);
            m = mn;
            if (hk == 0)
                qm[0] = (E)(-m);
            l *= alpha;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                sc[r] -= dm;
            if (other) // half b's scores, computed against the old m
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    (*other)[r] -= dm;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    oacc[dt][r] *= alpha;
            float ls = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                pw[j] = X::pack(__builtin_amdgcn_exp2f(sc[2 * j]), __builtin_amdgcn_exp2f(sc[2 * j + 1]));
                ls = X::sum2(pw[j], ls);
            }
            lh = ls;
        };
        const int k0 = t * kKT;
#pragma unroll
        for (int g = 0; g < LA; ++g)
            rd(g);
        __builtin_amdgcn_sched_barrier(0);
        s_a = X::mfma(HOLE ? kbias(k0 + r32) : kone, qm, f32x16{}, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        // the next tile's direct loads (past the end: the last tile again, discarded) go out one after each S^T
        // MFMA of half a, not as one burst after the barrier (a burst from every wave stalls their issue)
        constexpr int ND = RK + RV, PER = (ND + DS - 1) / DS;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            s_a = X::mfma(fk[ds], qf[ds], s_a, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            rd(ds + LA);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = ds * PER; i < (ds + 1) * PER && i < ND; ++i)
                dma1(t + 1, buf ^ 1, i);
            __builtin_amdgcn_sched_barrier(0);
        }
        s_b = X::mfma(HOLE ? kbias(k0 + 32 + r32) : kone, qm, f32x16{}, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t pa[8], pbw[8];
        float la = 0.0f, lb = 0.0f;
        // S^T of half b || softmax of half a
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            s_b = X::mfma(fk[DS + ds], qf[ds], s_b, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            rd(DS + ds + LA);
            __builtin_amdgcn_sched_barrier(0);
            chunk(s_a, k0, pa, la, ds);
            __builtin_amdgcn_sched_barrier(0);
        }
        // a score more than kLazy above m makes its P, and so the lane's row-sum part, exceed 2^kLazy (P >= 0, and
        // an overflow is +inf); a larger sum of smaller P only redoes a half that needed none
        if (t == 0 || __any(la > kLazyP))
            redo(s_a, pa, la, t == 0, &s_b);
        l += la;
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 pA[2] = {u32x4{pa[0], pa[1], pa[2], pa[3]}, u32x4{pa[4], pa[5], pa[6], pa[7]}};
        // P V of half a || softmax of half b
#pragma unroll
        for (int j = 0; j < 2 * DT; ++j) {
            const int dt = j % DT, st = j / DT;
            oacc[dt] = X::mfma(fv[j], __builtin_bit_cast(V8, pA[st]), oacc[dt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            rd(2 * DS + j + LA);
            __builtin_amdgcn_sched_barrier(0);
            chunk(s_b, k0 + 32, pbw, lb, j);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (__any(lb > kLazyP))
            redo(s_b, pbw, lb, false, nullptr);
        l += lb;
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 pB[2] = {u32x4{pbw[0], pbw[1], pbw[2], pbw[3]}, u32x4{pbw[4], pbw[5], pbw[6], pbw[7]}};
#pragma unroll
        for (int j = 0; j < 2 * DT; ++j) {
            const int dt = j % DT, st = j / DT;
            oacc[dt] = X::mfma(fv[2 * DT + j], __builtin_bit_cast(V8, pB[st]),
                                                               oacc[dt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            rd(2 * DS + 2 * DT + j + LA);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    int t = 0;
    if constexpr (U) {
        // a tile needs masking when it passes the key end or, under the causal prefix, reaches past the wave's
        // first query
        auto run = [&](int tt, auto buf_c) {
            const int e = tt * kKT + kKT - 1;
            if (e >= int(p.n_k) || (wave_causal && e > int(p.q_pos0) + q0) || hits_hole(tt * kKT, kKT))
                tile_u(tt, buf_c, std::true_type{});
            else
                tile_u(tt, buf_c, std::false_type{});
        };
        for (; t + 1 < ntiles; t += 2) {
            run(t, std::integral_constant<int, 0>{});
            run(t + 1, std::integral_constant<int, 1>{});
        }
        if (t < ntiles)
            run(t, std::integral_constant<int, 0>{});
    } else {
        for (; t + 1 < ntiles; t += 2) {
            tile(t, std::integral_constant<int, 0>{});
            tile(t + 1, std::integral_constant<int, 1>{});
        }
        if (t < ntiles)
            tile(t, std::integral_constant<int, 0>{});
    }
    __builtin_amdgcn_s_waitcnt(0);

    const float lt = add_xor32(l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int qi = q0 + r32;
    if (qi >= int(p.n_q))
        return;
    uint16_t* o = p.out + int64_t(bi) * p.so + int64_t(qi) * p.ldo + int64_t(head) * D;
    // one branch on the output type around stores specialised for each (a test at every pair becomes a branch each)
    auto store = [&](auto h_c) {
        auto pk = [](float a, float b) { return decltype(h_c)::value ? pack_f16x2(a, b) : cvt_bf16x2(a, b); };
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x16& a = oacc[dt];
                *reinterpret_cast<u32x2*>(o + dt * 32 + 8 * i + 4 * hk) =
                    u32x2{pk(a[4 * i] * inv, a[4 * i + 1] * inv), pk(a[4 * i + 2] * inv, a[4 * i + 3] * inv)};
            }
    };
    if (p.out_f16)
        store(std::true_type{});
    else
        store(std::false_type{});
}

} // namespace
} // namespace mk

using namespace mk;

namespace mk {
mk_status attention_to(const void* q, const void* k, const void* vt, void* out, uint32_t dtype, uint32_t batch,
                       uint32_t heads, uint32_t kv_heads, uint32_t d, uint32_t n_q, uint32_t q_pad, uint32_t n_k,
                       uint32_t k_pad, int64_t ldo, int64_t stride_o, uint32_t q_pos0, uint32_t block, float scale,
                       const uint32_t* key_hole, uint32_t out_dtype, void* stream)
{
    if (!q || !k || !vt || !out)
        return fail(MK_ERR_ARG, "attention: null pointer");
    if (out_dtype != MK_BF16 && out_dtype != MK_F16)
        return fail(MK_ERR_ARG, "attention: output bf16 or f16");
    if (dtype != MK_BF16 && dtype != MK_F16)
        return fail(MK_ERR_ARG, "attention: q, k, v must be bf16 or f16");
    if (!heads || !kv_heads || heads % kv_heads)
        return fail(MK_ERR_ARG, "attention: kv_heads must divide heads");
    if (d != 64 && d != 128)
        return fail(MK_ERR_ARG, "attention: head dim must be 64 or 128");
    if (n_q == 0 || n_k == 0 || n_q > q_pad || k_pad % kKT || n_k > k_pad)
        return fail(MK_ERR_ARG, "attention: need 0 < n_q <= q_pad, 0 < n_k <= k_pad, k_pad a multiple of 64");
    if (ldo % 4 || (reinterpret_cast<uintptr_t>(out) & 7))
        return fail(MK_ERR_ARG, "attention: output rows must be 8-byte aligned");
    if (key_hole && batch > uint32_t(kMaxHoleBatch))
        return fail(MK_ERR_ARG, "attention: masked key ranges for at most 8 batch items");
    AttnP p{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(vt),
            static_cast<uint16_t*>(out), heads, heads / kv_heads, batch, n_q, q_pad, n_k, k_pad, q_pos0, block, ldo,
            stride_o,
            scale * 1.4426950408889634f, {}, out_dtype == MK_F16 ? 1u : 0u};
    if (key_hole)
        for (uint32_t b = 0; b < batch; ++b) {
            p.hole[b][0] = key_hole[2 * b];
            p.hole[b][1] = key_hole[2 * b + 1];
            // the first key stays visible (every query row needs one finite score in the first tile)
            if (p.hole[b][0] == 0 && p.hole[b][1] > 0)
                return fail(MK_ERR_ARG, "attention: a masked key range must leave key 0 visible");
        }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool unit = scale == 0.0f;
    // 64-dim heads in launches of fewer 128-query blocks than two a CU take 64-query workgroups (four a CU)
    int cus = 0, dev = 0;
    MK_HIP(hipGetDevice(&dev));
    MK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const bool narrow = d == 64 && uint64_t(cdiv(n_q, 128)) * heads * batch < 2 * uint64_t(cus > 0 ? cus : 1);
    const dim3 grid(cdiv(n_q, 128) * heads * batch), grid2(cdiv(n_q, 64) * heads * batch);
#define MK_ATTN(F16, HOLE)                                                                                         \
    if (d == 128)                                                                                                  \
        unit ? attn2_kernel<128, true, F16, HOLE><<<grid, 256, 0, s>>>(p)                                          \
             : attn2_kernel<128, false, F16, HOLE><<<grid, 256, 0, s>>>(p);                                        \
    else if (narrow)                                                                                               \
        unit ? attn2_kernel<64, true, F16, HOLE, 2><<<grid2, 128, 0, s>>>(p)                                       \
             : attn2_kernel<64, false, F16, HOLE, 2><<<grid2, 128, 0, s>>>(p);                                     \
    else                                                                                                           \
        unit ? attn2_kernel<64, true, F16, HOLE><<<grid, 256, 0, s>>>(p)                                           \
             : attn2_kernel<64, false, F16, HOLE><<<grid, 256, 0, s>>>(p)
    bool hole = false;
    for (uint32_t b = 0; key_hole && b < batch; ++b)
        hole = hole || key_hole[2 * b] < key_hole[2 * b + 1];
    if (dtype == MK_F16) {
        if (hole) {
            MK_ATTN(true, true);
        } else {
            MK_ATTN(true, false);
        }
    } else {
        if (hole) {
            MK_ATTN(false, true);
        } else {
            MK_ATTN(false, false);
        }
    }
#undef MK_ATTN
    MK_LAUNCH_CHECK("attention");
    return MK_OK;
}
} // namespace mk

extern "C" mk_status mk_attention(const void* q, const void* k, const void* vt, void* out, uint32_t dtype,
                                  uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t d, uint32_t n_q,
                                  uint32_t q_pad, uint32_t n_k, uint32_t k_pad, int64_t ldo, int64_t stride_o,
                                  uint32_t q_pos0, uint32_t block, float scale, const uint32_t* key_hole,
                                  void* stream)
{
    return attention_to(q, k, vt, out, dtype, batch, heads, kv_heads, d, n_q, q_pad, n_k, k_pad, ldo, stride_o, q_pos0,
                        block, scale, key_hole, MK_BF16, stream);
}
