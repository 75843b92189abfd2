// The engine: one model family's denoiser with its weights resident on the device, driving the kernel-dispatch
// surface of the C ABI on one stream. It mirrors the reference's Engine subclasses:
//   - load / upload_rows: named checkpoint tensors, q|k|v and gate|up fused along output rows at load
//     (src/image/qwen_image.cpp:79-111, src/image/sdxl.cpp:264-310);
//   - begin(prompt, h, w, slot): the RoPE table and per-slot text state (qwen_image.cpp:113-142; sdxl.cpp:672-720);
//   - step(latents, sigma, slot): one transformer pass (qwen_image.cpp:144-293), here for three graphs over one kernel
//     set: the dual-stream MMDiT (text and image weight sets, shift/scale/gate adaLN, GELU-tanh FFN), Qwen-Image 2.1
//     as the reference runs it (shared weights, scale + tanh gate, SwiGLU, causal text prefix, text K/V cached after
//     the first step), and the SDXL spatial transformer (sdxl.cpp:742-796);
//   - the guided Euler step of the sampler loop (engine.cpp:471-503) with both guidance passes as one batch of 2.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <map>
#include <random>
#include <string>
#include <unordered_map>
#include <memory>
#include <vector>

namespace mk {

namespace {

// Device buffer that grows (zero-filled) on demand.
struct Buf {
    void* p = nullptr;
    size_t bytes = 0;
    Buf() = default;
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    ~Buf()
    {
        if (p)
            (void)hipFree(p);
    }
    mk_status ensure(size_t b)
    {
        if (b <= bytes)
            return MK_OK;
        if (p)
            MK_HIP(hipFree(p));
        p = nullptr;
        bytes = 0;
        MK_HIP(hipMalloc(&p, b));
        MK_HIP(hipMemset(p, 0, b));
        // the null stream's fill must be done before the engine's non-blocking stream uses the buffer
        MK_HIP(hipStreamSynchronize(nullptr));
        bytes = b;
        return MK_OK;
    }
    float* f() const { return static_cast<float*>(p); }
    uint16_t* h() const { return static_cast<uint16_t*>(p); }
};

// A linear layer on the device: W [out][in] (bf16 or fp8 with per-row scale), optional bias.
struct Linear {
    void* w = nullptr;
    uint32_t dtype = MK_BF16;
    float* scale = nullptr;
    float* bias = nullptr;
    uint32_t out = 0, in = 0;
};

// Where a checkpoint tensor goes: a device region (part of a fused tensor) and how to synthesise it.
struct Dest {
    void* p = nullptr;     // first element of this tensor's rows
    uint32_t dtype = MK_F32;
    uint64_t rows = 0, cols = 0;
    float* scale = nullptr; // fp8: per-row scale destination
    double mean = 0, std = 0.02;
};

// Bookkeeping of kernel time per class (events on the step's stream).
struct Timing {
    bool on = false;
    struct Ev {
        hipEvent_t a, b;
        int cls;
        double flops;
    };
    hipEvent_t ref = nullptr; // recorded on the engine's stream before the step's first timed launch
    std::vector<Ev> evs;
    std::vector<std::string> names;
    std::vector<float> ms;
    std::vector<uint32_t> launches;
    std::vector<double> flops;
    int cls(const char* n)
    {
        for (size_t i = 0; i < names.size(); ++i)
            if (names[i] == n)
                return int(i);
        names.push_back(n);
        ms.push_back(0);
        launches.push_back(0);
        flops.push_back(0);
        return int(names.size() - 1);
    }
};

// The rope3 angles of one position (qwen_image.cpp:33-45): axes of 16, 56 and 56 dims, theta 10000, pairs (cos, sin).
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

} // namespace
} // namespace mk

using namespace mk;

// The table begin builds (qwen_image.cpp:113-142): text row t at (t, t, t), image row S + y w + x at frame S and the
// grid position centred as (y - (h - h / 2), x - (w - w / 2)).
extern "C" mk_status mk_rope_table(uint32_t S, uint32_t h, uint32_t w, float* out)
{
    if (!out)
        return fail(MK_ERR_ARG, "rope_table: null");
    for (uint32_t t = 0; t < S; ++t)
        rope3(out + uint64_t(t) * 128, t, t, t);
    for (uint32_t y = 0; y < h; ++y)
        for (uint32_t x = 0; x < w; ++x)
            rope3(out + (uint64_t(S) + uint64_t(y) * w + x) * 128, S, int64_t(y) - int64_t(h - h / 2),
                  int64_t(x) - int64_t(w - w / 2));
    return MK_OK;
}

struct mk_engine {
    // 1 / sqrt(128) * log2(e): the QKV epilogue scales K by it, so attention takes its scores in log2 units
    static constexpr float kScaleLog2 = 0.12751743082459868f;
    mk_config cfg{};
    hipStream_t stream = nullptr;
    // The per-block modulation GEMVs (HBM-bound, 36 us each) run on a second stream, block i's on event mod_ready[i]:
    // their workgroups fill compute units the block GEMMs' partial last rounds leave idle. Default priority, like the
    // main stream; the side stream starts a step only after temb_ready, recorded on the main stream after all of
    // the previous step's work, so it never overwrites modulation a running block still reads.
    hipStream_t side = nullptr;
    hipEvent_t temb_ready = nullptr;
    std::vector<hipEvent_t> mod_ready;
    uint32_t cus = 256; // compute units of the engine's device
    std::vector<void*> allocs; // weight storage
    std::map<std::string, Dest> dests;
    uint64_t weight_bytes = 0;

    // ---- weights (dual: index 0 image stream, 1 text stream) ----
    Linear img_in, txt_in, t_lin1, t_lin2, norm_out, proj_out, mods;
    Linear txt_in1, txt_in2;        // Q21 text in
    float* txt_norm = nullptr;      // Q21: stored zero-centred, +1 applied by the kernel
    struct Block {
        Linear qkv[2], o[2], ff1[2], ff2[2];
        float *nq[2] = {}, *nk[2] = {};
        // SDXL
        Linear q2, kv2;
        float *n1g = nullptr, *n1b = nullptr, *n2g = nullptr, *n2b = nullptr, *n3g = nullptr, *n3b = nullptr;
    };
    std::vector<Block> blocks;
    // SDXL transformer ends
    float *gn_g = nullptr, *gn_b = nullptr;
    Linear proj_in;

    // ---- begin state ----
    struct Slot {
        bool begun = false;
        uint32_t S = 0, steps = 0;
        Buf prompt;               // [S][text_dim] fp32
        Buf kcache, vcache;       // Q21: [blocks][H][S][128] K and [blocks][H][128][S] V^T
        Buf ck, cvt;              // SDXL: per-block cross K [blocks][H][s_pad][64], V^T [blocks][H][64][s_pad]
    } slots[2];
    uint32_t gh = 0, gw = 0;
    std::vector<float> rope_host;
    Buf rope;                     // [tables][S + N][64][2]
    std::vector<uint32_t> rope_key; // (S, h, w, the samples' prompt rows) the table was built for

    // ---- scratch ----
    Buf x_img, x_txt, xn_img, xn_txt, q, k, vt, att, hid, out, lat, lat_bf, tn, tproj, temb_h, temb, mod, omod, qkv;
    Buf vpos; // the positive pass's velocity when guidance runs as two passes
    Buf host_in, host_out; // mk_step_cfg's device copies of the caller's latents (kept: no allocation a step)
    // ordering against a caller's stream (mk_step_cfg_device with another stream): created once, reused
    hipEvent_t ord_in = nullptr, ord_out = nullptr;

    // ---- probe / timing ----
    mk_probe_fn probe = nullptr;
    void* probe_user = nullptr;
    Timing timing;

    // ---------------------------------------------------------------------------------------------------------
    mk_status alloc_w(size_t bytes, void** p)
    {
        MK_HIP(hipMalloc(p, bytes));
        MK_HIP(hipMemset(*p, 0, bytes));
        MK_HIP(hipStreamSynchronize(nullptr));
        allocs.push_back(*p);
        weight_bytes += bytes;
        return MK_OK;
    }
    static size_t esize(uint32_t dt) { return dt == MK_F32 ? 4 : (dt == MK_BF16 || dt == MK_F16) ? 2 : 1; }

    // A fused linear layer from `parts` checkpoint names stacked along output rows (upload_rows).
    mk_status linear(Linear& L, const std::vector<std::string>& parts, uint32_t rows_each, uint32_t in, bool bias,
                     uint32_t dtype = MK_BF16)
    {
        L.out = rows_each * uint32_t(parts.size());
        L.in = in;
        L.dtype = dtype;
        MK_TRY(alloc_w(size_t(L.out) * in * esize(dtype), &L.w));
        if (dtype == MK_FP8_E4M3)
            MK_TRY(alloc_w(size_t(L.out) * 4, reinterpret_cast<void**>(&L.scale)));
        if (bias)
            MK_TRY(alloc_w(size_t(L.out) * 4, reinterpret_cast<void**>(&L.bias)));
        for (size_t i = 0; i < parts.size(); ++i) {
            Dest d;
            d.p = static_cast<char*>(L.w) + i * size_t(rows_each) * in * esize(dtype);
            d.dtype = dtype;
            d.rows = rows_each;
            d.cols = in;
            d.scale = L.scale ? L.scale + i * rows_each : nullptr;
            dests[parts[i] + ".weight"] = d;
            if (bias) {
                Dest b;
                b.p = L.bias + i * rows_each;
                b.rows = rows_each;
                b.cols = 1;
                dests[parts[i] + ".bias"] = b;
            }
        }
        return MK_OK;
    }
    mk_status vec(float** p, const std::string& name, uint32_t n, double mean)
    {
        MK_TRY(alloc_w(size_t(n) * 4, reinterpret_cast<void**>(p)));
        Dest d;
        d.p = *p;
        d.rows = n;
        d.cols = 1;
        d.mean = mean;
        dests[name] = d;
        return MK_OK;
    }

    mk_status build()
    {
        const uint32_t D = cfg.dim, F = cfg.ffn, E = cfg.text_dim, L = cfg.latent, hd = cfg.head_dim;
        const uint32_t wdt = cfg.weight_dtype;
        blocks.resize(cfg.blocks);
        if (cfg.family == MK_FAMILY_DUAL) {
            MK_TRY(linear(img_in, {"img_in"}, D, L, true));
            MK_TRY(vec(&txt_norm, "txt_norm.weight", E, 1.0));
            MK_TRY(linear(txt_in, {"txt_in"}, D, E, true));
            MK_TRY(linear(t_lin1, {"time_text_embed.timestep_embedder.linear_1"}, D, 256, true));
            MK_TRY(linear(t_lin2, {"time_text_embed.timestep_embedder.linear_2"}, D, D, true));
            MK_TRY(linear(norm_out, {"norm_out.linear"}, 2 * D, D, true));
            MK_TRY(linear(proj_out, {"proj_out"}, L, D, true));
            // Every block's image and text modulation stacked: [blocks][2][6D] rows, one GEMV a step.
            std::vector<std::string> mparts;
            for (uint32_t i = 0; i < cfg.blocks; ++i) {
                const std::string b = "transformer_blocks." + std::to_string(i) + ".";
                mparts.push_back(b + "img_mod.1");
                mparts.push_back(b + "txt_mod.1");
            }
            MK_TRY(linear(mods, mparts, 6 * D, D, true));
            for (uint32_t i = 0; i < cfg.blocks; ++i) {
                const std::string b = "transformer_blocks." + std::to_string(i) + ".";
                Block& B = blocks[i];
                MK_TRY(linear(B.qkv[0], {b + "attn.to_q", b + "attn.to_k", b + "attn.to_v"}, D, D, true, wdt));
                MK_TRY(linear(B.qkv[1], {b + "attn.add_q_proj", b + "attn.add_k_proj", b + "attn.add_v_proj"}, D, D,
                              true, wdt));
                MK_TRY(linear(B.o[0], {b + "attn.to_out.0"}, D, D, true, wdt));
                MK_TRY(linear(B.o[1], {b + "attn.to_add_out"}, D, D, true, wdt));
                MK_TRY(vec(&B.nq[0], b + "attn.norm_q.weight", hd, 1.0));
                MK_TRY(vec(&B.nk[0], b + "attn.norm_k.weight", hd, 1.0));
                MK_TRY(vec(&B.nq[1], b + "attn.norm_added_q.weight", hd, 1.0));
                MK_TRY(vec(&B.nk[1], b + "attn.norm_added_k.weight", hd, 1.0));
                MK_TRY(linear(B.ff1[0], {b + "img_mlp.net.0.proj"}, F, D, true, wdt));
                MK_TRY(linear(B.ff2[0], {b + "img_mlp.net.2"}, D, F, true, wdt));
                MK_TRY(linear(B.ff1[1], {b + "txt_mlp.net.0.proj"}, F, D, true, wdt));
                MK_TRY(linear(B.ff2[1], {b + "txt_mlp.net.2"}, D, F, true, wdt));
            }
        } else if (cfg.family == MK_FAMILY_Q21) {
            MK_TRY(linear(img_in, {"img_in"}, D, L, false));
            MK_TRY(vec(&txt_norm, "txt_in.text_norm.weight", E, 0.0));
            MK_TRY(linear(txt_in1, {"txt_in.in_layer"}, D, E, false));
            MK_TRY(linear(txt_in2, {"txt_in.out_layer"}, D, D, false));
            MK_TRY(linear(t_lin1, {"time_text_embed.timestep_embedder.linear_1"}, D, 256, false));
            MK_TRY(linear(t_lin2, {"time_text_embed.timestep_embedder.linear_2"}, D, D, false));
            MK_TRY(linear(mods, {"modulation.1"}, 4 * D, D, false));
            MK_TRY(linear(norm_out, {"norm_out.linear"}, D, D, false));
            MK_TRY(linear(proj_out, {"proj_out"}, L, D, false));
            for (uint32_t i = 0; i < cfg.blocks; ++i) {
                const std::string b = "transformer_blocks." + std::to_string(i) + ".";
                Block& B = blocks[i];
                MK_TRY(linear(B.qkv[0], {b + "attn.to_q", b + "attn.to_k", b + "attn.to_v"}, D, D, false, wdt));
                MK_TRY(linear(B.o[0], {b + "attn.to_out.0"}, D, D, false, wdt));
                MK_TRY(vec(&B.nq[0], b + "attn.norm_q.weight", hd, 1.0));
                MK_TRY(vec(&B.nk[0], b + "attn.norm_k.weight", hd, 1.0));
                // gate rows first (qwen_image.cpp:104-105, 315-316)
                MK_TRY(linear(B.ff1[0], {b + "img_mlp.gate_layer", b + "img_mlp.proj"}, F, D, false, wdt));
                MK_TRY(linear(B.ff2[0], {b + "img_mlp.out"}, D, F, false, wdt));
            }
        } else if (cfg.family == MK_FAMILY_SDXL) {
            // weight_dtype F16: the matrices Sdxl::load_trans reads through Engine::matrix (sdxl.cpp:267-306) are
            // half, as that keeps an F16 checkpoint's (engine.cpp:292-302); q|k|v and the context's k|v (upload_rows)
            // stay bf16
            const uint32_t mdt = wdt == MK_F16 ? MK_F16 : wdt, rdt = wdt == MK_F16 ? MK_BF16 : wdt;
            MK_TRY(vec(&gn_g, "norm.weight", D, 1.0));
            MK_TRY(vec(&gn_b, "norm.bias", D, 0.0));
            MK_TRY(linear(proj_in, {"proj_in"}, D, D, true, wdt == MK_F16 ? MK_F16 : MK_BF16));
            MK_TRY(linear(proj_out, {"proj_out"}, D, D, true, wdt == MK_F16 ? MK_F16 : MK_BF16));
            for (uint32_t i = 0; i < cfg.blocks; ++i) {
                const std::string b = "transformer_blocks." + std::to_string(i) + ".";
                Block& B = blocks[i];
                MK_TRY(vec(&B.n1g, b + "norm1.weight", D, 1.0));
                MK_TRY(vec(&B.n1b, b + "norm1.bias", D, 0.0));
                MK_TRY(vec(&B.n2g, b + "norm2.weight", D, 1.0));
                MK_TRY(vec(&B.n2b, b + "norm2.bias", D, 0.0));
                MK_TRY(vec(&B.n3g, b + "norm3.weight", D, 1.0));
                MK_TRY(vec(&B.n3b, b + "norm3.bias", D, 0.0));
                MK_TRY(linear(B.qkv[0], {b + "attn1.to_q", b + "attn1.to_k", b + "attn1.to_v"}, D, D, false, rdt));
                MK_TRY(linear(B.o[0], {b + "attn1.to_out.0"}, D, D, true, mdt));
                MK_TRY(linear(B.q2, {b + "attn2.to_q"}, D, D, false, mdt));
                MK_TRY(linear(B.kv2, {b + "attn2.to_k", b + "attn2.to_v"}, D, E, false, rdt));
                MK_TRY(linear(B.o[1], {b + "attn2.to_out.0"}, D, D, true, mdt));
                MK_TRY(linear(B.ff1[0], {b + "ff.net.0.proj"}, 2 * F, D, true, mdt));
                MK_TRY(linear(B.ff2[0], {b + "ff.net.2"}, D, F, true, mdt));
            }
        } else {
            return fail(MK_ERR_ARG, "engine: unknown family");
        }
        return MK_OK;
    }

    // ---------------------------------------------------------------------------------------------------------
    // launches with optional timing: events around the launch on its stream (the engine's, or `on`)
    template <typename F>
    mk_status timed(const char* cls, double flops, F&& f, hipStream_t on = nullptr)
    {
        if (!timing.on)
            return f();
        if (timing.evs.empty()) {
            if (!timing.ref)
                MK_HIP(hipEventCreate(&timing.ref));
            MK_HIP(hipEventRecord(timing.ref, stream));
        }
        Timing::Ev ev{};
        MK_HIP(hipEventCreate(&ev.a));
        MK_HIP(hipEventCreate(&ev.b));
        ev.cls = timing.cls(cls);
        ev.flops = flops;
        MK_HIP(hipEventRecord(ev.a, on ? on : stream));
        mk_status s = f();
        MK_HIP(hipEventRecord(ev.b, on ? on : stream));
        timing.evs.push_back(ev);
        return s;
    }
    // Per class: the summed launch durations; and the step's attention and GEMM time as the union of their launches'
    // intervals (class "union:attention+gemm"): the summed durations less any overlap of launches on other streams.
    mk_status finish_timing()
    {
        if (!timing.on)
            return MK_OK;
        MK_HIP(hipStreamSynchronize(stream));
        for (size_t i = 0; i < timing.names.size(); ++i) {
            timing.ms[i] = 0;
            timing.launches[i] = 0;
            timing.flops[i] = 0;
        }
        std::vector<std::pair<float, float>> iv;
        double uflops = 0;
        for (auto& e : timing.evs) {
            float ms = 0, t0 = 0, t1 = 0;
            MK_HIP(hipEventElapsedTime(&ms, e.a, e.b));
            timing.ms[e.cls] += ms;
            timing.launches[e.cls] += 1;
            timing.flops[e.cls] += e.flops;
            const std::string& n = timing.names[e.cls];
            if (n == "attention" || n.compare(0, 4, "gemm") == 0) {
                MK_HIP(hipEventElapsedTime(&t0, timing.ref, e.a));
                MK_HIP(hipEventElapsedTime(&t1, timing.ref, e.b));
                iv.emplace_back(t0, t1);
                uflops += e.flops;
            }
            (void)hipEventDestroy(e.a);
            (void)hipEventDestroy(e.b);
        }
        timing.evs.clear();
        std::sort(iv.begin(), iv.end());
        double uni = 0, lo = 0, hi = -1;
        for (const auto& [a, b] : iv) {
            if (a > hi) {
                uni += hi > lo ? hi - lo : 0;
                lo = a;
                hi = b;
            } else if (b > hi) {
                hi = b;
            }
        }
        uni += hi > lo ? hi - lo : 0;
        const int u = timing.cls("union:attention+gemm");
        timing.ms[u] = float(uni);
        timing.launches[u] = uint32_t(iv.size());
        timing.flops[u] = uflops;
        return MK_OK;
    }

    // GEMM: C[batch][M][ldc] (epilogue) = A[batch][M][lda] W^T
    mk_status gemm(const Linear& L, const void* A, int64_t lda, int64_t sa, uint32_t M, uint32_t batch, void* C,
                   int64_t ldc, int64_t sc, uint32_t epi, uint32_t cdt, const float* gate = nullptr,
                   int64_t gate_alt = 0, uint32_t split = 0, uint32_t seg = 0, const mk_heads_args* heads = nullptr,
                   const char* cls = "gemm")
    {
        const mk_gemm_args g = gemm_args(L, A, lda, sa, M, batch, C, ldc, sc, epi, cdt, gate, gate_alt, split, seg,
                                         heads);
        return timed(cls, 2.0 * M * L.out * L.in * batch, [&] { return mk_gemm(&g, stream); });
    }
    // Two GEMMs of equal N, K and epilogue kind (a block's image and text projections) in one launch.
    // Two GEMMs of equal N, K and epilogue kind (a block's image and text projections): one launch when that takes
    // fewer waves of tiles than two (the text's few tiles fill the image's last wave), else two.
    // Timing classes: `cls` for the grouped launch, cls + ".img" / ".txt" when the two go separately.
    mk_status gemm2(const mk_gemm_args (&g)[2], const char* cls)
    {
        const bool one = launch_cost(g, 2) < launch_cost(g, 1) + launch_cost(g + 1, 1);
        if (one) {
            const double fl = 2.0 * g[0].N * g[0].K * (double(g[0].M) * g[0].batch + double(g[1].M) * g[1].batch);
            return timed(cls, fl, [&] { return mk_gemm_grouped(g, 2, stream); });
        }
        for (int i = 0; i < 2; ++i) {
            const std::string c = std::string(cls) + (i ? ".txt" : ".img");
            MK_TRY(timed(c.c_str(), 2.0 * g[i].N * g[i].K * double(g[i].M) * g[i].batch,
                         [&] { return mk_gemm_grouped(g + i, 1, stream); }));
        }
        return MK_OK;
    }
    // Estimated duration of a launch (the GEMM dispatch's own plan: tile width, waves, stream-K).
    double launch_cost(const mk_gemm_args* g, int n) const { return gemm_cost(g, uint32_t(n), cus); }
    static mk_gemm_args gemm_args(const Linear& L, const void* A, int64_t lda, int64_t sa, uint32_t M, uint32_t batch,
                                  void* C, int64_t ldc, int64_t sc, uint32_t epi, uint32_t cdt,
                                  const float* gate = nullptr, int64_t gate_alt = 0, uint32_t split = 0,
                                  uint32_t seg = 0, const mk_heads_args* heads = nullptr)
    {
        mk_gemm_args g{};
        g.a = A;
        g.w = L.w;
        g.wscale = L.scale;
        g.bias = L.bias;
        g.c = C;
        g.gate = gate;
        g.gate_alt = gate_alt;
        g.split = split;
        g.seg_rows = seg;
        g.M = M;
        g.N = L.out;
        g.K = L.in;
        g.lda = lda;
        g.ldc = ldc;
        g.stride_a = sa;
        g.stride_c = sc;
        g.batch = batch;
        g.w_dtype = L.dtype;
        g.c_dtype = cdt;
        g.epilogue = epi;
        g.heads = heads;
        return g;
    }

    mk_status probe_f32(const char* name, int layer, const float* d, size_t n)
    {
        if (!probe)
            return MK_OK;
        std::vector<float> h(n);
        MK_HIP(hipStreamSynchronize(stream));
        MK_HIP(hipMemcpy(h.data(), d, n * 4, hipMemcpyDeviceToHost));
        probe(probe_user, name, layer, h.data(), n);
        return MK_OK;
    }
    mk_status probe_bf16(const char* name, int layer, const uint16_t* d, size_t n)
    {
        if (!probe)
            return MK_OK;
        std::vector<uint16_t> h(n);
        std::vector<float> f(n);
        MK_HIP(hipStreamSynchronize(stream));
        MK_HIP(hipMemcpy(h.data(), d, n * 2, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < n; ++i)
            f[i] = bf2f_bits(h[i]);
        probe(probe_user, name, layer, f.data(), n);
        return MK_OK;
    }

    // The RoPE table(s) of a step: one table of S + h w rows (mk_rope_table) when n = 1; n tables for samples whose
    // prompts have Sb[b] <= S rows, all padded to S text rows: table b holds the text positions 0 .. S - 1 and, from
    // row S on, its image rows at frame Sb[b].
    mk_status make_rope(const uint32_t* Sb, uint32_t n, uint32_t S)
    {
        std::vector<uint32_t> key{S, gh, gw};
        key.insert(key.end(), Sb, Sb + n);
        if (key == rope_key)
            return MK_OK;
        const uint64_t N = uint64_t(gh) * gw, rows = S + N;
        std::vector<float> base(rows * 128), t;
        MK_TRY(mk_rope_table(S, gh, gw, base.data()));
        rope_host.assign(n * rows * 128, 0.0f);
        for (uint32_t b = 0; b < n; ++b) {
            float* tab = rope_host.data() + b * rows * 128;
            if (Sb[b] == S) {
                std::copy(base.begin(), base.end(), tab);
            } else {
                std::copy(base.begin(), base.begin() + S * 128, tab); // the text positions 0 .. S - 1
                t.assign((Sb[b] + N) * 128, 0.0f);
                MK_TRY(mk_rope_table(Sb[b], gh, gw, t.data()));
                std::copy(t.begin() + Sb[b] * 128, t.end(), tab + S * 128); // the image rows at frame Sb[b]
            }
        }
        MK_TRY(rope.ensure(rope_host.size() * 4));
        MK_HIP(hipMemcpy(rope.p, rope_host.data(), rope_host.size() * 4, hipMemcpyHostToDevice));
        rope_key = key;
        return MK_OK;
    }
    mk_status make_rope(uint32_t S) { return make_rope(&S, 1, S); }

    // Sinusoidal embedding, cos half first (qwen_image.cpp:179-187), of v (= 1000 sigma) for each row.
    static void sinusoid(float v, float* out)
    {
        for (uint32_t i = 0; i < 128; ++i) {
            const float freq = std::exp(-std::log(10000.0f) * float(i) / 128.0f);
            out[i] = std::cos(v * freq);
            out[128 + i] = std::sin(v * freq);
        }
    }

    // ---------------------------------------------------------------------------------------------------------
    // Dual-stream step over `nb` samples sharing sigma: lat [nb][N][L] fp32 (device) -> out [nb][N][L] fp32.
    // slot_of[b] names the text state of sample b; all samples' texts have S rows.
    mk_status dual_step(const float* lat_dev, float sigma, const uint32_t* slot_of, uint32_t nb)
    {
        const uint32_t D = cfg.dim, H = cfg.heads, F = cfg.ffn, E = cfg.text_dim, L = cfg.latent;
        // a guidance batch whose prompts differ in length: every sample's text takes S = the longest prompt's rows,
        // a shorter prompt's rows [S_b, S) are zero on input and masked as keys; sample b's image rows keep their
        // RoPE frame S_b (one table a sample)
        uint32_t Sb[2] = {slots[slot_of[0]].S, nb > 1 ? slots[slot_of[1]].S : 0};
        const uint32_t S = nb > 1 ? std::max(Sb[0], Sb[1]) : Sb[0], N = gh * gw, T = S + N;
        const bool ragged = nb > 1 && Sb[0] != Sb[1];
        const uint32_t q_pad = uint32_t(round_up(T, 256)), k_pad = uint32_t(round_up(T, 64));
        const float eps = 1e-6f;
        MK_TRY(make_rope(Sb, ragged ? nb : 1, S));
        uint32_t hole[4] = {Sb[0], S, Sb[1], S}; // keys [S_b, S) of sample b
        // scratch
        MK_TRY(x_img.ensure(size_t(nb) * N * D * 4));
        MK_TRY(x_txt.ensure(size_t(nb) * S * D * 4));
        MK_TRY(xn_img.ensure(size_t(nb) * N * D * 2));
        MK_TRY(xn_txt.ensure(size_t(nb) * S * D * 2));
        MK_TRY(q.ensure(size_t(nb) * H * q_pad * 128 * 2));
        MK_TRY(k.ensure(size_t(nb) * H * k_pad * 128 * 2));
        MK_TRY(vt.ensure(size_t(nb) * H * 128 * k_pad * 2));
        MK_TRY(att.ensure(size_t(nb) * T * D * 2));
        MK_TRY(hid.ensure(size_t(nb) * (N + S) * F * 2)); // image rows, then text rows
        MK_TRY(out.ensure(size_t(nb) * N * L * 4));
        MK_TRY(lat_bf.ensure(size_t(nb) * N * L * 2));
        MK_TRY(tn.ensure(size_t(nb) * S * E * 2));
        MK_TRY(tproj.ensure(256 * 4));
        MK_TRY(temb_h.ensure(size_t(D) * 4));
        MK_TRY(temb.ensure(size_t(D) * 4));
        MK_TRY(mod.ensure(size_t(cfg.blocks) * 12 * D * 4));
        MK_TRY(omod.ensure(size_t(2) * D * 4));
        if (k_pad_last != k_pad) {
            // a new key padding: the padded keys / values must be zero
            MK_TRY(fill_zero(k.p, k.bytes, stream));
            MK_TRY(fill_zero(vt.p, vt.bytes, stream));
            k_pad_last = k_pad;
        }
        // time embedding -> every block's modulation (silu(temb) feeds them all) and the output norm's
        float tp[256];
        sinusoid(1000.0f * sigma, tp);
        MK_HIP(hipMemcpyAsync(tproj.p, tp, sizeof(tp), hipMemcpyHostToDevice, stream));
        MK_TRY(timed("gemv", 2.0 * D * 256, [&] { return mk_gemv(tproj.f(), 1, 256, t_lin1.w, t_lin1.bias, D, temb_h.f(), 0, stream); }));
        MK_TRY(timed("gemv", 2.0 * D * D, [&] { return mk_gemv(temb_h.f(), 1, D, t_lin2.w, t_lin2.bias, D, temb.f(), 1, stream); }));
        MK_TRY(probe_f32("temb", -1, temb.f(), D));
        // every block's modulation: one GEMV over the stacked matrix when timing or probing (serial, measured), else
        // one GEMV a block on the side stream
        const bool side_mods = !timing.on && !probe && side && mod_ready.size() >= cfg.blocks;
        if (side_mods) {
            MK_HIP(hipEventRecord(temb_ready, stream));
            MK_HIP(hipStreamWaitEvent(side, temb_ready, 0));
            for (uint32_t i = 0; i < cfg.blocks; ++i) {
                const size_t r0 = size_t(i) * 12 * D;
                MK_TRY(mk_gemv(temb.f(), 1, D, static_cast<const uint16_t*>(mods.w) + r0 * D,
                               mods.bias ? mods.bias + r0 : nullptr, 12 * D, mod.f() + r0, 1, side));
                MK_HIP(hipEventRecord(mod_ready[i], side));
            }
        } else {
            MK_TRY(timed("gemv", 2.0 * mods.out * D, [&] { return mk_gemv(temb.f(), 1, D, mods.w, mods.bias, mods.out, mod.f(), 1, stream); }));
            MK_TRY(probe_f32("modulation", -1, mod.f(), size_t(cfg.blocks) * 12 * D));
        }
        MK_TRY(timed("gemv", 2.0 * 2 * D * D, [&] { return mk_gemv(temb.f(), 1, D, norm_out.w, norm_out.bias, 2 * D, omod.f(), 1, stream); }));
        // text in: RMSNorm(w) -> Linear; image in: Linear
        for (uint32_t b = 0; b < nb; ++b) {
            MK_TRY(timed("norm", 0, [&] {
                return mk_rms_norm(slots[slot_of[b]].prompt.f(), Sb[b], E, txt_norm, 0.0f, eps,
                                   tn.h() + size_t(b) * S * E, stream);
            }));
            if (Sb[b] < S)
                MK_TRY(fill_zero(tn.h() + (size_t(b) * S + Sb[b]) * E, size_t(S - Sb[b]) * E * 2, stream));
        }
        MK_TRY(gemm(txt_in, tn.p, E, 0, nb * S, 1, x_txt.p, D, 0, MK_EPI_STORE, MK_F32));
        MK_TRY(timed("convert", 0, [&] { return mk_f32_to_bf16(lat_dev, size_t(nb) * N * L, lat_bf.p, stream); }));
        MK_TRY(gemm(img_in, lat_bf.p, L, 0, nb * N, 1, x_img.p, D, 0, MK_EPI_STORE, MK_F32));
        if (probe)
            for (uint32_t b = 0; b < nb; ++b) {
                MK_TRY(probe_f32("txt_in", int(b), x_txt.f() + size_t(b) * S * D, size_t(S) * D));
                MK_TRY(probe_f32("img_in", int(b), x_img.f() + size_t(b) * N * D, size_t(N) * D));
            }
        const double attn_flops = 4.0 * double(T) * T * 128 * H * nb;
        for (uint32_t i = 0; i < cfg.blocks; ++i) {
            if (side_mods)
                MK_HIP(hipStreamWaitEvent(stream, mod_ready[i], 0));
            const Block& B = blocks[i];
            const float* mi = mod.f() + size_t(i) * 12 * D; // image: shift1, scale1, gate1, shift2, scale2, gate2
            const float* mt = mi + 6 * D;                    // text
            struct St {
                Buf *x, *xn;
                uint32_t rows, row0, which;
                const float* m;
                uint16_t* hid;
            } st[2] = {{&x_img, &xn_img, N, S, 0, mi, hid.h()}, {&x_txt, &xn_txt, S, 0, 1, mt, hid.h() + size_t(nb) * N * F}};
            mk_heads_args ha[2];
            mk_gemm_args g[2];
            // both streams' norms in one launch: scale m + D, shift m (and below m + 4D, m + 3D)
            auto ln2 = [&](int scale_off, int shift_off) {
                LnArgs la[2];
                for (int j = 0; j < 2; ++j)
                    la[j] = LnArgs{st[j].x->f(), st[j].m + scale_off, st[j].m + shift_off, 0, nb * st[j].rows, 0, 1,
                                   st[j].xn->p};
                return timed("ln_modulate", 0, [&] { return ln_modulate_group(la, 2, D, eps, stream); });
            };
            MK_TRY(ln2(D, 0));
            for (int j = 0; j < 2; ++j) {
                const St& s = st[j];
                ha[j] = mk_heads_args{};
                ha[j].q = q.p;
                ha[j].k = k.p;
                ha[j].vt = vt.p;
                ha[j].heads = H;
                ha[j].head_dim = 128;
                ha[j].q_pad = q_pad;
                ha[j].k_pad = k_pad;
                ha[j].row0 = s.row0;
                ha[j].q_row0 = s.row0;
                ha[j].norm_q = B.nq[s.which];
                ha[j].norm_k = B.nk[s.which];
                ha[j].rope = rope.f();
                ha[j].rope_stride = ragged ? int64_t(T) * 128 : 0;
                ha[j].rope_mode = 2;
                ha[j].eps = eps;
                ha[j].k_scale = kScaleLog2; // K carries the softmax scale: attention runs with scale 0
                g[j] = gemm_args(B.qkv[s.which], s.xn->p, D, int64_t(s.rows) * D, s.rows, nb, nullptr, 0, 0,
                                 MK_EPI_HEADS, MK_BF16, nullptr, 0, 0, 0, &ha[j]);
            }
            MK_TRY(gemm2(g, "gemm.qkv"));
            MK_TRY(timed("attention", attn_flops, [&] {
                return mk_attention(q.p, k.p, vt.p, att.p, MK_BF16, nb, H, H, 128, T, q_pad, T, k_pad, D,
                                    int64_t(T) * D, 0, 0, 0.0f, ragged ? hole : nullptr, stream);
            }));
            for (int j = 0; j < 2; ++j) {
                const St& s = st[j];
                const uint16_t* a = att.h() + size_t(s.row0) * D; // image rows after the text's
                g[j] = gemm_args(B.o[s.which], a, D, int64_t(T) * D, s.rows, nb, s.x->p, D, int64_t(s.rows) * D,
                                 MK_EPI_GATE_ADD, MK_F32, s.m + 2 * D);
            }
            MK_TRY(gemm2(g, "gemm.o"));
            MK_TRY(ln2(4 * D, 3 * D));
            for (int j = 0; j < 2; ++j) {
                const St& s = st[j];
                g[j] = gemm_args(B.ff1[s.which], s.xn->p, D, 0, nb * s.rows, 1, s.hid, F, 0, MK_EPI_GELU_TANH, MK_BF16);
            }
            MK_TRY(gemm2(g, "gemm.ff1"));
            for (int j = 0; j < 2; ++j) {
                const St& s = st[j];
                g[j] = gemm_args(B.ff2[s.which], s.hid, F, 0, nb * s.rows, 1, s.x->p, D, 0, MK_EPI_GATE_ADD, MK_F32,
                                 s.m + 5 * D);
            }
            MK_TRY(gemm2(g, "gemm.ff2"));
            if (probe)
                for (uint32_t b = 0; b < nb; ++b)
                    MK_TRY(probe_f32("block", int(i * nb + b), x_img.f() + size_t(b) * N * D, size_t(N) * D));
        }
        // output norm (scale first, then shift: AdaLayerNormContinuous) -> proj_out on the image rows
        MK_TRY(timed("ln_modulate", 0, [&] {
            return mk_ln_modulate(x_img.f(), nb * N, D, omod.f(), omod.f() + D, 0, 0, 1, eps, xn_img.p, stream);
        }));
        if (probe)
            for (uint32_t b = 0; b < nb; ++b)
                MK_TRY(probe_bf16("norm_out", int(b), xn_img.h() + size_t(b) * N * D, size_t(N) * D));
        MK_TRY(gemm(proj_out, xn_img.p, D, 0, nb * N, 1, out.p, L, 0, MK_EPI_STORE, MK_F32));
        return MK_OK;
    }
    uint32_t k_pad_last = 0;

    // ---------------------------------------------------------------------------------------------------------
    // Qwen-Image 2.1 step for one slot (qwen_image.cpp:144-293): the first step runs [text; image] and keeps the
    // text's K / V per block; later steps run the image rows against them.
    mk_status q21_step(const float* lat_dev, float sigma, uint32_t slot)
    {
        Slot& g = slots[slot];
        const uint32_t D = cfg.dim, H = cfg.heads, F = cfg.ffn, E = cfg.text_dim, L = cfg.latent;
        const uint32_t N = gh * gw, S = g.S;
        const bool first = g.steps++ == 0;
        const uint32_t T = first ? S + N : N, row0 = first ? 0 : S, n_k = S + N;
        const uint32_t q_pad = uint32_t(round_up(T, 256)), k_pad = uint32_t(round_up(n_k, 64)),
                       split = first ? S : 0;
        const float eps = 1e-6f;
        MK_TRY(make_rope(S));
        MK_TRY(x_img.ensure(size_t(T) * D * 4));
        MK_TRY(xn_img.ensure(size_t(T) * D * 2));
        MK_TRY(q.ensure(size_t(H) * q_pad * 128 * 2));
        MK_TRY(k.ensure(size_t(H) * k_pad * 128 * 2));
        MK_TRY(vt.ensure(size_t(H) * 128 * k_pad * 2));
        MK_TRY(att.ensure(size_t(T) * D * 2));
        MK_TRY(hid.ensure(size_t(T) * F * 2));
        MK_TRY(out.ensure(size_t(T) * L * 4));
        MK_TRY(lat_bf.ensure(size_t(N) * L * 2));
        MK_TRY(tn.ensure(size_t(S) * E * 2));
        MK_TRY(tproj.ensure(2 * 256 * 4));
        MK_TRY(temb_h.ensure(size_t(2) * D * 4));
        MK_TRY(temb.ensure(size_t(2) * D * 4));
        MK_TRY(mod.ensure(size_t(2) * 4 * D * 4));
        MK_TRY(omod.ensure(size_t(2) * D * 4));
        if (k_pad_last != k_pad) { // padding keys zero (the heads epilogue writes rows < n only)
            MK_TRY(fill_zero(k.p, k.bytes, stream));
            MK_TRY(fill_zero(vt.p, vt.bytes, stream));
            k_pad_last = k_pad;
        }
        const uint32_t S16 = uint32_t(round_up(S, 16)); // V^T cache columns: whole groups of 16 keys
        if (first) {
            MK_TRY(g.kcache.ensure(size_t(cfg.blocks) * H * S * 128 * 2));
            MK_TRY(g.vcache.ensure(size_t(cfg.blocks) * H * 128 * S16 * 2));
        }
        // rows [sigma, t = 0]: t_lin1 -> silu -> t_lin2 -> (probe) -> silu -> modulation / out_lin
        float tp[512];
        sinusoid(1000.0f * sigma, tp);
        sinusoid(0.0f, tp + 256);
        MK_HIP(hipMemcpyAsync(tproj.p, tp, sizeof(tp), hipMemcpyHostToDevice, stream));
        MK_TRY(timed("gemv", 0, [&] { return mk_gemv(tproj.f(), 2, 256, t_lin1.w, nullptr, D, temb_h.f(), 0, stream); }));
        MK_TRY(timed("gemv", 0, [&] { return mk_gemv(temb_h.f(), 2, D, t_lin2.w, nullptr, D, temb.f(), 1, stream); }));
        MK_TRY(probe_f32("temb", -1, temb.f(), 2 * D));
        MK_TRY(timed("gemv", 0, [&] { return mk_gemv(temb.f(), 2, D, mods.w, nullptr, 4 * D, mod.f(), 1, stream); }));
        MK_TRY(probe_f32("modulation", -1, mod.f(), 8 * D));
        MK_TRY(timed("gemv", 0, [&] { return mk_gemv(temb.f(), 2, D, norm_out.w, nullptr, D, omod.f(), 1, stream); }));
        if (first) {
            MK_TRY(timed("norm", 0, [&] { return mk_rms_norm(g.prompt.f(), S, E, txt_norm, 1.0f, eps, tn.p, stream); }));
            MK_TRY(gemm(txt_in1, tn.p, E, 0, S, 1, hid.p, D, 0, MK_EPI_GELU_TANH, MK_BF16));
            MK_TRY(gemm(txt_in2, hid.p, D, 0, S, 1, x_img.p, D, 0, MK_EPI_STORE, MK_F32));
            MK_TRY(probe_f32("txt_in", -1, x_img.f(), size_t(S) * D));
        }
        MK_TRY(timed("convert", 0, [&] { return mk_f32_to_bf16(lat_dev, size_t(N) * L, lat_bf.p, stream); }));
        float* ximg = x_img.f() + size_t(T - N) * D;
        MK_TRY(gemm(img_in, lat_bf.p, L, 0, N, 1, ximg, D, 0, MK_EPI_STORE, MK_F32));
        MK_TRY(probe_f32("img_in", -1, ximg, size_t(N) * D));
        // attention flops: image rows see all keys; text rows (first step) see their causal prefix
        const double pairs = double(N) * n_k + (first ? double(S) * (S + 1) / 2 : 0.0);
        for (uint32_t i = 0; i < cfg.blocks; ++i) {
            const Block& B = blocks[i];
            MK_TRY(timed("ln_modulate", 0, [&] {
                return mk_ln_modulate(x_img.f(), T, D, mod.f(), nullptr, 4 * D, split, T, eps, xn_img.p, stream);
            }));
            mk_heads_args ha{};
            ha.q = q.p;
            ha.k = k.p;
            ha.vt = vt.p;
            ha.heads = H;
            ha.head_dim = 128;
            ha.q_pad = q_pad;
            ha.k_pad = k_pad;
            ha.row0 = row0;
            ha.q_row0 = 0;
            ha.norm_q = B.nq[0];
            ha.norm_k = B.nk[0];
            ha.rope = rope.f();
            ha.rope_mode = 2;
            ha.eps = eps;
            ha.k_scale = kScaleLog2;
            ha.dtype = MK_F16; // the reference's heads_norm_half / heads_half
            // the text's keys and values (heads_rows): kept after the first step's q/k/v, restored before the later
            // steps'. V^T keeps whole groups of 16 keys (its columns permute keys within a group); a group shared
            // with image keys is rewritten by the image rows' q/k/v that follow the restore.
            uint16_t* kc = g.kcache.h() + size_t(i) * H * S * 128;
            uint16_t* vc = g.vcache.h() + size_t(i) * H * 128 * S16;
            if (!first) {
                MK_HIP(hipMemcpy2DAsync(k.p, size_t(k_pad) * 256, kc, size_t(S) * 256, size_t(S) * 256, H,
                                        hipMemcpyDeviceToDevice, stream));
                MK_HIP(hipMemcpy2DAsync(vt.p, size_t(k_pad) * 2, vc, size_t(S16) * 2, size_t(S16) * 2,
                                        size_t(H) * 128, hipMemcpyDeviceToDevice, stream));
            }
            MK_TRY(gemm(B.qkv[0], xn_img.p, D, 0, T, 1, nullptr, 0, 0, MK_EPI_HEADS, MK_BF16, nullptr, 0, 0, 0, &ha,
                        "gemm.qkv"));
            if (first) {
                MK_HIP(hipMemcpy2DAsync(kc, size_t(S) * 256, k.p, size_t(k_pad) * 256, size_t(S) * 256, H,
                                        hipMemcpyDeviceToDevice, stream));
                MK_HIP(hipMemcpy2DAsync(vc, size_t(S16) * 2, vt.p, size_t(k_pad) * 2, size_t(S16) * 2,
                                        size_t(H) * 128, hipMemcpyDeviceToDevice, stream));
            }
            MK_TRY(timed("attention", 4.0 * pairs * 128 * H, [&] {
                return mk_attention(q.p, k.p, vt.p, att.p, MK_F16, 1, H, H, 128, T, q_pad, n_k, k_pad, D, 0, row0, S, 0.0f,
                                    nullptr, stream);
            }));
            MK_TRY(gemm(B.o[0], att.p, D, 0, T, 1, x_img.p, D, 0, MK_EPI_GATE_TANH, MK_F32, mod.f() + D, 4 * D, split,
                        T, nullptr, "gemm.o"));
            MK_TRY(timed("ln_modulate", 0, [&] {
                return mk_ln_modulate(x_img.f(), T, D, mod.f() + 2 * D, nullptr, 4 * D, split, T, eps, xn_img.p,
                                      stream);
            }));
            // gate|up -> swiglu_rows fused: the GEMM's epilogue takes silu(gate) up on the fp32 accumulators
            MK_TRY(gemm(B.ff1[0], xn_img.p, D, 0, T, 1, hid.p, F, 0, MK_EPI_SWIGLU, MK_BF16, nullptr, 0, 0, 0, nullptr,
                        "gemm.ff1"));
            MK_TRY(gemm(B.ff2[0], hid.p, F, 0, T, 1, x_img.p, D, 0, MK_EPI_GATE_TANH, MK_F32, mod.f() + 3 * D, 4 * D,
                        split, T, nullptr, "gemm.ff2"));
            MK_TRY(probe_f32("block", int(i), x_img.f(), size_t(T) * D));
        }
        MK_TRY(timed("ln_modulate", 0, [&] {
            return mk_ln_modulate(x_img.f(), T, D, omod.f(), nullptr, D, split, T, eps, xn_img.p, stream);
        }));
        MK_TRY(probe_bf16("norm_out", -1, xn_img.h(), size_t(T) * D));
        MK_TRY(gemm(proj_out, xn_img.h() + size_t(T - N) * D, D, 0, N, 1, out.p, L, 0, MK_EPI_STORE, MK_F32));
        return MK_OK;
    }

    // ---------------------------------------------------------------------------------------------------------
    // SDXL: the context's keys / values per block for a slot (sdxl.cpp:693-719).
    mk_status sdxl_begin(uint32_t slot)
    {
        Slot& g = slots[slot];
        const uint32_t c = cfg.dim, H = c / 64, E = cfg.text_dim, S = g.S, s_pad = uint32_t(round_up(S, 64));
        MK_TRY(tn.ensure(size_t(S) * E * 2));
        MK_TRY(qkv.ensure(size_t(S) * 2 * c * 2));
        // layout [blocks][slot][H][s_pad][64] (K) and [blocks][slot][H][64][s_pad] (V^T): both slots of a block
        // form a batch of 2 for the cross attention.
        MK_TRY(slots[0].ck.ensure(size_t(cfg.blocks) * 2 * H * s_pad * 64 * 2));
        MK_TRY(slots[0].cvt.ensure(size_t(cfg.blocks) * 2 * H * 64 * s_pad * 2));
        sdxl_spad = s_pad;
        MK_TRY(timed("convert", 0, [&] { return mk_f32_to_bf16(g.prompt.f(), size_t(S) * E, tn.p, stream); }));
        for (uint32_t i = 0; i < cfg.blocks; ++i) {
            // the reference's half heads of the fp32 projection (heads_half, sdxl.cpp:697-708): the k|v GEMM's
            // epilogue rounds its accumulators to half once, straight into K and V^T
            mk_heads_args ha{};
            ha.k = slots[0].ck.h() + (size_t(i) * 2 + slot) * H * s_pad * 64;
            ha.vt = slots[0].cvt.h() + (size_t(i) * 2 + slot) * H * 64 * s_pad;
            ha.heads = H;
            ha.head_dim = 64;
            ha.k_pad = s_pad;
            ha.dtype = MK_F16;
            MK_TRY(gemm(blocks[i].kv2, tn.p, E, 0, S, 1, nullptr, 0, 0, MK_EPI_HEADS, MK_BF16, nullptr, 0, 0, 0, &ha));
        }
        return MK_OK;
    }
    uint32_t sdxl_spad = 0;

    // trans_fwd (sdxl.cpp:742-796) for nb samples: x [nb][n][c] fp32 -> y [nb][n][c] fp32.
    mk_status sdxl_forward(const float* x, uint32_t nb, uint32_t n, float* y)
    {
        const uint32_t c = cfg.dim, H = c / 64, F = cfg.ffn, S = slots[0].S;
        const uint32_t q_pad = uint32_t(round_up(n, 256)), k_pad = uint32_t(round_up(n, 64)), s_pad = sdxl_spad;
        MK_TRY(xn_img.ensure(size_t(nb) * n * c * 2));
        MK_TRY(x_img.ensure(size_t(nb) * n * c * 4));
        MK_TRY(q.ensure(size_t(nb) * H * q_pad * 64 * 2));
        MK_TRY(k.ensure(size_t(nb) * H * k_pad * 64 * 2));
        MK_TRY(vt.ensure(size_t(nb) * H * 64 * k_pad * 2));
        MK_TRY(att.ensure(size_t(nb) * n * c * 2));
        MK_TRY(hid.ensure(size_t(nb) * n * F * 2));
        if (k_pad_last != k_pad) { // padding keys zero (the heads epilogue writes rows < n only)
            MK_TRY(fill_zero(k.p, k.bytes, stream));
            MK_TRY(fill_zero(vt.p, vt.bytes, stream));
            k_pad_last = k_pad;
        }
        // Q, K, V^T as half (the reference's heads_half, sdxl.cpp:439-448), written by the projections' epilogue
        mk_heads_args ha{};
        ha.q = q.p;
        ha.k = k.p;
        ha.vt = vt.p;
        ha.heads = H;
        ha.head_dim = 64;
        ha.q_pad = q_pad;
        ha.k_pad = k_pad;
        ha.dtype = MK_F16;
        mk_heads_args hq = ha; // the cross attention's Q alone
        hq.k = hq.vt = nullptr;
        // the self attention's K carries its softmax scale in log2 units (1 / sqrt(64) * log2(e)), so it runs the
        // unit-scale attention (scores arrive as S - m from the matrix core; the softmax in the MFMAs' shadow)
        ha.k_scale = 0.18033688011112042f;
        float* hs = x_img.f();
        const int64_t nc = int64_t(n) * c;
        // the type of a GEMM's input: half for a half matrix (both matrix-core operands take one type), else bf16;
        // the norms, the attention and the GEGLU epilogue write their outputs in the type of the GEMM they feed
        auto in_dt = [](const Linear& L) { return L.dtype == MK_F16 ? uint32_t(MK_F16) : uint32_t(MK_BF16); };
        MK_TRY(timed("norm", 0, [&] {
            return group_norm_to(x, nb, n, c, 32, gn_g, gn_b, 1e-6f, xn_img.p, in_dt(proj_in), stream);
        }));
        MK_TRY(gemm(proj_in, xn_img.p, c, 0, nb * n, 1, hs, c, 0, MK_EPI_STORE, MK_F32));
        const float scale = 0.125f;
        for (uint32_t i = 0; i < cfg.blocks; ++i) {
            const Block& B = blocks[i];
            MK_TRY(timed("norm", 0, [&] {
                return layer_norm_to(hs, nb * n, c, B.n1g, B.n1b, 1e-5f, xn_img.p, in_dt(B.qkv[0]), stream);
            }));
            MK_TRY(gemm(B.qkv[0], xn_img.p, c, nc, n, nb, nullptr, 0, 0, MK_EPI_HEADS, MK_BF16, nullptr, 0, 0, 0, &ha,
                        "gemm.qkv"));
            MK_TRY(timed("attention", 4.0 * double(n) * n * 64 * H * nb, [&] {
                return attention_to(q.p, k.p, vt.p, att.p, MK_F16, nb, H, H, 64, n, q_pad, n, k_pad, c, nc, 0, 0, 0.0f,
                                    nullptr, in_dt(B.o[0]), stream);
            }));
            MK_TRY(gemm(B.o[0], att.p, c, 0, nb * n, 1, hs, c, 0, MK_EPI_ADD, MK_F32, nullptr, 0, 0, 0, nullptr,
                        "gemm.o"));
            MK_TRY(timed("norm", 0, [&] {
                return layer_norm_to(hs, nb * n, c, B.n2g, B.n2b, 1e-5f, xn_img.p, in_dt(B.q2), stream);
            }));
            MK_TRY(gemm(B.q2, xn_img.p, c, nc, n, nb, nullptr, 0, 0, MK_EPI_HEADS, MK_BF16, nullptr, 0, 0, 0, &hq,
                        "gemm.q2"));
            // cross attention: batch b reads slot b's context keys (consecutive in the cache)
            const uint16_t* kc = slots[0].ck.h() + size_t(i) * 2 * H * s_pad * 64;
            const uint16_t* vc = slots[0].cvt.h() + size_t(i) * 2 * H * 64 * s_pad;
            MK_TRY(timed("attention", 4.0 * double(n) * S * 64 * H * nb, [&] {
                return attention_to(q.p, kc, vc, att.p, MK_F16, nb, H, H, 64, n, q_pad, S, s_pad, c, nc, 0, 0, scale,
                                    nullptr, in_dt(B.o[1]), stream);
            }));
            MK_TRY(gemm(B.o[1], att.p, c, 0, nb * n, 1, hs, c, 0, MK_EPI_ADD, MK_F32, nullptr, 0, 0, 0, nullptr,
                        "gemm.o2"));
            MK_TRY(timed("norm", 0, [&] {
                return layer_norm_to(hs, nb * n, c, B.n3g, B.n3b, 1e-5f, xn_img.p, in_dt(B.ff1[0]), stream);
            }));
            // ff.net.0 -> geglu_rows fused into the GEMM's epilogue
            MK_TRY(gemm(B.ff1[0], xn_img.p, c, 0, nb * n, 1, hid.p, F, 0, MK_EPI_GEGLU, in_dt(B.ff2[0]), nullptr, 0, 0,
                        0, nullptr, "gemm.ff1"));
            MK_TRY(gemm(B.ff2[0], hid.p, F, 0, nb * n, 1, hs, c, 0, MK_EPI_ADD, MK_F32, nullptr, 0, 0, 0, nullptr,
                        "gemm.ff2"));
        }
        // proj_out + bias + the transformer's input
        MK_HIP(hipMemcpyAsync(y, x, size_t(nb) * nc * 4, hipMemcpyDeviceToDevice, stream));
        MK_TRY(timed("convert", 0, [&] {
            return in_dt(proj_out) == MK_F16 ? f32_to_f16(hs, size_t(nb) * nc, xn_img.p, stream)
                                             : mk_f32_to_bf16(hs, size_t(nb) * nc, xn_img.p, stream);
        }));
        MK_TRY(gemm(proj_out, xn_img.p, c, 0, nb * n, 1, y, c, 0, MK_EPI_ADD, MK_F32));
        return MK_OK;
    }
};

// =====================================================================================================================
// C ABI: engine
// =====================================================================================================================

namespace {

bool fill_dest(mk_engine* e, const std::string& name, const Dest& d, uint64_t seed, mk_status& st)
{
    const uint64_t key = tensor_key(seed, name.c_str());
    const uint64_t n = d.rows * d.cols;
    if (d.dtype == MK_FP8_E4M3) {
        // bf16 N(0, 0.02), then per-row fp8 quantisation (the CPU reference's rule)
        void* tmp = nullptr;
        if (hipMalloc(&tmp, n * 2) != hipSuccess) {
            st = fail(MK_ERR_NOMEM, "init_random: temporary");
            return false;
        }
        st = mk_fill_normal(tmp, n, MK_BF16, key, d.mean, d.std, e->stream);
        if (st == MK_OK)
            st = mk_quantize_fp8_rows(tmp, d.rows, d.cols, d.p, d.scale, e->stream);
        (void)hipStreamSynchronize(e->stream);
        (void)hipFree(tmp);
        return st == MK_OK;
    }
    st = mk_fill_normal(d.p, n, d.dtype, key, d.mean, d.std, e->stream);
    return st == MK_OK;
}

} // namespace

extern "C" {

mk_status mk_engine_create(const mk_config* cfg, mk_engine** out)
{
    if (!cfg || !out)
        return fail(MK_ERR_ARG, "engine_create: null");
    *out = nullptr;
    const mk_config& c = *cfg;
    if (c.family > MK_FAMILY_SDXL || !c.blocks || !c.dim || !c.heads || !c.ffn || !c.text_dim)
        return fail(MK_ERR_ARG, "engine_create: bad family or zero size");
    if (c.family != MK_FAMILY_SDXL && (c.head_dim != 128 || c.heads * 128 != c.dim || c.latent != 64))
        return fail(MK_ERR_ARG, "engine_create: MMDiT families need heads x 128 = dim and 64 latent channels");
    if (c.family == MK_FAMILY_SDXL && (c.head_dim != 64 || c.dim % 64))
        return fail(MK_ERR_ARG, "engine_create: SDXL needs heads of 64");
    if ((c.family == MK_FAMILY_SDXL ? c.dim % 64 : c.dim % 256) || c.ffn % 64 || c.text_dim % 64 || c.dim > 4096 ||
        c.text_dim > 4096)
        return fail(MK_ERR_ARG, "engine_create: dim a multiple of 256 (SDXL: 64) up to 4096, ffn and text_dim "
                                "multiples of 64");
    if (c.weight_dtype != MK_BF16 && c.weight_dtype != MK_FP8_E4M3 &&
        !(c.weight_dtype == MK_F16 && c.family == MK_FAMILY_SDXL))
        return fail(MK_ERR_ARG, "engine_create: weights bf16 or fp8-e4m3 (SDXL: also f16)");
    auto e = std::make_unique<mk_engine>();
    e->cfg = c;
    if (!e->cfg.max_batch)
        e->cfg.max_batch = 2;
    MK_HIP(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    MK_HIP(hipStreamCreateWithFlags(&e->side, hipStreamNonBlocking));
    MK_HIP(hipEventCreateWithFlags(&e->temb_ready, hipEventDisableTiming));
    e->mod_ready.resize(e->cfg.blocks);
    for (auto& ev : e->mod_ready)
        MK_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    int dev = 0, ncu = 0;
    MK_HIP(hipGetDevice(&dev));
    MK_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    e->cus = ncu > 0 ? uint32_t(ncu) : 256;
    mk_status s = e->build();
    if (s != MK_OK)
        return s;
    *out = e.release();
    return MK_OK;
}

mk_status mk_engine_destroy(mk_engine* e)
{
    if (!e)
        return MK_OK;
    (void)hipStreamSynchronize(e->stream);
    if (e->side)
        (void)hipStreamSynchronize(e->side);
    for (void* p : e->allocs)
        (void)hipFree(p);
    for (hipEvent_t ev : e->mod_ready)
        (void)hipEventDestroy(ev);
    if (e->temb_ready)
        (void)hipEventDestroy(e->temb_ready);
    if (e->timing.ref)
        (void)hipEventDestroy(e->timing.ref);
    if (e->ord_in)
        (void)hipEventDestroy(e->ord_in);
    if (e->ord_out)
        (void)hipEventDestroy(e->ord_out);
    if (e->side)
        (void)hipStreamDestroy(e->side);
    (void)hipStreamDestroy(e->stream);
    delete e;
    return MK_OK;
}

mk_status mk_engine_load(mk_engine* e, const char* name, const void* data, uint32_t dtype, uint64_t rows,
                         uint64_t cols)
{
    if (!e || !name || !data)
        return fail(MK_ERR_ARG, "engine_load: null");
    std::string n(name);
    bool is_scale = false;
    if (n.size() > 6 && n.compare(n.size() - 6, 6, ".scale") == 0) {
        n = n.substr(0, n.size() - 6);
        is_scale = true;
    }
    auto it = e->dests.find(n);
    if (it == e->dests.end())
        return fail(MK_ERR_ARG, "engine_load: no tensor named " + std::string(name));
    const Dest& d = it->second;
    if (is_scale) {
        if (d.dtype != MK_FP8_E4M3 || dtype != MK_F32 || rows * cols != d.rows)
            return fail(MK_ERR_ARG, "engine_load: " + std::string(name) + ": a scale is fp32 per row of an fp8 matrix");
        MK_HIP(hipMemcpy(d.scale, data, d.rows * 4, hipMemcpyHostToDevice));
        return MK_OK;
    }
    if (dtype != d.dtype || rows * cols != d.rows * d.cols)
        return fail(MK_ERR_ARG, "engine_load: " + std::string(name) + ": expected " + std::to_string(d.rows) + " x " +
                                    std::to_string(d.cols) + " of dtype " + std::to_string(d.dtype));
    MK_HIP(hipMemcpy(d.p, data, d.rows * d.cols * mk_engine::esize(d.dtype), hipMemcpyHostToDevice));
    return MK_OK;
}

mk_status mk_engine_init_random(mk_engine* e, uint64_t seed)
{
    if (!e)
        return fail(MK_ERR_ARG, "engine_init_random: null");
    for (const auto& [name, d] : e->dests) {
        mk_status st;
        if (!fill_dest(e, name, d, seed, st))
            return st;
    }
    MK_HIP(hipStreamSynchronize(e->stream));
    return MK_OK;
}

mk_status mk_engine_weight_bytes(const mk_engine* e, uint64_t* bytes)
{
    if (!e || !bytes)
        return fail(MK_ERR_ARG, "engine_weight_bytes: null");
    *bytes = e->weight_bytes;
    return MK_OK;
}

mk_status mk_begin(mk_engine* e, const float* prompt, size_t rows, uint32_t h, uint32_t w, uint32_t slot)
{
    if (!e || !prompt)
        return fail(MK_ERR_ARG, "begin: null");
    if (slot > 1)
        return fail(MK_ERR_ARG, "slot must be 0 or 1");
    if (!rows)
        return fail(MK_ERR_ARG, "prompt embeddings must be rows of " + std::to_string(e->cfg.text_dim));
    if (!h || !w)
        return fail(MK_ERR_ARG, "begin: empty latent grid");
    auto& g = e->slots[slot];
    if (e->gh != h || e->gw != w)
        e->rope_key.clear();
    e->gh = h;
    e->gw = w;
    g.S = uint32_t(rows);
    g.steps = 0;
    MK_TRY(g.prompt.ensure(rows * e->cfg.text_dim * 4));
    MK_HIP(hipMemcpy(g.prompt.p, prompt, rows * e->cfg.text_dim * 4, hipMemcpyHostToDevice));
    g.begun = true;
    if (e->cfg.family == MK_FAMILY_SDXL)
        MK_TRY(e->sdxl_begin(slot));
    return MK_OK;
}

mk_status mk_step(mk_engine* e, const float* latents, size_t n, float sigma, uint32_t slot, float* out)
{
    if (!e || !latents || !out)
        return fail(MK_ERR_ARG, "step: null");
    if (slot > 1)
        return fail(MK_ERR_ARG, "slot must be 0 or 1");
    if (e->cfg.family == MK_FAMILY_SDXL)
        return fail(MK_ERR_UNSUPPORTED, "step: the SDXL family runs mk_sdxl_forward");
    auto& g = e->slots[slot];
    if (!g.begun)
        return fail(MK_ERR_STATE, "step before begin");
    const size_t N = size_t(e->gh) * e->gw, L = e->cfg.latent;
    if (n != N * L)
        return fail(MK_ERR_ARG, "latents must be [h * w][" + std::to_string(L) + "]");
    MK_TRY(e->lat.ensure(N * L * 4));
    MK_HIP(hipMemcpyAsync(e->lat.p, latents, N * L * 4, hipMemcpyHostToDevice, e->stream));
    if (e->cfg.family == MK_FAMILY_DUAL) {
        const uint32_t so[1] = {slot};
        MK_TRY(e->dual_step(e->lat.f(), sigma, so, 1));
    } else {
        MK_TRY(e->q21_step(e->lat.f(), sigma, slot));
    }
    MK_HIP(hipMemcpyAsync(out, e->out.p, N * L * 4, hipMemcpyDeviceToHost, e->stream));
    MK_HIP(hipStreamSynchronize(e->stream));
    MK_TRY(gemm_take_error(e->stream));
    MK_TRY(e->finish_timing());
    return MK_OK;
}

mk_status mk_step_cfg_device(mk_engine* e, const float* lat, float sigma, float sigma_next, float guidance,
                             float* lat_out, void* stream)
{
    if (!e || !lat || !lat_out)
        return fail(MK_ERR_ARG, "step_cfg: null");
    if (e->cfg.family != MK_FAMILY_DUAL && e->cfg.family != MK_FAMILY_Q21)
        return fail(MK_ERR_UNSUPPORTED, "step_cfg: MMDiT families only");
    if (!e->slots[0].begun || !e->slots[1].begun)
        return fail(MK_ERR_STATE, "step_cfg: begin both slots first");
    const size_t N = size_t(e->gh) * e->gw, L = e->cfg.latent;
    if (stream && stream != e->stream) {
        // order after the caller's stream
        if (!e->ord_in)
            MK_HIP(hipEventCreateWithFlags(&e->ord_in, hipEventDisableTiming));
        MK_HIP(hipEventRecord(e->ord_in, static_cast<hipStream_t>(stream)));
        MK_HIP(hipStreamWaitEvent(e->stream, e->ord_in, 0));
    }
    const float dt = sigma_next - sigma;
    if (e->cfg.family == MK_FAMILY_DUAL) {
        // both guidance passes as one batch of 2 (prompts of different lengths padded to the longer one)
        MK_TRY(e->lat.ensure(2 * N * L * 4));
        MK_HIP(hipMemcpyAsync(e->lat.p, lat, N * L * 4, hipMemcpyDeviceToDevice, e->stream));
        MK_HIP(hipMemcpyAsync(e->lat.f() + N * L, lat, N * L * 4, hipMemcpyDeviceToDevice, e->stream));
        const uint32_t so[2] = {0, 1};
        MK_TRY(e->dual_step(e->lat.f(), sigma, so, 2));
        MK_TRY(e->timed("cfg_euler", 0, [&] {
            return mk_cfg_euler(lat, e->out.f(), e->out.f() + N * L, N * L, guidance, dt, lat_out, e->stream);
        }));
    } else {
        // two passes (the 2.1 graph, whose slots keep their own K / V): the positive velocity waits in a buffer of
        // the engine's
        Buf& pos = e->vpos;
        MK_TRY(pos.ensure(N * L * 4));
        MK_TRY(e->lat.ensure(N * L * 4));
        MK_HIP(hipMemcpyAsync(e->lat.p, lat, N * L * 4, hipMemcpyDeviceToDevice, e->stream));
        for (uint32_t s = 0; s < 2; ++s) {
            MK_TRY(e->q21_step(e->lat.f(), sigma, s));
            if (s == 0)
                MK_HIP(hipMemcpyAsync(pos.p, e->out.p, N * L * 4, hipMemcpyDeviceToDevice, e->stream));
        }
        MK_TRY(e->timed("cfg_euler", 0, [&] {
            return mk_cfg_euler(lat, pos.f(), e->out.f(), N * L, guidance, dt, lat_out, e->stream);
        }));
    }
    if (stream && stream != e->stream) {
        if (!e->ord_out)
            MK_HIP(hipEventCreateWithFlags(&e->ord_out, hipEventDisableTiming));
        MK_HIP(hipEventRecord(e->ord_out, e->stream));
        MK_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), e->ord_out, 0));
    }
    if (e->timing.on)
        MK_TRY(e->finish_timing());
    return MK_OK;
}

mk_status mk_step_cfg(mk_engine* e, const float* latents, size_t n, float sigma, float sigma_next, float guidance,
                      float* latents_out)
{
    if (!e || !latents || !latents_out)
        return fail(MK_ERR_ARG, "step_cfg: null");
    const size_t N = size_t(e->gh) * e->gw, L = e->cfg.latent;
    if (n != N * L)
        return fail(MK_ERR_ARG, "latents must be [h * w][" + std::to_string(L) + "]");
    // the engine's buffers (grown once, then reused: a steady-state call allocates nothing)
    MK_TRY(e->host_in.ensure(n * 4));
    MK_TRY(e->host_out.ensure(n * 4));
    MK_HIP(hipMemcpyAsync(e->host_in.p, latents, n * 4, hipMemcpyHostToDevice, e->stream));
    MK_TRY(mk_step_cfg_device(e, e->host_in.f(), sigma, sigma_next, guidance, e->host_out.f(), nullptr));
    MK_HIP(hipMemcpyAsync(latents_out, e->host_out.p, n * 4, hipMemcpyDeviceToHost, e->stream));
    MK_HIP(hipStreamSynchronize(e->stream));
    MK_TRY(gemm_take_error(e->stream));
    return MK_OK;
}

mk_status mk_noise(uint64_t seed, float* out, size_t n)
{
    if (!out && n)
        return fail(MK_ERR_ARG, "noise: null");
    // the reference's two lines (engine.cpp:399-400, 406-407): one engine, one distribution, the values in order
    std::mt19937_64 rng(seed);
    std::normal_distribution<float> nd;
    for (size_t i = 0; i < n; ++i)
        out[i] = nd(rng);
    return MK_OK;
}

mk_status mk_sigmas(uint32_t steps, uint32_t tokens, const mk_schedule* sched, float* out)
{
    if (!out)
        return fail(MK_ERR_ARG, "sigmas: null");
    const mk_schedule d{256.0, 4096.0, 0.5, 1.15, 0.0, 0, 0.0};
    const mk_schedule& s = sched ? *sched : d;
    if (!s.has_mu && s.max_seq == s.base_seq)
        return fail(MK_ERR_ARG, "sigmas: max_seq == base_seq");
    // the shift: fixed, or on the line through (base_seq, base_shift) and (max_seq, max_shift)
    const double slope = s.has_mu ? 0.0 : (s.max_shift - s.base_shift) / (s.max_seq - s.base_seq);
    const double mu = s.has_mu ? s.mu : double(tokens) * slope + (s.base_shift - slope * s.base_seq);
    const double em = std::exp(mu);
    for (uint32_t i = 0; i < steps; ++i) {
        // t on linspace(1, 1 / steps, steps), held in float as the scheduler holds it
        const float t = steps == 1 ? 1.0f : float(1.0 + (1.0 / steps - 1.0) * double(i) / double(steps - 1));
        out[i] = float(em / (em + (1.0 / double(t) - 1.0)));
    }
    // stretched so that the last level is the terminal one (nothing to stretch when it is 1)
    if (s.terminal > 0 && steps > 0 && out[steps - 1] < 1.0f) {
        const float k = (1.0f - out[steps - 1]) / (1.0f - float(s.terminal));
        for (uint32_t i = 0; i < steps; ++i)
            out[i] = 1.0f - (1.0f - out[i]) / k;
    }
    out[steps] = 0.0f;
    return MK_OK;
}

mk_status mk_generate(mk_engine* e, const float* noise, size_t n, const float* sigmas, uint32_t steps, float guidance,
                      float* latents_out)
{
    if (!e || !noise || !sigmas || !latents_out)
        return fail(MK_ERR_ARG, "generate: null");
    if (e->cfg.family != MK_FAMILY_DUAL && e->cfg.family != MK_FAMILY_Q21)
        return fail(MK_ERR_UNSUPPORTED, "generate: MMDiT families only");
    const bool guided = guidance != 1.0f;
    if (!e->slots[0].begun || (guided && !e->slots[1].begun))
        return fail(MK_ERR_STATE, guided ? "generate: begin both slots first" : "generate: begin slot 0 first");
    const size_t N = size_t(e->gh) * e->gw, L = e->cfg.latent;
    if (n != N * L)
        return fail(MK_ERR_ARG, "latents must be [h * w][" + std::to_string(L) + "]");
    Buf x[2];
    MK_TRY(x[0].ensure(n * 4));
    MK_TRY(x[1].ensure(n * 4));
    MK_HIP(hipMemcpyAsync(x[0].p, noise, n * 4, hipMemcpyHostToDevice, e->stream));
    for (uint32_t i = 0; i < steps; ++i) {
        float* cur = x[i % 2].f();
        float* nxt = x[(i + 1) % 2].f();
        const float dt = sigmas[i + 1] - sigmas[i];
        if (guided) {
            MK_TRY(mk_step_cfg_device(e, cur, sigmas[i], sigmas[i + 1], guidance, nxt, nullptr));
        } else {
            if (e->cfg.family == MK_FAMILY_DUAL) {
                const uint32_t so[1] = {0};
                MK_TRY(e->dual_step(cur, sigmas[i], so, 1));
            } else {
                MK_TRY(e->q21_step(cur, sigmas[i], 0));
            }
            // guidance 1: neg + 1 (pos - neg) with pos = neg is the prompt's own velocity
            MK_TRY(e->timed("cfg_euler", 0, [&] {
                return mk_cfg_euler(cur, e->out.f(), e->out.f(), n, 1.0f, dt, nxt, e->stream);
            }));
            if (e->timing.on)
                MK_TRY(e->finish_timing());
        }
    }
    MK_HIP(hipMemcpyAsync(latents_out, x[steps % 2].p, n * 4, hipMemcpyDeviceToHost, e->stream));
    MK_HIP(hipStreamSynchronize(e->stream));
    return gemm_take_error(e->stream);
}

mk_status mk_engine_stream(mk_engine* e, void** stream)
{
    if (!e || !stream)
        return fail(MK_ERR_ARG, "engine_stream: null");
    *stream = e->stream;
    return MK_OK;
}

mk_status mk_engine_set_probe(mk_engine* e, mk_probe_fn fn, void* user)
{
    if (!e)
        return fail(MK_ERR_ARG, "set_probe: null");
    e->probe = fn;
    e->probe_user = user;
    return MK_OK;
}

mk_status mk_engine_set_timing(mk_engine* e, int on)
{
    if (!e)
        return fail(MK_ERR_ARG, "set_timing: null");
    e->timing.on = on != 0;
    return MK_OK;
}

mk_status mk_engine_timing(mk_engine* e, uint32_t i, const char** name, float* ms, uint32_t* launches, double* flops)
{
    if (!e || !name || !ms || !launches || !flops)
        return fail(MK_ERR_ARG, "engine_timing: null");
    if (i >= e->timing.names.size())
        return fail(MK_ERR_ARG, "engine_timing: no such class");
    *name = e->timing.names[i].c_str();
    *ms = e->timing.ms[i];
    *launches = e->timing.launches[i];
    *flops = e->timing.flops[i];
    return MK_OK;
}

mk_status mk_sdxl_forward(mk_engine* e, const float* x, uint32_t batch, uint32_t n, float* y, void* stream)
{
    if (!e || !x || !y)
        return fail(MK_ERR_ARG, "sdxl_forward: null");
    if (e->cfg.family != MK_FAMILY_SDXL)
        return fail(MK_ERR_UNSUPPORTED, "sdxl_forward: not an SDXL engine");
    if (batch == 0 || batch > 2 || !n)
        return fail(MK_ERR_ARG, "sdxl_forward: batch 1 or 2, n > 0");
    for (uint32_t b = 0; b < batch; ++b)
        if (!e->slots[b].begun)
            return fail(MK_ERR_STATE, "sdxl_forward: begin slot " + std::to_string(b) + " first");
    if (batch == 2 && e->slots[0].S != e->slots[1].S)
        return fail(MK_ERR_ARG, "sdxl_forward: both slots' contexts must have the same length");
    (void)stream;
    MK_TRY(e->sdxl_forward(x, batch, n, y));
    MK_HIP(hipStreamSynchronize(e->stream));
    MK_TRY(gemm_take_error(e->stream));
    MK_TRY(e->finish_timing());
    return MK_OK;
}

} // extern "C"

namespace {

float f16_to_f32(uint16_t h)
{
    const int e = (h >> 10) & 31, m = h & 1023;
    const float v = e == 0 ? std::ldexp(float(m), -24)
                    : e == 31 ? (m ? NAN : INFINITY)
                              : std::ldexp(float(1024 + m), e - 25);
    return h & 0x8000 ? -v : v;
}

const char* dtype_label(uint32_t dt)
{
    return dt == MK_F32 ? "F32" : dt == MK_BF16 ? "BF16" : dt == MK_F16 ? "F16" : dt == MK_FP8_E4M3 ? "F8_E4M3" : "?";
}

// n values of dtype `from` (F32, BF16 or F16) as `to` (F32, BF16 or F16, nearest even).
void convert_host(const void* src, uint32_t from, void* dst, uint32_t to, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        const float v = from == MK_F32    ? static_cast<const float*>(src)[i]
                        : from == MK_BF16 ? bf2f_bits(static_cast<const uint16_t*>(src)[i])
                                          : f16_to_f32(static_cast<const uint16_t*>(src)[i]);
        if (to == MK_F32)
            static_cast<float*>(dst)[i] = v;
        else
            static_cast<uint16_t*>(dst)[i] = to == MK_F16 ? f2h_bits(v) : f2bf_bits(v);
    }
}

// Streams tensors from a checkpoint into device memory: file -> pinned host buffer (converted there when the
// dtypes differ) -> async copy on the engine's stream, two buffers in turn so a read overlaps the previous copy.
struct Streamer {
    static constexpr size_t kChunk = size_t(64) << 20;
    const mk_st* st;
    hipStream_t stream;
    void* pin[2] = {};
    hipEvent_t ev[2] = {};
    int cur = 0;
    std::vector<char> raw;
    Buf stage; // bf16 rows on their way to fp8 quantisation

    ~Streamer()
    {
        if (stream)
            (void)hipStreamSynchronize(stream);
        for (int i = 0; i < 2; ++i) {
            if (pin[i])
                (void)hipHostFree(pin[i]);
            if (ev[i])
                (void)hipEventDestroy(ev[i]);
        }
    }
    mk_status init()
    {
        for (int i = 0; i < 2; ++i) {
            MK_HIP(hipHostMalloc(&pin[i], kChunk, hipHostMallocDefault));
            MK_HIP(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
        }
        return MK_OK;
    }
    // The tensor's elements as dtype `to` at device address d.
    mk_status upload(const mk_st_tensor& t, void* d, uint32_t to)
    {
        const size_t es_in = mk_engine::esize(t.dtype == MK_F16 ? MK_BF16 : t.dtype), es_out = mk_engine::esize(to);
        const uint64_t n = t.bytes / es_in;
        const uint64_t per = kChunk / std::max(es_in, es_out);
        for (uint64_t i = 0; i < n; i += per) {
            const uint64_t m = std::min<uint64_t>(per, n - i);
            MK_HIP(hipEventSynchronize(ev[cur]));
            if (t.dtype == to) {
                if (!st_read(st, t, pin[cur], m * es_in, i * es_in))
                    return fail(MK_ERR_ARG, std::string("safetensors: cannot read ") + t.name);
            } else {
                raw.resize(m * es_in);
                if (!st_read(st, t, raw.data(), m * es_in, i * es_in))
                    return fail(MK_ERR_ARG, std::string("safetensors: cannot read ") + t.name);
                convert_host(raw.data(), t.dtype, pin[cur], to, m);
            }
            MK_HIP(hipMemcpyAsync(static_cast<char*>(d) + i * es_out, pin[cur], m * es_out, hipMemcpyHostToDevice,
                                  stream));
            MK_HIP(hipEventRecord(ev[cur], stream));
            cur ^= 1;
        }
        return MK_OK;
    }
    // A small tensor (<= 1024 values) read and converted to fp32 on the host.
    mk_status host_f32(const mk_st_tensor& t, std::vector<float>& out)
    {
        const size_t es = mk_engine::esize(t.dtype == MK_F16 ? MK_BF16 : t.dtype);
        const size_t n = t.bytes / es;
        raw.resize(t.bytes);
        if (!st_read(st, t, raw.data(), t.bytes, 0))
            return fail(MK_ERR_ARG, std::string("safetensors: cannot read ") + t.name);
        out.resize(n);
        convert_host(raw.data(), t.dtype, out.data(), MK_F32, n);
        return MK_OK;
    }
};

uint64_t numel(const mk_st_tensor& t)
{
    uint64_t n = 1;
    for (uint32_t i = 0; i < t.ndim; ++i)
        n *= t.dims[i];
    return n;
}

bool float_dtype(uint32_t dt) { return dt == MK_F32 || dt == MK_BF16 || dt == MK_F16; }

// Checkpoint name under the prefixes single-file checkpoints use.
const char* const kPrefixes[] = {"", "model.diffusion_model.", "transformer."};

bool find_prefixed(const mk_st* st, const std::string& name, mk_st_tensor* t, const std::string& first = "")
{
    // a caller-given prefix (an SDXL spatial transformer's place in its UNet) first, then the defaults
    if (!first.empty() && mk_st_find(st, (first + name).c_str(), t) == MK_OK)
        return true;
    for (const char* p : kPrefixes) {
        const std::string n = p + name;
        if (mk_st_find(st, n.c_str(), t) == MK_OK)
            return true;
    }
    set_error("");
    return false;
}

struct StClose {
    void operator()(mk_st* s) const { mk_st_close(s); }
};

} // namespace

extern "C" {

mk_status mk_engine_load_safetensors(mk_engine* e, const char* path, uint64_t* loaded)
{
    return mk_engine_load_safetensors_at(e, path, nullptr, loaded);
}

mk_status mk_engine_load_safetensors_at(mk_engine* e, const char* path, const char* prefix, uint64_t* loaded)
{
    if (!e || !path)
        return fail(MK_ERR_ARG, "engine_load_safetensors: null");
    const std::string pre = prefix ? prefix : "";
    mk_st* raw_st = nullptr;
    MK_TRY(mk_st_open(path, &raw_st));
    std::unique_ptr<mk_st, StClose> st(raw_st);
    // a checkpoint with more blocks than the engine was made for (with a prefix: the blocks under it)
    size_t count = 0;
    MK_TRY(mk_st_count(st.get(), &count, nullptr));
    for (size_t i = 0; i < count; ++i) {
        mk_st_tensor t;
        MK_TRY(mk_st_at(st.get(), i, &t));
        std::string n = t.name;
        if (!pre.empty()) {
            if (n.rfind(pre, 0) != 0)
                continue;
            n = n.substr(pre.size());
        }
        for (const char* p : kPrefixes)
            if (*p && n.rfind(p, 0) == 0)
                n = n.substr(strlen(p));
        static const std::string blk = "transformer_blocks.";
        if (n.rfind(blk, 0) == 0) {
            const unsigned long b = strtoul(n.c_str() + blk.size(), nullptr, 10);
            if (b >= e->cfg.blocks)
                return fail(MK_ERR_ARG, "load_safetensors: the checkpoint has " + std::string(t.name) +
                                            " but the engine has " + std::to_string(e->cfg.blocks) + " blocks");
        }
    }
    // every tensor the engine holds must be there, with its shape and a usable dtype: checked before any upload
    struct Job {
        const Dest* d;
        mk_st_tensor t, scale;
        bool has_scale = false;
    };
    std::vector<Job> jobs;
    for (const auto& [name, d] : e->dests) {
        Job j{&d, {}, {}};
        if (!find_prefixed(st.get(), name, &j.t, pre))
            return fail(MK_ERR_ARG, "load_safetensors: the checkpoint has no tensor " + pre + name);
        const mk_st_tensor& t = j.t;
        const bool matrix = d.cols > 1;
        const bool shape_ok = matrix ? t.ndim == 2 && t.dims[0] == d.cols && t.dims[1] == d.rows
                                     : t.ndim <= 2 && numel(t) == d.rows;
        if (!shape_ok) {
            std::string dims;
            for (uint32_t k = 0; k < t.ndim; ++k)
                dims += (k ? ", " : "") + std::to_string(t.dims[k]);
            return fail(MK_ERR_ARG, "load_safetensors: " + name + " has dims {" + dims + "}, the engine needs " +
                                        (matrix ? "{" + std::to_string(d.cols) + ", " + std::to_string(d.rows) + "}"
                                                : "{" + std::to_string(d.rows) + "}"));
        }
        if (t.dtype == MK_FP8_E4M3) {
            if (d.dtype != MK_FP8_E4M3)
                return fail(MK_ERR_ARG, "load_safetensors: " + name + " is F8_E4M3 but the engine stores it as " +
                                            dtype_label(d.dtype));
            if (!find_prefixed(st.get(), name + ".scale", &j.scale, pre) || numel(j.scale) != d.rows ||
                !float_dtype(j.scale.dtype))
                return fail(MK_ERR_ARG, "load_safetensors: F8_E4M3 " + name + " needs its per-row scale " + name +
                                            ".scale (" + std::to_string(d.rows) + " values)");
            j.has_scale = true;
        } else if (!float_dtype(t.dtype)) {
            return fail(MK_ERR_ARG, "load_safetensors: " + name + " has dtype " + t.dtype_name);
        }
        jobs.push_back(j);
    }
    Streamer s{st.get(), e->stream};
    MK_TRY(s.init());
    for (const Job& j : jobs) {
        const Dest& d = *j.d;
        if (d.dtype != MK_FP8_E4M3) {
            MK_TRY(s.upload(j.t, d.p, d.dtype));
        } else if (j.has_scale) {
            MK_TRY(s.upload(j.t, d.p, MK_FP8_E4M3));
            MK_TRY(s.upload(j.scale, d.scale, MK_F32));
        } else {
            if (d.rows * d.cols * 2 > s.stage.bytes)
                MK_HIP(hipStreamSynchronize(e->stream)); // the previous quantisation may still read the stage
            MK_TRY(s.stage.ensure(d.rows * d.cols * 2));
            MK_TRY(s.upload(j.t, s.stage.p, MK_BF16));
            MK_TRY(mk_quantize_fp8_rows(s.stage.p, d.rows, d.cols, d.p, d.scale, e->stream));
        }
    }
    MK_HIP(hipStreamSynchronize(e->stream));
    if (loaded)
        *loaded = jobs.size();
    return MK_OK;
}

mk_status mk_engine_add_lora(mk_engine* e, const char* path, float scale, uint64_t* merged, uint64_t* skipped)
{
    if (!e || !path)
        return fail(MK_ERR_ARG, "engine_add_lora: null");
    mk_st* raw_st = nullptr;
    MK_TRY(mk_st_open(path, &raw_st));
    std::unique_ptr<mk_st, StClose> st(raw_st);
    size_t count = 0;
    MK_TRY(mk_st_count(st.get(), &count, nullptr));
    // modules and their down (A) / up (B) / alpha tensors
    struct Mod {
        int a = -1, b = -1, alpha = -1;
        bool other = false;
    };
    std::map<std::string, Mod> mods;
    static const struct {
        const char* suffix;
        int part; // 0 A, 1 B, 2 alpha
    } kParts[] = {{".lora_A.weight", 0},        {".lora_B.weight", 1},         {".lora_A.default.weight", 0},
                  {".lora_B.default.weight", 1}, {".lora_down.weight", 0},      {".lora_up.weight", 1},
                  {".alpha", 2}};
    std::vector<mk_st_tensor> ts(count);
    for (size_t i = 0; i < count; ++i) {
        MK_TRY(mk_st_at(st.get(), i, &ts[i]));
        const std::string n = ts[i].name;
        bool hit = false;
        for (const auto& p : kParts) {
            const size_t L = strlen(p.suffix);
            if (n.size() > L && n.compare(n.size() - L, L, p.suffix) == 0) {
                Mod& m = mods[n.substr(0, n.size() - L)];
                (p.part == 0 ? m.a : p.part == 1 ? m.b : m.alpha) = int(i);
                hit = true;
                break;
            }
        }
        if (!hit) {
            const size_t dot = n.rfind('.');
            mods[dot == std::string::npos ? n : n.substr(0, dot)].other = true;
        }
    }
    // '_' and '.' alike: engine module names with dots turned to underscores
    std::unordered_map<std::string, std::string> flat;
    for (const auto& [name, d] : e->dests)
        if (d.cols > 1 && name.size() > 7 && name.compare(name.size() - 7, 7, ".weight") == 0) {
            std::string m = name.substr(0, name.size() - 7);
            std::string f = m;
            for (char& c : f)
                if (c == '.')
                    c = '_';
            flat[f] = m;
        }
    struct Merge {
        std::string module;
        Dest d;
        const mk_st_tensor *a, *b;
        uint32_t rank;
        float factor;
    };
    std::vector<Merge> plan;
    uint64_t n_skipped = 0;
    Streamer s{st.get(), e->stream};
    for (const auto& [module, m] : mods) {
        std::string mod = module;
        for (const char* p : {"base_model.model.", "model.diffusion_model.", "diffusion_model.", "transformer.",
                              "lora_unet_", "lora_transformer_"})
            if (mod.rfind(p, 0) == 0)
                mod = mod.substr(strlen(p));
        if (m.a < 0 && m.b < 0) {
            ++n_skipped; // no LoRA pair here (a full-weight diff, a DoRA scale, ...)
            continue;
        }
        if (m.a < 0 || m.b < 0)
            return fail(MK_ERR_ARG, "add_lora: " + module + " has only one of its down / up matrices");
        if (m.other) // a DoRA magnitude, a bias difference, ...: merging the pair alone would be wrong
            return fail(MK_ERR_UNSUPPORTED, "add_lora: " + module + " has parts beside its down / up matrices "
                                                                    "(DoRA / bias diffs are not merged)");
        // the target: the module's rows in the fused tensor (QwenImage::lora_target); Q21's fused gate_up spans
        // the gate rows and the up rows that follow them
        Dest d{};
        bool found = false;
        auto it = e->dests.find(mod + ".weight");
        if (it == e->dests.end()) {
            auto f = flat.find(mod);
            if (f != flat.end())
                it = e->dests.find(f->second + ".weight");
        }
        if (it != e->dests.end() && it->second.cols > 1) {
            d = it->second;
            found = true;
        } else if (e->cfg.family == MK_FAMILY_Q21 && mod.size() > 16 &&
                   mod.compare(mod.size() - 16, 16, ".img_mlp.gate_up") == 0) {
            auto g = e->dests.find(mod.substr(0, mod.size() - 7) + "gate_layer.weight");
            if (g != e->dests.end()) {
                d = g->second;
                d.rows *= 2;
                found = true;
            }
        }
        if (!found) {
            ++n_skipped;
            continue;
        }
        const mk_st_tensor& A = ts[size_t(m.a)];
        const mk_st_tensor& B = ts[size_t(m.b)];
        if (A.ndim != 2 || B.ndim != 2 || !float_dtype(A.dtype) || !float_dtype(B.dtype))
            return fail(MK_ERR_ARG, "add_lora: " + module + ": down / up must be 2-d F32, BF16 or F16 matrices");
        const uint64_t r = A.dims[1];
        if (A.dims[0] != d.cols || B.dims[1] != d.rows || B.dims[0] != r || r == 0 || r > 1024)
            return fail(MK_ERR_ARG, "add_lora: " + module + ": down {" + std::to_string(A.dims[0]) + ", " +
                                        std::to_string(A.dims[1]) + "}, up {" + std::to_string(B.dims[0]) + ", " +
                                        std::to_string(B.dims[1]) + "} do not fit a " + std::to_string(d.rows) +
                                        " x " + std::to_string(d.cols) + " weight at rank <= 1024");
        float factor = scale;
        if (m.alpha >= 0) {
            const mk_st_tensor& al = ts[size_t(m.alpha)];
            std::vector<float> v;
            if (numel(al) != 1 || !float_dtype(al.dtype))
                return fail(MK_ERR_ARG, "add_lora: " + module + ".alpha must be one F32, BF16 or F16 value");
            MK_TRY(s.host_f32(al, v));
            factor = scale * v[0] / float(r);
        }
        plan.push_back({module, d, &A, &B, uint32_t(r), factor});
    }
    if (!plan.empty()) {
        MK_TRY(s.init());
        Buf ab; // one module's A then B, fp32; the merge of a module finishes before the next one's upload
        for (const Merge& p : plan) {
            const size_t na = size_t(p.rank) * p.d.cols, nb = size_t(p.d.rows) * p.rank;
            if ((na + nb) * 4 > ab.bytes)
                MK_HIP(hipStreamSynchronize(e->stream)); // the previous merge may still read the buffer
            MK_TRY(ab.ensure((na + nb) * 4));
            MK_TRY(s.upload(*p.a, ab.f(), MK_F32));
            MK_TRY(s.upload(*p.b, ab.f() + na, MK_F32));
            MK_TRY(mk_lora_merge(p.d.p, p.d.dtype, p.d.scale, p.d.rows, p.d.cols, ab.f(), ab.f() + na, p.rank,
                                 p.factor, e->stream));
        }
        MK_HIP(hipStreamSynchronize(e->stream));
    }
    if (merged)
        *merged = plan.size();
    if (skipped)
        *skipped = n_skipped;
    return MK_OK;
}

mk_status mk_engine_tensor_count(const mk_engine* e, size_t* n)
{
    if (!e || !n)
        return fail(MK_ERR_ARG, "engine_tensor_count: null");
    *n = e->dests.size();
    return MK_OK;
}

mk_status mk_engine_tensor_at(const mk_engine* e, size_t i, const char** name, uint32_t* dtype, uint64_t* rows,
                              uint64_t* cols)
{
    if (!e || !name || !dtype || !rows || !cols)
        return fail(MK_ERR_ARG, "engine_tensor_at: null");
    if (i >= e->dests.size())
        return fail(MK_ERR_ARG, "engine_tensor_at: index " + std::to_string(i) + " of " +
                                    std::to_string(e->dests.size()));
    auto it = std::next(e->dests.begin(), std::ptrdiff_t(i));
    *name = it->first.c_str();
    *dtype = it->second.dtype;
    *rows = it->second.rows;
    *cols = it->second.cols;
    return MK_OK;
}

mk_status mk_engine_fetch(const mk_engine* e, const char* name, void* data, size_t bytes)
{
    if (!e || !name || !data)
        return fail(MK_ERR_ARG, "engine_fetch: null");
    std::string n(name);
    const bool is_scale = n.size() > 6 && n.compare(n.size() - 6, 6, ".scale") == 0;
    auto it = e->dests.find(is_scale ? n.substr(0, n.size() - 6) : n);
    if (it == e->dests.end() || (is_scale && it->second.dtype != MK_FP8_E4M3))
        return fail(MK_ERR_ARG, "engine_fetch: no tensor named " + n);
    const Dest& d = it->second;
    const size_t want = is_scale ? d.rows * 4 : d.rows * d.cols * mk_engine::esize(d.dtype);
    if (bytes != want)
        return fail(MK_ERR_ARG, "engine_fetch: " + n + " holds " + std::to_string(want) + " bytes");
    MK_HIP(hipStreamSynchronize(e->stream));
    MK_HIP(hipMemcpy(data, is_scale ? static_cast<const void*>(d.scale) : d.p, want, hipMemcpyDeviceToHost));
    return MK_OK;
}

} // extern "C"
