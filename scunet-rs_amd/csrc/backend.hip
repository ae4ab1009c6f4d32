// The MI355X backend behind the C ABI of include/scunet_hip.h: weight upload and
// repacking, the per-geometry device arena, the graph walker, probes, and profiling.
//
// The walker is the reference's Cuda::forward (src/cuda.rs:1606-1848) / cpu::forward_dump
// (src/cpu.rs:1175-1321) stage for stage; what differs is the device's own design:
//   * activations are pixel-major [P][c]; a block's conv half and transformer half are
//     column ranges of one buffer, so split, concat, gather and scatter do not exist as
//     kernels (the attention kernel reads windows through the shifted index map);
//   * whole-plane launches, no token chunking, skips and the head stay on the device;
//   * 9 launches per ConvTransBlock: conv1_1, 3x3+ReLU, 3x3+residual, LN1+qkv, attention,
//     proj+residual, LN2+mlp.0+GELU, mlp.2+residual, conv1_2+residual.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/scunet_hip.h"
#include "kernels.h"
#include "weights.h"

using namespace scunet;

// The forward's scratch for callers that cannot allocate device memory
// (scunet_hip_run_device_noalloc): every arena role of one forward, carved out of this
// array. Each device the library runs on holds its own copy until the process ends. In
// host code `scratch` is only a stand-in for the symbol: its device address comes from
// hipGetSymbolAddress, resolved once per device when a handle is created on it.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(256) << 20;
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

thread_local std::string g_create_error;

// Per-device address of `scratch` (null until resolved) and the error of a failed resolve.
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[MAX_DEVICES] = {};
std::string g_scratch_err[MAX_DEVICES];

// With `device` current: look up the device address of `scratch` once for that device.
void resolve_scratch(int device) {
    if (device < 0 || device >= MAX_DEVICES) return;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        hipGetLastError();
        g_scratch_err[device] = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
        return;
    }
    g_scratch_ptr[device] = static_cast<float*>(p);
    g_scratch_err[device].clear();
}

const char* STAGE[7] = {"down1", "down2", "down3", "body", "up3", "up2", "up1"};

struct ProfRec {
    std::string name;
    hipEvent_t e0, e1;
    double flop, bytes;
};

}  // namespace

struct scunet_hip {
    Weights wt;
    hipStream_t stream = nullptr;
    int device = 0;
    std::string err;
    float scale = 0.f;

    // Device weights: one allocation, name -> pointer (repacked where the kernels want it).
    float* wblob = nullptr;
    size_t wbytes = 0;
    std::map<std::string, float*> w;
    std::map<std::string, float*> tab;   // block prefix -> lane-ordered rel-pos bias table
    std::map<std::string, float*> atab;  // block prefix -> the attention kernel's 4-variant table

    // Arena: role -> (pointer, bytes), grown on demand, kept across calls.
    std::map<std::string, std::pair<float*, size_t>> arena;
    // During scunet_hip_run_device_noalloc: role -> (pointer into the static scratch, bytes);
    // buf() then serves only these and never allocates.
    std::map<std::string, std::pair<float*, size_t>> fixed;
    bool fixed_active = false;

    bool prof = false;
    bool unfused_msa = false;            // route every level through the 3-launch attention half
    bool direct3x3 = false;              // the direct implicit-GEMM 3x3 instead of Winograd
    bool wino16 = false;                 // Winograd with 16 output channels per unit only
    bool wino_pair = false;              // 16-channel Winograd always in 8 x 16 pair units
    bool wino2 = false;                  // the 32-bit-offset Winograd forms wherever the plane allows
    bool wino3_all = false;              // k_wino3 at every level (32-channel units below 64 channels)
    bool attn64 = false;                 // the attention kernel with 64-bit offsets at every size
    int attn_qs = 0;                     // the attention kernel's query parts (0: automatic)
    bool gemm2 = false;                  // one tile per workgroup GEMM (no persistent walker)
    bool gemm1x1 = false;                // the tiled GEMM for every 1x1 (no resident weights, no chaining)
    bool separate_mlp = false;           // the MLP as its own kernel also at t = 32
    int h16 = 0;                         // 1: fp16 MFMA operands, fp32 accumulation and planes
    // The k-permuted fp16 weight copies (built when the fp16 mode is first selected).
    half_t* h16blob = nullptr;
    size_t h16bytes = 0;
    std::map<std::string, const half_t*> hw;
    std::map<const float*, const half_t*> hw_of;   // fp32 device pointer -> its fp16 copy
    // The split-operand fp32 products (x6, the default fp32 mode): three bf16 part planes per
    // matrix weight, built at create; x6 = false (SCUNET_HIP_FP32_MFMA) sends every fp32
    // product to the fp32 matrix cores instead.
    bool x6 = false;
    bf16_t* x6blob = nullptr;
    size_t x6bytes = 0;
    std::map<std::string, const bf16_t*> xw;
    std::map<const float*, const bf16_t*> xw_of;
    std::string tag;                     // appended to profiler class names ("@L0".."@L3")
    std::vector<ProfRec> recs;
    std::vector<hipEvent_t> ev_pool;
    hipEvent_t chain = nullptr;          // the last profiled launch's end event (shared start)
    size_t ev_used = 0;
    std::vector<std::string> report_names;

    ~scunet_hip() {
        if (stream) hipStreamSynchronize(stream);
        for (auto& kv : arena)
            if (kv.second.first) hipFree(kv.second.first);
        if (wblob) hipFree(wblob);
        if (h16blob) hipFree(h16blob);
        if (x6blob) hipFree(x6blob);
        for (auto e : ev_pool) hipEventDestroy(e);
        if (stream) hipStreamDestroy(stream);
    }
};

namespace {

bool fail(scunet_hip* h, const std::string& m) {
    h->err = m;
    return false;
}

bool ck(scunet_hip* h, hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    return fail(h, std::string(what) + ": " + hipGetErrorString(e));
}

bool launched(scunet_hip* h, const char* what) {
    return ck(h, hipGetLastError(), what);
}

float* buf(scunet_hip* h, const std::string& role, size_t floats) {
    size_t bytes = std::max<size_t>(floats, 1) * sizeof(float);
    if (h->fixed_active) {
        auto it = h->fixed.find(role);
        if (it == h->fixed.end() || it->second.second < bytes) {
            fail(h, "no-alloc forward: scratch role `" + role + "` (" + std::to_string(bytes) +
                        " bytes) is not in the planned layout");
            return nullptr;
        }
        return it->second.first;
    }
    auto& slot = h->arena[role];
    if (slot.second >= bytes) return slot.first;
    if (slot.first) {
        hipStreamSynchronize(h->stream);
        hipFree(slot.first);
        slot = {nullptr, 0};
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        hipGetLastError();
        size_t held = 0;
        for (auto& kv : h->arena) held += kv.second.second;
        fail(h, "device allocation of " + std::to_string(bytes >> 20) + " MiB for `" + role +
                    "` failed (" + hipGetErrorString(e) + "): " + std::to_string(held >> 20) +
                    " MiB of scratch and " + std::to_string(h->wbytes >> 20) + " MiB of weights held");
        return nullptr;
    }
    slot = {static_cast<float*>(p), bytes};
    return slot.first;
}

// Profiling (cuda.rs:263-273): HIP events around every launch when on. Consecutive
// launches share the event between them (one launch's end is the next one's start), which
// halves the events in the stream; a launch's time then includes the dispatch gap before
// it. The chain restarts at each forward.
struct Span {
    scunet_hip* h;
    std::string name;
    double flop, bytes;
    hipEvent_t e0 = nullptr;
    Span(scunet_hip* hh, const char* n, double f, double b) : h(hh), name(std::string(n) + hh->tag), flop(f), bytes(b) {
        if (!h->prof) return;
        if (h->chain) {
            e0 = h->chain;
        } else {
            e0 = next();
            hipEventRecord(e0, h->stream);
        }
    }
    hipEvent_t next() {
        if (h->ev_used == h->ev_pool.size()) {
            // Timing-only events: no system-scope fence (cache writeback and invalidate) at
            // each record; the report synchronizes the stream before reading them.
            hipEvent_t e;
            hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
            h->ev_pool.push_back(e);
        }
        return h->ev_pool[h->ev_used++];
    }
    ~Span() {
        if (!h->prof) return;
        hipEvent_t e1 = next();
        hipEventRecord(e1, h->stream);
        h->recs.push_back({name, e0, e1, flop, bytes});
        h->chain = e1;
    }
};

const float* W(scunet_hip* h, const std::string& name) {
    auto it = h->w.find(name);
    return it == h->w.end() ? nullptr : it->second;
}

// The fp16 copy of weight `name` when the handle is in the fp16 mode, else null (which
// selects a kernel's fp32 path).
const half_t* W16(scunet_hip* h, const std::string& name) {
    if (!h->h16) return nullptr;
    auto it = h->hw.find(name);
    return it == h->hw.end() ? nullptr : it->second;
}

// The split planes of weight `name` when the handle computes fp32 products in split form,
// else null (which selects a kernel's fp32-MFMA path).
const bf16_t* WX(scunet_hip* h, const std::string& name) {
    if (h->h16 || !h->x6) return nullptr;
    auto it = h->xw.find(name);
    return it == h->xw.end() ? nullptr : it->second;
}

// Upload every tensor once (cuda.rs:466-472 uploads lazily; here all at create), in the
// layout its kernel reads:
//   3x3 conv_block weights [co][ci][3][3] -> [tap][co][ci], and as Winograd filters [16][co][ci]
//   down-conv m_downN.K.weight [co][ci][2][2] -> [co][tap*ci]        (tap = ky*2 + kx)
//   up-conv   m_upN.0.weight  [ci][co][2][2] -> [tap*co + co'][ci]
//   everything else as stored; rel-pos tables -> lane-ordered bias tables.
bool upload_weights(scunet_hip* h) {
    const Weights& wt = h->wt;
    std::vector<std::pair<std::string, std::vector<float>>> host;
    auto is_down = [&](const std::string& n) {
        for (int k = 0; k < 3; ++k)
            if (n == "m_" + std::string(STAGE[k]) + "." + std::to_string(wt.config[k]) + ".weight") return true;
        return false;
    };
    auto is_up = [&](const std::string& n) {
        for (int k = 4; k < 7; ++k)
            if (n == "m_" + std::string(STAGE[k]) + ".0.weight") return true;
        return false;
    };
    for (auto& kv : wt.all()) {
        const std::string& n = kv.first;
        const Tensor& t = kv.second;
        std::vector<float> v(t.data, t.data + t.numel);
        if (n.find(".conv_block.") != std::string::npos) {
            size_t co = t.shape[0], ci = t.shape[1];
            for (size_t o = 0; o < co; ++o)
                for (size_t i = 0; i < ci; ++i)
                    for (size_t tap = 0; tap < 9; ++tap) v[(tap * co + o) * ci + i] = t.data[(o * ci + i) * 9 + tap];
            std::vector<float> u(16 * co * ci);
            winograd_filter(t.data, int(co), int(ci), u.data());
            if (ci % 8 == 0) {
                std::vector<float> u8(16 * co * ci);
                winograd_filter_slices(u.data(), int(co), int(ci), u8.data());
                host.push_back({"@wino8:" + n, std::move(u8)});
            }
            host.push_back({"@wino:" + n, std::move(u)});
        } else if (is_down(n)) {
            size_t co = t.shape[0], ci = t.shape[1];
            for (size_t o = 0; o < co; ++o)
                for (size_t i = 0; i < ci; ++i)
                    for (size_t tap = 0; tap < 4; ++tap) v[o * 4 * ci + tap * ci + i] = t.data[(o * ci + i) * 4 + tap];
        } else if (is_up(n)) {
            size_t ci = t.shape[0], co = t.shape[1];
            for (size_t i = 0; i < ci; ++i)
                for (size_t o = 0; o < co; ++o)
                    for (size_t tap = 0; tap < 4; ++tap) v[(tap * co + o) * ci + i] = t.data[(i * co + o) * 4 + tap];
        } else if (n.find("relative_position_params") != std::string::npos) {
            int heads = int(t.shape[0]);
            std::vector<float> tab(size_t(heads) * 64 * 64);
            build_bias_table(t.data, heads, tab.data());
            std::string prefix = n.substr(0, n.find(".trans_block"));
            host.push_back({"@tab:" + prefix, std::move(tab)});
            std::vector<float> atab(size_t(heads) * 225);
            build_attn_table(t.data, heads, atab.data());
            host.push_back({"@atab:" + prefix, std::move(atab)});
        }
        host.push_back({n, std::move(v)});
    }
    {
        std::vector<float> gt(GELU_TABLE);
        build_gelu_table(gt.data());
        host.push_back({"@gelu", std::move(gt)});
    }
    size_t total = 0;
    for (auto& e : host) total += (e.second.size() * 4 + 255) / 256 * 256;
    void* p = nullptr;
    if (!ck(h, hipMalloc(&p, total), "weight upload: hipMalloc")) return false;
    h->wblob = static_cast<float*>(p);
    h->wbytes = total;
    char* at = static_cast<char*>(p);
    for (auto& e : host) {
        if (!ck(h, hipMemcpy(at, e.second.data(), e.second.size() * 4, hipMemcpyHostToDevice), "weight upload"))
            return false;
        if (e.first.rfind("@tab:", 0) == 0) h->tab[e.first.substr(5)] = reinterpret_cast<float*>(at);
        else if (e.first.rfind("@atab:", 0) == 0) h->atab[e.first.substr(6)] = reinterpret_cast<float*>(at);
        else h->w[e.first] = reinterpret_cast<float*>(at);   // "@wino:" / "@wino8:" Winograd filters, "@gelu"
        at += (e.second.size() * 4 + 255) / 256 * 256;
    }
    return true;
}

// The matrix weights the 16-bit layouts cover: every weight whose reduction width K is a
// multiple of 32, as [rows][K] in the layout the fp32 kernels read (after the repacking above).
struct MatItem { const float* src; long rows; int K; std::string name; };
std::vector<MatItem> matrix_weights(scunet_hip* h) {
    const Weights& wt = h->wt;
    using Item = MatItem;
    std::vector<Item> items;
    for (auto& kv : wt.all()) {
        const std::string& n = kv.first;
        const Tensor& t = kv.second;
        if (n.size() < 7 || n.compare(n.size() - 7, 7, ".weight") != 0) continue;
        long rows = 0;
        int K = 0;
        if (t.shape.size() == 2) {
            rows = long(t.shape[0]); K = int(t.shape[1]);                      // linear [out][in]
        } else if (t.shape.size() == 4 && n.find(".conv_block.") != std::string::npos) {
            rows = 9L * long(t.shape[0]); K = int(t.shape[1]);                 // [tap][co][ci]
        } else if (t.shape.size() == 4 && t.shape[2] == 1 && t.shape[3] == 1) {
            rows = long(t.shape[0]); K = int(t.shape[1]);                      // 1x1 [co][ci]
        } else if (t.shape.size() == 4 && t.shape[2] == 2 && t.shape[3] == 2) {
            const bool up = n.find("m_up") == 0 && n.find(".0.weight") != std::string::npos;
            if (up) { rows = 4L * long(t.shape[1]); K = int(t.shape[0]); }    // [tap*co][ci]
            else { rows = long(t.shape[0]); K = 4 * int(t.shape[1]); }         // [co][tap*ci]
        }
        if (rows <= 0 || K % 32 != 0 || long(rows) * K != long(t.numel)) continue;
        const float* src = W(h, n);
        if (!src) continue;
        items.push_back({src, rows, K, n});
    }
    return items;
}

// The fp16 mode's weight copies, converted and k-permuted on the device.
bool build_h16_weights(scunet_hip* h) {
    if (h->h16blob) return true;
    const std::vector<MatItem> items = matrix_weights(h);
    size_t total = 0;
    for (auto& it : items) total += (size_t(it.rows) * it.K * 2 + 255) / 256 * 256;
    void* p = nullptr;
    if (!ck(h, hipMalloc(&p, std::max<size_t>(total, 256)), "fp16 weights: hipMalloc")) return false;
    h->h16blob = static_cast<half_t*>(p);
    h->h16bytes = total;
    char* at = static_cast<char*>(p);
    for (auto& it : items) {
        h16_permute(it.src, reinterpret_cast<half_t*>(at), it.rows, it.K, h->stream);
        if (!launched(h, "fp16 weights")) return false;
        h->hw[it.name] = reinterpret_cast<const half_t*>(at);
        h->hw_of[it.src] = reinterpret_cast<const half_t*>(at);
        at += (size_t(it.rows) * it.K * 2 + 255) / 256 * 256;
    }
    return ck(h, hipStreamSynchronize(h->stream), "fp16 weights");
}

// The split weight planes (three bf16 planes per matrix weight, k-permuted like the fp16 copy).
bool build_x6_weights(scunet_hip* h) {
    if (h->x6blob) return true;
    const std::vector<MatItem> items = matrix_weights(h);
    size_t total = 0;
    for (auto& it : items) total += (size_t(it.rows) * it.K * 6 + 255) / 256 * 256;
    void* p = nullptr;
    if (!ck(h, hipMalloc(&p, std::max<size_t>(total, 256)), "split weights: hipMalloc")) return false;
    h->x6blob = static_cast<bf16_t*>(p);
    h->x6bytes = total;
    char* at = static_cast<char*>(p);
    for (auto& it : items) {
        x6_permute(it.src, reinterpret_cast<bf16_t*>(at), it.rows, it.K, h->stream);
        if (!launched(h, "split weights")) return false;
        h->xw[it.name] = reinterpret_cast<const bf16_t*>(at);
        h->xw_of[it.src] = reinterpret_cast<const bf16_t*>(at);
        at += (size_t(it.rows) * it.K * 6 + 255) / 256 * 256;
    }
    return ck(h, hipStreamSynchronize(h->stream), "split weights");
}

// Algorithmic FLOP / bytes for the profiler (fp32, 2 FLOP per multiply-add; bytes =
// inputs read once + outputs written once).
double gemm_flop(long M, int N, int K) { return 2.0 * double(M) * N * K; }

bool run_gemm(scunet_hip* h, const char* cls, const GemmArgs& g, GemmA a, GemmE e) {
    double bytes = 4.0 * (double(g.M) * g.K * (a == A_ADD2 ? 2 : 1) + double(g.N) * g.K +
                          double(g.M) * g.N * (e == E_RESID ? 2 : (e == E_DUAL ? 2 : 1)));
    Span sp(h, cls, gemm_flop(g.M, g.N, g.K), bytes);
    const char* why = nullptr;
    GemmArgs gg = g;
    gg.persistent = h->gemm2 ? 0 : 1;
    if (h->h16 && !h->gemm2) {
        auto it = h->hw_of.find(g.W);
        if (it != h->hw_of.end()) gg.W16 = it->second;
    } else if (h->x6 && !h->gemm2) {
        auto it = h->xw_of.find(g.W);
        if (it != h->xw_of.end()) gg.WX = it->second;
    }
    if (!gemm(gg, a, e, h->stream, &why)) return fail(h, std::string(cls) + ": " + why);
    return launched(h, cls);
}

// A conv_block 3x3 convolution `name` (".weight" appended): Winograd F(2x2,3x3) unless the
// handle was created with the direct kernel selected. FLOP are counted as the direct
// form's (18 cin cout per pixel), so both paths report comparable rates.
bool run_conv3(scunet_hip* h, const std::string& name, Conv3Args c, bool relu) {
    long P = long(c.H) * c.W;
    const char* why = nullptr;
    const float* u = W(h, "@wino:" + name + ".weight");
    const half_t* w16 = W16(h, name + ".weight");
    const bool h16 = w16 && c.cin == c.cout && (c.cin == 32 || c.cin == 64 || c.cin == 128 || c.cin == 256);
    const bool wino = !h16 && !h->direct3x3 && u && c.cin % 16 == 0 && c.cout % 16 == 0 && c.H % 2 == 0 &&
                      c.W % 2 == 0;
    if (h16) {
        c.w16 = w16;
    } else if (wino) {
        c.w = u;
        c.w8 = W(h, "@wino8:" + name + ".weight");
        c.cblock = h->wino16 ? 16 : 0;
        c.pair = h->wino_pair ? 1 : 0;
        c.wino3 = h->wino2 ? 0 : h->wino3_all ? 2 : 1;
        c.split = h->x6 && !h->h16 && !h->wino2 ? 1 : 0;
    } else {
        c.w = W(h, name + ".weight");
    }
    // The split-operand form is its own profile class (its products run on the bf16 matrix
    // cores, the other Winograd kernels' on the fp32 ones).
    const char* cls = wino && conv3x3_winograd_split(c) ? "conv3x3_split" : "conv3x3";
    Span sp(h, cls, 18.0 * double(P) * c.cin * c.cout,
            4.0 * (double(P) * (c.cin + c.cout * (relu ? 1 : 2)) + 9.0 * c.cin * c.cout));
    if (h16) {
        if (!conv3x3_h16(c, relu, h->stream, &why)) return fail(h, why);
    } else if (wino) {
        if (!conv3x3_winograd(c, relu, h->stream, &why)) return fail(h, why);
    } else {
        if (!conv3x3(c, relu, h->stream, &why)) return fail(h, why);
    }
    return launched(h, cls);
}

// Scratch of one ConvTransBlock at width t on P pixels: y [P][2t], s1 [P][t],
// qkv [P][3t], o [P][t].
struct BlockScratch {
    float *y, *s1, *qkv, *o;
};

bool block_scratch(scunet_hip* h, long P, int t, BlockScratch* s) {
    float* b = buf(h, "block", size_t(P) * 7 * t);
    if (!b) return false;
    s->y = b;
    s->s1 = s->y + size_t(P) * 2 * t;
    s->qkv = s->s1 + size_t(P) * t;
    s->o = s->qkv + size_t(P) * 3 * t;
    return true;
}

// The window-attention half as three launches (LN1+qkv GEMM, attention kernel,
// proj GEMM with the residual): the path for t >= 128, where the token plane is small.
bool msa_unfused(scunet_hip* h, const std::string& p, float* yt, int c, int t, int H, int Wd, int shift,
                 const BlockScratch& s) {
    const long P = long(H) * Wd;
    const std::string tp = p + ".trans_block";
    GemmArgs g;
    g.A = yt; g.lda = c; g.ln_g = W(h, tp + ".ln1.weight"); g.ln_b = W(h, tp + ".ln1.bias");
    g.W = W(h, tp + ".msa.embedding_layer.weight"); g.bias = W(h, tp + ".msa.embedding_layer.bias");
    g.C = s.qkv; g.ldc = 3 * t; g.M = P; g.N = 3 * t; g.K = t;
    if (!run_gemm(h, "qkv_ln", g, A_LN, E_STORE)) return false;
    {
        AttnArgs a;
        a.qkv = s.qkv; a.ldq = 3 * t; a.out = s.o; a.ldo = t; a.tab = h->atab[p];
        a.C = t; a.heads = t / h->wt.head_dim; a.nwh = H / 8; a.nww = Wd / 8; a.H = H; a.W = Wd;
        a.shift = shift; a.pixel_mode = 1; a.scale = h->scale; a.wide = h->attn64; a.qsplit = h->attn_qs; a.split = !h->h16 && h->x6;
        long nw = long(a.nwh) * a.nww;
        Span sp(h, "attention", 16384.0 * t * nw, 4.0 * 64.0 * nw * 4 * t);
        const char* why = nullptr;
        if (!attention(a, h->stream, &why)) return fail(h, why);
        if (!launched(h, "attention")) return false;
    }
    g = GemmArgs{};
    g.A = s.o; g.lda = t; g.W = W(h, tp + ".msa.linear.weight"); g.bias = W(h, tp + ".msa.linear.bias");
    g.C = yt; g.ldc = c; g.R = yt; g.ldr = c; g.M = P; g.N = t; g.K = t;
    return run_gemm(h, "proj", g, A_ROWS, E_RESID);
}

// A block's 1x1 convolution through the resident-weight kernel; FLOP and bytes as for
// the GEMM form (the chained form counts both products and both outputs).
bool run_pconv(scunet_hip* h, const PconvArgs& a, PconvMode mode) {
    const double P = double(a.M), c = a.c;
    const double flop = 2.0 * P * c * c * (mode == PC_CHAIN ? 2 : 1);
    const double bytes = 4.0 * (P * c * (mode == PC_STORE ? 2 : mode == PC_RESID ? 3 : 4) +
                                c * c * (mode == PC_CHAIN ? 2 : 1));
    Span sp(h, mode == PC_CHAIN ? "conv1x1_chain" : "conv1x1", flop, bytes);
    const char* why = nullptr;
    PconvArgs aa = a;
    aa.h16 = h->h16;
    if (!h->h16 && h->x6) {
        auto find = [&](const float* w) -> const bf16_t* {
            auto it = h->xw_of.find(w);
            return it == h->xw_of.end() ? nullptr : it->second;
        };
        aa.x = find(a.W);
        aa.x1 = a.W1 ? find(a.W1) : nullptr;
        if (mode == PC_CHAIN && a.c == 128 && aa.x && aa.x1) {
            // The split chained form does not fit the LDS at 128 channels: the block output
            // goes through HBM between the two products.
            PconvArgs second = aa;
            second.A = a.C; second.W = a.W1; second.b = a.b1; second.C = a.C2; second.x = aa.x1;
            second.R = nullptr; second.W1 = nullptr; second.x1 = nullptr; second.C2 = nullptr;
            if (!pconv(aa, PC_RESID, h->stream, &why) || !pconv(second, PC_STORE, h->stream, &why))
                return fail(h, why);
            return launched(h, "conv1x1");
        }
    }
    if (!pconv(aa, mode, h->stream, &why)) return fail(h, why);
    return launched(h, "conv1x1");
}

// One ConvTransBlock in place on x [P][c] (cpu.rs:869-970; cuda.rs:1063-1146).
// y_ready: the previous block's chained epilogue already wrote this block's conv1_1
// output into the block scratch. next: the following block of the same stage, whose
// conv1_1 is then chained onto this block's conv1_2 (empty for the last block).
bool block(scunet_hip* h, const std::string& p, float* x, int H, int Wd, int shift, bool y_ready = false,
           const std::string& next = std::string(), int nimg = 1) {
    auto dims = h->wt.block_dims(p);
    const int t = dims.second, conv = dims.first, c = conv + t;
    if (conv != t) return fail(h, p + ": conv and trans halves of different widths are not supported");
    // nimg images of H x Wd stacked along y: the per-pixel work sees one plane of P pixels.
    const long P = long(H) * Wd * nimg;
    BlockScratch s;
    if (!block_scratch(h, P, t, &s)) return false;
    const std::string tp = p + ".trans_block";

    const bool resident = pconv_supported(c) && !h->gemm1x1;
    if (y_ready && !resident) return fail(h, p + ": chained conv1_1 needs the resident-weight kernel");
    GemmArgs g;
    // conv1_1: y = x W^T + b.
    if (resident && !y_ready) {
        PconvArgs a;
        a.A = x; a.W = W(h, p + ".conv1_1.weight"); a.b = W(h, p + ".conv1_1.bias"); a.C = s.y; a.M = P; a.c = c;
        if (!run_pconv(h, a, PC_STORE)) return false;
    } else if (!resident) {
        g.A = x; g.lda = c; g.W = W(h, p + ".conv1_1.weight"); g.bias = W(h, p + ".conv1_1.bias");
        g.C = s.y; g.ldc = c; g.M = P; g.N = c; g.K = c;
        if (!run_gemm(h, "conv1x1", g, A_ROWS, E_STORE)) return false;
    }
    // conv half: s1 = relu(conv3x3(y[:, :t])); y[:, :t] += conv3x3(s1).
    Conv3Args cv;
    cv.in = s.y; cv.ldi = c; cv.out = s.s1; cv.ldo = t;
    cv.H = H * nimg; cv.W = Wd; cv.cin = t; cv.cout = t; cv.img_h = nimg > 1 ? H : 0;
    if (!run_conv3(h, p + ".conv_block.0", cv, true)) return false;
    cv.in = s.s1; cv.ldi = t; cv.out = s.y; cv.ldo = c;
    if (!run_conv3(h, p + ".conv_block.2", cv, false)) return false;
    // transformer half, tokens = pixels of y[:, t:2t].
    float* yt = s.y + t;
    const double mlp_flop = 16.0 * double(P) * t * t;
    // At t <= 64 the MLP runs inside the window kernel, on the window's tokens.
    // In the split-operand mode the t = 64 MLP runs as its own kernel, whose LDS-staged
    // weight slices feed 128 rows (inside the window kernel every window reads the weight
    // planes from L2 again): 572 -> 464 us per level-1 block (attention half + MLP).
    const bool mlp_in_msa = (t <= 32 || (t == 64 && !(h->x6 && !h->h16))) && !h->unfused_msa && !h->separate_mlp;
    if (t <= 256 && !h->unfused_msa) {
        MsaArgs m;
        m.x = yt; m.ldx = c; m.ln_g = W(h, tp + ".ln1.weight"); m.ln_b = W(h, tp + ".ln1.bias");
        m.wqkv = W(h, tp + ".msa.embedding_layer.weight"); m.bqkv = W(h, tp + ".msa.embedding_layer.bias");
        m.wp = W(h, tp + ".msa.linear.weight"); m.bp = W(h, tp + ".msa.linear.bias"); m.tab = h->tab[p];
        m.t = t; m.nwh = H / 8; m.nww = Wd / 8; m.H = H; m.W = Wd; m.shift = shift; m.scale = h->scale;
        m.nimg = nimg;
        m.hqkv = W16(h, tp + ".msa.embedding_layer.weight"); m.hp = W16(h, tp + ".msa.linear.weight");
        m.xqkv = WX(h, tp + ".msa.embedding_layer.weight"); m.xp = WX(h, tp + ".msa.linear.weight");
        if (mlp_in_msa) {
            m.ln2_g = W(h, tp + ".ln2.weight"); m.ln2_b = W(h, tp + ".ln2.bias");
            m.w0 = W(h, tp + ".mlp.0.weight"); m.b0 = W(h, tp + ".mlp.0.bias");
            m.w2 = W(h, tp + ".mlp.2.weight"); m.b2 = W(h, tp + ".mlp.2.bias");
            m.h0 = W16(h, tp + ".mlp.0.weight"); m.h2 = W16(h, tp + ".mlp.2.weight");
            m.x0 = WX(h, tp + ".mlp.0.weight"); m.x2 = WX(h, tp + ".mlp.2.weight");
            m.gelu = W(h, "@gelu");
        }
        const double nw = double(m.nwh) * m.nww * nimg;
        const double msa_flop = 64.0 * nw * (8.0 * t * t) + 16384.0 * t * nw;
        Span sp(h, mlp_in_msa ? "tblock_fused" : "msa_fused", msa_flop + (mlp_in_msa ? mlp_flop : 0.0),
                4.0 * (2.0 * P * t + 4.0 * t * t + (mlp_in_msa ? 8.0 * t * t : 0.0)));
        const char* why = nullptr;
        if (!msa_fused(m, h->stream, &why)) return fail(h, why);
        if (!launched(h, "msa_fused")) return false;
    } else if (!msa_unfused(h, p, yt, c, t, H, Wd, shift, s)) {
        return false;
    }
    if (!mlp_in_msa) {
        MlpArgs m;
        m.x = yt; m.ldx = c; m.ln_g = W(h, tp + ".ln2.weight"); m.ln_b = W(h, tp + ".ln2.bias");
        m.w0 = W(h, tp + ".mlp.0.weight"); m.b0 = W(h, tp + ".mlp.0.bias");
        m.w2 = W(h, tp + ".mlp.2.weight"); m.b2 = W(h, tp + ".mlp.2.bias"); m.M = P; m.t = t;
        m.h0 = W16(h, tp + ".mlp.0.weight"); m.h2 = W16(h, tp + ".mlp.2.weight");
        m.x0 = WX(h, tp + ".mlp.0.weight"); m.x2 = WX(h, tp + ".mlp.2.weight");
        m.gelu = W(h, "@gelu");
        Span sp(h, "mlp_fused", mlp_flop, 4.0 * (2.0 * P * t + 8.0 * t * t + 5.0 * t));
        const char* why = nullptr;
        if (!mlp(m, h->stream, &why)) return fail(h, why);
        if (!launched(h, "mlp")) return false;
    }
    // conv1_2 on the concatenation, residual over the block: x += y W^T + b; chained with
    // the next block's conv1_1 (y = x W1^T + b1) when there is one.
    if (resident) {
        PconvArgs a;
        a.A = s.y; a.W = W(h, p + ".conv1_2.weight"); a.b = W(h, p + ".conv1_2.bias");
        a.R = x; a.C = x; a.M = P; a.c = c;
        if (next.empty()) return run_pconv(h, a, PC_RESID);
        a.W1 = W(h, next + ".conv1_1.weight"); a.b1 = W(h, next + ".conv1_1.bias"); a.C2 = s.y;
        return run_pconv(h, a, PC_CHAIN);
    }
    g = GemmArgs{};
    g.A = s.y; g.lda = c; g.W = W(h, p + ".conv1_2.weight"); g.bias = W(h, p + ".conv1_2.bias");
    g.C = x; g.ldc = c; g.R = x; g.ldr = c; g.M = P; g.N = c; g.K = c;
    return run_gemm(h, "conv1x1", g, A_ROWS, E_RESID);
}

// The `count` blocks `prefix` first .. first+count-1 of one stage, in place on x; block i
// uses the shifted windows when i is odd (cpu.rs:1216-1222, 1298-1302). With the resident-weight 1x1
// kernel, each block's conv1_2 is chained with the next block's conv1_1.
bool stage_blocks(scunet_hip* h, const std::string& prefix, int first, int count, float* x, int H, int Wd,
                  int nimg = 1) {
    const int win = h->wt.window;
    const int c = h->wt.block_dims(prefix + std::to_string(first)).first * 2;
    const bool chain = pconv_supported(c) && !h->gemm1x1;
    for (int i = 0; i < count; ++i) {
        const std::string next = chain && i + 1 < count ? prefix + std::to_string(first + i + 1) : std::string();
        if (!block(h, prefix + std::to_string(first + i), x, H, Wd, (i & 1) ? win / 2 : 0, chain && i > 0, next, nimg))
            return false;
    }
    return true;
}

bool dump_plane(scunet_hip* h, scunet_stage_hook hook, void* user, const char* name, const float* plane,
                int c, long P) {
    if (!hook) return true;
    float* tmp = buf(h, "dump", size_t(c) * P);
    if (!tmp) return false;
    nhwc_to_nchw(plane, tmp, c, P, c, h->stream);
    if (!launched(h, "dump")) return false;
    std::vector<float> host(size_t(c) * P);
    if (!ck(h, hipMemcpyAsync(host.data(), tmp, host.size() * 4, hipMemcpyDeviceToHost, h->stream), "dump D2H"))
        return false;
    if (!ck(h, hipStreamSynchronize(h->stream), "dump sync")) return false;
    hook(name, host.data(), host.size(), user);
    return true;
}

// The walker. x: NCHW image of size hh x ww (hh == H, ww == W when already padded);
// y: NCHW [in_nc][oh][ow] (the crop is fused into m_tail).
bool walk(scunet_hip* h, const float* x, int hh, int ww, int H, int Wd, float* y, int oh, int ow,
          scunet_stage_hook hook, void* user, int nimg = 1) {
    const Weights& wt = h->wt;
    const int dim = wt.dim, in_nc = wt.in_nc;
    if (H % 64 || Wd % 64) return fail(h, "the padded plane must be a multiple of 64 on each axis");
    long P[4];
    int Hs[4], Ws[4];
    for (int k = 0; k < 4; ++k) {
        Hs[k] = H >> k;
        Ws[k] = Wd >> k;
        P[k] = long(Hs[k]) * Ws[k] * nimg;
    }
    h->chain = nullptr;
    float* cur[4];
    float* skip[4] = {nullptr, nullptr, nullptr, nullptr};
    for (int k = 0; k < 4; ++k) {
        cur[k] = buf(h, "cur" + std::to_string(k), size_t(P[k]) * (dim << k));
        if (!cur[k]) return false;
        if (k > 0) {
            skip[k] = buf(h, "skip" + std::to_string(k), size_t(P[k]) * (dim << k));
            if (!skip[k]) return false;
        }
    }
    h->tag.clear();
    {
        Span sp(h, "head", 2.0 * 9 * in_nc * dim * double(P[0]), 4.0 * (in_nc + dim) * double(P[0]));
        if (!head_conv(x, in_nc, hh, ww, H, Wd, W(h, "m_head.0.weight"), dim, cur[0], false, h->stream, nimg))
            return fail(h, "m_head: unsupported shape");
        if (!launched(h, "m_head")) return false;
    }
    if (!dump_plane(h, hook, user, "m_head", cur[0], dim, P[0])) return false;
    for (int k = 0; k < 3; ++k) {
        const std::string name = STAGE[k];
        const int count = wt.config[k];
        const int c = dim << k;
        h->tag = "@L" + std::to_string(k);
        if (!stage_blocks(h, "m_" + name + ".", 0, count, cur[k], Hs[k], Ws[k], nimg)) return false;
        if (!dump_plane(h, hook, user, ("m_" + name + "_blocks").c_str(), cur[k], c, P[k])) return false;
        GemmArgs g;
        g.A = cur[k]; g.lda = c; g.W = W(h, "m_" + name + "." + std::to_string(count) + ".weight");
        g.C = skip[k + 1]; g.C2 = cur[k + 1]; g.ldc = 2 * c; g.M = P[k + 1]; g.N = 2 * c; g.K = 4 * c;
        g.in_w = Ws[k]; g.cin = c;
        if (!run_gemm(h, "down2x2", g, A_S2D, E_DUAL)) return false;
        if (!dump_plane(h, hook, user, ("m_" + name).c_str(), skip[k + 1], 2 * c, P[k + 1])) return false;
    }
    h->tag = "@L3";
    if (!stage_blocks(h, "m_body.", 0, wt.config[3], cur[3], Hs[3], Ws[3], nimg)) return false;
    if (!dump_plane(h, hook, user, "m_body", cur[3], dim << 3, P[3])) return false;
    for (int k = 0; k < 3; ++k) {
        const std::string name = STAGE[4 + k];
        const int lvl = 2 - k;               // up3 -> level 2, up2 -> 1, up1 -> 0
        const int co = dim << lvl, ci = 2 * co;
        h->tag = "@L" + std::to_string(lvl);
        GemmArgs g;
        g.A = cur[lvl + 1]; g.A2 = skip[lvl + 1]; g.lda = ci;
        g.W = W(h, "m_" + name + ".0.weight");
        g.C = cur[lvl]; g.M = P[lvl + 1]; g.N = 4 * co; g.K = ci; g.in_w = Ws[lvl + 1]; g.cout = co;
        if (!run_gemm(h, "up2x2", g, A_ADD2, E_D2S)) return false;
        if (!dump_plane(h, hook, user, ("m_" + name + "_up").c_str(), cur[lvl], co, P[lvl])) return false;
        if (!stage_blocks(h, "m_" + name + ".", 1, wt.config[4 + k], cur[lvl], Hs[lvl], Ws[lvl], nimg)) return false;
        if (!dump_plane(h, hook, user, ("m_" + name).c_str(), cur[lvl], co, P[lvl])) return false;
    }
    h->tag.clear();
    {
        Span sp(h, "head", 2.0 * 9 * in_nc * dim * double(P[0]), 4.0 * (in_nc + 2 * dim) * double(P[0]));
        if (!head_conv(x, in_nc, hh, ww, H, Wd, W(h, "m_head.0.weight"), dim, cur[0], true, h->stream, nimg))
            return fail(h, "m_head: unsupported shape");
        if (!launched(h, "m_head (tail input)")) return false;
    }
    if (!dump_plane(h, hook, user, "m_tail_in", cur[0], dim, P[0])) return false;
    {
        Span sp(h, "tail", 2.0 * 9 * in_nc * dim * double(P[0]), 4.0 * (in_nc + dim) * double(P[0]));
        // The split-product tail in the default and fp16 modes (exact to fp32 level); the
        // fp32-MFMA mode keeps the fp32 FMA form.
        if (!tail_conv(cur[0], dim, H, Wd, W(h, "m_tail.0.weight"), in_nc, y, oh, ow, h->stream, nimg,
                       h->x6 || h->h16))
            return fail(h, "m_tail: unsupported width");
        if (!launched(h, "m_tail")) return false;
    }
    if (hook) {
        std::vector<float> host(size_t(in_nc) * oh * ow);
        if (!ck(h, hipMemcpyAsync(host.data(), y, host.size() * 4, hipMemcpyDeviceToHost, h->stream), "dump D2H"))
            return false;
        if (!ck(h, hipStreamSynchronize(h->stream), "dump sync")) return false;
        hook("m_tail", host.data(), host.size(), user);
    }
    return true;
}

bool check_arch(scunet_hip* h) {
    const Weights& wt = h->wt;
    if (wt.window != 8) return fail(h, "window " + std::to_string(wt.window) + ": the attention kernel is built for 8x8 windows");
    if (wt.head_dim != 32) return fail(h, "head_dim " + std::to_string(wt.head_dim) + ": the attention kernel is built for head_dim 32");
    if (wt.in_nc > 4) return fail(h, "in_nc > 4 is not supported by the m_tail kernel");
    if (wt.dim != 64) return fail(h, "dim " + std::to_string(wt.dim) + ": only the published dim = 64 is supported");
    return true;
}

size_t pad64(size_t v) { return (v + 63) / 64 * 64; }

// plan.rs:105-118.
bool check_min_size(scunet_hip* h, size_t hh, size_t ww) {
    size_t hp = pad64(hh), wp = pad64(ww), win = size_t(h->wt.window);
    if (hh == 0 || ww == 0) return fail(h, "empty image");
    if (hp < 8 * win || wp < 8 * win)
        return fail(h, std::to_string(hh) + "x" + std::to_string(ww) + " pads to " + std::to_string(hp) + "x" +
                           std::to_string(wp) + ", but the 1/8-resolution body needs at least " +
                           std::to_string(win) + "x" + std::to_string(win) + " pixels there");
    return true;
}

template <typename F>
int guard(scunet_hip* h, F&& f) {
    if (!h) return -1;
    h->err.clear();
    h->chain = nullptr;   // a profiled launch never shares an event across API calls
    try {
        return f() ? 0 : 1;
    } catch (const std::exception& e) {
        h->err = e.what();
        return 1;
    }
}

bool to_device(scunet_hip* h, const char* role, const float* src, size_t n, float** out) {
    *out = buf(h, role, n);
    if (!*out) return false;
    return ck(h, hipMemcpyAsync(*out, src, n * 4, hipMemcpyHostToDevice, h->stream), "H2D");
}

bool to_host(scunet_hip* h, float* dst, const float* src, size_t n) {
    if (!ck(h, hipMemcpyAsync(dst, src, n * 4, hipMemcpyDeviceToHost, h->stream), "D2H")) return false;
    return ck(h, hipStreamSynchronize(h->stream), "sync");
}

// The scratch a forward of the padded H x W plane requests, role by role, exactly as walk()
// and block() ask buf() for it: the four level planes and three skips (dim 2^k channels at
// P / 4^k pixels), one ConvTransBlock scratch sized for level 0 (7 t floats per pixel), the
// stage-dump staging plane when a hook is given, and the host entry points' input/output
// staging copies (io floats each).
std::vector<std::pair<std::string, size_t>> arena_plan(const scunet_hip* h, size_t H, size_t W, size_t io,
                                                       bool dump) {
    const size_t dim = size_t(h->wt.dim);
    std::vector<std::pair<std::string, size_t>> r;
    size_t block = 0;
    for (int k = 0; k < 4; ++k) {
        const size_t P = (H >> k) * (W >> k), c = dim << k;
        r.push_back({"cur" + std::to_string(k), P * c});
        if (k > 0) r.push_back({"skip" + std::to_string(k), P * c});
        block = std::max(block, P * 7 * (c / 2));
    }
    r.push_back({"block", block});
    if (dump) r.push_back({"dump", H * W * dim});
    if (io) {
        r.push_back({"io_x", io});
        r.push_back({"io_y", io});
    }
    return r;
}

// (bytes the arena holds for that plan, bytes not held yet). The arena keeps each role's
// largest size, so a role already big enough costs nothing.
std::pair<size_t, size_t> arena_need(const scunet_hip* h, const std::vector<std::pair<std::string, size_t>>& plan) {
    size_t total = 0, more = 0;
    for (auto& r : plan) {
        const size_t bytes = std::max<size_t>(r.second, 1) * sizeof(float);
        auto it = h->arena.find(r.first);
        const size_t held = it == h->arena.end() ? 0 : it->second.second;
        total += std::max(bytes, held);
        // A grown role frees its old buffer just before allocating the new one, so the roles'
        // growths add up: their sum is both the extra footprint and the peak extra demand.
        if (bytes > held) more += bytes - held;
    }
    for (auto& kv : h->arena) {
        bool planned = false;
        for (auto& r : plan) planned = planned || r.first == kv.first;
        if (!planned) total += kv.second.second;
    }
    return {total, more};
}

// The memguard.rs:66-74 question, asked before the first allocation of a forward: does the
// scratch it still needs fit in the device's free memory? Refuses with the sizes named.
bool preflight(scunet_hip* h, size_t H, size_t W, size_t io, bool dump) {
    const auto need = arena_need(h, arena_plan(h, H, W, io, dump));
    if (need.second == 0) return true;
    size_t free_b = 0, total_b = 0;
    if (!ck(h, hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo")) return false;
    if (need.second <= free_b) return true;
    return fail(h, "a " + std::to_string(H) + "x" + std::to_string(W) + " forward needs " +
                       std::to_string(need.second >> 20) + " MiB more device memory (" +
                       std::to_string(need.first >> 20) + " MiB of scratch in all, plus " +
                       std::to_string((h->wbytes + h->h16bytes + h->x6bytes) >> 20) + " MiB of weights); the device has " +
                       std::to_string(free_b >> 20) + " MiB free of " + std::to_string(total_b >> 20) + " MiB");
}

bool shape_ok(scunet_hip* h, size_t c, size_t hp, size_t wp) {
    if (c != size_t(h->wt.in_nc))
        return fail(h, "expected " + std::to_string(h->wt.in_nc) + " channels, got " + std::to_string(c));
    if (hp % 64 || wp % 64 || hp == 0 || wp == 0)
        return fail(h, "forward takes the padded plane: " + std::to_string(hp) + "x" + std::to_string(wp) +
                           " is not a multiple of 64 on each axis");
    return true;
}

}  // namespace

extern "C" {

const char* scunet_hip_create_error(void) { return g_create_error.c_str(); }

static int create_handle(const char* path, const scunet_hip_arch_info* arch, scunet_hip_tensor_lookup lookup,
                         void* user, scunet_hip** out);

// No C++ exception leaves the C ABI: a failed host allocation while reading or repacking the
// checkpoint is reported like any other create error.
int scunet_hip_create(const char* path, scunet_hip** out) {
    g_create_error.clear();
    if (!out) {
        g_create_error = "null output handle";
        return 1;
    }
    *out = nullptr;
    try {
        return create_handle(path, nullptr, nullptr, nullptr, out);
    } catch (const std::exception& e) {
        g_create_error = std::string("scunet_hip_create: ") + e.what();
        return 1;
    }
}

int scunet_hip_create_from_tensors(const scunet_hip_arch_info* arch, scunet_hip_tensor_lookup lookup, void* user,
                                   scunet_hip** out) {
    g_create_error.clear();
    if (!out) {
        g_create_error = "null output handle";
        return 1;
    }
    *out = nullptr;
    if (!arch) {
        g_create_error = "weights: no architecture given";
        return 1;
    }
    try {
        return create_handle(nullptr, arch, lookup, user, out);
    } catch (const std::exception& e) {
        g_create_error = std::string("scunet_hip_create_from_tensors: ") + e.what();
        return 1;
    }
}

// From a file (path) or from the caller's tensors (arch + lookup, borrowed until the upload).
static int create_handle(const char* path, const scunet_hip_arch_info* arch, scunet_hip_tensor_lookup lookup,
                         void* user, scunet_hip** out) {
    std::unique_ptr<scunet_hip> h(new scunet_hip());
    std::string err;
    if (arch) {
        ArchInfo a;
        a.variant = arch->variant ? arch->variant : "";
        auto clamp = [](size_t v) { return long(std::min<size_t>(v, size_t(1) << 40)); };
        a.in_nc = clamp(arch->in_nc);
        a.dim = clamp(arch->dim);
        a.head_dim = clamp(arch->head_dim);
        a.window = clamp(arch->window);
        for (int i = 0; i < 7; ++i) a.config[i] = clamp(arch->config[i]);
        if (!h->wt.borrow(a, lookup, user, &err)) {
            g_create_error = err;
            return 1;
        }
    } else if (!h->wt.load(path ? path : "", &err)) {
        g_create_error = err;
        return 1;
    }
    if (!check_arch(h.get())) {
        g_create_error = h->err;
        return 1;
    }
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0) {
        g_create_error = std::string("no HIP device: ") + hipGetErrorString(e);
        return 1;
    }
    hipGetDevice(&h->device);
    resolve_scratch(h->device);
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
        g_create_error = "hipStreamCreate failed";
        return 1;
    }
    h->scale = std::pow(float(h->wt.head_dim), -0.5f);
    // A/B switch: run the window-attention half as three launches at every level.
    h->unfused_msa = std::getenv("SCUNET_HIP_UNFUSED_MSA") != nullptr;
    // A/B switch: the direct implicit-GEMM 3x3 kernel instead of Winograd F(2x2,3x3).
    h->direct3x3 = std::getenv("SCUNET_HIP_DIRECT3X3") != nullptr;
    h->wino16 = std::getenv("SCUNET_HIP_WINO16") != nullptr;
    // A/B switch: 16-channel Winograd units always as pairs of 8 x 16 half-tiles.
    h->wino_pair = std::getenv("SCUNET_HIP_WINO_PAIR") != nullptr;
    // A/B switch: k_wino2 / k_wino at every level whose plane fits 32-bit offsets (no k_wino3).
    h->wino2 = std::getenv("SCUNET_HIP_WINO2") != nullptr;
    // A/B switch: k_wino3 at every level, including 32-channel units at level 0.
    h->wino3_all = std::getenv("SCUNET_HIP_WINO3") != nullptr;
    // A/B switch: the attention kernel's 64-bit-offset form at every size.
    h->attn64 = std::getenv("SCUNET_HIP_ATTN64") != nullptr;
    // A/B switch: the attention kernel with 1 or 2 query parts per (window, head).
    if (const char* q = std::getenv("SCUNET_HIP_ATTN_QS")) h->attn_qs = std::atoi(q) == 2 ? 2 : 1;
    h->gemm2 = std::getenv("SCUNET_HIP_GEMM2") != nullptr;
    h->gemm1x1 = std::getenv("SCUNET_HIP_GEMM1X1") != nullptr;
    h->separate_mlp = std::getenv("SCUNET_HIP_SEPARATE_MLP") != nullptr;
    if (!upload_weights(h.get())) {
        g_create_error = h->err;
        return 1;
    }
    // The default fp32 mode forms products from split operands where a kernel can.
    h->x6 = true;
    if (!build_x6_weights(h.get())) {
        g_create_error = h->err;
        return 1;
    }
    if (arch) h->wt.forget_data();   // the caller's buffers are not ours beyond this call
    *out = h.release();
    return 0;
}

void scunet_hip_destroy(scunet_hip* h) { delete h; }

const char* scunet_hip_last_error(const scunet_hip* h) { return h ? h->err.c_str() : "null handle"; }

const char* scunet_hip_name(const scunet_hip*) { return "hip"; }

int scunet_hip_set_precision(scunet_hip* h, int mode) {
    if (!h) return 1;
    if (mode != SCUNET_HIP_FP32 && mode != SCUNET_HIP_FP16 && mode != SCUNET_HIP_FP32_MFMA) {
        fail(h, "scunet_hip_set_precision: mode must be SCUNET_HIP_FP32 (0), SCUNET_HIP_FP16 (1) or "
                "SCUNET_HIP_FP32_MFMA (2)");
        return 1;
    }
    try {
        if (mode == SCUNET_HIP_FP16 && !build_h16_weights(h)) return 1;
        if (mode == SCUNET_HIP_FP32 && !build_x6_weights(h)) return 1;
    } catch (const std::exception& e) {
        fail(h, std::string("scunet_hip_set_precision: ") + e.what());
        return 1;
    }
    h->h16 = mode == SCUNET_HIP_FP16 ? 1 : 0;
    h->x6 = mode == SCUNET_HIP_FP32;
    return 0;
}

int scunet_hip_precision(const scunet_hip* h) {
    if (!h) return -1;
    return h->h16 ? SCUNET_HIP_FP16 : h->x6 ? SCUNET_HIP_FP32 : SCUNET_HIP_FP32_MFMA;
}

int scunet_hip_arch(const scunet_hip* h, int* in_nc, int* dim, int* head_dim, int* window, int* config) {
    if (!h) return -1;
    if (in_nc) *in_nc = h->wt.in_nc;
    if (dim) *dim = h->wt.dim;
    if (head_dim) *head_dim = h->wt.head_dim;
    if (window) *window = h->wt.window;
    if (config)
        for (int i = 0; i < 7; ++i) config[i] = h->wt.config[i];
    return 0;
}

const char* scunet_hip_variant(const scunet_hip* h) { return h ? h->wt.variant.c_str() : ""; }

int scunet_hip_forward_device(scunet_hip* h, const float* x, size_t c, size_t hp, size_t wp, float* y) {
    return guard(h, [&] {
        if (!shape_ok(h, c, hp, wp)) return false;
        if (!preflight(h, hp, wp, 0, false)) return false;
        return walk(h, x, int(hp), int(wp), int(hp), int(wp), y, int(hp), int(wp), nullptr, nullptr);
    });
}

int scunet_hip_forward_dump(scunet_hip* h, const float* x, size_t c, size_t hp, size_t wp, float* y,
                            scunet_stage_hook hook, void* user) {
    return guard(h, [&] {
        if (!shape_ok(h, c, hp, wp)) return false;
        size_t n = c * hp * wp;
        if (!preflight(h, hp, wp, n, hook != nullptr)) return false;
        float *dx, *dy;
        if (!to_device(h, "io_x", x, n, &dx)) return false;
        dy = buf(h, "io_y", n);
        if (!dy) return false;
        if (!walk(h, dx, int(hp), int(wp), int(hp), int(wp), dy, int(hp), int(wp), hook, user)) return false;
        return to_host(h, y, dy, n);
    });
}

int scunet_hip_forward(scunet_hip* h, const float* x, size_t c, size_t hp, size_t wp, float* y) {
    return scunet_hip_forward_dump(h, x, c, hp, wp, y, nullptr, nullptr);
}

int scunet_hip_run_device(scunet_hip* h, const float* x, size_t c, size_t hh, size_t ww, float* y) {
    return guard(h, [&] {
        if (!check_min_size(h, hh, ww)) return false;
        if (c != size_t(h->wt.in_nc))
            return fail(h, "expected " + std::to_string(h->wt.in_nc) + " channels, got " + std::to_string(c));
        size_t hp = pad64(hh), wp = pad64(ww);
        if (!preflight(h, hp, wp, 0, false)) return false;
        return walk(h, x, int(hh), int(ww), int(hp), int(wp), y, int(hh), int(ww), nullptr, nullptr);
    });
}

// scunet_hip_run_device with the arena in the static `scratch` array: no device memory is
// allocated or freed. The roles of arena_plan() are laid out back to back (256-byte
// aligned); nothing in them needs clearing, since every role is written before it is read
// within the forward. Profiling events are not recorded during the call.
int scunet_hip_run_device_noalloc(scunet_hip* h, const float* x, size_t c, size_t hh, size_t ww, float* y) {
    return guard(h, [&] {
        if (!check_min_size(h, hh, ww)) return false;
        if (c != size_t(h->wt.in_nc))
            return fail(h, "expected " + std::to_string(h->wt.in_nc) + " channels, got " + std::to_string(c));
        const size_t hp = pad64(hh), wp = pad64(ww);
        float* base = nullptr;
        {
            std::lock_guard<std::mutex> lock(g_scratch_mu);
            if (h->device >= 0 && h->device < MAX_DEVICES) {
                base = g_scratch_ptr[h->device];
                if (!base) return fail(h, "no-alloc forward: " + g_scratch_err[h->device]);
            }
        }
        if (!base) return fail(h, "no-alloc forward: device " + std::to_string(h->device) + " has no scratch");
        std::map<std::string, std::pair<float*, size_t>> roles;
        size_t at = 0;
        for (auto& r : arena_plan(h, hp, wp, 0, false)) {
            const size_t bytes = std::max<size_t>(r.second, 1) * sizeof(float);
            roles[r.first] = {base + at / sizeof(float), bytes};
            at += (bytes + 255) / 256 * 256;
        }
        if (at > NOALLOC_SCRATCH_BYTES)
            return fail(h, "no-alloc forward: a " + std::to_string(hh) + "x" + std::to_string(ww) + " image (padded " +
                               std::to_string(hp) + "x" + std::to_string(wp) + ") needs " + std::to_string(at) +
                               " bytes of scratch; the static scratch holds " +
                               std::to_string(NOALLOC_SCRATCH_BYTES) + " (use scunet_hip_run_device)");
        struct Restore {
            scunet_hip* h;
            bool prof;
            ~Restore() {
                h->fixed_active = false;
                h->fixed.clear();
                h->prof = prof;
            }
        } restore{h, h->prof};
        h->fixed = std::move(roles);
        h->fixed_active = true;
        h->prof = false;
        return walk(h, x, int(hh), int(ww), int(hp), int(wp), y, int(hh), int(ww), nullptr, nullptr);
    });
}

int scunet_hip_run(scunet_hip* h, const float* x, size_t c, size_t hh, size_t ww, float* y) {
    return guard(h, [&] {
        if (!check_min_size(h, hh, ww)) return false;
        if (c != size_t(h->wt.in_nc))
            return fail(h, "expected " + std::to_string(h->wt.in_nc) + " channels, got " + std::to_string(c));
        size_t hp = pad64(hh), wp = pad64(ww), n = c * hh * ww;
        if (!preflight(h, hp, wp, n, false)) return false;
        float *dx, *dy;
        if (!to_device(h, "io_x", x, n, &dx)) return false;
        dy = buf(h, "io_y", n);
        if (!dy) return false;
        if (!walk(h, dx, int(hh), int(ww), int(hp), int(wp), dy, int(hh), int(ww), nullptr, nullptr)) return false;
        return to_host(h, y, dy, n);
    });
}

int scunet_hip_run_batch(scunet_hip* h, const float* x, size_t nimg, size_t c, size_t hh, size_t ww, float* y) {
    return guard(h, [&] {
        if (!check_min_size(h, hh, ww)) return false;
        if (c != size_t(h->wt.in_nc))
            return fail(h, "expected " + std::to_string(h->wt.in_nc) + " channels, got " + std::to_string(c));
        if (nimg == 0) return true;
        size_t hp = pad64(hh), wp = pad64(ww), n = c * hh * ww;
        if (!preflight(h, hp * nimg, wp, n * nimg, false)) return false;
        float *dx, *dy;
        if (!to_device(h, "io_x", x, n * nimg, &dx)) return false;
        dy = buf(h, "io_y", n * nimg);
        if (!dy) return false;
        if (h->direct3x3 || h->unfused_msa) {
            // The A/B kernels take one image at a time.
            for (size_t i = 0; i < nimg; ++i)
                if (!walk(h, dx + i * n, int(hh), int(ww), int(hp), int(wp), dy + i * n, int(hh), int(ww), nullptr,
                          nullptr))
                    return false;
        } else if (!walk(h, dx, int(hh), int(ww), int(hp), int(wp), dy, int(hh), int(ww), nullptr, nullptr,
                         int(nimg))) {
            return false;
        }
        return to_host(h, y, dy, n * nimg);
    });
}

int scunet_hip_device_need(const scunet_hip* h, size_t c, size_t hh, size_t ww, int host_io, size_t* scratch_bytes,
                           size_t* more_bytes) {
    if (!h || hh == 0 || ww == 0) return 1;
    try {
        const auto need = arena_need(h, arena_plan(h, pad64(hh), pad64(ww), host_io ? c * hh * ww : 0, false));
        if (scratch_bytes) *scratch_bytes = need.first;
        if (more_bytes) *more_bytes = need.second;
    } catch (const std::exception&) {
        return 1;
    }
    return 0;
}

int scunet_hip_footprint(const scunet_hip* h, size_t* weight_bytes, size_t* scratch_bytes) {
    if (!h) return -1;
    size_t s = 0;
    for (auto& kv : h->arena) s += kv.second.second;
    if (weight_bytes) *weight_bytes = h->wbytes + h->h16bytes + h->x6bytes;
    if (scratch_bytes) *scratch_bytes = s;
    return 0;
}

int scunet_hip_release_scratch(scunet_hip* h) {
    return guard(h, [&] {
        if (!ck(h, hipStreamSynchronize(h->stream), "sync")) return false;
        for (auto& kv : h->arena)
            if (kv.second.first) hipFree(kv.second.first);
        h->arena.clear();
        return true;
    });
}

int scunet_hip_synchronize(scunet_hip* h) {
    return guard(h, [&] { return ck(h, hipStreamSynchronize(h->stream), "hipStreamSynchronize"); });
}

void* scunet_hip_stream(scunet_hip* h) { return h ? static_cast<void*>(h->stream) : nullptr; }

int scunet_hip_profile(scunet_hip* h, int on) {
    return guard(h, [&] {
        if (!ck(h, hipStreamSynchronize(h->stream), "sync")) return false;
        h->prof = on != 0;
        h->recs.clear();
        h->ev_used = 0;
        h->chain = nullptr;
        return true;
    });
}

int scunet_hip_profile_report(scunet_hip* h, const char** names, long* launches, double* ms, double* flop,
                              double* bytes, int cap, int* n) {
    return guard(h, [&] {
        if (!ck(h, hipStreamSynchronize(h->stream), "sync")) return false;
        struct Agg { long n = 0; double ms = 0, flop = 0, bytes = 0; };
        std::map<std::string, Agg> agg;
        for (auto& r : h->recs) {
            float t = 0.f;
            if (!ck(h, hipEventElapsedTime(&t, r.e0, r.e1), "hipEventElapsedTime")) return false;
            auto& a = agg[r.name];
            a.n += 1;
            a.ms += t;
            a.flop += r.flop;
            a.bytes += r.bytes;
        }
        std::vector<std::pair<std::string, Agg>> v(agg.begin(), agg.end());
        std::sort(v.begin(), v.end(), [](auto& a, auto& b) { return a.second.ms > b.second.ms; });
        h->report_names.clear();
        for (auto& e : v) h->report_names.push_back(e.first);
        int k = 0;
        for (; k < int(v.size()) && k < cap; ++k) {
            if (names) names[k] = h->report_names[size_t(k)].c_str();
            if (launches) launches[k] = v[size_t(k)].second.n;
            if (ms) ms[k] = v[size_t(k)].second.ms;
            if (flop) flop[k] = v[size_t(k)].second.flop;
            if (bytes) bytes[k] = v[size_t(k)].second.bytes;
        }
        if (n) *n = int(v.size());
        h->recs.clear();
        h->ev_used = 0;
        h->chain = nullptr;
        return true;
    });
}

int scunet_hip_malloc(scunet_hip* h, void** p, size_t bytes) {
    return guard(h, [&] { return ck(h, hipMalloc(p, std::max<size_t>(bytes, 1)), "hipMalloc"); });
}
int scunet_hip_free(scunet_hip* h, void* p) {
    return guard(h, [&] {
        if (!ck(h, hipStreamSynchronize(h->stream), "sync")) return false;
        return ck(h, hipFree(p), "hipFree");
    });
}
int scunet_hip_h2d(scunet_hip* h, void* dst, const void* src, size_t bytes) {
    return guard(h, [&] {
        if (!ck(h, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, h->stream), "H2D")) return false;
        return ck(h, hipStreamSynchronize(h->stream), "sync");
    });
}
int scunet_hip_d2h(scunet_hip* h, void* dst, const void* src, size_t bytes) {
    return guard(h, [&] {
        if (!ck(h, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, h->stream), "D2H")) return false;
        return ck(h, hipStreamSynchronize(h->stream), "sync");
    });
}

int scunet_hip_copy(scunet_hip* h, void* dst, const void* src, size_t bytes) {
    return guard(h, [&] {
        if (bytes % 16 || (reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16)
            return fail(h, "scunet_hip_copy: bytes and pointers must be 16-byte aligned");
        Span sp(h, "copy", 0.0, 2.0 * double(bytes));
        copy_f4(src, dst, long(bytes / 16), h->stream);
        return launched(h, "copy");
    });
}

// ---------------------------------------------------------------------------
// Probes
// ---------------------------------------------------------------------------

int scunet_hip_block_probe(scunet_hip* h, const char* prefix, size_t hh, size_t ww, size_t shift, const float* x,
                           float* out) {
    return guard(h, [&] {
        std::string p = prefix;
        if (!h->wt.has(p + ".conv1_1.weight")) return fail(h, "no block `" + p + "`");
        if (hh % 8 || ww % 8 || hh == 0 || ww == 0) return fail(h, "block planes must be multiples of 8");
        auto d = h->wt.block_dims(p);
        int c = d.first + d.second;
        long P = long(hh) * long(ww);
        float *dx, *xt;
        if (!to_device(h, "probe_in", x, size_t(c) * P, &dx)) return false;
        xt = buf(h, "probe_x", size_t(c) * P);
        if (!xt) return false;
        nchw_to_nhwc(dx, xt, c, P, c, h->stream);
        if (!block(h, p, xt, int(hh), int(ww), int(shift))) return false;
        float* o = buf(h, "probe_out", size_t(c) * P);
        if (!o) return false;
        nhwc_to_nchw(xt, o, c, P, c, h->stream);
        if (!launched(h, "block probe")) return false;
        return to_host(h, out, o, size_t(c) * P);
    });
}

int scunet_hip_op_probe(scunet_hip* h, const char* op, const char* name, const float* x, size_t c_in, size_t c_out,
                        size_t hh, size_t ww, float* out) {
    return guard(h, [&] {
        std::string o = op, n = name;
        const float* wp = W(h, n + ".weight");
        if (!wp) return fail(h, "no weight `" + n + ".weight`");
        const float* bp = W(h, n + ".bias");
        long P = long(hh) * long(ww);
        float* dx;
        if (!to_device(h, "probe_in", x, c_in * size_t(P), &dx)) return false;
        float* xt = buf(h, "probe_x", c_in * size_t(P));
        if (!xt) return false;
        long Po = P;
        if (o == "conv2x2s2") Po = P / 4;
        if (o == "conv_t2x2") Po = P * 4;
        float* yt = buf(h, "probe_y", c_out * size_t(Po));
        float* yo = buf(h, "probe_out", c_out * size_t(Po));
        if (!yt || !yo) return false;
        if (o == "conv3x3" && n == "m_head.0") {
            if (!head_conv(dx, int(c_in), int(hh), int(ww), int(hh), int(ww), wp, int(c_out), yt, false, h->stream))
                return fail(h, "m_head: unsupported shape");
        } else if (o == "conv3x3" && n == "m_tail.0") {
            nchw_to_nhwc(dx, xt, int(c_in), P, long(c_in), h->stream);
            if (!tail_conv(xt, int(c_in), int(hh), int(ww), wp, int(c_out), yo, int(hh), int(ww), h->stream, 1,
                           h->x6 || h->h16))
                return fail(h, "m_tail: unsupported width");
            if (!launched(h, "op probe")) return false;
            return to_host(h, out, yo, c_out * size_t(P));
        } else {
            nchw_to_nhwc(dx, xt, int(c_in), P, long(c_in), h->stream);
            if (o == "conv3x3") {
                Conv3Args cv;
                cv.in = xt; cv.ldi = long(c_in); cv.out = yt; cv.ldo = long(c_out);
                cv.H = int(hh); cv.W = int(ww); cv.cin = int(c_in); cv.cout = int(c_out);
                if (!ck(h, hipMemsetAsync(yt, 0, c_out * size_t(P) * 4, h->stream), "memset")) return false;
                if (!run_conv3(h, n, cv, false)) return false;
            } else {
                GemmArgs g;
                g.A = xt; g.lda = long(c_in); g.W = wp; g.C = yt; g.ldc = long(c_out);
                g.N = int(c_out);
                if (o == "conv1x1" && c_in == c_out && pconv_supported(int(c_in)) && bp && !h->gemm1x1) {
                    PconvArgs a;
                    a.A = xt; a.W = wp; a.b = bp; a.C = yt; a.M = P; a.c = int(c_in);
                    if (!run_pconv(h, a, PC_STORE)) return false;
                } else if (o == "conv1x1") {
                    g.bias = bp; g.M = P; g.K = int(c_in);
                    if (!run_gemm(h, "conv1x1", g, A_ROWS, E_STORE)) return false;
                } else if (o == "conv2x2s2") {
                    g.M = P / 4; g.K = int(4 * c_in); g.in_w = int(ww); g.cin = int(c_in);
                    if (!run_gemm(h, "down2x2", g, A_S2D, E_STORE)) return false;
                } else if (o == "conv_t2x2") {
                    g.M = P; g.K = int(c_in); g.N = int(4 * c_out); g.in_w = int(ww); g.cout = int(c_out);
                    g.ldc = 0;
                    float* zero = buf(h, "probe_zero", c_in * size_t(P));
                    if (!zero) return false;
                    if (!ck(h, hipMemsetAsync(zero, 0, c_in * size_t(P) * 4, h->stream), "memset")) return false;
                    g.A2 = zero;
                    if (!run_gemm(h, "up2x2", g, A_ADD2, E_D2S)) return false;
                } else {
                    return fail(h, "op_probe: no such op `" + o + "`");
                }
            }
        }
        nhwc_to_nchw(yt, yo, int(c_out), Po, long(c_out), h->stream);
        if (!launched(h, "op probe")) return false;
        return to_host(h, out, yo, c_out * size_t(Po));
    });
}

int scunet_hip_linear_probe(scunet_hip* h, const char* name, const float* x, size_t rows, size_t c_in, size_t c_out,
                            float* out) {
    return guard(h, [&] {
        std::string n = name;
        const float* wp = W(h, n + ".weight");
        if (!wp) return fail(h, "no weight `" + n + ".weight`");
        float* dx;
        if (!to_device(h, "probe_in", x, rows * c_in, &dx)) return false;
        float* y = buf(h, "probe_out", rows * c_out);
        if (!y) return false;
        GemmArgs g;
        g.A = dx; g.lda = long(c_in); g.W = wp; g.bias = W(h, n + ".bias"); g.C = y; g.ldc = long(c_out);
        g.M = long(rows); g.N = int(c_out); g.K = int(c_in);
        if (!run_gemm(h, "linear", g, A_ROWS, E_STORE)) return false;
        return to_host(h, out, y, rows * c_out);
    });
}

// LayerNorm through the GEMM's own LN prologue against an identity weight: every output
// is one normalised value times 1 plus zeros, so the GEMM adds nothing of its own.
int scunet_hip_layer_norm_probe(scunet_hip* h, const char* name, const float* x, size_t rows, size_t c, float* out) {
    return guard(h, [&] {
        std::string n = name;
        const float* gw = W(h, n + ".weight");
        const float* gb = W(h, n + ".bias");
        if (!gw || !gb) return fail(h, "no LayerNorm `" + n + "`");
        float* dx;
        if (!to_device(h, "probe_in", x, rows * c, &dx)) return false;
        std::vector<float> eye(c * c, 0.f);
        for (size_t i = 0; i < c; ++i) eye[i * c + i] = 1.f;
        float* de;
        if (!to_device(h, "probe_eye", eye.data(), c * c, &de)) return false;
        float* y = buf(h, "probe_out", rows * c);
        if (!y) return false;
        GemmArgs g;
        g.A = dx; g.lda = long(c); g.ln_g = gw; g.ln_b = gb; g.W = de; g.C = y; g.ldc = long(c);
        g.M = long(rows); g.N = int(c); g.K = int(c);
        if (!run_gemm(h, "layer_norm", g, A_LN, E_STORE)) return false;
        return to_host(h, out, y, rows * c);
    });
}

int scunet_hip_attention_kernel_probe(scunet_hip* h, size_t hh, size_t ww, size_t c, size_t heads, size_t hd,
                                      size_t shift, const float* qkv, const float* rp, float* out) {
    return guard(h, [&] {
        if (hd != 32 || c != heads * hd) return fail(h, "the attention kernel needs head_dim 32");
        if (hh % 8 || ww % 8) return fail(h, "the plane must be a multiple of the 8x8 window");
        size_t nw = (hh / 8) * (ww / 8), nt = nw * 64;
        float *dq, *dt;
        if (!to_device(h, "probe_in", qkv, nt * 3 * c, &dq)) return false;
        std::vector<float> tab(heads * 225);
        build_attn_table(rp, int(heads), tab.data());
        if (!to_device(h, "probe_tab", tab.data(), tab.size(), &dt)) return false;
        float* y = buf(h, "probe_out", nt * c);
        if (!y) return false;
        AttnArgs a;
        a.qkv = dq; a.ldq = long(3 * c); a.out = y; a.ldo = long(c); a.tab = dt; a.C = int(c); a.heads = int(heads);
        a.nwh = int(hh / 8); a.nww = int(ww / 8); a.H = int(hh); a.W = int(ww); a.shift = int(shift);
        a.pixel_mode = 0; a.scale = std::pow(float(hd), -0.5f); a.wide = h->attn64; a.qsplit = h->attn_qs; a.split = !h->h16 && h->x6;
        const char* why = nullptr;
        if (!attention(a, h->stream, &why)) return fail(h, why);
        if (!launched(h, "attention probe")) return false;
        return to_host(h, out, y, nt * c);
    });
}

int scunet_hip_gather_probe(scunet_hip* h, size_t hh, size_t ww, size_t c, size_t shift, const float* x, float* tok) {
    return guard(h, [&] {
        if (hh % 8 || ww % 8) return fail(h, "the plane must be a multiple of the 8x8 window");
        long P = long(hh) * long(ww);
        float* dx;
        if (!to_device(h, "probe_in", x, c * size_t(P), &dx)) return false;
        float* xt = buf(h, "probe_x", c * size_t(P));
        float* y = buf(h, "probe_out", c * size_t(P));
        if (!xt || !y) return false;
        nchw_to_nhwc(dx, xt, int(c), P, long(c), h->stream);
        window_gather(xt, y, int(c), int(hh), int(ww), int(shift), h->stream);
        if (!launched(h, "gather probe")) return false;
        return to_host(h, tok, y, c * size_t(P));
    });
}

int scunet_hip_window_round_trip(scunet_hip* h, size_t hh, size_t ww, size_t c, size_t shift, const float* x,
                                 float* out) {
    return guard(h, [&] {
        if (hh % 8 || ww % 8) return fail(h, "the plane must be a multiple of the 8x8 window");
        long P = long(hh) * long(ww);
        float* dx;
        if (!to_device(h, "probe_in", x, c * size_t(P), &dx)) return false;
        float* xt = buf(h, "probe_x", c * size_t(P));
        float* tk = buf(h, "probe_y", c * size_t(P));
        float* y = buf(h, "probe_out", c * size_t(P));
        if (!xt || !tk || !y) return false;
        nchw_to_nhwc(dx, xt, int(c), P, long(c), h->stream);
        window_gather(xt, tk, int(c), int(hh), int(ww), int(shift), h->stream);
        hipMemsetAsync(xt, 0, c * size_t(P) * 4, h->stream);
        window_scatter(tk, xt, int(c), int(hh), int(ww), int(shift), h->stream);
        nhwc_to_nchw(xt, y, int(c), P, long(c), h->stream);
        if (!launched(h, "round trip")) return false;
        return to_host(h, out, y, c * size_t(P));
    });
}

int scunet_hip_attention_probe(scunet_hip* h, const char* prefix, size_t hh, size_t ww, size_t c, size_t shift,
                               const float* x, float* tok) {
    return guard(h, [&] {
        std::string tp = std::string(prefix) + ".trans_block";
        if (!W(h, tp + ".ln1.weight")) return fail(h, "no block `" + std::string(prefix) + "`");
        if (hh % 8 || ww % 8) return fail(h, "the plane must be a multiple of the 8x8 window");
        long P = long(hh) * long(ww);
        int t = int(c);
        float* dx;
        if (!to_device(h, "probe_in", x, c * size_t(P), &dx)) return false;
        float* xt = buf(h, "probe_x", c * size_t(P));
        float* qkv = buf(h, "probe_qkv", 3 * c * size_t(P));
        float* att = buf(h, "probe_att", c * size_t(P));
        float* o = buf(h, "probe_y", c * size_t(P));
        float* y = buf(h, "probe_out", c * size_t(P));
        if (!xt || !qkv || !att || !o || !y) return false;
        nchw_to_nhwc(dx, xt, t, P, t, h->stream);
        GemmArgs g;
        g.A = xt; g.lda = t; g.ln_g = W(h, tp + ".ln1.weight"); g.ln_b = W(h, tp + ".ln1.bias");
        g.W = W(h, tp + ".msa.embedding_layer.weight"); g.bias = W(h, tp + ".msa.embedding_layer.bias");
        g.C = qkv; g.ldc = 3 * t; g.M = P; g.N = 3 * t; g.K = t;
        if (!run_gemm(h, "qkv_ln", g, A_LN, E_STORE)) return false;
        AttnArgs a;
        a.qkv = qkv; a.ldq = 3 * t; a.out = att; a.ldo = t; a.tab = h->atab[prefix]; a.C = t;
        a.heads = t / h->wt.head_dim; a.nwh = int(hh / 8); a.nww = int(ww / 8); a.H = int(hh); a.W = int(ww);
        a.shift = int(shift); a.pixel_mode = 1; a.scale = h->scale; a.wide = h->attn64; a.qsplit = h->attn_qs; a.split = !h->h16 && h->x6;
        const char* why = nullptr;
        if (!attention(a, h->stream, &why)) return fail(h, why);
        g = GemmArgs{};
        g.A = att; g.lda = t; g.W = W(h, tp + ".msa.linear.weight"); g.bias = W(h, tp + ".msa.linear.bias");
        g.C = o; g.ldc = t; g.M = P; g.N = t; g.K = t;
        if (!run_gemm(h, "proj", g, A_ROWS, E_STORE)) return false;
        window_gather(o, y, t, int(hh), int(ww), int(shift), h->stream);
        if (!launched(h, "attention probe")) return false;
        return to_host(h, tok, y, c * size_t(P));
    });
}

int scunet_hip_bench_attn(scunet_hip* h, const float* qkv, const float* rp, float* out, size_t nwh, size_t nww,
                          size_t c, size_t heads, size_t shift, int iters, double* ms) {
    return guard(h, [&] {
        if (c != heads * 32) return fail(h, "the attention kernel needs head_dim 32");
        std::vector<float> tab(heads * 225);
        build_attn_table(rp, int(heads), tab.data());
        float* dt;
        if (!to_device(h, "bench_tab", tab.data(), tab.size(), &dt)) return false;
        AttnArgs a;
        a.qkv = qkv; a.ldq = long(3 * c); a.out = out; a.ldo = long(c); a.tab = dt; a.C = int(c);
        a.heads = int(heads); a.nwh = int(nwh); a.nww = int(nww); a.H = int(nwh * 8); a.W = int(nww * 8);
        a.shift = int(shift); a.pixel_mode = 0; a.scale = h->scale; a.wide = h->attn64; a.qsplit = h->attn_qs; a.split = !h->h16 && h->x6;
        const char* why = nullptr;
        for (int i = 0; i < 3; ++i)
            if (!attention(a, h->stream, &why)) return fail(h, why);
        hipEvent_t e0, e1;
        hipEventCreate(&e0);
        hipEventCreate(&e1);
        hipEventRecord(e0, h->stream);
        for (int i = 0; i < iters; ++i) attention(a, h->stream, &why);
        hipEventRecord(e1, h->stream);
        bool ok = launched(h, "attention bench") && ck(h, hipEventSynchronize(e1), "sync");
        float t = 0.f;
        if (ok) ok = ck(h, hipEventElapsedTime(&t, e0, e1), "elapsed");
        hipEventDestroy(e0);
        hipEventDestroy(e1);
        if (ok && ms) *ms = double(t) / std::max(iters, 1);
        return ok;
    });
}

}  // extern "C"
