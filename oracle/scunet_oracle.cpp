// TEST INFRASTRUCTURE - NOT PART OF THE PRODUCT.
//
// A CPU restatement of the reference's fp32 path, src/cpu.rs (jacobsparts/scunet-rs),
// used in three places only: as the parity oracle the HIP backend is tested against
// (tests/), as the checker inside __graft_entry__.smoke(), and as the timed CPU
// baseline in bench.py. The product library never links, loads or calls it.
//
// Faithfulness rules, taken from src/cpu.rs's own header (cpu.rs:38-44):
//   * every loop that is split across threads (OpenMP here, rayon there) is split over
//     INDEPENDENT OUTPUT ELEMENTS, and each output accumulates its terms in the same
//     order the serial loop does, so the result does not depend on the thread count;
//   * sums run in the order cpu.rs writes them (cited per function below);
//   * built with -O3 -ffp-contract=off and no fast-math, so no FMA contraction and no
//     reassociation - Rust never contracts either; expf/sqrtf/powf/exp come from libm,
//     which is what Rust's f32::exp / f64::exp call on Linux.
//
// The two chunkings in cpu.rs (TOKEN_BUDGET windows, cpu.rs:381-392, and
// MLP_CHUNK_BYTES of hidden, cpu.rs:376-379) are arithmetic-neutral by construction
// (each window and each token is computed independently) and are not reproduced.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>
#include <cfloat>
#include <stdexcept>
#include <omp.h>

namespace {

const float LN_EPS = 1e-5f;                       // cpu.rs:50
const float MASK_SENTINEL = -FLT_MAX / 4.0f;      // cpu.rs:370
const size_t PAR_MIN = size_t(1) << 14;           // cpu.rs:55
const size_t CONV1X1_BLK = 1024;                  // cpu.rs:459

inline bool par_on(size_t n) { return n >= PAR_MIN && omp_get_max_threads() > 1; }

// cpu.rs:72-137. Output channel `co`, row `yy`: dst = 0, then input channel ascending,
// ky, kx, each tap applied to the row of output columns whose source is inside the
// plane (zero padding = skipped tap).
void conv3x3(const float* x, size_t c_in, size_t c_out, size_t h, size_t w, const float* wt,
             float* out) {
    auto run = [&](size_t co) {
        float* row = out + co * h * w;
        for (size_t yy = 0; yy < h; ++yy) {
            float* dst = row + yy * w;
            for (size_t i = 0; i < w; ++i) dst[i] = 0.0f;
            for (size_t ci = 0; ci < c_in; ++ci) {
                const float* p = x + ci * h * w;
                const float* k = wt + (co * c_in + ci) * 9;
                for (size_t ky = 0; ky < 3; ++ky) {
                    long sy = long(yy) + long(ky) - 1;
                    if (sy < 0 || sy >= long(h)) continue;
                    const float* s = p + size_t(sy) * w;
                    for (size_t kx = 0; kx < 3; ++kx) {
                        float kk = k[ky * 3 + kx];
                        long x0 = std::max(1L - long(kx), 0L);
                        long x1 = std::min(long(w) + 1 - long(kx), long(w));
                        const float* src = s + x0 + long(kx) - 1;
                        for (long i = 0; i < x1 - x0; ++i) dst[x0 + i] += kk * src[i];
                    }
                }
            }
        }
    };
    if (par_on(c_out * h * w)) {
#pragma omp parallel for schedule(static)
        for (long co = 0; co < long(c_out); ++co) run(size_t(co));
    } else {
        for (size_t co = 0; co < c_out; ++co) run(co);
    }
}

// cpu.rs:141-170. acc over ci ascending, the four taps (0,0),(0,1),(1,0),(1,1) inner.
void conv2x2s2(const float* x, size_t c_in, size_t c_out, size_t h, size_t w, const float* wt,
               float* out) {
    size_t oh = h / 2, ow = w / 2;
    auto run = [&](size_t co) {
        float* row = out + co * oh * ow;
        for (size_t y = 0; y < oh; ++y)
            for (size_t xx = 0; xx < ow; ++xx) {
                float acc = 0.0f;
                for (size_t ci = 0; ci < c_in; ++ci) {
                    const float* p = x + ci * h * w;
                    const float* k = wt + (co * c_in + ci) * 4;
                    acc += k[0] * p[(2 * y) * w + 2 * xx];
                    acc += k[1] * p[(2 * y) * w + 2 * xx + 1];
                    acc += k[2] * p[(2 * y + 1) * w + 2 * xx];
                    acc += k[3] * p[(2 * y + 1) * w + 2 * xx + 1];
                }
                row[y * ow + xx] = acc;
            }
    };
    if (par_on(c_out * oh * ow)) {
#pragma omp parallel for schedule(static)
        for (long co = 0; co < long(c_out); ++co) run(size_t(co));
    } else {
        for (size_t co = 0; co < c_out; ++co) run(co);
    }
}

// cpu.rs:175-217. dst = bias, then += k[ci] * x[ci] for ci ascending.
void conv1x1(const float* x, size_t c_in, size_t c_out, size_t n, const float* wt,
             const float* bias, float* out) {
    auto run = [&](size_t co) {
        const float* k = wt + co * c_in;
        float b = bias ? bias[co] : 0.0f;
        float* row = out + co * n;
        for (size_t jb = 0; jb < n; jb += CONV1X1_BLK) {
            size_t je = std::min(jb + CONV1X1_BLK, n);
            for (size_t j = jb; j < je; ++j) row[j] = b;
            for (size_t ci = 0; ci < c_in; ++ci) {
                float kk = k[ci];
                const float* src = x + ci * n;
                for (size_t j = jb; j < je; ++j) row[j] += kk * src[j];
            }
        }
    };
    if (par_on(c_out * n)) {
#pragma omp parallel for schedule(static)
        for (long co = 0; co < long(c_out); ++co) run(size_t(co));
    } else {
        for (size_t co = 0; co < c_out; ++co) run(co);
    }
}

// cpu.rs:232-263. ConvTranspose2d(2, stride 2), weight [c_in][c_out][2][2], no tap flip.
void conv_t2x2(const float* x, size_t c_in, size_t c_out, size_t h, size_t w, const float* wt,
               float* out) {
    size_t oh = 2 * h, ow = 2 * w;
    auto run = [&](size_t co) {
        float* row = out + co * oh * ow;
        for (size_t i = 0; i < oh * ow; ++i) row[i] = 0.0f;
        for (size_t ci = 0; ci < c_in; ++ci) {
            const float* p = x + ci * h * w;
            const float* k = wt + (ci * c_out + co) * 4;
            for (size_t y = 0; y < h; ++y)
                for (size_t xx = 0; xx < w; ++xx) {
                    float v = p[y * w + xx];
                    row[(2 * y) * ow + 2 * xx] += k[0] * v;
                    row[(2 * y) * ow + 2 * xx + 1] += k[1] * v;
                    row[(2 * y + 1) * ow + 2 * xx] += k[2] * v;
                    row[(2 * y + 1) * ow + 2 * xx + 1] += k[3] * v;
                }
        }
    };
    if (par_on(c_out * oh * ow)) {
#pragma omp parallel for schedule(static)
        for (long co = 0; co < long(c_out); ++co) run(size_t(co));
    } else {
        for (size_t co = 0; co < c_out; ++co) run(co);
    }
}

// cpu.rs:271-280: y += x.
void add_into(const float* x, float* y, size_t n) {
    if (par_on(n)) {
#pragma omp parallel for schedule(static)
        for (long i = 0; i < long(n); ++i) y[i] += x[i];
    } else {
        for (size_t i = 0; i < n; ++i) y[i] += x[i];
    }
}

// cpu.rs:284-288.
void relu(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = std::max(x[i], 0.0f);
}

}  // namespace

// cpu.rs:318-332: Abramowitz & Stegun 7.1.26 in f64, |error| < 1.5e-7.
extern "C" double oracle_erf(double x) {
    double t = 1.0 / (1.0 + 0.3275911 * std::fabs(x));
    double y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t +
                      0.254829592) *
                         t * std::exp(-x * x);
    return x >= 0.0 ? y : -y;
}

namespace {

// cpu.rs:293-311: 0.5 * t * (1 + erf(t / sqrt(2))) in f64, cast to f32.
void gelu_erf_inplace(float* x, size_t n) {
    const double SQRT_2 = 1.4142135623730951;
    auto one = [&](size_t i) {
        double t = double(x[i]);
        x[i] = float(0.5 * t * (1.0 + oracle_erf(t / SQRT_2)));
    };
    if (par_on(n)) {
#pragma omp parallel for schedule(static)
        for (long i = 0; i < long(n); ++i) one(size_t(i));
    } else {
        for (size_t i = 0; i < n; ++i) one(i);
    }
}

// cpu.rs:338-357. mu = sequential sum / c, var = sequential sum of squares / c,
// inv = 1/sqrt(var + eps), dst = (src - mu) * inv * w + b.
void layer_norm(const float* x, size_t rows, size_t c, const float* wg, const float* bs,
                float* out) {
    auto run = [&](size_t r) {
        const float* src = x + r * c;
        float* dst = out + r * c;
        float sum = 0.0f;
        for (size_t i = 0; i < c; ++i) sum += src[i];
        float mu = sum / float(c);
        float sq = 0.0f;
        for (size_t i = 0; i < c; ++i) sq += (src[i] - mu) * (src[i] - mu);
        float var = sq / float(c);
        float inv = 1.0f / std::sqrt(var + LN_EPS);
        for (size_t i = 0; i < c; ++i) dst[i] = (src[i] - mu) * inv * wg[i] + bs[i];
    };
    if (par_on(rows * c)) {
#pragma omp parallel for schedule(static)
        for (long r = 0; r < long(rows); ++r) run(size_t(r));
    } else {
        for (size_t r = 0; r < rows; ++r) run(r);
    }
}

// cpu.rs:412-431 / 438-453: [c][n] <-> [n][c].
void to_hwc(const float* src, size_t c, size_t n, float* dst) {
#pragma omp parallel for schedule(static) if (par_on(n * c))
    for (long i = 0; i < long(n); ++i)
        for (size_t ci = 0; ci < c; ++ci) dst[size_t(i) * c + ci] = src[ci * n + size_t(i)];
}
void from_hwc(const float* src, size_t c, size_t n, float* dst) {
#pragma omp parallel for schedule(static) if (par_on(n * c))
    for (long ci = 0; ci < long(c); ++ci)
        for (size_t i = 0; i < n; ++i) dst[size_t(ci) * n + i] = src[i * c + size_t(ci)];
}

// cpu.rs:514-520: sequential dot product from 0.0.
inline float dot(const float* a, const float* b, size_t n) {
    float acc = 0.0f;
    for (size_t i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}

}  // namespace

// cpu.rs:532-546: entry (p, q) = params[(py - qy + win - 1) * span + (px - qx + win - 1)].
extern "C" void oracle_rel_pos_table(const float* params, size_t win, float* out) {
    size_t n = win * win, span = 2 * win - 1;
    for (size_t p = 0; p < n; ++p) {
        size_t py = p / win, px = p % win;
        for (size_t q = 0; q < n; ++q) {
            size_t qy = q / win, qx = q % win;
            size_t dy = py + win - 1 - qy, dx = px + win - 1 - qx;
            out[p * n + q] = params[dy * span + dx];
        }
    }
}

// cpu.rs:558-586: the shifted-window mask; each edge compares the same axis.
extern "C" int oracle_mask_hit(size_t p, size_t t, size_t wh, size_t ww, size_t nwh, size_t nww,
                               size_t win) {
    size_t s = win - win / 2;
    size_t pr = p / win, pc = p % win, tr = t / win, tc = t % win;
    bool row_edge = wh == nwh - 1, col_edge = ww == nww - 1;
    bool row = (pr < s && tr >= s) || (pr >= s && tr < s);
    bool col = (pc < s && tc >= s) || (pc >= s && tc < s);
    return ((row_edge && row) || (col_edge && col)) ? 1 : 0;
}

// cpu.rs:602-758. x and out are [h][w][c] token planes. Split over windows; each window
// does its own qkv, scores, softmax, PV and projection, then scatters to the rolled
// pixel positions.
extern "C" void oracle_attention(const float* x, size_t h, size_t w, size_t c, size_t win,
                                 size_t shift, const float* emb_w, const float* emb_b,
                                 const float* lin_w, const float* lin_b, const float* rp,
                                 size_t heads, float* out) {
    size_t n = win * win, nwh = h / win, nww = w / win, span = 2 * win - 1;
    size_t hd = c / heads;
    float scale = std::pow(float(hd), -0.5f);
    bool shifted = shift != 0;
    size_t nw = nwh * nww;
#pragma omp parallel if (par_on(nw * n * c))
    {
        std::vector<float> q(n * hd), k(n * hd), v(n * hd), sim(n * n), rel(n * n), o(n * c),
            dst(n * c);
        std::vector<size_t> pix(n);
#pragma omp for schedule(static)
        for (long wil = 0; wil < long(nw); ++wil) {
            size_t wi = size_t(wil);
            size_t wh = wi / nww, ww = wi % nww;
            for (size_t t = 0; t < n; ++t) {
                size_t i = t / win, j = t % win;
                pix[t] = ((wh * win + i + shift) % h) * w + (ww * win + j + shift) % w;
            }
            for (size_t head = 0; head < heads; ++head) {
                size_t base = head * hd;
                for (size_t t = 0; t < n; ++t) {
                    const float* xv = x + pix[t] * c;
                    for (size_t r = 0; r < hd; ++r) {
                        q[t * hd + r] = dot(emb_w + (base + r) * c, xv, c) + emb_b[base + r];
                        k[t * hd + r] = dot(emb_w + (c + base + r) * c, xv, c) + emb_b[c + base + r];
                        v[t * hd + r] =
                            dot(emb_w + (2 * c + base + r) * c, xv, c) + emb_b[2 * c + base + r];
                    }
                }
                oracle_rel_pos_table(rp + head * span * span, win, rel.data());
                for (size_t p = 0; p < n; ++p) {
                    float* row = sim.data() + p * n;
                    for (size_t t = 0; t < n; ++t) {
                        float s = dot(&q[p * hd], &k[t * hd], hd) * scale;
                        s += rel[p * n + t];
                        if (shifted && oracle_mask_hit(p, t, wh, ww, nwh, nww, win)) s = MASK_SENTINEL;
                        row[t] = s;
                    }
                    float mx = -INFINITY;
                    for (size_t t = 0; t < n; ++t) mx = std::fmax(mx, row[t]);
                    float sum = 0.0f;
                    for (size_t t = 0; t < n; ++t) {
                        row[t] = std::exp(row[t] - mx);
                        sum += row[t];
                    }
                    float inv = 1.0f / sum;
                    for (size_t t = 0; t < n; ++t) row[t] *= inv;
                    for (size_t r = 0; r < hd; ++r) {
                        float acc = 0.0f;
                        for (size_t t = 0; t < n; ++t) acc += row[t] * v[t * hd + r];
                        o[p * c + base + r] = acc;
                    }
                }
            }
            for (size_t p = 0; p < n; ++p)
                for (size_t r = 0; r < c; ++r)
                    dst[p * c + r] = dot(lin_w + r * c, &o[p * c], c) + lin_b[r];
            for (size_t t = 0; t < n; ++t)
                std::memcpy(out + pix[t] * c, &dst[t * c], c * sizeof(float));
        }
    }
}

namespace {

struct Weights {
    std::unordered_map<std::string, std::pair<const float*, size_t>> t;
    int in_nc = 3, dim = 64, head_dim = 32, window = 8;
    int config[7] = {4, 4, 4, 4, 4, 4, 4};
    const float* get(const std::string& name) const {
        auto it = t.find(name);
        if (it == t.end()) throw std::runtime_error("oracle: weight `" + name + "` missing");
        return it->second.first;
    }
    size_t numel(const std::string& name) const {
        auto it = t.find(name);
        if (it == t.end()) throw std::runtime_error("oracle: weight `" + name + "` missing");
        return it->second.second;
    }
    // weights.rs:196-200: (conv, trans) read off conv1_1.weight [c][c][1][1] and
    // msa.linear.weight [t][t].
    std::pair<size_t, size_t> block_dims(const std::string& p) const {
        size_t total = size_t(std::llround(std::sqrt(double(numel(p + ".conv1_1.weight")))));
        size_t trans =
            size_t(std::llround(std::sqrt(double(numel(p + ".trans_block.msa.linear.weight")))));
        return {total - trans, trans};
    }
};

}  // namespace

extern "C" {

typedef struct {
    int n;
    const char* const* names;
    const float* const* ptrs;
    const size_t* numel;
    int in_nc, dim, head_dim, window;
    int config[7];
} oracle_weights;

typedef void (*oracle_hook)(const char* name, const float* plane, size_t n, void* user);

void oracle_set_threads(int n) { omp_set_num_threads(n); }
int oracle_get_threads(void) { return omp_get_max_threads(); }

void oracle_conv3x3(const float* x, size_t c_in, size_t c_out, size_t h, size_t w,
                    const float* wt, float* out) {
    conv3x3(x, c_in, c_out, h, w, wt, out);
}
void oracle_conv2x2s2(const float* x, size_t c_in, size_t c_out, size_t h, size_t w,
                      const float* wt, float* out) {
    conv2x2s2(x, c_in, c_out, h, w, wt, out);
}
void oracle_conv1x1(const float* x, size_t c_in, size_t c_out, size_t n, const float* wt,
                    const float* bias, float* out) {
    conv1x1(x, c_in, c_out, n, wt, bias, out);
}
void oracle_conv_t2x2(const float* x, size_t c_in, size_t c_out, size_t h, size_t w,
                      const float* wt, float* out) {
    conv_t2x2(x, c_in, c_out, h, w, wt, out);
}
void oracle_layer_norm(const float* x, size_t rows, size_t c, const float* wg, const float* bs,
                       float* out) {
    layer_norm(x, rows, c, wg, bs, out);
}
void oracle_gelu_inplace(float* x, size_t n) { gelu_erf_inplace(x, n); }

// plan.rs:67-82: replicate (edge-clamp) [c][h][w] -> [c][hp][wp].
void oracle_pad_replicate(const float* x, size_t c, size_t h, size_t w, size_t hp, size_t wp,
                          float* out) {
    for (size_t ch = 0; ch < c; ++ch)
        for (size_t y = 0; y < hp; ++y) {
            size_t sy = y < h ? y : h - 1;
            const float* src = x + (ch * h + sy) * w;
            float* dst = out + (ch * hp + y) * wp;
            std::memcpy(dst, src, w * sizeof(float));
            for (size_t i = w; i < wp; ++i) dst[i] = src[w - 1];
        }
}

// plan.rs:85-94.
void oracle_crop(const float* x, size_t c, size_t h, size_t w, size_t hp, size_t wp, float* out) {
    for (size_t ch = 0; ch < c; ++ch)
        for (size_t y = 0; y < h; ++y)
            std::memcpy(out + (ch * h + y) * w, x + (ch * hp + y) * wp, w * sizeof(float));
}

// cpu.rs:782-861: pre-norm window attention then pre-norm MLP, both residual, on the
// [h][w][c] token plane.
void oracle_trans_block(const float* x, size_t h, size_t w, size_t c, size_t win, size_t shift,
                        const float* ln1_w, const float* ln1_b, const float* emb_w,
                        const float* emb_b, const float* lin_w, const float* lin_b,
                        const float* rp, size_t heads, const float* ln2_w, const float* ln2_b,
                        const float* mlp0_w, const float* mlp0_b, const float* mlp2_w,
                        const float* mlp2_b, float* out, float* msa_out) {
    size_t n = h * w;
    std::vector<float> norm(c * n), att(c * n);
    layer_norm(x, n, c, ln1_w, ln1_b, norm.data());
    oracle_attention(norm.data(), h, w, c, win, shift, emb_w, emb_b, lin_w, lin_b, rp, heads,
                     att.data());
    if (msa_out) std::memcpy(msa_out, att.data(), c * n * sizeof(float));
    std::memcpy(out, x, c * n * sizeof(float));
    add_into(att.data(), out, c * n);
    layer_norm(out, n, c, ln2_w, ln2_b, norm.data());
    size_t four = 4 * c;
#pragma omp parallel if (par_on(n * four))
    {
        std::vector<float> hb(four);
#pragma omp for schedule(static)
        for (long tl = 0; tl < long(n); ++tl) {
            size_t t = size_t(tl);
            const float* src = norm.data() + t * c;
            for (size_t r = 0; r < four; ++r) hb[r] = dot(mlp0_w + r * c, src, c) + mlp0_b[r];
            for (size_t r = 0; r < four; ++r) {
                double tt = double(hb[r]);
                hb[r] = float(0.5 * tt * (1.0 + oracle_erf(tt / 1.4142135623730951)));
            }
            float* dst = att.data() + t * c;
            for (size_t r = 0; r < c; ++r) dst[r] = dot(mlp2_w + r * four, hb.data(), four) + mlp2_b[r];
        }
    }
    add_into(att.data(), out, c * n);
}

}  // extern "C"

namespace {

Weights make_weights(const oracle_weights* ow) {
    Weights W;
    for (int i = 0; i < ow->n; ++i) W.t[ow->names[i]] = {ow->ptrs[i], ow->numel[i]};
    W.in_nc = ow->in_nc;
    W.dim = ow->dim;
    W.head_dim = ow->head_dim;
    W.window = ow->window;
    for (int i = 0; i < 7; ++i) W.config[i] = ow->config[i];
    return W;
}

struct BlockDump {
    float* expand = nullptr;
    float* conv_half = nullptr;
    float* trans_half = nullptr;
    float* msa = nullptr;
    float* res = nullptr;
};

// cpu.rs:869-953 (+ the residual of 963-970 / 976-983): 1x1 expand, 3x3-ReLU-3x3 +
// residual on the conv half, the transformer half through [h][w][c], 1x1 project.
void block_project(const float* x, std::pair<size_t, size_t> dims, size_t h, size_t w,
                   size_t win, size_t shift, const Weights& wt, const std::string& prefix,
                   std::vector<float>& proj, const BlockDump* dump) {
    size_t conv = dims.first, trans = dims.second, c = conv + trans, n = h * w;
    std::vector<float> y(c * n), c1(conv * n), c2(conv * n), tok(trans * n), bt(trans * n);
    proj.assign(c * n, 0.0f);
    conv1x1(x, c, c, n, wt.get(prefix + ".conv1_1.weight"), wt.get(prefix + ".conv1_1.bias"),
            y.data());
    if (dump && dump->expand) std::memcpy(dump->expand, y.data(), c * n * 4);
    conv3x3(y.data(), conv, conv, h, w, wt.get(prefix + ".conv_block.0.weight"), c1.data());
    relu(c1.data(), conv * n);
    conv3x3(c1.data(), conv, conv, h, w, wt.get(prefix + ".conv_block.2.weight"), c2.data());
    add_into(y.data(), c2.data(), conv * n);
    std::memcpy(y.data(), c2.data(), conv * n * 4);
    if (dump && dump->conv_half) std::memcpy(dump->conv_half, c2.data(), conv * n * 4);
    to_hwc(y.data() + conv * n, trans, n, tok.data());
    std::string tp = prefix + ".trans_block";
    size_t heads = wt.numel(tp + ".msa.relative_position_params") / size_t((2 * win - 1) * (2 * win - 1));
    oracle_trans_block(tok.data(), h, w, trans, win, shift, wt.get(tp + ".ln1.weight"),
                       wt.get(tp + ".ln1.bias"), wt.get(tp + ".msa.embedding_layer.weight"),
                       wt.get(tp + ".msa.embedding_layer.bias"), wt.get(tp + ".msa.linear.weight"),
                       wt.get(tp + ".msa.linear.bias"), wt.get(tp + ".msa.relative_position_params"),
                       heads, wt.get(tp + ".ln2.weight"), wt.get(tp + ".ln2.bias"),
                       wt.get(tp + ".mlp.0.weight"), wt.get(tp + ".mlp.0.bias"),
                       wt.get(tp + ".mlp.2.weight"), wt.get(tp + ".mlp.2.bias"), bt.data(),
                       dump ? dump->msa : nullptr);
    from_hwc(bt.data(), trans, n, y.data() + conv * n);
    if (dump && dump->trans_half) std::memcpy(dump->trans_half, y.data() + conv * n, trans * n * 4);
    conv1x1(y.data(), c, c, n, wt.get(prefix + ".conv1_2.weight"), wt.get(prefix + ".conv1_2.bias"),
            proj.data());
    if (dump && dump->res) std::memcpy(dump->res, proj.data(), c * n * 4);
}

const char* STAGE_NAMES[7] = {"down1", "down2", "down3", "body", "up3", "up2", "up1"};

thread_local std::string g_error;

template <typename F>
int guarded(F&& f) {
    g_error.clear();
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}

void conv_trans_block_impl(const oracle_weights* ow, const char* prefix, const float* x, size_t h,
                           size_t w, size_t shift, float* out, float* expand, float* conv_half,
                           float* trans_half, float* msa, float* res);
void forward_dump_impl(const oracle_weights* ow, const float* x, size_t hp, size_t wp,
                       float* out_final, oracle_hook hook, void* user);

}  // namespace

extern "C" {

// cpu.rs:976-983 (conv_trans_block) with the interior dump of cpu.rs:1000-1081.
// Any of the dump pointers may be NULL.
// Errors (a missing weight) return 1 with the message in oracle_last_error(): the oracle
// shares its process with the GPU test session, which one bad input must not end.
int oracle_conv_trans_block(const oracle_weights* ow, const char* prefix, const float* x,
                            size_t h, size_t w, size_t shift, float* out, float* expand,
                            float* conv_half, float* trans_half, float* msa, float* res) {
    return guarded([&] { conv_trans_block_impl(ow, prefix, x, h, w, shift, out, expand, conv_half,
                                                trans_half, msa, res); });
}

int oracle_forward_dump(const oracle_weights* ow, const float* x, size_t hp, size_t wp,
                        float* out_final, oracle_hook hook, void* user) {
    return guarded([&] { forward_dump_impl(ow, x, hp, wp, out_final, hook, user); });
}

const char* oracle_last_error(void) { return g_error.c_str(); }

}  // extern "C"

namespace {

void conv_trans_block_impl(const oracle_weights* ow, const char* prefix, const float* x, size_t h,
                           size_t w, size_t shift, float* out, float* expand, float* conv_half,
                           float* trans_half, float* msa, float* res) {
    Weights wt = make_weights(ow);
    auto dims = wt.block_dims(prefix);
    size_t c = dims.first + dims.second, n = h * w;
    std::vector<float> proj;
    BlockDump d{expand, conv_half, trans_half, msa, res};
    block_project(x, dims, h, w, size_t(wt.window), shift, wt, prefix, proj, &d);
    std::memcpy(out, x, c * n * 4);
    add_into(proj.data(), out, c * n);
}

// cpu.rs:1175-1321: the walker with the 16-name stage hook. `x` is the padded
// [in_nc][hp][wp] plane; `out` receives [in_nc][hp][wp].
void forward_dump_impl(const oracle_weights* ow, const float* x, size_t hp, size_t wp,
                       float* out_final, oracle_hook hook, void* user) {
    Weights wt = make_weights(ow);
    size_t dim = size_t(wt.dim), in_nc = size_t(wt.in_nc), win = size_t(wt.window);
    size_t n = hp * wp;
    auto f = [&](const std::string& name, const std::vector<float>& v) {
        if (hook) hook(name.c_str(), v.data(), v.size(), user);
    };
    std::vector<float> cur(dim * n);
    conv3x3(x, in_nc, dim, hp, wp, wt.get("m_head.0.weight"), cur.data());
    f("m_head", cur);
    std::vector<std::vector<float>> skips;
    size_t hh = hp, ww = wp;
    std::vector<float> proj;
    for (int k = 0; k < 3; ++k) {
        std::string name = STAGE_NAMES[k];
        int count = wt.config[k];
        size_t width = 2 * wt.block_dims("m_" + name + ".0").first;
        for (int i = 0; i < count; ++i) {
            std::string prefix = "m_" + name + "." + std::to_string(i);
            auto dims = wt.block_dims(prefix);
            block_project(cur.data(), dims, hh, ww, win, (i % 2 == 1) ? win / 2 : 0, wt, prefix,
                          proj, nullptr);
            add_into(proj.data(), cur.data(), cur.size());
        }
        size_t oh = hh / 2, ow2 = ww / 2, out_w = 2 * width;
        std::vector<float> down(out_w * oh * ow2);
        conv2x2s2(cur.data(), width, out_w, hh, ww,
                  wt.get("m_" + name + "." + std::to_string(count) + ".weight"), down.data());
        f("m_" + name + "_blocks", cur);
        f("m_" + name, down);
        skips.push_back(down);
        cur = std::move(down);
        hh = oh;
        ww = ow2;
    }
    for (int i = 0; i < wt.config[3]; ++i) {
        std::string prefix = "m_body." + std::to_string(i);
        auto dims = wt.block_dims(prefix);
        block_project(cur.data(), dims, hh, ww, win, (i % 2 == 1) ? win / 2 : 0, wt, prefix, proj,
                      nullptr);
        add_into(proj.data(), cur.data(), cur.size());
    }
    f("m_body", cur);
    for (int k = 0; k < 3; ++k) {
        std::string name = STAGE_NAMES[4 + k];
        int count = wt.config[4 + k];
        auto d1 = wt.block_dims("m_" + name + ".1");
        size_t co = d1.first + d1.second, ci = 2 * co;
        std::vector<float> skip = std::move(skips.back());
        skips.pop_back();
        add_into(skip.data(), cur.data(), cur.size());
        size_t nh = hh * 2, nw = ww * 2;
        std::vector<float> up(co * nh * nw);
        conv_t2x2(cur.data(), ci, co, hh, ww, wt.get("m_" + name + ".0.weight"), up.data());
        f("m_" + name + "_up", up);
        cur = std::move(up);
        for (int i = 0; i < count; ++i) {
            std::string prefix = "m_" + name + "." + std::to_string(i + 1);
            auto dims = wt.block_dims(prefix);
            block_project(cur.data(), dims, nh, nw, win, (i % 2 == 1) ? win / 2 : 0, wt, prefix,
                          proj, nullptr);
            add_into(proj.data(), cur.data(), cur.size());
        }
        f("m_" + name, cur);
        hh = nh;
        ww = nw;
    }
    std::vector<float> head(dim * n);
    conv3x3(x, in_nc, dim, hp, wp, wt.get("m_head.0.weight"), head.data());
    add_into(head.data(), cur.data(), cur.size());
    f("m_tail_in", cur);
    std::vector<float> out(in_nc * n);
    conv3x3(cur.data(), dim, in_nc, hp, wp, wt.get("m_tail.0.weight"), out.data());
    f("m_tail", out);
    std::memcpy(out_final, out.data(), out.size() * 4);
}

}  // namespace
