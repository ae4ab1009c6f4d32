// Launchers for the gfx950 kernels (kernels.hip). Host code only sees these.
//
// Activation layout on the device is pixel-major ("NHWC"): element (pixel p, channel c)
// of a plane with row stride ld lives at base[p * ld + c], p = y * W + x.
// Several images are one plane stacked along y: image b owns rows [b img_h, (b + 1) img_h).
// The spatial kernels (3x3 convolutions, windows, head, tail) take img_h and treat each
// image's edges as plane edges; per-pixel kernels and the 2x2 convolutions need nothing
// (img_h is even at every level, so 2x2 pairs never straddle two images). A block's
// conv half and transformer half are the column ranges [0, t) and [t, 2t) of one
// [P][2t] buffer, so the split and the concatenation of the reference
// (cpu.rs:867-868) cost nothing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace scunet {

// The fp16-operand mode. Matrix weights are kept a second time as fp16, rows [rows][K]
// (K a multiple of 32) with k permuted inside each block of 32: position 32b + 8g + j holds
// k = 32b + 4g + j for j < 4 and k = 32b + 16 + 4g + (j - 4) for j >= 4 (g = 0..3). That is
// the order in which the kernels' f16 products consume k (each lane packs the 4 consecutive
// k of two adjacent 16-wide k groups), so a lane's 8 operand halves are one 16-byte load.
// Non-null h* pointers in the argument structs below select a kernel's fp16 path.
using half_t = _Float16;
void h16_permute(const float* src, half_t* dst, long rows, int K, hipStream_t s);

// The split-operand fp32 products (the default fp32 mode where a kernel has them): an fp32
// weight is kept as three bf16 parts h + m + l equal to it exactly, in three planes of the
// fp16 copy's layout and k permutation, plane p at element offset p * rows * K. Each product
// is formed from the six part products larger than 2^-25 |ab| on the bf16 matrix cores with
// fp32 accumulation (the kernels split their activation operand the same way in registers).
// Non-null x* / WX pointers in the argument structs below select a kernel's split path.
using bf16_t = __bf16;
void x6_permute(const float* src, bf16_t* dst, long rows, int K, hipStream_t s);

// A-operand loaders of the GEMM.
enum GemmA {
    A_ROWS = 0,   // A[m][k] = A[m*lda + k]
    A_LN = 1,     // LayerNorm(A row)[k] (eps 1e-5, gamma/beta), K = the row width (<= 256)
    A_S2D = 2,    // 2x2 stride-2 patches: A[m][tap*cin + ci] = in[(2y+ky, 2x+kx)][ci]
    A_ADD2 = 3,   // A[m][k] = A[m*lda + k] + A2[m*lda + k] (the skip join before an up-conv)
};
// Epilogues (bias is always added; out = sum_k A[m][k] W[n][k] + bias[n]).
enum GemmE {
    E_STORE = 0,  // C[m*ldc + n] = out
    E_DUAL = 1,   // C and C2 both (the down-conv output that is also the stage skip)
    E_GELU = 2,   // C = gelu_erf(out)
    E_RESID = 3,  // C[m*ldc + n] = R[m*ldr + n] + out (C may equal R: in place)
    E_D2S = 4,    // 2x2 transposed conv: n = tap*cout + co -> out pixel (2i+dy, 2j+dx)
};

struct GemmArgs {
    const float* A = nullptr;
    const float* A2 = nullptr;
    long lda = 0;
    const float* W = nullptr;      // [N][K] row-major
    const float* bias = nullptr;   // [N] or null
    const float* ln_g = nullptr;
    const float* ln_b = nullptr;
    float* C = nullptr;
    float* C2 = nullptr;
    long ldc = 0;
    const float* R = nullptr;
    long ldr = 0;
    long M = 0;
    int N = 0, K = 0;
    int in_w = 0;   // A_S2D: input plane width; E_D2S: input plane width
    int cin = 0;    // A_S2D
    int cout = 0;   // E_D2S
    int persistent = 1;   // the persistent tile walker for non-LN operands (0: one tile per workgroup)
    // fp16 mode: W k-permuted. Used by the persistent walker for N % 64 == 0, K % 32 == 0 and
    // the row, patch and skip-sum operands; other shapes keep fp32 products.
    const half_t* W16 = nullptr;
    // Split-operand fp32 products: W as three k-permuted bf16 planes (N * K elements apart),
    // same shape conditions as W16.
    const bf16_t* WX = nullptr;
};

// Returns false (and a reason) if no tile configuration fits the shape.
bool gemm(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s, const char** why);

// A block's 1x1 convolutions over c channels (in = out = c, row stride c) with the whole
// weight matrix resident in LDS, for c in {64, 128}:
//   PC_STORE: C = A W^T + b                     (conv1_1, cpu.rs:869-872)
//   PC_RESID: C = R + A W^T + b                 (conv1_2 + the block residual, cpu.rs:960-968)
//   PC_CHAIN: C = R + A W^T + b, then C2 = C W1^T + b1: one block's conv1_2 and residual
//             followed by the next block's conv1_1, without the block output leaving the CU.
// In place is allowed (C == R, C2 == A): every row is read and written by one wave only.
enum PconvMode { PC_STORE = 0, PC_RESID = 1, PC_CHAIN = 2 };
struct PconvArgs {
    const float* A = nullptr;
    const float* W = nullptr;      // [c][c]
    const float* b = nullptr;      // [c]
    const float* R = nullptr;
    float* C = nullptr;
    const float* W1 = nullptr;     // PC_CHAIN: [c][c]
    const float* b1 = nullptr;
    float* C2 = nullptr;
    long M = 0;
    int c = 0;
    int h16 = 0;                   // fp16 MFMA operands (fp32 accumulation)
    // Split-operand products: W (and W1) as three bf16 planes (c * c elements apart). The
    // chained form at c = 128 has no split configuration (its six planes exceed the LDS).
    const bf16_t* x = nullptr;
    const bf16_t* x1 = nullptr;
};
// False (and a reason) for channel counts without a resident-weight configuration.
bool pconv_supported(int c);
bool pconv(const PconvArgs& a, PconvMode mode, hipStream_t s, const char** why);

// The transformer half's MLP with its pre-norm and residual, fused (cpu.rs:800-860):
// x[m] += W2 gelu(W0 LN(x[m]) + b0) + b2 for each row m of a [M][ldx] plane with t = T
// columns. The 4t-wide hidden layer never leaves the CU.
struct MlpArgs {
    float* x = nullptr;
    long ldx = 0;
    const float* ln_g = nullptr;
    const float* ln_b = nullptr;
    const float* w0 = nullptr;     // [4t][t]
    const float* b0 = nullptr;     // [4t]
    const float* w2 = nullptr;     // [t][4t]
    const float* b2 = nullptr;     // [t]
    const half_t* h0 = nullptr;    // fp16 mode: W0, W2 k-permuted
    const half_t* h2 = nullptr;
    const bf16_t* x0 = nullptr;    // split products (t = 128, 256): W0, W2 as three planes each
    const bf16_t* x2 = nullptr;
    const float* gelu = nullptr;   // the GELU table (build_gelu_table), GELU_TABLE floats
    long M = 0;
    int t = 0;
};
bool mlp(const MlpArgs& a, hipStream_t s, const char** why);

// GELU as the fused kernels evaluate it: Phi(v) = (1 + erf(v / sqrt 2)) / 2 with the
// reference's Abramowitz & Stegun 7.1.26 erf (cpu.rs:318-332), tabulated in double on the
// host as GELU_PIECES cubic pieces of width 1/16 over [-6, 6) (coefficients a, b, c, d of
// a + f (b + f (c + f d)), f the position in the piece), and gelu(v) = v Phi(v) with the
// argument clamped to the table (Phi is within 1e-9 of 0 or 1 outside it). The table holds
// the A&S function to 2e-8 of Phi; evaluated in fp32 the result is within 1.7e-7 |v| of the
// A&S GELU. It replaces the fp32 A&S evaluation (two transcendental instructions and a
// dozen VALU ones) by a 16-byte LDS read and a cubic: on gfx950 VALU work delays the fp32
// matrix products it is interleaved with, and it bounds the fp16-mode window kernels.
constexpr int GELU_PIECES = 192;
constexpr int GELU_TABLE = 4 * GELU_PIECES;
void build_gelu_table(float* tab);

struct Conv3Args {
    const float* in = nullptr;
    long ldi = 0;                  // channels [0, cin) of a [P][ldi] plane
    const float* w = nullptr;      // repacked [9][cout][cin]
    float* out = nullptr;
    long ldo = 0;
    int H = 0, W = 0, cin = 0, cout = 0;
    int img_h = 0;                 // rows per image (0: the whole plane is one image)
    int cblock = 0;                // Winograd: output channels per unit (0 = 32 below 256 input channels, else 16; 16)
    int pair = 0;                  // Winograd, 16-channel units: 0 = 8 x 16 pair units when they take fewer rounds, 1 = always
    const half_t* w16 = nullptr;   // fp16 mode: [9][cout][cin] k-permuted (conv3x3_h16)
    const float* w8 = nullptr;     // Winograd: U as [cin / 8][16][cout][8] (k_wino3; null: not used)
    int wino3 = 1;                 // Winograd: 1 k_wino3 at >= 64 channels; 0 the 32-bit-offset forms
                                   // where the plane allows; 2 k_wino3 everywhere
    int split = 0;                 // Winograd at cin = cout = 32: split-operand products (k_wino6)
};
// relu=true: out = relu(conv); relu=false: out += conv (the conv half's residual).
bool conv3x3(const Conv3Args& a, bool relu, hipStream_t s, const char** why);
// The same convolution by Winograd F(2x2, 3x3); a.w is the transformed filter
// U = G g G^T laid out [16][cout][cin] (see winograd_filter). cin, cout multiples of 16.
bool conv3x3_winograd(const Conv3Args& a, bool relu, hipStream_t s, const char** why);
// Whether conv3x3_winograd runs `a` with split-operand products (k_wino6).
bool conv3x3_winograd_split(const Conv3Args& a);
// The fp16-operand direct convolution, cin = cout in {32, 64, 128, 256}; a.w16 holds the
// filters [9][cout][cin] k-permuted (a.w is not read).
bool conv3x3_h16(const Conv3Args& a, bool relu, hipStream_t s, const char** why);
// Host-side filter transform: g [cout][cin][3][3] -> U [16][cout][cin] (in double).
void winograd_filter(const float* g, int cout, int cin, float* u);
// U [16][cout][cin] -> [cin / 8][16][cout][8] (cin a multiple of 8), k_wino3's layout.
void winograd_filter_slices(const float* u, int cout, int cin, float* u8);

struct AttnArgs {
    const float* qkv = nullptr;    // rows of [q | k | v], each C wide
    long ldq = 0;
    float* out = nullptr;          // rows of C
    long ldo = 0;
    const float* tab = nullptr;    // [heads][15][15] from build_attn_table
    int C = 0, heads = 0;
    int nwh = 0, nww = 0;          // window grid
    int H = 0, W = 0;              // plane (pixel mode)
    int shift = 0;
    int pixel_mode = 1;            // 1: rows are pixels y*W+x; 0: rows are window*64+token
    float scale = 0.f;
    int wide = 0;                  // 1: 64-bit element offsets even where 32-bit ones would do
    int qsplit = 0;                // query parts per (window, head): 0 automatic, 1 or 2
    int split = 0;                 // 1: split-operand products (the default fp32 mode)
};
// 8x8 windows, head_dim 32, at most 8 heads.
bool attention(const AttnArgs& a, hipStream_t s, const char** why);

// The whole window-attention half of a Swin block, fused per window (cpu.rs:791-799):
// x += proj(attention(qkv(LN1(x)))) + proj bias, x being the [P][ldx] token plane with
// t = T columns. q/k/v, the logits and the attention output never leave the CU.
struct MsaArgs {
    float* x = nullptr;
    long ldx = 0;
    const float* ln_g = nullptr;
    const float* ln_b = nullptr;
    const float* wqkv = nullptr;   // [3t][t]
    const float* bqkv = nullptr;   // [3t]
    const float* wp = nullptr;     // [t][t]
    const float* bp = nullptr;     // [t]
    const float* tab = nullptr;    // [heads][64][64] lane-ordered rel-pos bias
    // Optional: the MLP with its pre-norm and residual (as MlpArgs), applied to the
    // window's tokens after the attention residual, in the same kernel (w0 != null).
    const float* ln2_g = nullptr;
    const float* ln2_b = nullptr;
    const float* w0 = nullptr;     // [4t][t]
    const float* b0 = nullptr;
    const float* w2 = nullptr;     // [t][4t]
    const float* b2 = nullptr;
    // fp16 mode: the k-permuted weights (hqkv, hp always; h0, h2 with the MLP option).
    const half_t* hqkv = nullptr;
    const half_t* hp = nullptr;
    const half_t* h0 = nullptr;
    const half_t* h2 = nullptr;
    // Split-operand products: the same weights as three bf16 planes each (xqkv, xp always;
    // x0, x2 with the MLP option).
    const bf16_t* xqkv = nullptr;
    const bf16_t* xp = nullptr;
    const bf16_t* x0 = nullptr;
    const bf16_t* x2 = nullptr;
    const float* gelu = nullptr;   // with the MLP option: the GELU table (build_gelu_table)
    int t = 0;
    int nwh = 0, nww = 0, H = 0, W = 0, shift = 0;   // nwh, H: one image's window rows and rows
    int nimg = 1;                                     // images stacked along y
    float scale = 0.f;
};
// t = 32 (one wave per window, all heads) or 64, 128, 256 (one workgroup per window, one
// wave per head); false otherwise. The MLP option is available at t = 32, 64.
bool msa_fused(const MsaArgs& a, hipStream_t s, const char** why);
// Host-side construction of the lane-ordered bias table from rp [heads][15][15].
void build_bias_table(const float* rp, int heads, float* tab);
// The attention kernel's table: rp [heads][15][15] scaled by log2(e).
void build_attn_table(const float* rp, int heads, float* tab);

// m_head (in_nc -> dim, 3x3, zero pad) reading an NCHW image of size hh x ww that is
// replicate-padded on the fly to H x W; writes (or, with add, accumulates into) the
// pixel-major [H*W][dim] plane.
// With nimg > 1, x holds nimg such images back to back and out their stacked planes.
bool head_conv(const float* x, int cin, int hh, int ww, int H, int W, const float* w, int dim,
               float* out, bool add, hipStream_t s, int nimg = 1);
// m_tail (dim -> cout, 3x3, zero pad) from pixel-major [H*W][dim] into NCHW [cout][oh][ow]
// for the top-left oh x ow corner (oh <= H, ow <= W: the crop is fused).
// With nimg > 1, in holds nimg stacked H x W planes and out nimg [cout][oh][ow] images.
// split: the products on the bf16 matrix cores from split operands (k_tail6); else fp32 FMAs.
bool tail_conv(const float* in, int dim, int H, int W, const float* w, int cout, float* out,
               int oh, int ow, hipStream_t s, int nimg = 1, bool split = false);

// A streaming copy of n float4 (the counter-calibration kernel).
void copy_f4(const void* src, void* dst, long n, hipStream_t s);

// Layout changes for the host boundary, probes and stage dumps.
void nchw_to_nhwc(const float* src, float* dst, int c, long P, long ld, hipStream_t s);
void nhwc_to_nchw(const float* src, float* dst, int c, long P, long ld, hipStream_t s);
// The window index map: tok[(wi*64 + t)*c + ch] = x[pix(wi, t)*c + ch] and its inverse.
void window_gather(const float* x, float* tok, int c, int H, int W, int shift, hipStream_t s);
void window_scatter(const float* tok, float* x, int c, int H, int W, int shift, hipStream_t s);

}  // namespace scunet
