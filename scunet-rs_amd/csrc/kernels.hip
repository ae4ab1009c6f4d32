// gfx950 (MI355X, CDNA4) kernels of the SCUNet forward. All arithmetic is fp32; every
// contraction runs on the fp32 matrix cores through v_mfma_f32_16x16x4_f32.
//
// MFMA 16x16x4 f32 operand/result layout (wave64, lane l, li = l % 16, lg = l / 16):
//   A operand: lane holds A[li][lg]       (16 x 4)
//   B operand: lane holds B[lg][li]       (4 x 16)
//   C/D      : lane holds C[4*lg + r][li] for r = 0..3 (4 accumulator registers)
// The K order inside a 16-wide slice is permuted so that each lane fetches 4
// consecutive k values with one 16-byte load: at MFMA step s the lane with group lg
// supplies k = 16*kk + 4*lg + s for both operands. Any K permutation is valid as long
// as A and B agree on it.
#include "kernels.h"

#include <atomic>
#include <type_traits>

#include <algorithm>
#include <cmath>
#include <cstdint>

namespace scunet {

typedef float f4 __attribute__((ext_vector_type(4)));

#define DEVI __device__ __forceinline__

DEVI f4 mfma4(float a, float b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// The 16-bit operand mode: v_mfma_f32_16x16x32_f16 (fp16 operands, fp32 accumulation),
// lane l supplying A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16], j = 0..7 (checked
// on the device). The fp32 kernels hand each lane 4 consecutive k of a 16-wide k group
// (k = 16 kg + 4 lg + s); one f16 product takes the lane's float4s of two adjacent groups
// 2kk and 2kk + 1, i.e. k = 32 kk + {4 lg .. 4 lg + 3} u {16 + 4 lg .. 16 + 4 lg + 3}. Both
// operands see the same permutation of k, so the sum is unchanged, and an accumulator
// (4 consecutive output channels per lane) is already the next product's operand.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
DEVI h8 pack8(f4 lo, f4 hi) {
    return h8{(_Float16)lo.x, (_Float16)lo.y, (_Float16)lo.z, (_Float16)lo.w,
              (_Float16)hi.x, (_Float16)hi.y, (_Float16)hi.z, (_Float16)hi.w};
}
DEVI f4 mfma16(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
DEVI h8 ldh8(const _Float16* p) { return *reinterpret_cast<const h8*>(p); }
DEVI void sth8(_Float16* p, h8 v) { *reinterpret_cast<h8*>(p) = v; }

// Split-operand fp32 products on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, the same
// lane layout as the f16 product above). An fp32 value x is carried as three bf16 parts with
// h + m + l == x exactly: h = rne(x), m = rne(x - h), l = x - h - m (both differences are
// exact in fp32, and l has at most 8 significant bits). A product ab is then the sum of the
// six part products whose size can exceed 2^-24 |ab|: hh + hm + mh + hl + lh + mm; the three
// dropped (ml, lm, ll) are below 2^-25 |ab| together, under fp32's own rounding of one
// product, and every part product is exact in the fp32 accumulator's input. Operands that
// are weights are split once at upload (x6_permute); activations are split in registers.
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef short s8v __attribute__((ext_vector_type(8)));
struct x8 {
    b8 h, m, l;
};
DEVI f4 mfmab(b8 a, b8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
// Two floats -> their rne bf16 parts packed in one register, and the exact remainders.
// Default form: each part unpacked by a shift or mask, then subtracted (five instructions a
// pair). DOT form (three a pair): each remainder is one v_dot2c_f32_bf16, x - h as the dot of
// the packed parts with (-1, 0) or (0, -1) accumulated onto x; both products are exact and
// x - h is representable, so the sum is exact, bit-equal to the default form for normal
// values (denormal inputs may be flushed). The DOT form is used where it measured faster:
// the level-0 split Winograd and the resident-weight 1x1. In the window, MLP and tile-GEMM
// kernels it measured slower, with more registers or spills, and they keep the default.
template <bool DOT = false>
DEVI unsigned split2(float& x0, float& x1) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    typedef float fl2 __attribute__((ext_vector_type(2)));
    const b2 p = __builtin_convertvector(fl2{x0, x1}, b2);
    if (DOT) {
        // The (-1, 0) pair goes in through an SGPR: the compiler encodes it as the inline
        // constant -1.0, which this operand does not read as that pair.
        unsigned c0 = 0x0000bf80u, c1 = 0xbf800000u;
        asm("" : "+s"(c0), "+s"(c1));
        x0 = __builtin_amdgcn_fdot2_f32_bf16(p, __builtin_bit_cast(b2, c0), x0, false);
        x1 = __builtin_amdgcn_fdot2_f32_bf16(p, __builtin_bit_cast(b2, c1), x1, false);
        return __builtin_bit_cast(unsigned, p);
    }
    const unsigned u = __builtin_bit_cast(unsigned, p);
    x0 -= __builtin_bit_cast(float, u << 16);
    x1 -= __builtin_bit_cast(float, u & 0xffff0000u);
    return u;
}
DEVI unsigned pack2(float x0, float x1) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    typedef float fl2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(unsigned, __builtin_convertvector(fl2{x0, x1}, b2));
}
// The lane's 8 k values (the f4s of two adjacent k groups, as pack8) in split form.
template <bool DOT = false>
DEVI x8 split8(f4 lo, f4 hi) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    u4 H, M, L;
#pragma unroll
    for (int i = 0; i < 4; ++i) H[i] = split2<DOT>(v[2 * i], v[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) M[i] = split2<DOT>(v[2 * i], v[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) L[i] = pack2(v[2 * i], v[2 * i + 1]);
    return x8{__builtin_bit_cast(b8, H), __builtin_bit_cast(b8, M), __builtin_bit_cast(b8, L)};
}
// c += a b over the lane's 8 k values, a and b in split form (smallest terms first).
DEVI f4 mfma6(const x8& a, const x8& b, f4 c) {
    c = mfmab(a.l, b.h, c);
    c = mfmab(a.h, b.l, c);
    c = mfmab(a.m, b.m, c);
    c = mfmab(a.m, b.h, c);
    c = mfmab(a.h, b.m, c);
    return mfmab(a.h, b.h, c);
}
DEVI b8 ldb8(const __bf16* p) { return *reinterpret_cast<const b8*>(p); }
DEVI void stb8(__bf16* p, b8 v) { *reinterpret_cast<b8*>(p) = v; }
// The three parts of a split weight fragment: part planes `ps` elements apart.
DEVI x8 ldx8(const __bf16* p, long ps) { return x8{ldb8(p), ldb8(p + ps), ldb8(p + 2 * ps)}; }

DEVI f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
// LDS row pitches: a wave's 16-byte LDS reads are conflict-free when, within each 32-lane
// half, the 16-byte slot indices are distinct mod 32. The MFMA operand reads here have
// lane li (0..15) on a row and lane group lg (0..1 per half) on 4 consecutive floats of
// it, so a row pitch of P floats is conflict-free when P = 8 (mod 16) (P/4 twice an odd
// number). Pitches below are the row width + 8 for that reason.
DEVI void st4(float* p, f4 v) { *reinterpret_cast<f4*>(p) = v; }

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on XCD b % 8),
// and each XCD has its own L2. Remap so every XCD processes one contiguous range of
// logical tiles: tiles that share an input (the N-blocks of one M-tile, neighbouring
// spatial tiles) then meet in the same L2.
DEVI long xcd_swizzle(long b, long nb) {
    long q = nb >> 3, r = nb & 7;
    long xcd = b & 7, j = b >> 3;
    long start = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
    return start + j;
}

// GELU with the Abramowitz & Stegun 7.1.26 erf the reference's CPU path uses
// (cpu.rs:293-332), evaluated in fp32 (|erf error| < 1.5e-7 + fp32 rounding).
// With x = v/sqrt(2), t = 1/(1 + p|x|) and q = 0.5 t poly(t) e^(-x^2) (so that
// erf(|x|) = 1 - 2q), gelu(v) = 0.5 v (1 + erf(x)) is v - v q for v >= 0 and v q for v < 0,
// i.e. max(v, 0) - |v| q in both cases. The 1/sqrt(2) is folded into p and into the
// exponent's constant (e^(-v^2/2) = 2^(-v^2 log2(e)/2)), the 0.5 into the coefficients.
DEVI float gelu_as(float v) {
    const float av = fabsf(v);
    // v_rcp_f32 (1 ulp) instead of an IEEE division: t enters a polynomial whose own
    // approximation error is 1.5e-7, so a 1-ulp reciprocal changes nothing measurable.
    const float t = __builtin_amdgcn_rcpf(fmaf(av, 0.3275911f * 0.70710678118654752440f, 1.0f));
    const float p = ((((0.5f * 1.061405429f) * t - 0.5f * 1.453152027f) * t + 0.5f * 1.421413741f) * t -
                     0.5f * 0.284496736f) * t + 0.5f * 0.254829592f;
    const float e = __builtin_amdgcn_exp2f(v * (v * (-0.5f * 1.4426950408889634f)));
    const float q = p * t * e;
    return fmaf(-av, q, fmaxf(v, 0.0f));
}

// The table form of the same GELU (build_gelu_table): tab is the table in LDS.
DEVI float gelu_lut(const float* tab, float v) {
    const float u = fminf(fmaxf(fmaf(v, 16.0f, 96.0f), 0.0f), 191.99998f);   // piece index + fraction
    const int i = int(u);
    const float f = __builtin_amdgcn_fractf(u);
    const f4 c = ld4(tab + 4 * i);
    return v * fmaf(fmaf(fmaf(c.w, f, c.z), f, c.y), f, c.x);
}
// A workgroup copies the table from global memory into its LDS (callers sync before use).
DEVI void load_gelu_table(float* tab, const float* g, int tid, int nthreads) {
    for (int i = tid; i < GELU_TABLE / 4; i += nthreads) st4(tab + 4 * i, ld4(g + 4 * i));
}

// ---------------------------------------------------------------------------
// GEMM: C[m][n] = epi(sum_k A[m][k] W[n][k] + bias[n]), M pixels, N and K small.
// Tile BM x BN x 32, 256 threads = 4 waves, each wave WM x WN of 16x16 MFMA tiles.
// Global -> registers (prefetch of the next K slice) -> LDS -> MFMA.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN, int AM, int EP>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g) {
    constexpr int BK = 32, LDK = BK + 4;   // +4 floats: ds_read_b128 rows hit distinct banks
    constexpr int NWN = BN / WN;
    constexpr int MT = WM / 16, NT = WN / 16;
    constexpr int AV = BM * BK / 4 / 256;  // float4 per thread per A slice
    constexpr int BV = (BN * BK / 4 + 255) / 256;
    static_assert((BM / WM) * (BN / WN) == 4, "4 waves");
    static_assert(AV >= 1, "BM too small");
    __shared__ float As[BM * LDK];
    __shared__ float Bs[BN * LDK];
    __shared__ float s_mu[AM == A_LN ? BM : 1];
    __shared__ float s_rs[AM == A_LN ? BM : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int ntn = g.N / BN;
    const long tile = xcd_swizzle(blockIdx.x, gridDim.x);
    const long m0 = (tile / ntn) * BM;
    const int n0 = int(tile % ntn) * BN;
    const int wm = wave / NWN, wn = wave % NWN;

    if constexpr (AM == A_LN) {
        // Row statistics, two-pass as cpu.rs:338-357: mu = sum/K, var = sum (x-mu)^2 / K.
        const int L = g.K >> 2;            // lanes per row (K <= 256 -> L <= 64)
        const int rpp = 64 / L;            // rows per pass
        const int per_wave = BM / 4;
        for (int base = 0; base < per_wave; base += rpp) {
            int r = wave * per_wave + base + lane / L;
            int j = lane % L;
            long gm = m0 + r;
            f4 v = {0.f, 0.f, 0.f, 0.f};
            bool ok = (base + lane / L) < per_wave && gm < g.M;
            if (ok) v = ld4(g.A + gm * g.lda + j * 4);
            float s = (v.x + v.y) + (v.z + v.w);
            for (int o = L >> 1; o > 0; o >>= 1) s += __shfl_xor(s, o);
            float mu = s / float(g.K);
            f4 d = v - mu;
            float q = (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            for (int o = L >> 1; o > 0; o >>= 1) q += __shfl_xor(q, o);
            float var = q / float(g.K);
            if (j == 0 && (base + lane / L) < per_wave) {
                s_mu[r] = mu;
                s_rs[r] = 1.0f / sqrtf(var + 1e-5f);
            }
        }
        __syncthreads();
    }

    f4 ra[AV], rb[BV];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            int f = tid + i * 256;
            int row = f >> 3, c4 = f & 7;
            long gm = m0 + row;
            int k = k0 + c4 * 4;
            f4 v = {0.f, 0.f, 0.f, 0.f};
            if (gm < g.M) {
                if constexpr (AM == A_S2D) {
                    int tap = k / g.cin, ci = k - tap * g.cin;
                    int ow = g.in_w >> 1;
                    long oy = gm / ow, ox = gm - oy * ow;
                    long ip = (2 * oy + (tap >> 1)) * long(g.in_w) + 2 * ox + (tap & 1);
                    v = ld4(g.A + ip * g.cin + ci);
                } else if constexpr (AM == A_ADD2) {
                    v = ld4(g.A + gm * g.lda + k) + ld4(g.A2 + gm * g.lda + k);
                } else {
                    v = ld4(g.A + gm * g.lda + k);
                }
            }
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            int f = tid + i * 256;
            if (f < BN * 8) {
                int row = f >> 3, c4 = f & 7;
                rb[i] = ld4(g.W + long(n0 + row) * g.K + k0 + c4 * 4);
            }
        }
    };
    auto stash = [&](int k0) {
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            int f = tid + i * 256;
            int row = f >> 3, c4 = f & 7;
            f4 v = ra[i];
            if constexpr (AM == A_LN) {
                int k = k0 + c4 * 4;
                float mu = s_mu[row], rs = s_rs[row];
                f4 gg = ld4(g.ln_g + k), bb = ld4(g.ln_b + k);
                v = (v - mu) * rs * gg + bb;
                if (m0 + row >= g.M) v = f4{0.f, 0.f, 0.f, 0.f};
            }
            st4(&As[row * LDK + c4 * 4], v);
        }
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            int f = tid + i * 256;
            if (f < BN * 8) {
                int row = f >> 3, c4 = f & 7;
                st4(&Bs[row * LDK + c4 * 4], rb[i]);
            }
        }
    };

    f4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    load(0);
    stash(0);
    __syncthreads();
    for (int k0 = 0; k0 < g.K; k0 += BK) {
        const bool more = k0 + BK < g.K;
        if (more) load(k0 + BK);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            f4 a[MT], b[NT];
#pragma unroll
            for (int i = 0; i < MT; ++i) a[i] = ld4(&As[(wm * WM + i * 16 + li) * LDK + kk * 16 + lg * 4]);
#pragma unroll
            for (int j = 0; j < NT; ++j) b[j] = ld4(&Bs[(wn * WN + j * 16 + li) * LDK + kk * 16 + lg * 4]);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < NT; ++j) acc[i][j] = mfma4(a[i][s], b[j][s], acc[i][j]);
        }
        __syncthreads();
        if (more) {
            stash(k0 + BK);
            __syncthreads();
        }
    }

    // Epilogue: lane holds rows 4*lg + r of each 16x16 tile, column li.
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int col = n0 + wn * WN + j * 16 + li;
        const float bv = g.bias ? g.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const long row = m0 + wm * WM + i * 16 + lg * 4 + r;
                if (row >= g.M) continue;
                float v = acc[i][j][r] + bv;
                if constexpr (EP == E_STORE) {
                    g.C[row * g.ldc + col] = v;
                } else if constexpr (EP == E_DUAL) {
                    g.C[row * g.ldc + col] = v;
                    g.C2[row * g.ldc + col] = v;
                } else if constexpr (EP == E_GELU) {
                    g.C[row * g.ldc + col] = gelu_as(v);
                } else if constexpr (EP == E_RESID) {
                    g.C[row * g.ldc + col] = g.R[row * g.ldr + col] + v;
                } else {  // E_D2S
                    long ii = row / g.in_w, jj = row - ii * g.in_w;
                    int tap = col / g.cout, co = col - tap * g.cout;
                    long oy = 2 * ii + (tap >> 1), ox = 2 * jj + (tap & 1);
                    g.C[(oy * 2 * g.in_w + ox) * g.cout + co] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMM, "A-direct" form: each wave owns 16*MT rows and all BN columns of its
// workgroup and loads its A fragments straight from HBM into MFMA registers (a row's
// 4 consecutive k values per lane, 64 contiguous bytes per row per instruction); only
// the weight slice [BN][KC], shared by the 4 waves, goes through LDS, double-buffered.
// The next A slice and the next weight slice are loaded while the current one is
// multiplied. LN mode (KLN = K > 0) holds the whole row in registers, normalises it
// there (two-pass, cpu.rs:338-357) and streams only the weights.
// ---------------------------------------------------------------------------
template <int MT, int BN, int KC, int AM, int EP, int KLN>
__global__ __launch_bounds__(256) void k_gemm2(GemmArgs g) {
    constexpr int NT = BN / 16, KG = KC / 16, LDB = KC + 8;
    constexpr int BV = BN * KC / 4 / 256;
    static_assert(BN * KC / 4 % 256 == 0, "weight slice must split evenly over 256 threads");
    constexpr bool LN = AM == A_LN;
    constexpr int XKG = LN ? KLN / 16 : 1;
    __shared__ float Bs[2 * BN * LDB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int ntn = g.N / BN;
    const long tile = xcd_swizzle(blockIdx.x, gridDim.x);
    const long m0 = (tile / ntn) * (64 * MT) + wave * 16 * MT;
    const int n0 = int(tile % ntn) * BN;

    auto a_addr = [&](long row, int k) -> const float* {
        if constexpr (AM == A_S2D) {
            const int tap = k / g.cin, ci = k - tap * g.cin;
            const int ow = g.in_w >> 1;
            const long oy = row / ow, ox = row - oy * ow;
            const long ip = (2 * oy + (tap >> 1)) * long(g.in_w) + 2 * ox + (tap & 1);
            return g.A + ip * g.cin + ci;
        } else {
            return g.A + row * g.lda + k;
        }
    };
    auto a_get = [&](long row, int k) -> f4 {
        if (row >= g.M) return f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (AM == A_ADD2) return ld4(g.A + row * g.lda + k) + ld4(g.A2 + row * g.lda + k);
        return ld4(a_addr(row, k));
    };

    f4 xl[LN ? MT : 1][XKG];
    if constexpr (LN) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const long r = m0 + mt * 16 + li;
#pragma unroll
            for (int kg = 0; kg < XKG; ++kg) xl[mt][kg] = a_get(r, kg * 16 + lg * 4);
            float sm = 0.f;
#pragma unroll
            for (int kg = 0; kg < XKG; ++kg) sm += (xl[mt][kg].x + xl[mt][kg].y) + (xl[mt][kg].z + xl[mt][kg].w);
            sm += __shfl_xor(sm, 16);
            sm += __shfl_xor(sm, 32);
            const float mu = sm / float(KLN);
            float q = 0.f;
#pragma unroll
            for (int kg = 0; kg < XKG; ++kg) {
                f4 d = xl[mt][kg] - mu;
                q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            }
            q += __shfl_xor(q, 16);
            q += __shfl_xor(q, 32);
            const float rs = __builtin_amdgcn_rsqf(q * (1.0f / float(KLN)) + 1e-5f);
#pragma unroll
            for (int kg = 0; kg < XKG; ++kg) {
                f4 gg = ld4(g.ln_g + kg * 16 + lg * 4), bb = ld4(g.ln_b + kg * 16 + lg * 4);
                xl[mt][kg] = (xl[mt][kg] - mu) * rs * gg + bb;
            }
        }
    }

    f4 bpre[BV];
    auto bload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            const int f = tid + i * 256;
            const int row = f / (KC / 4), c4 = f % (KC / 4);
            bpre[i] = ld4(g.W + long(n0 + row) * g.K + k0 + c4 * 4);
        }
    };
    auto bstore = [&](int b) {
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            const int f = tid + i * 256;
            const int row = f / (KC / 4), c4 = f % (KC / 4);
            st4(&Bs[b * BN * LDB + row * LDB + c4 * 4], bpre[i]);
        }
    };
    f4 acur[LN ? 1 : MT][LN ? 1 : KG], anext[LN ? 1 : MT][LN ? 1 : KG];
    auto aload = [&](int k0, f4 (&dst)[LN ? 1 : MT][LN ? 1 : KG]) {
        if constexpr (!LN) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int kg = 0; kg < KG; ++kg) dst[mt][kg] = a_get(m0 + mt * 16 + li, k0 + kg * 16 + lg * 4);
        }
    };

    f4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

    auto step = [&](int c, bool more) {
        const float* B = Bs + (c & 1) * BN * LDB;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) {
            f4 b[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) b[nt] = ld4(B + (nt * 16 + li) * LDB + kg * 16 + lg * 4);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    float av;
                    if constexpr (LN) av = xl[mt][c * KG + kg][s4];
                    else av = acur[mt][kg][s4];
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mfma4(b[nt][s4], av, acc[mt][nt]);
                }
        }
        if (more) bstore((c + 1) & 1);
        __syncthreads();
    };

    bload(0);
    bstore(0);
    aload(0, acur);
    __syncthreads();
    if constexpr (LN) {
        constexpr int NCH = KLN / KC;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (c + 1 < NCH) bload((c + 1) * KC);
            step(c, c + 1 < NCH);
        }
    } else {
        const int nch = g.K / KC;
        for (int c = 0; c < nch; ++c) {
            const bool more = c + 1 < nch;
            if (more) {
                bload((c + 1) * KC);
                aload((c + 1) * KC, anext);
            }
            step(c, more);
            if (more) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int kg = 0; kg < KG; ++kg) acur[mt][kg] = anext[mt][kg];
            }
        }
    }

    // The product was computed transposed (weights as the M rows), so each lane holds 4
    // consecutive output columns of one row: one 16-byte store per row and N tile.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int col = n0 + nt * 16 + lg * 4;
        const f4 bv = g.bias ? ld4(g.bias + col) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const long row = m0 + mt * 16 + li;
            if (row >= g.M) continue;
            f4 v = acc[mt][nt] + bv;
            if constexpr (EP == E_STORE) {
                st4(g.C + row * g.ldc + col, v);
            } else if constexpr (EP == E_DUAL) {
                st4(g.C + row * g.ldc + col, v);
                st4(g.C2 + row * g.ldc + col, v);
            } else if constexpr (EP == E_GELU) {
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = gelu_as(v[r]);
                st4(g.C + row * g.ldc + col, v);
            } else if constexpr (EP == E_RESID) {
                st4(g.C + row * g.ldc + col, ld4(g.R + row * g.ldr + col) + v);
            } else {
                const long ii = row / g.in_w, jj = row - ii * g.in_w;
                const int tap = col / g.cout, co = col - tap * g.cout;
                const long oy = 2 * ii + (tap >> 1), ox = 2 * jj + (tap & 1);
                st4(g.C + (oy * 2 * g.in_w + ox) * g.cout + co, v);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Persistent form of k_gemm2 for the row and patch (A_S2D) A operands: as
// many workgroups as fit on the chip walk the output tiles with a grid stride. In the last
// K slice of a tile the next tile's first A rows and weight slice are already loaded, and
// a residual the epilogue adds is read at the start of that slice, so neither a tile's
// start nor its epilogue waits on memory. One barrier per K slice (the weight slices are
// double-buffered in LDS; the epilogue uses registers only). Tile t = 8 j + xcd: the
// N-blocks of one M-tile are consecutive j on one XCD and share its L2.
// ---------------------------------------------------------------------------
// Widest N the persistent GEMM serves (its bias is staged in LDS): the 2x2 transposed conv
// at 256 output channels, N = 4 * 256.
constexpr int GEMM3_NMAX = 1024;
template <int MT, int BN, int KC, int AM, int EP, bool H16, bool X6 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm3(GemmArgs g, long tiles) {
    // fp16 mode: a K slice is one 32-wide k block of the k-permuted weights, staged as halves
    // with rows of 48 (2 mod 4 sixteen-byte slots: conflict-free 128-bit reads). The split
    // products (X6) stage the three bf16 part planes of the slice the same way.
    static_assert(!H16 || KC == 32, "fp16 slices are one k block");
    static_assert(!X6 || H16, "split products use the 16-bit layout");
    constexpr int NT = BN / 16, KG = KC / 16, LDB = H16 ? 48 : KC + 8;
    constexpr int EV = H16 ? 8 : 4;               // elements per 16-byte chunk
    constexpr int NP = X6 ? 3 : 1;                // weight planes
    constexpr int BV = BN * KC / EV / 256;
    static_assert(BN * KC / EV % 256 == 0, "weight slice must split evenly over 256 threads");
    // The residual is read ahead when its registers fit (up to 8 float4 per lane).
    constexpr bool RPRE = EP == E_RESID && MT * NT <= 8;
    using ET = std::conditional_t<X6, __bf16, std::conditional_t<H16, _Float16, float>>;
    __shared__ __align__(16) ET Bs[2 * NP * BN * LDB];
    // The bias of every column, staged once per (persistent) workgroup: read from global
    // memory in the epilogue, each column block's read was waited for before its stores,
    // and that wait also covered the next tile's operands, requested during the last slice.
    __shared__ __align__(16) float bsh[GEMM3_NMAX];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int ntn = g.N / BN, nch = g.K / KC;
    const long mtiles = (g.M + 64 * MT - 1) / (64 * MT);
    const long G = gridDim.x;
    // Rows of this wave in tile t (g.M when the tile is past the end: no loads, no stores).
    // Tile indices fit 32 bits (fewer than 2^31 tiles), so the divisions are 32-bit.
    auto decode = [&](long t, long& m0, int& n0) {
        const unsigned tt = unsigned(t), xcd = tt & 7u, j = tt >> 3;
        const unsigned q = j / unsigned(ntn), mt = q * 8u + xcd;
        n0 = int(j - q * unsigned(ntn)) * BN;
        m0 = long(mt) < mtiles ? long(mt) * 64 * MT + wave * 16 * MT : g.M;
    };
    // The patch operand (A_S2D) finds its 2x2 input patch per load. (Patch bases kept per
    // tile, with the tap per slice, measured slower at level 0 of the forward: 300 against
    // 270 us, though faster at level 2.)
    // Rows past the end read row M - 1 and are replaced by zeros (no load under a branch).
    auto a_get = [&](long row, int k) -> f4 {
        const long rc = row < g.M ? row : g.M - 1;
        f4 v;
        if constexpr (AM == A_S2D) {
            const int tap = k / g.cin, ci = k - tap * g.cin;
            const int ow = g.in_w >> 1;
            const long oy = rc / ow, ox = rc - oy * ow;
            const long ip = (2 * oy + (tap >> 1)) * long(g.in_w) + 2 * ox + (tap & 1);
            v = ld4(g.A + ip * g.cin + ci);
        } else {
            v = ld4(g.A + rc * g.lda + k);
        }
        return row < g.M ? v : f4{0.f, 0.f, 0.f, 0.f};
    };
    f4 bpre[NP * BV];
    const long wps = long(g.N) * g.K;   // X6: part plane stride
    auto bload = [&](int n0, int k0) {
#pragma unroll
        for (int i = 0; i < BV; ++i) {
            const int f = tid + i * 256;
            const int row = f / (KC / EV), c = f % (KC / EV);
            if constexpr (X6) {
#pragma unroll
                for (int p = 0; p < NP; ++p)
                    bpre[p * BV + i] = ld4(reinterpret_cast<const float*>(g.WX + p * wps + long(n0 + row) * g.K + k0 + c * 8));
            } else if constexpr (H16) {
                bpre[i] = ld4(reinterpret_cast<const float*>(g.W16 + long(n0 + row) * g.K + k0 + c * 8));
            } else {
                bpre[i] = ld4(g.W + long(n0 + row) * g.K + k0 + c * 4);
            }
        }
    };
    auto bstore = [&](int b) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int i = 0; i < BV; ++i) {
                const int f = tid + i * 256;
                const int row = f / (KC / EV), c = f % (KC / EV);
                st4(reinterpret_cast<float*>(&Bs[(b * NP + p) * BN * LDB + row * LDB + c * EV]), bpre[p * BV + i]);
            }
    };
    // The skip-sum operand (A_ADD2) keeps its two loads apart until the slice is used, so the
    // sum does not wait on memory where the loads are issued; its rows past the end read row
    // M - 1 (their products only reach output rows that are not stored).
    constexpr int A2N = AM == A_ADD2 ? MT : 1;
    f4 acur[MT][KG], anext[MT][KG], anext2[A2N][KG];
    auto aload = [&](long m0, int k0, f4 (&dst)[MT][KG]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                if constexpr (AM == A_ADD2) {
                    const long row = m0 + mt * 16 + li < g.M ? m0 + mt * 16 + li : g.M - 1;
                    const int k = k0 + kg * 16 + lg * 4;
                    dst[mt][kg] = ld4(g.A + row * g.lda + k);
                    anext2[mt][kg] = ld4(g.A2 + row * g.lda + k);
                } else {
                    dst[mt][kg] = a_get(m0 + mt * 16 + li, k0 + kg * 16 + lg * 4);
                }
            }
    };
    f4 acc[MT][NT], res[MT][NT];

    long t = blockIdx.x;
    if (t >= tiles) return;
    long m0;
    int n0;
    decode(t, m0, n0);
    bload(n0, 0);
    aload(m0, 0, acur);
    if constexpr (AM == A_ADD2) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) acur[mt][kg] += anext2[mt][kg];
    }
    bstore(0);
    for (int i = tid; i < g.N; i += 256) bsh[i] = g.bias ? g.bias[i] : 0.0f;
    // The first tile's rows arrive before the loop: with loads still pending on its entry
    // edge, every slice would wait for its own prefetch before its products.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int kb = 0;
    for (;;) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
        const long tn = t + G;
        long m0n = g.M;
        int n0n = 0;
        if (tn < tiles) decode(tn, m0n, n0n);
        for (int c = 0; c < nch; ++c) {
            const bool last = c + 1 == nch;
            const bool more = !last || tn < tiles;
            // The next slice (the next tile's first at the last slice) is requested on every
            // path, past the last tile too (then column block 0's weights and rows past the
            // end, unused): with loads on some paths only, the wait before the products
            // would have to cover the loads just issued.
            bload(last ? n0n : n0, last ? 0 : (c + 1) * KC);
            aload(last ? m0n : m0, last ? 0 : (c + 1) * KC, anext);
            // ... and kept here, ahead of the products (the scheduler would otherwise sink
            // them next to their LDS stores at the end of the slice).
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (RPRE) {
                if (last) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const long row = m0 + mt * 16 + li < g.M ? m0 + mt * 16 + li : g.M - 1;
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt) res[mt][nt] = ld4(g.R + row * g.ldr + n0 + nt * 16 + lg * 4);
                    }
                }
            }
            const ET* B = Bs + kb * NP * BN * LDB;
            if constexpr (X6) {
                x8 ap[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) ap[mt] = split8(acur[mt][0], acur[mt][1]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const x8 bx = ldx8(B + (nt * 16 + li) * LDB + lg * 8, BN * LDB);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma6(bx, ap[mt], acc[mt][nt]);
                }
            } else if constexpr (H16) {
                h8 ap[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) ap[mt] = pack8(acur[mt][0], acur[mt][1]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const h8 bh = ldh8(B + (nt * 16 + li) * LDB + lg * 8);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma16(bh, ap[mt], acc[mt][nt]);
                }
            } else {
#pragma unroll
                for (int kg = 0; kg < KG; ++kg) {
                    f4 b[NT];
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) b[nt] = ld4(B + (nt * 16 + li) * LDB + kg * 16 + lg * 4);
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                            for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mfma4(b[nt][s4], acur[mt][kg][s4], acc[mt][nt]);
                }
            }
            if (more) bstore(kb ^ 1);
            __syncthreads();
            kb ^= 1;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int kg = 0; kg < KG; ++kg) {
                    if constexpr (AM == A_ADD2) acur[mt][kg] = anext[mt][kg] + anext2[mt][kg];
                    else acur[mt][kg] = anext[mt][kg];
                }
        }
        // Epilogue: each lane holds 4 consecutive output columns of one row. The bias and the
        // read-ahead residual are added for every row before the row bound is tested: a load
        // still pending after a skipped branch would make the next tile's slice loop wait on
        // every slice (the wait analysis is conservative across the loop head). The
        // depth-to-space form finds its output pixels once per row (a 32-bit division while
        // the rows fit) and steps (tap, co) through the 16-column blocks (cout is a multiple
        // of 16, so no block straddles two taps).
        long d2s_px[MT];
        int tap = 0, co = 0;
        // A residual not read ahead is read for the whole tile before the first store (rows
        // clamped), so its reads are in flight together.
        constexpr bool RLATE = EP == E_RESID && !RPRE && AM == A_ROWS;
        f4 rl[RLATE ? MT : 1][RLATE ? NT : 1];
        if constexpr (RLATE) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const long row = m0 + mt * 16 + li < g.M ? m0 + mt * 16 + li : g.M - 1;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) rl[mt][nt] = ld4(g.R + row * g.ldr + n0 + nt * 16 + lg * 4);
            }
        }
        if constexpr (EP == E_D2S) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const long row = m0 + mt * 16 + li;
                long ii, jj;
                if (g.M <= 0xffffffffL) {
                    const unsigned q = unsigned(row) / unsigned(g.in_w);
                    ii = q;
                    jj = unsigned(row) - q * unsigned(g.in_w);
                } else {
                    ii = row / g.in_w;
                    jj = row - ii * g.in_w;
                }
                d2s_px[mt] = 2 * ii * 2 * g.in_w + 2 * jj;   // output pixel of tap 0
            }
            tap = n0 / g.cout;
            co = n0 - tap * g.cout + lg * 4;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int col = n0 + nt * 16 + lg * 4;
            const f4 bv = ld4(bsh + col);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const long row = m0 + mt * 16 + li;
                f4 v = acc[mt][nt] + bv;
                if constexpr (RPRE) v = res[mt][nt] + v;
                if (row >= g.M) continue;
                if constexpr (EP == E_STORE) {
                    st4(g.C + row * g.ldc + col, v);
                } else if constexpr (EP == E_DUAL) {
                    st4(g.C + row * g.ldc + col, v);
                    st4(g.C2 + row * g.ldc + col, v);
                } else if constexpr (EP == E_GELU) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = gelu_as(v[r]);
                    st4(g.C + row * g.ldc + col, v);
                } else if constexpr (EP == E_RESID) {
                    st4(g.C + row * g.ldc + col, RPRE ? v : rl[RLATE ? mt : 0][RLATE ? nt : 0] + v);
                } else {
                    const long px = d2s_px[mt] + (tap >> 1) * 2 * g.in_w + (tap & 1);
                    st4(g.C + px * g.cout + co, v);
                }
            }
            if constexpr (EP == E_D2S) {
                co += 16;
                if (co >= g.cout) {
                    co -= g.cout;
                    ++tap;
                }
            }
        }
        if (tn >= tiles) break;
        t = tn;
        m0 = m0n;
        n0 = n0n;
    }
}

// Persistent grids size themselves to the chip: CU count and resident workgroups per CU of
// a kernel, queried at its first launch and kept in relaxed atomics (handles on several
// threads may launch concurrently; they compute and store the same values).
struct Occ {
    int cus, per_cu;
};
template <typename K>
static bool query_occ(K kernel, int threads, std::atomic<int>& cus_c, std::atomic<int>& pc_c, Occ* o) {
    int cus = cus_c.load(std::memory_order_relaxed), pc = pc_c.load(std::memory_order_relaxed);
    if (cus < 1 || pc < 1) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, kernel, threads, 0) != hipSuccess)
            return false;
        cus = std::max(cus, 1);
        pc = std::max(pc, 1);
        cus_c.store(cus, std::memory_order_relaxed);
        pc_c.store(pc, std::memory_order_relaxed);
    }
    *o = Occ{cus, pc};
    return true;
}

template <int MT, int BN, int KC, int AM, int EP, bool H16, bool X6>
static void launch_gemm3_k(const GemmArgs& g, hipStream_t s) {
    static std::atomic<int> cus_c{0}, pc_c{0};
    Occ oc;
    if (!query_occ(k_gemm3<MT, BN, KC, AM, EP, H16, X6>, 256, cus_c, pc_c, &oc)) oc = Occ{256, 1};
    const int cus = oc.cus, per_cu = oc.per_cu;
    const long mtiles = (g.M + 64 * MT - 1) / (64 * MT);
    const long tiles = ((mtiles + 7) / 8) * 8 * (g.N / BN);
    dim3 grid{unsigned(std::min<long>(tiles, long(cus) * per_cu)), 1u, 1u}, block{256u, 1u, 1u};
    hipLaunchKernelGGL((k_gemm3<MT, BN, KC, AM, EP, H16, X6>), grid, block, 0, s, g, tiles);
}

template <int MT, int BN, int KC, int AM, bool H16 = false, bool X6 = false>
static void launch_gemm3_e(const GemmArgs& g, GemmE e, hipStream_t s) {
    switch (e) {
        case E_STORE: launch_gemm3_k<MT, BN, KC, AM, E_STORE, H16, X6>(g, s); break;
        case E_DUAL: launch_gemm3_k<MT, BN, KC, AM, E_DUAL, H16, X6>(g, s); break;
        case E_GELU: launch_gemm3_k<MT, BN, KC, AM, E_GELU, H16, X6>(g, s); break;
        case E_RESID: launch_gemm3_k<MT, BN, KC, AM, E_RESID, H16, X6>(g, s); break;
        case E_D2S:
            if constexpr (AM != A_S2D) launch_gemm3_k<MT, BN, KC, AM, E_D2S, H16, X6>(g, s);
            break;
    }
}

template <int MT, int BN, int KC>
static void launch_gemm3_a(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s) {
    switch (a) {
        case A_ROWS: launch_gemm3_e<MT, BN, KC, A_ROWS>(g, e, s); break;
        case A_S2D: launch_gemm3_e<MT, BN, KC, A_S2D>(g, e, s); break;
        default: break;
    }
}

template <int MT, int BN>
static void launch_gemm3_h16(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s) {
    switch (a) {
        case A_ROWS: launch_gemm3_e<MT, BN, 32, A_ROWS, true>(g, e, s); break;
        case A_S2D: launch_gemm3_e<MT, BN, 32, A_S2D, true>(g, e, s); break;
        case A_ADD2: launch_gemm3_e<MT, BN, 32, A_ADD2, true>(g, e, s); break;
        default: break;
    }
}

template <int MT, int BN>
static void launch_gemm3_x6(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s) {
    switch (a) {
        case A_ROWS: launch_gemm3_e<MT, BN, 32, A_ROWS, true, true>(g, e, s); break;
        case A_S2D: launch_gemm3_e<MT, BN, 32, A_S2D, true, true>(g, e, s); break;
        case A_ADD2: launch_gemm3_e<MT, BN, 32, A_ADD2, true, true>(g, e, s); break;
        default: break;
    }
}

static bool launch_gemm3(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s) {
    // k_gemm3 decodes tile indices in 32 bits (at most 2^31 tiles of 16 rows or more). The
    // patch operand with the depth-to-space epilogue (no layer of the network) is left to
    // k_gemm2.
    if (g.M / 16 >= (1L << 31) || (a == A_S2D && e == E_D2S) || g.N > GEMM3_NMAX) return false;
    if (g.WX && a != A_LN && g.K % 32 == 0 && g.N % 64 == 0) {
        // Split products: at least two 16-row tiles per wave, so the three weight planes a
        // wave reads from LDS per k block feed twice as many products (one tile per wave
        // would need the whole LDS bandwidth).
        if (g.N % 128 == 0) launch_gemm3_x6<2, 128>(g, a, e, s);
        else launch_gemm3_x6<2, 64>(g, a, e, s);
        return true;
    }
    if (g.W16 && a != A_LN && g.K % 32 == 0 && g.N % 64 == 0) {
        // The level-0 down-conv (N = 128) reads its patches once with a 128-wide N block:
        // 382 -> 268 us per launch; the other shapes measured best as below.
        if (a == A_S2D && g.N == 128) launch_gemm3_h16<1, 128>(g, a, e, s);
        else if (g.N <= 128) launch_gemm3_h16<2, 64>(g, a, e, s);
        else if (g.N % 128 == 0) launch_gemm3_h16<2, 128>(g, a, e, s);
        else launch_gemm3_h16<4, 64>(g, a, e, s);
        return true;
    }
    // The LayerNorm operand keeps its row in registers (k_gemm2); the skip-sum operand with
    // the depth-to-space epilogue measured faster one tile per workgroup (k_gemm2).
    if (a == A_LN || a == A_ADD2) return false;
    // Measured on the 1080p forward: one 16-row tile per wave and a wide N block for the 1x1
    // at 256 and 512 channels (4-6 % faster than two tiles per wave), for the level-0
    // down-conv (N = 128: 9 %) and for the level-2 down-conv (N = 512: 322 -> 310 us); the
    // level-1 down-conv (N = 256) keeps two tiles per wave.
    if ((a == A_ROWS || a == A_S2D) && g.N >= 512 && g.N % 256 == 0) launch_gemm3_a<1, 256, 32>(g, a, e, s);
    else if ((a == A_ROWS && g.N == 256) || (a == A_S2D && g.N == 128)) launch_gemm3_a<1, 128, 32>(g, a, e, s);
    else if (g.N % 64 == 0 && g.N <= 128) launch_gemm3_a<2, 64, 32>(g, a, e, s);
    else if (g.N % 128 == 0) launch_gemm3_a<2, 128, 32>(g, a, e, s);
    else if (g.N % 96 == 0) launch_gemm3_a<2, 96, 32>(g, a, e, s);
    else if (g.N % 64 == 0) launch_gemm3_a<4, 64, 32>(g, a, e, s);
    else if (g.N % 32 == 0) launch_gemm3_a<4, 32, 32>(g, a, e, s);
    else return false;
    return true;
}

template <int MT, int BN, int KC, int AM, int KLN>
static void launch_gemm2_e(const GemmArgs& g, GemmE e, hipStream_t s) {
    const long tiles = ((g.M + 64 * MT - 1) / (64 * MT)) * (g.N / BN);
    dim3 grid{unsigned(tiles), 1u, 1u}, block{256u, 1u, 1u};
    switch (e) {
        case E_STORE: hipLaunchKernelGGL((k_gemm2<MT, BN, KC, AM, E_STORE, KLN>), grid, block, 0, s, g); break;
        case E_DUAL: hipLaunchKernelGGL((k_gemm2<MT, BN, KC, AM, E_DUAL, KLN>), grid, block, 0, s, g); break;
        case E_GELU: hipLaunchKernelGGL((k_gemm2<MT, BN, KC, AM, E_GELU, KLN>), grid, block, 0, s, g); break;
        case E_RESID: hipLaunchKernelGGL((k_gemm2<MT, BN, KC, AM, E_RESID, KLN>), grid, block, 0, s, g); break;
        case E_D2S: hipLaunchKernelGGL((k_gemm2<MT, BN, KC, AM, E_D2S, KLN>), grid, block, 0, s, g); break;
    }
}

template <int MT, int BN, int KC>
static void launch_gemm2_a(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s) {
    switch (a) {
        case A_ROWS: launch_gemm2_e<MT, BN, KC, A_ROWS, 0>(g, e, s); break;
        case A_S2D: launch_gemm2_e<MT, BN, KC, A_S2D, 0>(g, e, s); break;
        case A_ADD2: launch_gemm2_e<MT, BN, KC, A_ADD2, 0>(g, e, s); break;
        default: break;
    }
}

// Tile choice (32-wide K slices): see the comment in the body.
static bool launch_gemm2(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s) {
    if (a == A_LN) {
        switch (g.K) {
            case 32: if (g.N % 96 == 0) { launch_gemm2_e<4, 96, 32, A_LN, 32>(g, e, s); return true; } break;
            case 64: if (g.N % 96 == 0) { launch_gemm2_e<2, 96, 64, A_LN, 64>(g, e, s); return true; } break;
            case 128: if (g.N % 128 == 0) { launch_gemm2_e<1, 128, 64, A_LN, 128>(g, e, s); return true; } break;
            case 256: if (g.N % 128 == 0) { launch_gemm2_e<1, 128, 64, A_LN, 256>(g, e, s); return true; } break;
        }
        return false;
    }
    // Measured on the 1080p forward: for N <= 128, 64-wide N blocks and 32-row waves (more
    // waves per SIMD) beat wider tiles; above, 128-wide blocks.
    // The up-conv (skip-sum operand, depth-to-space epilogue): one 16-row tile per wave, at
    // four waves per SIMD (530 -> 480 us at level 0, 430 -> 400 us at level 1), and 16-wide
    // K slices (half the LDS per workgroup: 481 -> 456, 398 -> 380 and 370 -> 354 us at
    // levels 0, 1 and 2; the persistent GEMMs measured slower with them).
    if (a == A_ADD2 && g.N % 128 == 0) {
        launch_gemm2_a<1, 128, 16>(g, a, e, s);
        return true;
    }
    if (g.N % 64 == 0 && g.N <= 128) launch_gemm2_a<2, 64, 32>(g, a, e, s);
    else if (g.N % 128 == 0) launch_gemm2_a<2, 128, 32>(g, a, e, s);
    else if (g.N % 96 == 0) launch_gemm2_a<2, 96, 32>(g, a, e, s);
    else if (g.N % 64 == 0) launch_gemm2_a<4, 64, 32>(g, a, e, s);
    else if (g.N % 32 == 0) launch_gemm2_a<4, 32, 32>(g, a, e, s);
    else return false;
    return true;
}

template <int BM, int BN, int WM, int WN, int AM>
static void launch_gemm_e(const GemmArgs& g, GemmE e, hipStream_t s) {
    long tiles = ((g.M + BM - 1) / BM) * (g.N / BN);
    dim3 grid{unsigned(tiles), 1u, 1u}, block{256u, 1u, 1u};
    switch (e) {
        case E_STORE: hipLaunchKernelGGL((k_gemm<BM, BN, WM, WN, AM, E_STORE>), grid, block, 0, s, g); break;
        case E_DUAL: hipLaunchKernelGGL((k_gemm<BM, BN, WM, WN, AM, E_DUAL>), grid, block, 0, s, g); break;
        case E_GELU: hipLaunchKernelGGL((k_gemm<BM, BN, WM, WN, AM, E_GELU>), grid, block, 0, s, g); break;
        case E_RESID: hipLaunchKernelGGL((k_gemm<BM, BN, WM, WN, AM, E_RESID>), grid, block, 0, s, g); break;
        case E_D2S: hipLaunchKernelGGL((k_gemm<BM, BN, WM, WN, AM, E_D2S>), grid, block, 0, s, g); break;
    }
}

template <int BM, int BN, int WM, int WN>
static void launch_gemm_a(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s) {
    switch (a) {
        case A_ROWS: launch_gemm_e<BM, BN, WM, WN, A_ROWS>(g, e, s); break;
        case A_LN: launch_gemm_e<BM, BN, WM, WN, A_LN>(g, e, s); break;
        case A_S2D: launch_gemm_e<BM, BN, WM, WN, A_S2D>(g, e, s); break;
        case A_ADD2: launch_gemm_e<BM, BN, WM, WN, A_ADD2>(g, e, s); break;
    }
}

bool gemm(const GemmArgs& g, GemmA a, GemmE e, hipStream_t s, const char** why) {
    if (g.M <= 0) return true;
    if (g.K % 32 != 0) { *why = "gemm: K must be a multiple of 32"; return false; }
    if (a == A_LN && (g.K > 256 || (g.K & (g.K - 1)) != 0)) {
        *why = "gemm: the LayerNorm prologue needs K a power of two <= 256";
        return false;
    }
    if (a == A_S2D && (g.cin % 32 != 0 || g.K != 4 * g.cin || (g.in_w & 1))) {
        *why = "gemm: space-to-depth needs cin % 32 == 0, K == 4 cin, even width";
        return false;
    }
    if (e == E_D2S && (g.cout % 16 != 0 || g.N != 4 * g.cout)) {
        *why = "gemm: depth-to-space needs cout % 16 == 0 and N == 4 cout";
        return false;
    }
    if (g.persistent && launch_gemm3(g, a, e, s)) return true;
    if (launch_gemm2(g, a, e, s)) return true;
    if (g.N % 128 == 0) launch_gemm_a<128, 128, 64, 64>(g, a, e, s);
    else if (g.N % 96 == 0) launch_gemm_a<128, 96, 32, 96>(g, a, e, s);
    else if (g.N % 64 == 0) launch_gemm_a<256, 64, 64, 64>(g, a, e, s);
    else if (g.N % 32 == 0) launch_gemm_a<256, 32, 64, 32>(g, a, e, s);
    else { *why = "gemm: N must be a multiple of 32"; return false; }
    return true;
}

// ---------------------------------------------------------------------------
// Persistent 1x1 convolution with LDS-resident weights. A workgroup loads the [c][c]
// weight matrix (two of them when chaining) into LDS once; then each wave on its own
// walks 16*MT-row pixel groups with a grid stride: the next group's rows are loaded
// while the current group is multiplied, so the HBM stream never waits on a workgroup
// start-up or a barrier. The product is transposed as in k_gemm2 (weights as the MFMA
// M rows), which leaves each lane holding 4 consecutive output channels of one pixel:
// a float4 store, and, when chaining, exactly the pixel operand of the next product.
// ---------------------------------------------------------------------------
template <int C, int MT, int NW, int MODE, bool RPRE, bool H16, bool X6 = false>
__global__ __launch_bounds__(NW * 64) void k_pconv(PconvArgs a) {
    static_assert(!X6 || H16, "split products use the 16-bit layout");
    constexpr int NT = C / 16, KG = C / 16;
    // fp32 rows: pitch C + 8 floats; 16-bit rows: pitch C + 16 halves. Either way the pitch
    // is 2 mod 4 sixteen-byte slots, so the 16 rows x 2 slots a 32-lane half reads are
    // distinct mod 32: conflict-free 128-bit reads. Split weights: three such planes.
    constexpr int LDW = H16 ? C + 16 : C + 8;
    constexpr int NMAT = MODE == PC_CHAIN ? 2 : 1;
    constexpr int NP = X6 ? 3 : 1;
    constexpr int MSTR = NP * C * LDW;   // one matrix (all its planes)
    using WT = std::conditional_t<X6, __bf16, std::conditional_t<H16, _Float16, float>>;
    __shared__ __align__(16) WT Ws[NMAT * MSTR];
    // The biases sit in LDS too: a global read in the epilogue would make its wait cover the
    // next group's rows, issued just before.
    __shared__ __align__(16) float bs[NMAT * C];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    for (int f = tid; f < NMAT * C; f += NW * 64) bs[f] = f < C ? a.b[f] : a.b1[f - C];

    if constexpr (X6) {
        // The pre-split planes (already in the k order of the products), 16 bytes at a time.
        for (int f = tid; f < NMAT * NP * C * C / 8; f += NW * 64) {
            const int m = f / (NP * C * C / 8), p = (f / (C * C / 8)) % NP;
            const int r = (f / (C / 8)) % C, q = f % (C / 8);
            const __bf16* src = (m ? a.x1 : a.x) + long(p) * C * C + long(r) * C + q * 8;
            stb8(&Ws[m * MSTR + p * C * LDW + r * LDW + q * 8], ldb8(src));
        }
    } else if constexpr (H16) {
        // Halves in the order the f16 product reads them: slot q = 4 kk + lg of row r holds
        // W[r][32 kk + 4 lg + 0..3] and W[r][32 kk + 16 + 4 lg + 0..3].
        for (int f = tid; f < NMAT * C * C / 8; f += NW * 64) {
            const int m = f / (C * C / 8), r = (f / (C / 8)) % C, q = f % (C / 8);
            const float* src = (m ? a.W1 : a.W) + long(r) * C + 32 * (q >> 2) + 4 * (q & 3);
            sth8(&Ws[m * C * LDW + r * LDW + q * 8], pack8(ld4(src), ld4(src + 16)));
        }
    } else {
        for (int f = tid; f < NMAT * C * C / 4; f += NW * 64) {
            const int m = f / (C * C / 4), r = (f / (C / 4)) % C, c4 = f % (C / 4);
            const float* src = m ? a.W1 : a.W;
            st4(&Ws[m * C * LDW + r * LDW + c4 * 4], ld4(src + long(r) * C + c4 * 4));
        }
    }
    __syncthreads();

    const long groups = (a.M + 16 * MT - 1) / (16 * MT);
    const long stride = long(gridDim.x) * NW;
    long gi = long(blockIdx.x) * NW + wave;

    // Loads are issued on every path (rows past the end read row M - 1, whose products only
    // reach rows that are not stored; the last group re-reads itself as its "next"), so the
    // count of outstanding memory operations is the same on all paths and the wait for a
    // group's rows lands after the next group's loads are issued, not before.
    auto load = [&](long g, f4 (&dst)[MT][KG]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const long r = g * 16 * MT + mt * 16 + li, row = r < a.M ? r : a.M - 1;
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) dst[mt][kg] = ld4(a.A + row * C + kg * 16 + lg * 4);
        }
    };
    auto product = [&](const WT* Wm, const f4 (&x)[MT][KG], f4 (&acc)[MT][NT]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (X6) {
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) {
                x8 xv[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) xv[mt] = split8<true>(x[mt][2 * kk], x[mt][2 * kk + 1]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const x8 w = ldx8(Wm + (nt * 16 + li) * LDW + kk * 32 + lg * 8, C * LDW);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma6(w, xv[mt], acc[mt][nt]);
                }
            }
        } else if constexpr (H16) {
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) {
                h8 w[NT];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) w[nt] = ldh8(Wm + (nt * 16 + li) * LDW + kk * 32 + lg * 8);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const h8 xv = pack8(x[mt][2 * kk], x[mt][2 * kk + 1]);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mfma16(w[nt], xv, acc[mt][nt]);
                }
            }
        } else {
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                f4 w[NT];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) w[nt] = ld4(Wm + (nt * 16 + li) * LDW + kg * 16 + lg * 4);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mfma4(w[nt][s], x[mt][kg][s], acc[mt][nt]);
            }
        }
    };

    // The residual rows of a group: loaded with its A rows one group ahead (RPRE), or at
    // the start of the group's own products.
    auto rload = [&](long g, f4 (&dst)[MT][NT]) {
        if constexpr (MODE != PC_STORE) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const long r = g * 16 * MT + mt * 16 + li, row = r < a.M ? r : a.M - 1;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) dst[mt][nt] = ld4(a.R + row * C + nt * 16 + lg * 4);
            }
        }
    };
    // One group: its rows are in `cur` (and its residual rows in `rc`); the group one
    // stride ahead is loaded into `nxt` / `rn` before the product, so those loads overlap
    // this group's MFMAs and stores.
    auto body = [&](long g, const f4 (&cur)[MT][KG], f4 (&nxt)[MT][KG], const f4 (&rc)[MT][NT],
                    f4 (&rn)[MT][NT]) {
        if constexpr (!RPRE) rload(g, rn);
        {
            const long gn = g + stride < groups ? g + stride : g;
            load(gn, nxt);
            if constexpr (RPRE) rload(gn, rn);
        }
        // The weights are loop-invariant; an opaque zero offset keeps the compiler from
        // hoisting every LDS weight read out of the loop into registers.
        int wz = 0;
        asm volatile("" : "+v"(wz));
        const WT* Wg = Ws + wz;
        f4 acc[MT][NT];
        product(Wg, cur, acc);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f4 bv = ld4(bs + nt * 16 + lg * 4);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                acc[mt][nt] = acc[mt][nt] + bv;
                if constexpr (MODE != PC_STORE) acc[mt][nt] = (RPRE ? rc[mt][nt] : rn[mt][nt]) + acc[mt][nt];
                const long row = g * 16 * MT + mt * 16 + li;
                if (row < a.M) st4(a.C + row * C + nt * 16 + lg * 4, acc[mt][nt]);
            }
        }
        if constexpr (MODE == PC_CHAIN) {
            f4 acc2[MT][NT];
            product(Wg + MSTR, acc, acc2);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const f4 bv = ld4(bs + C + nt * 16 + lg * 4);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const long row = g * 16 * MT + mt * 16 + li;
                    if (row < a.M) st4(a.C2 + row * C + nt * 16 + lg * 4, acc2[mt][nt] + bv);
                }
            }
        }
    };

    f4 xa[MT][KG], xb[MT][KG];
    f4 ra[MT][NT], rb[MT][NT];   // unused (and eliminated) without a residual
    if (gi < groups) {
        load(gi, xa);
        if constexpr (RPRE) rload(gi, ra);
    }
    while (gi < groups) {
        body(gi, xa, xb, ra, rb);
        gi += stride;
        if (gi >= groups) break;
        body(gi, xb, xa, rb, ra);
        gi += stride;
    }
}

template <int C, int MT, int NW, int MODE, bool RPRE, bool H16 = false, bool X6 = false>
static bool launch_pconv(const PconvArgs& a, hipStream_t s) {
    static std::atomic<int> cus_c{0}, pc_c{0};
    Occ oc;
    if (!query_occ(k_pconv<C, MT, NW, MODE, RPRE, H16, X6>, NW * 64, cus_c, pc_c, &oc)) return false;
    const int cus = oc.cus, per_cu = oc.per_cu;
    const long groups = (a.M + 16 * MT - 1) / (16 * MT);
    const long waves = std::min<long>(groups, long(cus) * per_cu * NW);
    dim3 grid{unsigned((waves + NW - 1) / NW), 1u, 1u}, block{unsigned(NW * 64), 1u, 1u};
    hipLaunchKernelGGL((k_pconv<C, MT, NW, MODE, RPRE, H16, X6>), grid, block, 0, s, a);
    return true;
}

bool pconv_supported(int c) { return c == 64 || c == 128; }

bool pconv(const PconvArgs& a, PconvMode mode, hipStream_t s, const char** why) {
    if (a.M <= 0) return true;
    bool ok = false;
    if (a.x && a.c == 64) {
        // Split products, one 16-row group per wave (measured at level 0 against two: the
        // chained pair 552 -> 445 us, the 1x1 312 -> 248 us; two groups need ~270 registers).
        if (mode == PC_STORE) ok = launch_pconv<64, 1, 4, PC_STORE, false, true, true>(a, s);
        else if (mode == PC_RESID) ok = launch_pconv<64, 1, 4, PC_RESID, false, true, true>(a, s);
        else ok = launch_pconv<64, 1, 4, PC_CHAIN, false, true, true>(a, s);
    } else if (a.x && a.c == 128 && mode != PC_CHAIN) {
        if (mode == PC_STORE) ok = launch_pconv<128, 1, 8, PC_STORE, false, true, true>(a, s);
        else ok = launch_pconv<128, 1, 8, PC_RESID, false, true, true>(a, s);
    } else if (a.h16 && a.c == 64) {
        if (mode == PC_STORE) ok = launch_pconv<64, 1, 4, PC_STORE, false, true>(a, s);
        else if (mode == PC_RESID) ok = launch_pconv<64, 1, 4, PC_RESID, false, true>(a, s);
        else ok = launch_pconv<64, 1, 4, PC_CHAIN, false, true>(a, s);
    } else if (a.h16 && a.c == 128) {
        if (mode == PC_STORE) ok = launch_pconv<128, 1, 4, PC_STORE, false, true>(a, s);
        else if (mode == PC_RESID) ok = launch_pconv<128, 1, 4, PC_RESID, false, true>(a, s);
        else ok = launch_pconv<128, 1, 8, PC_CHAIN, false, true>(a, s);
    } else if (a.c == 64) {
        // One 16-row group per wave at 64 channels (measured: level-0 1x1 306 -> 275 us,
        // chained 505 -> 478 us against two groups per wave).
        if (mode == PC_STORE) ok = launch_pconv<64, 1, 4, PC_STORE, false>(a, s);
        else if (mode == PC_RESID) ok = launch_pconv<64, 1, 4, PC_RESID, false>(a, s);
        else ok = launch_pconv<64, 1, 4, PC_CHAIN, false>(a, s);
    } else if (a.c == 128) {
        if (mode == PC_STORE) ok = launch_pconv<128, 1, 4, PC_STORE, false>(a, s);
        else if (mode == PC_RESID) ok = launch_pconv<128, 1, 4, PC_RESID, false>(a, s);
        else ok = launch_pconv<128, 1, 8, PC_CHAIN, false>(a, s);
    } else {
        *why = "pconv: only 64 or 128 channels have a resident-weight configuration";
        return false;
    }
    if (!ok) *why = "pconv: device query failed";
    return ok;
}

// ---------------------------------------------------------------------------
// Fused MLP: x += W2 gelu(W0 LN(x) + b0) + b2, t = T channels, hidden 4T.
// Each wave owns 16*MT rows; LN runs on the rows in registers (the 4 lanes 16 apart hold
// one row between them). The hidden layer is produced HC units at a time and TRANSPOSED
// (H^T = W0c Xn^T, hidden units as the MFMA M rows), which leaves each lane holding
// H[row li][4 consecutive hidden units]: exactly the A operand of the second product, so
// the hidden never goes through LDS or HBM. W0/W2 slices are double-buffered in LDS.
// ---------------------------------------------------------------------------
template <int T, int MT, int HC, bool H16, int NWV = 4, bool KEEP = true, bool X6 = false, bool DB = true,
          bool XS = true>
__global__ __launch_bounds__(NWV * 64) void k_mlp(MlpArgs a) {
    constexpr int NTH = NWV * 64;
    constexpr int KG = T / 16, NT = T / 16, HT = HC / 16, NCH = 4 * T / HC;
    // Slice pitches: fp32 T + 8 / HC + 8 floats; 16-bit T + 16 / HC + 16 halves (2 mod 4
    // sixteen-byte slots either way: conflict-free 128-bit operand reads). Split products
    // (X6): three planes of each slice, [W0 planes][W2 planes] in a buffer.
    static_assert(!X6 || H16, "split products use the 16-bit layout");
    constexpr int L0 = H16 ? T + 16 : T + 8, L2 = H16 ? HC + 16 : HC + 8;
    constexpr int NP = X6 ? 3 : 1;
    constexpr int BUF = NP * (HC * L0 + T * L2);
    constexpr int EV = H16 ? 8 : 4;               // elements per 16-byte chunk
    constexpr int W0V = HC * T / EV;              // chunks in a W0 slice (and in a W2 slice)
    constexpr int PV = (2 * NP * W0V) / NTH;      // chunks per thread per slice (W0 then W2)
    static_assert((2 * NP * W0V) % NTH == 0 && (X6 || W0V % NTH == 0), "slice must split evenly");
    static_assert(!H16 || HC % 32 == 0, "fp16 slices are whole 32-wide k blocks");
    using ET = std::conditional_t<X6, __bf16, std::conditional_t<H16, _Float16, float>>;
    // DB: double-buffered slices (one barrier per slice); else one buffer, two barriers.
    __shared__ __align__(16) ET lds[(DB ? 2 : 1) * BUF];
    __shared__ __align__(16) float gtab[GELU_TABLE];
    // The hidden bias sits in LDS: a global read of it inside the slice loop would make its
    // wait cover the next slice's weights, issued at the top of the loop.
    __shared__ __align__(16) float b0s[4 * T];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    // The prologue's reads (GELU table, hidden bias, the rows, the LayerNorm parameters and
    // the first slice's weights, below) are issued as one batch before any of them is used or
    // stored: one at a time, each waited for, they were a chain of L2 round trips at the start
    // of every workgroup. Rows past the end read row M - 1 and are replaced by zeros.
    constexpr int NGT = (GELU_TABLE / 4 + NTH - 1) / NTH, NB0 = (4 * T + NTH - 1) / NTH;
    f4 gtv[NGT];
    float b0v[NB0];
#pragma unroll
    for (int j = 0; j < NGT; ++j) gtv[j] = ld4(a.gelu + 4 * min(tid + j * NTH, GELU_TABLE / 4 - 1));
#pragma unroll
    for (int j = 0; j < NB0; ++j) b0v[j] = a.b0[min(tid + j * NTH, 4 * T - 1)];
    const long row0 = long(blockIdx.x) * (16 * MT * NWV) + wave * 16 * MT;

    f4 xa[MT][KG];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const long r = row0 + mt * 16 + li, rc = r < a.M ? r : a.M - 1;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) {
            const f4 v = ld4(a.x + rc * a.ldx + kg * 16 + lg * 4);
            xa[mt][kg] = r < a.M ? v : f4{0.f, 0.f, 0.f, 0.f};
        }
    }
    // The LayerNorm parameters join the batch while they fit the registers (t <= 128).
    constexpr bool LNPRE = KG <= 8;
    f4 lng[LNPRE ? KG : 1], lnb[LNPRE ? KG : 1];
    if constexpr (LNPRE) {
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) {
            lng[kg] = ld4(a.ln_g + kg * 16 + lg * 4);
            lnb[kg] = ld4(a.ln_b + kg * 16 + lg * 4);
        }
    }
    // Slice ch: W0 rows ch HC .. + HC - 1 (all T columns) and W2 columns ch HC .. + HC - 1
    // (all T rows). In fp16 mode both come from the k-permuted copies, whose 32-wide k
    // blocks are whole within a slice.
    // HALF (split products, one buffer): W0's planes of the next slice are fetched during the
    // first product and W2's during the second, each stored after the barrier that frees its
    // region, so the prefetch registers hold one matrix's planes at a time.
    constexpr bool HALF = X6 && !DB;
    constexpr int PVH = NP * W0V / NTH;
    static_assert(!HALF || (NP * W0V) % NTH == 0, "half slice must split evenly");
    f4 pre[HALF ? PVH : PV];
    auto gload_half = [&](int ch, int which) {
#pragma unroll
        for (int i = 0; i < PVH; ++i) {
            const int f = tid + i * NTH, p = f / W0V, g = f % W0V;
            if (which == 0) {
                const int row = g / (T / 8), c = g % (T / 8);
                pre[i] = ld4(reinterpret_cast<const float*>(a.x0 + long(p) * 4 * T * T + long(ch * HC + row) * T + c * 8));
            } else {
                const int row = g / (HC / 8), c = g % (HC / 8);
                pre[i] = ld4(reinterpret_cast<const float*>(a.x2 + long(p) * 4 * T * T + long(row) * (4 * T) + ch * HC + c * 8));
            }
        }
    };
    auto lstore_half = [&](int which) {
#pragma unroll
        for (int i = 0; i < PVH; ++i) {
            const int f = tid + i * NTH, p = f / W0V, g = f % W0V;
            if (which == 0) {
                const int row = g / (T / 8), c = g % (T / 8);
                st4(reinterpret_cast<float*>(lds + p * HC * L0 + row * L0 + c * 8), pre[i]);
            } else {
                const int row = g / (HC / 8), c = g % (HC / 8);
                st4(reinterpret_cast<float*>(lds + NP * HC * L0 + p * T * L2 + row * L2 + c * 8), pre[i]);
            }
        }
    };
    auto gload = [&](int ch) {
#pragma unroll
        for (int i = 0; i < (HALF ? 0 : PV); ++i) {
            const int f = tid + i * NTH;
            if constexpr (X6) {
                const int which = f / (NP * W0V), rem = f % (NP * W0V), p = rem / W0V, g = rem % W0V;
                if (which == 0) {
                    const int row = g / (T / 8), c = g % (T / 8);
                    pre[i] = ld4(reinterpret_cast<const float*>(a.x0 + long(p) * 4 * T * T + long(ch * HC + row) * T + c * 8));
                } else {
                    const int row = g / (HC / 8), c = g % (HC / 8);
                    pre[i] = ld4(reinterpret_cast<const float*>(a.x2 + long(p) * 4 * T * T + long(row) * (4 * T) + ch * HC + c * 8));
                }
            } else if (f < W0V) {
                const int row = f / (T / EV), c = f % (T / EV);
                pre[i] = H16 ? ld4(reinterpret_cast<const float*>(a.h0 + long(ch * HC + row) * T + c * 8))
                             : ld4(a.w0 + long(ch * HC + row) * T + c * 4);
            } else {
                const int f2 = f - W0V;
                const int row = f2 / (HC / EV), c = f2 % (HC / EV);
                pre[i] = H16 ? ld4(reinterpret_cast<const float*>(a.h2 + long(row) * (4 * T) + ch * HC + c * 8))
                             : ld4(a.w2 + long(row) * (4 * T) + ch * HC + c * 4);
            }
        }
    };
    auto lstore = [&](int b) {
        ET* base = lds + b * BUF;
#pragma unroll
        for (int i = 0; i < (HALF ? 0 : PV); ++i) {
            const int f = tid + i * NTH;
            if constexpr (X6) {
                const int which = f / (NP * W0V), rem = f % (NP * W0V), p = rem / W0V, g = rem % W0V;
                if (which == 0) {
                    const int row = g / (T / 8), c = g % (T / 8);
                    st4(reinterpret_cast<float*>(base + p * HC * L0 + row * L0 + c * 8), pre[i]);
                } else {
                    const int row = g / (HC / 8), c = g % (HC / 8);
                    st4(reinterpret_cast<float*>(base + NP * HC * L0 + p * T * L2 + row * L2 + c * 8), pre[i]);
                }
            } else if (f < W0V) {
                const int row = f / (T / EV), c = f % (T / EV);
                st4(reinterpret_cast<float*>(base + row * L0 + c * EV), pre[i]);
            } else {
                const int f2 = f - W0V;
                const int row = f2 / (HC / EV), c = f2 % (HC / EV);
                st4(reinterpret_cast<float*>(base + HC * L0 + row * L2 + c * EV), pre[i]);
            }
        }
    };

    f4 acc2[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc2[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

    if constexpr (HALF) gload_half(0, 0);
    else gload(0);
    __builtin_amdgcn_sched_barrier(0);   // every prologue read above, its first use below
#pragma unroll
    for (int j = 0; j < NGT; ++j)
        if (tid + j * NTH < GELU_TABLE / 4) st4(gtab + 4 * (tid + j * NTH), gtv[j]);
#pragma unroll
    for (int j = 0; j < NB0; ++j)
        if (tid + j * NTH < 4 * T) b0s[tid + j * NTH] = b0v[j];
    // The raw rows stay in registers for the residual, unless they would crowd out the
    // accumulators (then they are read again at the end).
    constexpr bool KEEPX = KEEP && MT * KG <= 16;
    f4 xr[KEEPX ? MT : 1][KEEPX ? KG : 1];
    if constexpr (KEEPX) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) xr[mt][kg] = xa[mt][kg];
    }
    // LayerNorm, two-pass (cpu.rs:338-357).
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        float s = 0.f;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) s += (xa[mt][kg].x + xa[mt][kg].y) + (xa[mt][kg].z + xa[mt][kg].w);
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        const float mu = s / float(T);
        float q = 0.f;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) {
            f4 d = xa[mt][kg] - mu;
            q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
        q += __shfl_xor(q, 16);
        q += __shfl_xor(q, 32);
        const float rs = __builtin_amdgcn_rsqf(q * (1.0f / float(T)) + 1e-5f);
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) {
            const f4 g = LNPRE ? lng[LNPRE ? kg : 0] : ld4(a.ln_g + kg * 16 + lg * 4);
            const f4 b = LNPRE ? lnb[LNPRE ? kg : 0] : ld4(a.ln_b + kg * 16 + lg * 4);
            xa[mt][kg] = (xa[mt][kg] - mu) * rs * g + b;
        }
    }
    // 16-bit operands of the first product (k groups 2kk, 2kk + 1 packed), or their split form.
    h8 xh[H16 && !X6 ? MT : 1][H16 && !X6 ? KG / 2 : 1];
    // XS: the normalised rows kept in split form (else split again for every slice).
    x8 xs[X6 && XS ? MT : 1][X6 && XS ? KG / 2 : 1];
    if constexpr (X6 && XS) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) xs[mt][kk] = split8(xa[mt][2 * kk], xa[mt][2 * kk + 1]);
    } else if constexpr (H16) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) xh[mt][kk] = pack8(xa[mt][2 * kk], xa[mt][2 * kk + 1]);
    }

    if constexpr (HALF) {
        lstore_half(0);
        gload_half(0, 1);
        lstore_half(1);
    } else {
        lstore(0);
    }
    __syncthreads();
    for (int ch = 0; ch < NCH; ++ch) {
        const ET* cur = lds + (DB ? (ch & 1) * BUF : 0);
        // The next slice's weights are fetched on every pass (the last pass fetches its own
        // slice again and does not store it), so the number of memory operations in flight
        // does not depend on the path and the waits cover only what they must.
        const int chn = ch + 1 < NCH ? ch + 1 : ch;
        if constexpr (HALF) gload_half(chn, 0);
        else gload(chn);
        f4 acc1[HT][MT];
#pragma unroll
        for (int ht = 0; ht < HT; ++ht)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc1[ht][mt] = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (X6) {
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) {
                x8 xv[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    xv[mt] = XS ? xs[XS ? mt : 0][XS ? kk : 0] : split8(xa[mt][2 * kk], xa[mt][2 * kk + 1]);
#pragma unroll
                for (int ht = 0; ht < HT; ++ht) {
                    const x8 wv = ldx8(cur + (ht * 16 + li) * L0 + kk * 32 + lg * 8, HC * L0);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc1[ht][mt] = mfma6(wv, xv[mt], acc1[ht][mt]);
                }
            }
        } else if constexpr (H16) {
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk)
#pragma unroll
                for (int ht = 0; ht < HT; ++ht) {
                    const h8 wv = ldh8(cur + (ht * 16 + li) * L0 + kk * 32 + lg * 8);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc1[ht][mt] = mfma16(wv, xh[mt][kk], acc1[ht][mt]);
                }
        } else {
#pragma unroll
            for (int kg = 0; kg < KG; ++kg)
#pragma unroll
                for (int ht = 0; ht < HT; ++ht) {
                    const f4 wv = ld4(cur + (ht * 16 + li) * L0 + kg * 16 + lg * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc1[ht][mt] = mfma4(wv[s], xa[mt][kg][s], acc1[ht][mt]);
                }
        }
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
            const f4 bb = ld4(b0s + ch * HC + ht * 16 + lg * 4);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc1[ht][mt][r] = gelu_lut(gtab, acc1[ht][mt][r] + bb[r]);
        }
        if constexpr (HALF) {
            __syncthreads();   // every wave is past the first product: W0's region is free
            if (ch + 1 < NCH) lstore_half(0);
            gload_half(chn, 1);
        }
        if constexpr (X6) {
#pragma unroll
            for (int kb = 0; kb < HT / 2; ++kb)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const x8 hv = split8(acc1[2 * kb][mt], acc1[2 * kb + 1][mt]);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const x8 wv = ldx8(cur + NP * HC * L0 + (nt * 16 + li) * L2 + kb * 32 + lg * 8, T * L2);
                        acc2[mt][nt] = mfma6(wv, hv, acc2[mt][nt]);
                    }
                }
        } else if constexpr (H16) {
#pragma unroll
            for (int kb = 0; kb < HT / 2; ++kb)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const h8 hv = pack8(acc1[2 * kb][mt], acc1[2 * kb + 1][mt]);
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const h8 wv = ldh8(cur + HC * L0 + (nt * 16 + li) * L2 + kb * 32 + lg * 8);
                        acc2[mt][nt] = mfma16(wv, hv, acc2[mt][nt]);
                    }
                }
        } else {
#pragma unroll
            for (int ht = 0; ht < HT; ++ht)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const f4 wv = ld4(cur + HC * L0 + (nt * 16 + li) * L2 + ht * 16 + lg * 4);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc2[mt][nt] = mfma4(wv[r], acc1[ht][mt][r], acc2[mt][nt]);
                }
        }
        if constexpr (HALF) {
            __syncthreads();   // W2's region is free; W0's next planes are visible after this
            if (ch + 1 < NCH) lstore_half(1);
        } else if constexpr (DB) {
            if (ch + 1 < NCH) lstore((ch + 1) & 1);
            __syncthreads();
        } else {
            __syncthreads();
            if (ch + 1 < NCH) {
                lstore(0);
                __syncthreads();
            }
        }
    }
    // out^T = W2 H^T: each lane holds 4 consecutive output channels of one row. Without the
    // kept rows the row offset is formed again here (an opaque copy of the lane index keeps
    // the compiler from holding the prologue's 64-bit offset, and spilling it, through the loop).
    int lie = li, wve = wave;
    if constexpr (!KEEPX) asm volatile("" : "+v"(lie), "+v"(wve));
    const long row0e = long(blockIdx.x) * (16 * MT * NWV) + wve * 16 * MT;
    if constexpr (KEEPX) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const f4 bv = ld4(a.b2 + nt * 16 + lg * 4);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const long row = row0e + mt * 16 + lie;
                if (row < a.M) st4(a.x + row * a.ldx + nt * 16 + lg * 4, xr[mt][nt] + (acc2[mt][nt] + bv));
            }
        }
    } else {
        // The residual rows are read again, RG column groups at a time and all before their
        // stores (rows clamped), so the reads of a group are in flight together.
        constexpr int RG = NT < 8 ? NT : 8;
#pragma unroll
        for (int n0 = 0; n0 < NT; n0 += RG) {
            f4 bv[RG], rr[MT][RG];
#pragma unroll
            for (int j = 0; j < RG; ++j) bv[j] = ld4(a.b2 + (n0 + j) * 16 + lg * 4);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const long r = row0e + mt * 16 + lie, row = r < a.M ? r : a.M - 1;
#pragma unroll
                for (int j = 0; j < RG; ++j) rr[mt][j] = ld4(a.x + row * a.ldx + (n0 + j) * 16 + lg * 4);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const long row = row0e + mt * 16 + lie;
                if (row < a.M) {
#pragma unroll
                    for (int j = 0; j < RG; ++j)
                        st4(a.x + row * a.ldx + (n0 + j) * 16 + lg * 4, rr[mt][j] + (acc2[mt][n0 + j] + bv[j]));
                }
            }
        }
    }
}

bool mlp(const MlpArgs& a, hipStream_t s, const char** why) {
    if (a.M <= 0) return true;
    if (!a.gelu) {
        *why = "mlp: no GELU table";
        return false;
    }
    auto go = [&](auto kern, int rows_per_block, int threads = 256) {
        dim3 grid{unsigned((a.M + rows_per_block - 1) / rows_per_block), 1u, 1u};
        dim3 block{unsigned(threads), 1u, 1u};
        hipLaunchKernelGGL(kern, grid, block, 0, s, a);
    };
    if ((a.h0 && !a.h2) || (a.x0 && !a.x2)) {
        *why = "mlp: the 16-bit paths need both k-permuted weights";
        return false;
    }
    const bool h16 = a.h0 != nullptr;
    if (a.x0 && !h16 && a.t == 64) {
        // t = 64 (the split mode runs it outside the window kernel): 8 waves of two row tiles
        // share each double-buffered slice (68 KB of LDS). Measured at level 1 of 1080p:
        // 248 us with one row tile per wave, 227 us with two, 325 / 264 us on 4 waves.
        go(k_mlp<64, 2, 32, true, 8, true, true, true>, 256, 512);
        return true;
    }
    if (a.x0 && !h16 && (a.t == 128 || a.t == 256)) {
        // Split products: 8 waves of one row tile each share every streamed slice (three
        // planes per matrix). t = 128: double-buffered (129 KB of LDS), the normalised rows
        // kept in split form; t = 256: one buffer (126 KB), the rows split again per slice.
        // Measured at 1080p (levels 2 and 3): t = 128 310 -> 197 us per launch against the
        // fp32 products; t = 256 280 -> 264 us. Two row tiles per wave (8 or 4 waves) spill.
        if (a.t == 128) go(k_mlp<128, 1, 32, true, 8, false, true, true>, 128, 512);
        else go(k_mlp<256, 1, 32, true, 8, false, true, false, false>, 128, 512);
        return true;
    }
    switch (a.t) {
        case 32: h16 ? go(k_mlp<32, 4, 64, true>, 256) : go(k_mlp<32, 4, 64, false>, 256); break;
        case 64: h16 ? go(k_mlp<64, 2, 64, true>, 128) : go(k_mlp<64, 2, 64, false>, 128); break;
        // fp16: more rows per workgroup (8 waves at t = 128, 2 row tiles per wave at both), so
        // each streamed weight slice feeds 256 (t = 128) or 128 (t = 256) rows. fp32 at
        // t = 128: 16 hidden units per slice (317 -> 314 us per launch at level 2 of 1080p).
        case 128: h16 ? go(k_mlp<128, 2, 32, true, 8>, 256, 512) : go(k_mlp<128, 1, 16, false>, 64); break;
        // fp32 at t = 256: 8 waves of one row tile each share every 32-unit weight slice
        // (128 rows per workgroup; against two row tiles per wave on 4 waves 337 -> 307 us
        // per launch at level 3 of 1080p). Two waves per SIMD cap it at 256 VGPRs: keeping
        // the raw rows for the residual spilled 54 registers to scratch; reading the rows
        // again at the end fits in 248 without a spill (312 -> 280 us, bit-identical).
        case 256: h16 ? go(k_mlp<256, 2, 32, true>, 128) : go(k_mlp<256, 1, 32, false, 8, false>, 128, 512); break;
        default: *why = "mlp: t must be 32, 64, 128 or 256"; return false;
    }
    return true;
}

// ---------------------------------------------------------------------------
// 3x3 convolution, stride 1, zero padding 1, no bias, as an implicit GEMM:
// M = a 16x16 tile of output pixels, N = BN output channels, K = 9 taps x cin.
// Each 16-channel input slice of the tile's 18x18 halo and the matching weights go
// through LDS; a wave owns 4 tile rows (4 M-tiles of 16 pixels) x BN channels.
// ---------------------------------------------------------------------------
template <int BN, bool RELU>
__global__ __launch_bounds__(256) void k_conv3x3(Conv3Args a) {
    constexpr int BK = 16, LDC = BK + 4, HW = 18;
    constexpr int NT = BN / 16;
    constexpr int HV = (HW * HW * 4 + 255) / 256;   // halo float4 per thread
    constexpr int WV = (9 * BN * 4 + 255) / 256;    // weight float4 per thread
    __shared__ float Hs[HW * HW * LDC];
    __shared__ float Ws[9 * BN * LDC];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int tx = (a.W + 15) >> 4, ty = (a.H + 15) >> 4, nb = a.cout / BN;
    const long tile = xcd_swizzle(blockIdx.x, gridDim.x);
    const int nblk = int(tile % nb);
    const long sp = tile / nb;
    const int y0 = int(sp / tx) * 16, x0 = int(sp % tx) * 16;
    const int co0 = nblk * BN;
    (void)ty;

    f4 rh[HV], rw[WV];
    auto load = [&](int ci0) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            int f = tid + i * 256;
            f4 v = {0.f, 0.f, 0.f, 0.f};
            if (f < HW * HW * 4) {
                int px = f >> 2, c4 = f & 3;
                int gy = y0 - 1 + px / HW, gx = x0 - 1 + px % HW;
                if (gy >= 0 && gy < a.H && gx >= 0 && gx < a.W)
                    v = ld4(a.in + (long(gy) * a.W + gx) * a.ldi + ci0 + c4 * 4);
            }
            rh[i] = v;
        }
#pragma unroll
        for (int i = 0; i < WV; ++i) {
            int f = tid + i * 256;
            if (f < 9 * BN * 4) {
                int tap = f / (BN * 4), rem = f - tap * (BN * 4);
                int n = rem >> 2, c4 = rem & 3;
                rw[i] = ld4(a.w + (long(tap) * a.cout + co0 + n) * a.cin + ci0 + c4 * 4);
            }
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            int f = tid + i * 256;
            if (f < HW * HW * 4) st4(&Hs[(f >> 2) * LDC + (f & 3) * 4], rh[i]);
        }
#pragma unroll
        for (int i = 0; i < WV; ++i) {
            int f = tid + i * 256;
            if (f < 9 * BN * 4) {
                int tap = f / (BN * 4), rem = f - tap * (BN * 4);
                st4(&Ws[(tap * BN + (rem >> 2)) * LDC + (rem & 3) * 4], rw[i]);
            }
        }
    };

    f4 acc[4][NT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    load(0);
    stash();
    __syncthreads();
    for (int ci0 = 0; ci0 < a.cin; ci0 += BK) {
        const bool more = ci0 + BK < a.cin;
        if (more) load(ci0 + BK);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int ky = tap / 3, kx = tap % 3;
            f4 av[4], bv[NT];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = ld4(&Hs[((wave * 4 + i + ky) * HW + li + kx) * LDC + lg * 4]);
#pragma unroll
            for (int j = 0; j < NT; ++j) bv[j] = ld4(&Ws[(tap * BN + j * 16 + li) * LDC + lg * 4]);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < NT; ++j) acc[i][j] = mfma4(bv[j][s], av[i][s], acc[i][j]);
        }
        __syncthreads();
        if (more) {
            stash();
            __syncthreads();
        }
    }

    // Computed transposed (weights as the M rows): each lane holds output channels
    // co0 + 16j + 4lg .. +3 of pixel (y0 + 4*wave + i, x0 + li).
    const int x = x0 + li;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int y = y0 + wave * 4 + i;
        if (y >= a.H || x >= a.W) continue;
        float* o = a.out + (long(y) * a.W + x) * a.ldo + co0 + lg * 4;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            f4 v = acc[i][j];
            if constexpr (RELU) {
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = fmaxf(v[r], 0.0f);
                st4(o + j * 16, v);
            } else {
                st4(o + j * 16, ld4(o + j * 16) + v);
            }
        }
    }
}

bool conv3x3(const Conv3Args& a, bool relu, hipStream_t s, const char** why) {
    if (a.img_h > 0 && a.img_h < a.H) {
        *why = "conv3x3: the direct kernel does not take stacked images";
        return false;
    }
    if (a.cin % 16 != 0) { *why = "conv3x3: cin must be a multiple of 16"; return false; }
    long tiles = long((a.W + 15) / 16) * ((a.H + 15) / 16);
    if (a.cout % 64 == 0) {
        dim3 grid(unsigned(tiles * (a.cout / 64)));
        if (relu) hipLaunchKernelGGL((k_conv3x3<64, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_conv3x3<64, false>), grid, dim3(256), 0, s, a);
    } else if (a.cout % 32 == 0) {
        dim3 grid(unsigned(tiles * (a.cout / 32)));
        if (relu) hipLaunchKernelGGL((k_conv3x3<32, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_conv3x3<32, false>), grid, dim3(256), 0, s, a);
    } else {
        *why = "conv3x3: cout must be a multiple of 32";
        return false;
    }
    return true;
}

// ---------------------------------------------------------------------------
// 3x3 convolution by Winograd F(2x2, 3x3) on the matrix cores (Lavin & Gray 2016,
// "Fast Algorithms for Convolutional Neural Networks"): each 2x2 output tile is
// Y = A^T [ (G g G^T) .* (B^T d B) ] A summed over input channels, with d the tile's 4x4
// input patch and
//     B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
//     G   = [1 0 0; 1/2 1/2 1/2; 1/2 -1/2 1/2; 0 0 1]      (applied on the host)
//     A^T = [1 1 1 0; 0 1 -1 -1]
// so the channel sum becomes 16 independent products M[xi] = U[xi] V[xi] (xi = 4i + j over
// the transformed 4x4 positions), 2.25x fewer multiplies than the direct form.
// Unit of work: 16x16 output pixels (8x8 tiles) x 16 output channels, 4 waves; wave w owns
// tile rows 2w, 2w+1 (16 tiles, the MFMA N dimension: lane li = tile). Per 16-channel
// slice: the 18x18 halo and U[16][16 co][16 ci] go through LDS; each lane reads its tile's
// 4x4 patch for 4 consecutive channels (lane group lg), transforms it in registers into
// exactly the B operand it supplies, and M^T[xi] = U[xi] V[xi]^T accumulates in 16 x 4
// registers. Every lane then holds all 16 M[xi] for its tile and 4 consecutive channels,
// so the output transform and the float4 store are lane-local.
// The grid is persistent (as many workgroups as fit on the chip at once); a workgroup
// walks units with a grid stride, and the next (unit, slice) step's global loads are
// issued before the current step's products, across unit boundaries too, so a unit's
// first slice and its epilogue overlap the neighbouring steps. Units are numbered so that
// the cout blocks of one spatial tile run on the same XCD (they read the same halo).
// ---------------------------------------------------------------------------
struct WinoUnit {
    int y0, x0, co0;
    int y1 = -1, x1 = 0;   // pair units: the second 8 x 16 region (y1 = -1: none)
};
DEVI WinoUnit wino_unit(long u, int tx, int nb, long tiles, int cbw = 16) {
    // u = 8 j + xcd; within an XCD, consecutive j walk the cout blocks of one tile. Unit and
    // tile indices fit 32 bits (the launcher bounds the plane below 2^32 elements), so the
    // divisions are 32-bit.
    const unsigned uu = unsigned(u), xcd = uu & 7u, j = uu >> 3;
    const unsigned q = j / unsigned(nb), sp = q * 8u + xcd;
    WinoUnit w;
    w.co0 = int(j - q * unsigned(nb)) * cbw;
    const unsigned ty = sp / unsigned(tx);
    w.y0 = long(sp) < tiles ? int(ty) * 16 : -1;
    w.x0 = int(sp - ty * unsigned(tx)) * 16;
    return w;
}

// Pair units (PAIR): the plane is cut into 8 x 16-pixel half-tiles, and a unit is the
// half-tiles 2p and 2p + 1 of the row-major order (any two; waves 0-1 take the first, waves
// 2-3 the second) x 16 output channels: the same arithmetic per lane, with twice as many
// units of half the height. A 136-row plane (the 1/8 level of 1088 rows) then has no
// half-empty tile row, and 4 080 half-tiles x 16 channel blocks make 2 040 units: 3.98
// rounds of 512 workgroups instead of 2 160 units in 4.22 (run as 5).
DEVI WinoUnit wino_pair(long u, int tx, int nb, long pairs, long halfs) {
    const unsigned uu = unsigned(u), xcd = uu & 7u, j = uu >> 3;
    const unsigned q = j / unsigned(nb), sp = q * 8u + xcd;
    WinoUnit w;
    w.co0 = int(j - q * unsigned(nb)) * 16;
    const unsigned h0 = 2u * sp, h1 = h0 + 1u;
    const unsigned r0 = h0 / unsigned(tx), r1 = h1 / unsigned(tx);
    w.y0 = long(h0) < halfs ? int(r0) * 8 : -1;
    w.x0 = int(h0 - r0 * unsigned(tx)) * 16;
    w.y1 = long(h1) < halfs ? int(r1) * 8 : -1;
    w.x1 = int(h1 - r1 * unsigned(tx)) * 16;
    (void)pairs;
    return w;
}

template <bool RELU, bool BATCH, bool PAIR>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_wino(Conv3Args a, long tiles,
                                                                                         long units) {
    // Halo pixel (py, px) at Hs[(py * HP + px) * LDC]: 5 slots per pixel and 24-pixel rows
    // make the patch reads (lanes 2 pixels apart along a row, two tile rows 2 pixel rows
    // apart) hit 32 distinct slots mod 32 per half-wave; U rows are 24 floats apart.
    // Pair units keep their two 10 x 18 halos as LDS rows 0-9 and 10-19.
    constexpr int BK = 16, LDC = BK + 4, HW = 18, HP = 24, LDU = BK + 8;
    constexpr int HROWS = PAIR ? 20 : HW;            // halo rows in LDS
    constexpr int HPX = PAIR ? 2 * 10 * HW : HW * HW; // halo pixels per unit
    constexpr int HV = (HPX * 4 + 255) / 256;        // halo float4 per thread
    constexpr int UV = 16 * 16 * 4 / 256;            // U float4 per thread
    __shared__ float Hs[HROWS * HP * LDC];
    __shared__ float Us[16 * 16 * LDU];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int tx = (a.W + 15) >> 4, nb = a.cout / 16, nch = a.cin / BK;
    // The wave's tile row within its region and the region's first LDS halo row.
    const int tr = PAIR ? 2 * (wave & 1) + (li >> 3) : 2 * wave + (li >> 3), tc = li & 7;
    const int hrow0 = PAIR ? (wave >> 1) * 10 : 0;
    const long halfs = PAIR ? long((a.H + 7) >> 3) * tx : 0;
    auto unit_at = [&](long uu) { return PAIR ? wino_pair(uu, tx, nb, tiles, halfs) : wino_unit(uu, tx, nb, tiles); };
    // Origin of the wave's output region (y < 0: nothing to compute or store).
    auto ry0 = [&](const WinoUnit& w) { return PAIR && (wave >> 1) ? w.y1 : w.y0; };
    auto rx0 = [&](const WinoUnit& w) { return PAIR && (wave >> 1) ? w.x1 : w.x0; };

    // Load addressing: 32-bit element offsets per lane, fixed per kernel (U) or per unit
    // (halo); a slice only adds its uniform channel base, so the loop does no address
    // arithmetic. A plane of P pixels x ldi channels must have P * ldi < 2^32 (checked by
    // the launcher). NOFF marks a halo position outside the image: it loads zeros.
    constexpr unsigned NOFF = 0xffffffffu;
    unsigned uoff[UV];
#pragma unroll
    for (int i = 0; i < UV; ++i) {
        const int f = tid + i * 256;
        const int xi = f >> 6, rem = f & 63, co = rem >> 2, c4 = rem & 3;
        uoff[i] = (unsigned(xi) * unsigned(a.cout) + unsigned(co)) * unsigned(a.cin) + unsigned(c4 * 4);
    }
    auto halo_offsets = [&](const WinoUnit& w, unsigned (&ho)[HV]) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            const int f = tid + i * 256;
            const int px = f >> 2, c4 = f & 3;
            const bool second = PAIR && px >= 10 * HW;
            const int pp = second ? px - 10 * HW : px;
            const int oy = second ? w.y1 : w.y0, ox = second ? w.x1 : w.x0;
            const int gy = oy - 1 + pp / HW, gx = ox - 1 + pp % HW;
            const bool ok = f < HPX * 4 && oy >= 0 && gy >= 0 && gy < a.H && gx >= 0 && gx < a.W;
            ho[i] = ok ? (unsigned(gy) * unsigned(a.W) + unsigned(gx)) * unsigned(a.ldi) + unsigned(c4 * 4) : NOFF;
        }
    };
    f4 rh[HV], ru[UV];
    auto load = [&](const unsigned (&ho)[HV], int co0, int ci0) {
        const float* hb = a.in + ci0;
#pragma unroll
        for (int i = 0; i < HV; ++i) rh[i] = ho[i] != NOFF ? ld4(hb + ho[i]) : f4{0.f, 0.f, 0.f, 0.f};
        const float* ub = a.w + long(co0) * a.cin + ci0;
#pragma unroll
        for (int i = 0; i < UV; ++i) ru[i] = ld4(ub + uoff[i]);
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            const int f = tid + i * 256;
            if (f < HPX * 4) {
                const int px = f >> 2;   // pair units: pixel 180 + p is LDS row 10 + p / 18
                st4(&Hs[((px / HW) * HP + px % HW) * LDC + (f & 3) * 4], rh[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < UV; ++i) {
            const int f = tid + i * 256;
            st4(&Us[(f >> 2) * LDU + (f & 3) * 4], ru[i]);
        }
    };

    long u = blockIdx.x;
    if (u >= units) return;
    WinoUnit cur = unit_at(u);
    unsigned hcur[HV], hnxt[HV];
    halo_offsets(cur, hcur);
    load(hcur, cur.co0, 0);
    for (;;) {
        f4 acc[16];
#pragma unroll
        for (int xi = 0; xi < 16; ++xi) acc[xi] = f4{0.f, 0.f, 0.f, 0.f};
        const long un = u + gridDim.x;
        const WinoUnit nxt = unit_at(un);
        halo_offsets(nxt, hnxt);
        for (int c = 0; c < nch; ++c) {
            __syncthreads();
            stash();
            __syncthreads();
            if (c + 1 < nch) load(hcur, cur.co0, (c + 1) * BK);
            else if (un < units) load(hnxt, nxt.co0, 0);
            // T = B^T d column by column (each needs one column of the patch), then row i
            // of V = T B feeds the products for xi = 4i .. 4i+3 (channels 4lg .. 4lg+3).
            // Stacked images: the patch row above a tile that starts an image, or below one
            // that ends it, belongs to the neighbouring image and reads as zero padding.
            bool mtop = false, mbot = false;
            if constexpr (BATCH) {
                const int yo = ry0(cur) + 2 * tr;
                mtop = yo % a.img_h == 0;
                mbot = (yo + 2) % a.img_h == 0;
            }
            f4 t[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float* col = &Hs[((hrow0 + 2 * tr) * HP + 2 * tc + j) * LDC + lg * 4];
                f4 d0 = ld4(col), d1 = ld4(col + HP * LDC), d2 = ld4(col + 2 * HP * LDC),
                   d3 = ld4(col + 3 * HP * LDC);
                if constexpr (BATCH) {
                    if (mtop) d0 = f4{0.f, 0.f, 0.f, 0.f};
                    if (mbot) d3 = f4{0.f, 0.f, 0.f, 0.f};
                }
                t[0][j] = d0 - d2;
                t[1][j] = d1 + d2;
                t[2][j] = d2 - d1;
                t[3][j] = d1 - d3;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f4 v[4] = {t[i][0] - t[i][2], t[i][1] + t[i][2], t[i][2] - t[i][1], t[i][1] - t[i][3]};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f4 uu = ld4(&Us[((i * 4 + j) * 16 + li) * LDU + lg * 4]);
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4) acc[i * 4 + j] = mfma4(uu[s4], v[j][s4], acc[i * 4 + j]);
                }
            }
        }
        // Output transform: lane holds M[xi] for its tile, channels co0 + 4lg .. +3.
        if (ry0(cur) >= 0) {
            f4 s0[4], s1[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s0[j] = acc[j] + acc[4 + j] + acc[8 + j];
                s1[j] = acc[4 + j] - acc[8 + j] - acc[12 + j];
            }
            f4 yv[2][2];
            yv[0][0] = s0[0] + s0[1] + s0[2];
            yv[0][1] = s0[1] - s0[2] - s0[3];
            yv[1][0] = s1[0] + s1[1] + s1[2];
            yv[1][1] = s1[1] - s1[2] - s1[3];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int y = ry0(cur) + 2 * tr + i, x = rx0(cur) + 2 * tc + j;
                    if (y >= a.H || x >= a.W) continue;
                    float* o = a.out + (long(y) * a.W + x) * a.ldo + cur.co0 + lg * 4;
                    f4 v = yv[i][j];
                    if constexpr (RELU) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] = fmaxf(v[r], 0.0f);
                        st4(o, v);
                    } else {
                        st4(o, ld4(o) + v);
                    }
                }
        }
        if (un >= units) break;
        u = un;
        cur = nxt;
#pragma unroll
        for (int i = 0; i < HV; ++i) hcur[i] = hnxt[i];
    }
}

// Winograd F(2x2, 3x3) with 32 output channels per unit. 8 waves: wave pair p owns tile
// rows 2p, 2p+1 (16 tiles, lane li = tile), and within the pair wave half hh owns rows
// 2hh, 2hh+1 of the transformed 4x4 positions, for both 16-channel blocks. A wave thus
// needs 3 of the patch's 4 rows and half of the input transform per slice, for twice the
// output channels of k_wino: a quarter of the transform work and half of the halo loads per
// product. The output transform is linear in the rows, so each wave forms the partial 2x2
// outputs of its rows; the pair exchanges the partials of one channel block each through
// LDS, and each wave finishes (ReLU or residual) and stores one block.
// ---------------------------------------------------------------------------
template <bool RELU, bool URES, bool BATCH>
__global__ __launch_bounds__(512) void k_wino2(Conv3Args a, long tiles, long units) {
    // Two LDS buffers (halo + U each): slice k + 1 is written into one while slice k is read
    // from the other, so a slice costs one barrier. 18-pixel halo rows keep both buffers
    // within the CU's LDS (the patch reads then meet 2-way bank conflicts).
    // URES (cin = cout = 32): the whole U [16][32][32] is loaded into LDS once per workgroup
    // (unpadded, 16-byte slots XOR-swizzled by the row so that the operand reads stay
    // conflict-free), slices stage only the halo, and the exchange has its own area.
    constexpr int BK = 16, LDC = BK + 4, HW = 18, HP = 18, LDU = BK + 8, CB = 32, XP = 20;
    constexpr int HV = (HW * HW * 4 + 511) / 512;   // halo float4 per thread
    constexpr int UV = URES ? 0 : 16 * CB * 4 / 512;  // U float4 per thread and slice
    constexpr int HSZ = HW * HP * LDC, BSZ = URES ? HSZ : HSZ + 16 * CB * LDU;
    constexpr int USZ = URES ? 16 * CB * 32 : 0, XSZ = URES ? 8 * 64 * XP : 0;
    __shared__ float lds[2 * BSZ + USZ + XSZ];
    static_assert(URES || 8 * 64 * XP <= BSZ, "exchange must fit in one buffer");
    float* const ures = lds + 2 * BSZ;
    float* const xres = ures + USZ;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4, pair = wave >> 1, hh = wave & 1;
    const int tx = (a.W + 15) >> 4, nb = a.cout / CB, nch = a.cin / BK;
    const int tr = 2 * pair + (li >> 3), tc = li & 7;

    constexpr unsigned NOFF = 0xffffffffu;
    unsigned uoff[UV > 0 ? UV : 1];
#pragma unroll
    for (int i = 0; i < UV; ++i) {
        const int f = tid + i * 512;
        const int xi = f >> 7, rem = f & 127, co = rem >> 2, c4 = rem & 3;
        uoff[i] = (unsigned(xi) * unsigned(a.cout) + unsigned(co)) * unsigned(a.cin) + unsigned(c4 * 4);
    }
    auto halo_offsets = [&](const WinoUnit& w, unsigned (&ho)[HV]) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            const int f = tid + i * 512;
            const int px = f >> 2, c4 = f & 3;
            const int gy = w.y0 - 1 + px / HW, gx = w.x0 - 1 + px % HW;
            const bool ok = f < HW * HW * 4 && w.y0 >= 0 && gy >= 0 && gy < a.H && gx >= 0 && gx < a.W;
            ho[i] = ok ? (unsigned(gy) * unsigned(a.W) + unsigned(gx)) * unsigned(a.ldi) + unsigned(c4 * 4) : NOFF;
        }
    };
    f4 rh[HV], ru[UV > 0 ? UV : 1];
    auto load = [&](const unsigned (&ho)[HV], int co0, int ci0) {
        const float* hb = a.in + ci0;
#pragma unroll
        for (int i = 0; i < HV; ++i) rh[i] = ho[i] != NOFF ? ld4(hb + ho[i]) : f4{0.f, 0.f, 0.f, 0.f};
        const float* ub = a.w + long(co0) * a.cin + ci0;
#pragma unroll
        for (int i = 0; i < UV; ++i) ru[i] = ld4(ub + uoff[i]);
    };
    auto stash = [&](float* buf) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            const int f = tid + i * 512;
            if (f < HW * HW * 4) {
                const int px = f >> 2;
                st4(&buf[((px / HW) * HP + px % HW) * LDC + (f & 3) * 4], rh[i]);
            }
        }
        if constexpr (URES) return;
        float* us = buf + HSZ;
#pragma unroll
        for (int i = 0; i < UV; ++i) {
            const int f = tid + i * 512;
            st4(&us[(f >> 2) * LDU + (f & 3) * 4], ru[i]);
        }
    };
    // acc[cb][ii][j]: M[2hh + ii][j] for channel block cb (co0 + 16 cb + 4lg .. +3).
    f4 acc[2][2][4];
    // One slice: the two rows of V = B^T d B this half owns, then 2 x 4 x 2 x 4 products.
    // FIRST: the unit's first slice starts the sums (zero accumulator operand), so the
    // accumulators are never cleared with separate moves.
    auto slice = [&](auto HHc, auto FIRSTc, const float* buf, int ci0, bool mrow) {
        constexpr int H2 = decltype(HHc)::value;
        constexpr bool FIRST = decltype(FIRSTc)::value;
        const float* Us = buf + HSZ;
        f4 t[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float* col = &buf[((2 * tr + H2) * HP + 2 * tc + j) * LDC + lg * 4];
            f4 da = ld4(col), db = ld4(col + HP * LDC), dc = ld4(col + 2 * HP * LDC);
            // Stacked images: patch row 0 (H2 = 0: da) above a tile that starts an image, or
            // row 3 (H2 = 1: dc) below one that ends it, reads as zero padding.
            if constexpr (BATCH) {
                if (mrow) {
                    if constexpr (H2 == 0) da = f4{0.f, 0.f, 0.f, 0.f};
                    else dc = f4{0.f, 0.f, 0.f, 0.f};
                }
            }
            if constexpr (H2 == 0) {         // rows d0, d1, d2: T0 = d0 - d2, T1 = d1 + d2
                t[0][j] = da - dc;
                t[1][j] = db + dc;
            } else {                         // rows d1, d2, d3: T2 = d2 - d1, T3 = d1 - d3
                t[0][j] = db - da;
                t[1][j] = da - dc;
            }
        }
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const f4 v[4] = {t[ii][0] - t[ii][2], t[ii][1] + t[ii][2], t[ii][2] - t[ii][1], t[ii][1] - t[ii][3]};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    const int ur = ((2 * H2 + ii) * 4 + j) * CB + cb * 16 + li;
                    f4 uu;
                    if constexpr (URES)
                        uu = ld4(&ures[ur * 32 + 4 * (((ci0 >> 2) + lg) ^ (2 * ((ur >> 2) & 3)))]);
                    else
                        uu = ld4(&Us[ur * LDU + lg * 4]);
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4)
                        acc[cb][ii][j] = mfma4(uu[s4], v[j][s4],
                                               (FIRST && s4 == 0) ? f4{0.f, 0.f, 0.f, 0.f} : acc[cb][ii][j]);
                }
        }
    };

    // Partial outputs of this half's rows: with r_i[0] = M[i][0] + M[i][1] + M[i][2] and
    // r_i[1] = M[i][1] - M[i][2] - M[i][3], Y[0][b] = r_0 + r_1 + r_2 and
    // Y[1][b] = r_1 - r_2 - r_3 (A^T = [1 1 1 0; 0 1 -1 -1]). This wave finishes channel
    // block H2 and hands block 1 - H2 to its partner through LDS (the U buffer, free now).
    auto finish = [&](auto HHc, const WinoUnit& w, float* Us, const f4 (&res)[2][2]) {
        constexpr int H2 = decltype(HHc)::value;
        f4 yp[2][2][2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            f4 r[2][2];
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                r[ii][0] = acc[cb][ii][0] + acc[cb][ii][1] + acc[cb][ii][2];
                r[ii][1] = acc[cb][ii][1] - acc[cb][ii][2] - acc[cb][ii][3];
            }
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                if constexpr (H2 == 0) {
                    yp[cb][0][b] = r[0][b] + r[1][b];
                    yp[cb][1][b] = r[1][b];
                } else {
                    yp[cb][0][b] = r[0][b];
                    yp[cb][1][b] = f4{0.f, 0.f, 0.f, 0.f} - r[0][b] - r[1][b];
                }
            }
        }
        float* xo = &Us[((pair * 2 + (1 - H2)) * 64 + lane) * XP];
#pragma unroll
        for (int a0 = 0; a0 < 2; ++a0)
#pragma unroll
            for (int b = 0; b < 2; ++b) st4(xo + (a0 * 2 + b) * 4, yp[1 - H2][a0][b]);
        __syncthreads();
        if (w.y0 < 0) return;
        const float* xi = &Us[((pair * 2 + H2) * 64 + lane) * XP];
        const int co = w.co0 + H2 * 16 + lg * 4;
#pragma unroll
        for (int a0 = 0; a0 < 2; ++a0)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int y = w.y0 + 2 * tr + a0, x = w.x0 + 2 * tc + b;
                if (y >= a.H || x >= a.W) continue;
                f4 v = yp[H2][a0][b] + ld4(xi + (a0 * 2 + b) * 4);
                // 32-bit element offsets (the launcher bounds the plane below 2^32 elements).
                float* o = a.out + ((unsigned(y) * unsigned(a.W) + unsigned(x)) * unsigned(a.ldo) + unsigned(co));
                if constexpr (RELU) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = fmaxf(v[q], 0.0f);
                    st4(o, v);
                } else {
                    st4(o, res[a0][b] + v);
                }
            }
    };
    // The residual a unit's epilogue adds to (channel block hh of its 2x2 outputs), read at
    // the start of the unit's last slice so that its latency is hidden by the products.
    auto load_res = [&](const WinoUnit& w, f4 (&res)[2][2]) {
#pragma unroll
        for (int a0 = 0; a0 < 2; ++a0)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int y = w.y0 + 2 * tr + a0, x = w.x0 + 2 * tc + b;
                res[a0][b] = (w.y0 >= 0 && y < a.H && x < a.W)
                                 ? ld4(a.out + ((unsigned(y) * unsigned(a.W) + unsigned(x)) * unsigned(a.ldo) +
                                                unsigned(w.co0 + hh * 16 + lg * 4)))
                                 : f4{0.f, 0.f, 0.f, 0.f};
            }
    };

    long u = blockIdx.x;
    if (u >= units) return;
    if constexpr (URES) {
        // U [16 xi][32 co][32 ci]: row r = xi * 32 + co, 16-byte slot c4 of the row stored at
        // slot c4 ^ (2 ((r >> 2) & 3)).
        for (int f = tid; f < 16 * 32 * 8; f += 512) {
            const int r = f >> 3, c4 = f & 7;
            st4(&ures[r * 32 + 4 * (c4 ^ (2 * ((r >> 2) & 3)))], ld4(a.w + long(r) * 32 + c4 * 4));
        }
    }
    WinoUnit cur = wino_unit(u, tx, nb, tiles, CB);
    unsigned hcur[HV], hnxt[HV];
    halo_offsets(cur, hcur);
    load(hcur, cur.co0, 0);
    stash(lds);
    __syncthreads();
    int kb = 0;                              // buffer of the current slice
    for (;;) {
        const long un = u + gridDim.x;
        const WinoUnit nxt = wino_unit(un, tx, nb, tiles, CB);
        halo_offsets(nxt, hnxt);
        f4 res[2][2];
        for (int c = 0; c < nch; ++c) {
            // Buffer kb holds slice c. The next step's slice is loaded now and stashed into
            // the other buffer after this slice's products: that buffer was last read in the
            // previous step, which every wave finished before the last barrier.
            const bool more = c + 1 < nch || un < units;
            if (c + 1 < nch) load(hcur, cur.co0, (c + 1) * BK);
            else if (un < units) load(hnxt, nxt.co0, 0);
            if constexpr (!RELU) {
                if (c + 1 == nch) load_res(cur, res);
            }
            const float* buf = lds + kb * BSZ;
            bool mrow = false;
            if constexpr (BATCH) {
                const int yo = cur.y0 + 2 * tr;
                mrow = hh == 0 ? yo % a.img_h == 0 : (yo + 2) % a.img_h == 0;
            }
            using I0 = std::integral_constant<int, 0>;
            using I1 = std::integral_constant<int, 1>;
            using T1 = std::integral_constant<bool, true>;
            using T0 = std::integral_constant<bool, false>;
            if (c == 0) {
                if (hh == 0) slice(I0{}, T1{}, buf, c * BK, mrow);
                else slice(I1{}, T1{}, buf, c * BK, mrow);
            } else {
                if (hh == 0) slice(I0{}, T0{}, buf, c * BK, mrow);
                else slice(I1{}, T0{}, buf, c * BK, mrow);
            }
            if (more) stash(lds + (kb ^ 1) * BSZ);
            __syncthreads();
            kb ^= 1;
        }
        // The last slice's buffer (kb ^ 1) is free: every wave passed the barrier after
        // reading it. The exchange goes there; a barrier after the reads keeps the next
        // stash (into that buffer) from overwriting partials a wave has not read yet.
        float* xbuf = URES ? xres : lds + (kb ^ 1) * BSZ;
        if (hh == 0) finish(std::integral_constant<int, 0>{}, cur, xbuf, res);
        else finish(std::integral_constant<int, 1>{}, cur, xbuf, res);
        // The next stash goes into the exchange buffer unless it has its own area; the
        // partials are read before the next unit's exchange (several barriers later).
        if constexpr (!URES) __syncthreads();
        if (un >= units) break;
        u = un;
        cur = nxt;
#pragma unroll
        for (int i = 0; i < HV; ++i) hcur[i] = hnxt[i];
    }
}

// ---------------------------------------------------------------------------
// Winograd F(2x2, 3x3) at cin = cout = 32 with split-operand products (the default fp32
// mode's form of level 0's 3x3). A unit is a 16 x 16-pixel tile x all 32 output channels,
// 8 waves: wave pair p owns tile rows 2p, 2p + 1 (16 tiles, lane li = tile) and within the
// pair wave half hh owns rows 2hh, 2hh + 1 of the transformed 4x4 positions for both
// 16-channel blocks, so each V is formed and split once. With K = cin = 32 one split product
// covers a position's whole reduction.
//   - U = G g G^T, split into three bf16 planes, stays in LDS for the workgroup's lifetime:
//     rows [16 xi][32 co] of 32 ci (96 KB), 16-byte chunks XOR-swizzled by bit 3 of the row,
//     so that a half-wave's 16 rows x 2 chunks fall on distinct 16-byte slots mod 32;
//   - the unit's 18 x 18 x 32 fp32 halo sits in one LDS buffer with a pixel pitch of 9 and a
//     row pitch of 24 x 9 slots: the 8 tile columns of a half-wave (2 pixels apart) and its
//     two tile rows (2 pixel rows apart, 16 slots mod 32) read distinct slots. The next unit's
//     halo is loaded into registers during the products;
//   - per transformed row the wave reads the two patch rows B^T combines (4 columns, the
//     lane's 8 channels 4 lg .. + 3 and 16 + 4 lg .. + 3: the k order of the products), forms
//     t = (B^T d)_i, then V = t B for the row's four positions, splits V and multiplies;
//   - the output transform is linear in the rows: each wave forms the partial 2x2 outputs
//     of its two rows, and the pair exchanges one channel block each through the halo buffer
//     (free once every wave has read it), before the next halo is stashed there.
// ---------------------------------------------------------------------------
template <bool RELU, bool BATCH>
__global__ __launch_bounds__(512) void k_wino6(Conv3Args a, long tiles, long units) {
    constexpr int HW = 18, HP = 24, LDC = 36;           // halo pixels per row, pitches (floats)
    constexpr int HSZ = HW * HP * LDC;                   // 15 552 floats
    constexpr int UPL = 16 * 32 * 32;                    // one U plane, bf16 elements
    constexpr int HV = (HW * HW * 8 + 511) / 512;        // halo float4 per thread
    static_assert(8 * 1024 <= HSZ, "the exchange fits in the halo buffer");
    __shared__ __align__(16) float lds[HSZ + 3 * UPL / 2];
    float* const hs = lds;
    __bf16* const us = reinterpret_cast<__bf16*>(lds + HSZ);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4, pair = wave >> 1, hh = wave & 1;
    const int tx = (a.W + 15) >> 4;
    const int tr = 2 * pair + (li >> 3), tc = li & 7;

    long u = blockIdx.x;
    if (u >= units) return;
    // U planes: item (row r = xi * 32 + co, lane group g) holds ci 4g .. + 3 and 16 + 4g .. + 3.
    for (int f = tid; f < 16 * 32 * 4; f += 512) {
        const int r = f >> 2, g = f & 3;
        const float* src = a.w + long(r) * 32;
        const x8 v = split8<true>(ld4(src + 4 * g), ld4(src + 16 + 4 * g));
        __bf16* d = us + r * 32 + 8 * (g ^ (((r >> 3) & 1) << 1));
        stb8(d, v.h);
        stb8(d + UPL, v.m);
        stb8(d + 2 * UPL, v.l);
    }

    constexpr unsigned NOFF = 0xffffffffu;
    auto halo_offsets = [&](const WinoUnit& w, unsigned (&ho)[HV]) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            const int f = tid + i * 512;
            const int px = f >> 3, q = f & 7;
            const int gy = w.y0 - 1 + px / HW, gx = w.x0 - 1 + px % HW;
            const bool ok = f < HW * HW * 8 && w.y0 >= 0 && gy >= 0 && gy < a.H && gx >= 0 && gx < a.W;
            ho[i] = ok ? (unsigned(gy) * unsigned(a.W) + unsigned(gx)) * unsigned(a.ldi) + unsigned(q * 4) : NOFF;
        }
    };
    f4 rh[HV];
    // Every halo element is loaded (pixels outside the plane from offset 0) and zeroed when it
    // is stashed: with no load under a branch, and no use of the loaded values before the
    // stash, the waits neither stall the products nor cover the previous unit's stores.
    auto load = [&](const unsigned (&ho)[HV]) {
#pragma unroll
        for (int i = 0; i < HV; ++i) rh[i] = ld4(a.in + (ho[i] != NOFF ? ho[i] : 0u));
    };
    auto stash = [&](const unsigned (&ho)[HV]) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
            const int f = tid + i * 512;
            if (f < HW * HW * 8) {
                const int px = f >> 3;
                st4(hs + ((px / HW) * HP + px % HW) * LDC + (f & 7) * 4,
                    ho[i] != NOFF ? rh[i] : f4{0.f, 0.f, 0.f, 0.f});
            }
        }
    };
    // The residual of the accumulate form: this lane's 2 x 2 outputs of channel block hh.
    auto load_res = [&](const WinoUnit& w, f4 (&res)[2][2]) {
#pragma unroll
        for (int a0 = 0; a0 < 2; ++a0)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                // Pixels past the plane (not stored) read the last row / column.
                const int y = min(max(w.y0, 0) + 2 * tr + a0, a.H - 1), x = min(w.x0 + 2 * tc + b, a.W - 1);
                res[a0][b] = ld4(a.out + ((unsigned(y) * unsigned(a.W) + unsigned(x)) * unsigned(a.ldo) +
                                          unsigned(hh * 16 + lg * 4)));
            }
    };

    WinoUnit cur = wino_unit(u, tx, 1, tiles, 32);
    unsigned hcur[HV], hnxt[HV];
    halo_offsets(cur, hcur);
    load(hcur);
    stash(hcur);
    __syncthreads();   // U and the first halo
    const float* const base = hs + ((2 * tr) * HP + 2 * tc) * LDC;
    const __bf16* const ub = us + li * 32 + 8 * (lg ^ ((li >> 3) << 1));
    // Exchange slots: a wave's 4 partial outputs x 64 lanes, output-major, so that each
    // 16-byte store or load of the wave covers 1 KB of consecutive LDS.
    float* const xo = hs + (pair * 2 + (1 - hh)) * 1024 + lane * 4;
    const float* const xin = hs + (pair * 2 + hh) * 1024 + lane * 4;
    for (;;) {
        const long un = u + gridDim.x;
        // The next unit's halo is requested on every path (the last unit re-reads its own):
        // with the loads under a branch, the wait before the first products would have to
        // assume the path without them and cover them too.
        const WinoUnit nxt = wino_unit(un < units ? un : u, tx, 1, tiles, 32);
        halo_offsets(nxt, hnxt);
        load(hnxt);
        f4 res[2][2];
        if constexpr (!RELU) load_res(cur, res);
        // Stacked images: patch row 0 above a tile that starts an image, or row 3 below one
        // that ends it, reads as zero padding.
        bool top = false, bot = false;
        if constexpr (BATCH) {
            const int yo = cur.y0 + 2 * tr;
            top = yo % a.img_h == 0;
            bot = (yo + 2) % a.img_h == 0;
        }
        // Partial outputs of this half's rows (channels 16 cb + 4 lg .. + 3): keep[a0][b] for
        // the wave's own block cb = hh, give[a0][b] for its partner's.
        // A^T = [1 1 1 0; 0 1 -1 -1]: with r_i[0] = M[i][0] + M[i][1] + M[i][2] and
        // r_i[1] = M[i][1] - M[i][2] - M[i][3], Y[0][b] = r_0 + r_1 + r_2 and
        // Y[1][b] = r_1 - r_2 - r_3. Each row is folded in as soon as its products are done.
        f4 keep[2][2], give[2][2];
        auto rows = [&](auto HHc) __attribute__((always_inline)) {
            constexpr int H2 = decltype(HHc)::value;
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                // (B^T d)_i, i = 2 H2 + ii: rows (d0 - d2), (d1 + d2), (d2 - d1), (d1 - d3).
                constexpr int RA[4] = {0, 1, 2, 1}, RB[4] = {2, 2, 1, 3};
                const int i = 2 * H2 + ii;
                f4 t[4][2];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float* pa = base + (RA[i] * HP + j) * LDC;
                    const float* pb = base + (RB[i] * HP + j) * LDC;
                    f4 a0 = ld4(pa + 4 * lg), a1 = ld4(pa + 16 + 4 * lg);
                    f4 b0 = ld4(pb + 4 * lg), b1 = ld4(pb + 16 + 4 * lg);
                    if constexpr (BATCH) {
                        if (i == 0 && top) a0 = a1 = f4{0.f, 0.f, 0.f, 0.f};
                        if (i == 3 && bot) b0 = b1 = f4{0.f, 0.f, 0.f, 0.f};
                    }
                    t[j][0] = i == 1 ? a0 + b0 : a0 - b0;
                    t[j][1] = i == 1 ? a1 + b1 : a1 - b1;
                }
                f4 r[2][2];   // r[cb][b]
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    // (t B)_c: columns (t0 - t2), (t1 + t2), (t2 - t1), (t1 - t3).
                    f4 v0, v1;
                    if (c == 0) { v0 = t[0][0] - t[2][0]; v1 = t[0][1] - t[2][1]; }
                    if (c == 1) { v0 = t[1][0] + t[2][0]; v1 = t[1][1] + t[2][1]; }
                    if (c == 2) { v0 = t[2][0] - t[1][0]; v1 = t[2][1] - t[1][1]; }
                    if (c == 3) { v0 = t[1][0] - t[3][0]; v1 = t[1][1] - t[3][1]; }
                    const x8 xv = split8<true>(v0, v1);
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        const f4 m = mfma6(ldx8(ub + ((i * 4 + c) * 32 + cb * 16) * 32, UPL), xv,
                                           f4{0.f, 0.f, 0.f, 0.f});
                        if (c == 0) r[cb][0] = m;
                        if (c == 1) { r[cb][0] += m; r[cb][1] = m; }
                        if (c == 2) { r[cb][0] += m; r[cb][1] -= m; }
                        if (c == 3) r[cb][1] -= m;
                    }
                }
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        f4 (&yp)[2][2] = cb == H2 ? keep : give;
                        if (i == 0) yp[0][b] = r[cb][b];
                        if (i == 1) { yp[0][b] += r[cb][b]; yp[1][b] = r[cb][b]; }
                        if (i == 2) { yp[0][b] = r[cb][b]; yp[1][b] = f4{0.f, 0.f, 0.f, 0.f} - r[cb][b]; }
                        if (i == 3) yp[1][b] -= r[cb][b];
                    }
            }
        };
        if (hh == 0) rows(std::integral_constant<int, 0>{});
        else rows(std::integral_constant<int, 1>{});
        __syncthreads();   // every wave is done with this unit's halo: the exchange may use it
        // This wave finishes channel block hh and hands block 1 - hh to its partner.
#pragma unroll
        for (int q = 0; q < 4; ++q) st4(xo + q * 256, give[q >> 1][q & 1]);
        __syncthreads();
        f4 got[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) got[q] = ld4(xin + q * 256);
        __syncthreads();   // the partials are read: the next halo may overwrite them
        if (un < units) stash(hnxt);
        if (cur.y0 >= 0) {
#pragma unroll
            for (int a0 = 0; a0 < 2; ++a0)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int y = cur.y0 + 2 * tr + a0, x = cur.x0 + 2 * tc + b;
                    if (y >= a.H || x >= a.W) continue;
                    f4 v = keep[a0][b] + got[a0 * 2 + b];
                    float* o = a.out + ((unsigned(y) * unsigned(a.W) + unsigned(x)) * unsigned(a.ldo) +
                                        unsigned(hh * 16 + lg * 4));
                    if constexpr (RELU) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[q] = fmaxf(v[q], 0.0f);
                        st4(o, v);
                    } else {
                        st4(o, res[a0][b] + v);
                    }
                }
        }
        __syncthreads();   // the next unit's halo is visible
        if (un >= units) break;
        u = un;
        cur = nxt;
#pragma unroll
        for (int i = 0; i < HV; ++i) hcur[i] = hnxt[i];
    }
}

template <bool BATCH>
static bool launch_wino6(const Conv3Args& a, bool relu, hipStream_t s, const char** why) {
    static std::atomic<int> cus_c[2] = {}, pc_c[2] = {};
    Occ oc;
    if (!query_occ(relu ? k_wino6<true, BATCH> : k_wino6<false, BATCH>, 512, cus_c[relu ? 1 : 0],
                   pc_c[relu ? 1 : 0], &oc)) {
        *why = "conv3x3_winograd: device query failed";
        return false;
    }
    const long tiles = long((a.W + 15) / 16) * ((a.H + 15) / 16);
    const long units = ((tiles + 7) / 8) * 8;
    const long grid = std::min<long>(units, long(oc.cus) * oc.per_cu);
    dim3 g{unsigned(grid), 1u, 1u}, block{512u, 1u, 1u};
    if (relu) hipLaunchKernelGGL((k_wino6<true, BATCH>), g, block, 0, s, a, tiles, units);
    else hipLaunchKernelGGL((k_wino6<false, BATCH>), g, block, 0, s, a, tiles, units);
    return true;
}

// ---------------------------------------------------------------------------
// Winograd F(2x2, 3x3), the small-footprint form: a unit is 8 x 16 output pixels (4 x 8
// tiles) x CB output channels (CB = 32 or 64), 4 waves, and the input channels go in
// slices of 8 whose halo (10 x 18 pixels) and filter part (16 xi x CB x 8) are
// double-buffered in LDS: 46 KB at CB = 32 (three workgroups per CU), 78 KB at CB = 64
// (two per CU). On gfx950 the fp32 matrix instructions and the VALU do not overlap (each
// VALU instruction delays the products by about as long as it takes), so the design
// keeps VALU per product low and lets the independent workgroups of a CU cover each
// other's barriers and epilogues:
//   - wave pair p owns tile rows 2p, 2p + 1 (16 tiles, lane li = tile) and each wave of the
//     pair owns two of the four rows of the transformed 4x4 positions for all CB output
//     channels: the input transform costs 1 VALU instruction per product at CB = 32 and
//     0.5 at CB = 64;
//   - halo and filter slices come in through buffer loads whose per-thread byte offsets
//     are fixed (the filter slice) or fixed per unit (the halo; positions outside the image
//     get an offset past the buffer range, which loads zeros), on 64-bit unit bases, so the
//     plane may exceed 2^32 elements;
//   - the filters are read in the layout [cin / 8][16 xi][cout][8] (one contiguous block per
//     slice), their 8-byte LDS slots XOR-swizzled by (row >> 2) & 3 so that the operand
//     reads are at the two-pass minimum;
//   - the output transform is linear in the rows: each wave forms the partial 2x2 outputs
//     of its rows, the pair exchanges half of the channel blocks through LDS, and each
//     wave finishes (ReLU or residual) and stores its half.
// The next step's slice (across unit boundaries too) is loaded while the current one is
// multiplied; one barrier per slice.
// ---------------------------------------------------------------------------
typedef float f2 __attribute__((ext_vector_type(2)));
DEVI f2 ld2(const float* p) { return *reinterpret_cast<const f2*>(p); }
DEVI void st2(float* p, f2 v) { *reinterpret_cast<f2*>(p) = v; }
// Raw buffer loads: a descriptor (base, 2 GB range, the gfx9 word 3) in scalar registers and
// a 32-bit per-lane byte offset; offsets at or past the range load zeros.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
DEVI rsrc_t rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7fffffff, 0x00020000);
}
DEVI f4 bld4(rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

template <int CB, bool RELU, bool BATCH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(CB == 32 ? 3 : 2, CB == 32 ? 3 : 2))) void k_wino3(Conv3Args a, int tx, int nb, int spatial, int units) {
    // a.w8: the filters as [cin / 8][16][cout][8].
    constexpr int BK = 8, PP = 10, HC = 18, HR = 10, NCB = CB / 16, NU = CB / 8;
    constexpr int HSZ = HR * HC * PP;      // 1800 floats
    constexpr int USZ = 16 * CB * BK;      // 4096 floats
    constexpr int BSZ = HSZ + USZ;
    __shared__ __align__(16) float lds[2 * BSZ];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4, pair = wave >> 1, hh = wave & 1;
    const int tr = 2 * pair + (li >> 3), tc = li & 7;
    const int nch = a.cin / BK;
    const long W = a.W;

    struct Unit { int y0, x0, co0; };
    auto unit_at = [&](int u) {
        const unsigned uu = unsigned(u), xcd = uu & 7u, j = uu >> 3;
        const unsigned q = j / unsigned(nb), sp = q * 8u + xcd;
        Unit w;
        w.co0 = int(j - q * unsigned(nb)) * CB;
        const unsigned uy = sp / unsigned(tx);
        w.y0 = int(sp) < spatial ? int(uy) * 8 : -1;
        w.x0 = int(sp - uy * unsigned(tx)) * 16;
        return w;
    };
    // Halo f4 number f = tid + 256 i of the 10 x 18 x 8 slice (f < 360): byte offset from the
    // halo origin (y0 - 1, x0 - 1), fixed per thread; per unit it becomes NOFF (past the
    // buffer range: the load returns zeros) where the pixel is outside the image.
    // These per-thread constants are recomputed for every unit (a few integer instructions,
    // from an opaque copy of tid so that they are not hoisted back out of the unit loop)
    // rather than held for the kernel's lifetime: held, they were spilled at CB = 64.
    constexpr int NOFF = int(0x80000000u);
    auto halo_offsets = [&](const Unit& w, int (&ho)[2]) {
        int otid = tid;
        asm volatile("" : "+v"(otid));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int f = otid + 256 * i, px = f >> 1, hf = f & 1;
            const int hy = px / HC, hx = px - hy * HC;
            const int hfix = ((hy * int(a.W) + hx) * int(a.ldi) + hf * 4) * 4;
            const int hgy = f < HR * HC * 2 ? hy : -1000000;
            const int gy = w.y0 - 1 + hgy, gx = w.x0 - 1 + hx;
            bool ok = w.y0 >= 0 && gy >= 0 && gy < a.H && gx >= 0 && gx < a.W;
            if constexpr (BATCH) {
                if ((hgy == 0 && w.y0 % a.img_h == 0) || (hgy == HR - 1 && (w.y0 + 8) % a.img_h == 0)) ok = false;
            }
            ho[i] = ok ? hfix : NOFF;
        }
    };
    // Filter slice: f4 number f = tid + 256 i is row r = f >> 1 = (tid >> 1) + 128 i of the
    // [16 xi][CB co] x 8 ci slice, half tid & 1; byte offset fixed per thread plus i * ustep.
    const int uoff = ((((tid >> 1) / CB) * a.cout + ((tid >> 1) % CB)) * BK + (tid & 1) * 4) * 4;
    const int ustep = (128 / CB) * a.cout * BK * 4;
    f4 rh[2], ru[NU];
    auto load = [&](const Unit& w, const int (&ho)[2], int cs) {
        const float* hb = a.in + ((long(w.y0) - 1) * W + (w.x0 - 1)) * a.ldi + cs * BK;
        const rsrc_t hr = rsrc(hb);
#pragma unroll
        for (int i = 0; i < 2; ++i) rh[i] = bld4(hr, ho[i], 0);
        const rsrc_t ur = rsrc(a.w8 + (long(cs) * 16 * a.cout + w.co0) * BK);
#pragma unroll
        for (int i = 0; i < NU; ++i) ru[i] = bld4(ur, uoff, i * ustep);
    };
    // LDS stash bases (floats), fixed per thread: halo pixel (tid >> 1) + 128 i; filter row
    // (tid >> 1) + 128 i with its 8-byte slots XOR-swizzled by g = (row >> 2) & 3, which is
    // (tid >> 3) & 3 for every i.
    const int hl = (tid >> 1) * PP + (tid & 1) * 4;
    const int ug = (tid >> 3) & 3;
    const int ul0 = (tid >> 1) * 8 + 2 * ((2 * (tid & 1)) ^ ug);
    const int ul1 = (tid >> 1) * 8 + 2 * ((2 * (tid & 1) + 1) ^ ug);
    const bool h2nd = tid + 256 < HR * HC * 2;
    auto stash = [&](float* buf) {
        st2(buf + hl, f2{rh[0][0], rh[0][1]});
        st2(buf + hl + 2, f2{rh[0][2], rh[0][3]});
        if (h2nd) {
            st2(buf + hl + 128 * PP, f2{rh[1][0], rh[1][1]});
            st2(buf + hl + 128 * PP + 2, f2{rh[1][2], rh[1][3]});
        }
        float* us = buf + HSZ;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            st2(us + ul0 + i * 1024, f2{ru[i][0], ru[i][1]});
            st2(us + ul1 + i * 1024, f2{ru[i][2], ru[i][3]});
        }
    };
    const int gread = (li >> 2) & 3;
    const int pbase = ((2 * tr + hh) * HC + 2 * tc) * PP + 2 * lg;
    f4 acc[NCB][2][4];
    auto slice = [&](auto HHc, auto FIRSTc, const float* buf) {
        constexpr int H2 = decltype(HHc)::value;
        constexpr bool FIRST = decltype(FIRSTc)::value;
        const float* Us = buf + HSZ + li * 8 + 2 * (lg ^ gread);
        f2 t[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float* col = buf + pbase + j * PP;
            const f2 da = ld2(col), db = ld2(col + HC * PP), dc = ld2(col + 2 * HC * PP);
            if constexpr (H2 == 0) {
                t[0][j] = da - dc;
                t[1][j] = db + dc;
            } else {
                t[0][j] = db - da;
                t[1][j] = da - dc;
            }
        }
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const f2 v[4] = {t[ii][0] - t[ii][2], t[ii][1] + t[ii][2], t[ii][2] - t[ii][1], t[ii][1] - t[ii][3]};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) {
                    const int r = ((2 * H2 + ii) * 4 + j) * CB + cb * 16;
                    const f2 uu = ld2(Us + r * 8);
                    acc[cb][ii][j] = mfma4(uu[0], v[j][0], FIRST ? f4{0.f, 0.f, 0.f, 0.f} : acc[cb][ii][j]);
                    acc[cb][ii][j] = mfma4(uu[1], v[j][1], acc[cb][ii][j]);
                }
        }
    };
    // Each wave keeps NCB / 2 of its channel blocks (the ones of half hh) and hands the other
    // half's partial outputs to its partner through LDS.
    constexpr int NK = NCB / 2;
    auto finish = [&](auto HHc, const Unit& w, float* xb) {
        constexpr int H2 = decltype(HHc)::value;
        f4 yp[NCB][2][2];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            f4 r[2][2];
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                r[ii][0] = acc[cb][ii][0] + acc[cb][ii][1] + acc[cb][ii][2];
                r[ii][1] = acc[cb][ii][1] - acc[cb][ii][2] - acc[cb][ii][3];
            }
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                if constexpr (H2 == 0) {
                    yp[cb][0][b] = r[0][b] + r[1][b];
                    yp[cb][1][b] = r[1][b];
                } else {
                    yp[cb][0][b] = r[0][b];
                    yp[cb][1][b] = f4{0.f, 0.f, 0.f, 0.f} - r[0][b] - r[1][b];
                }
            }
        }
        float* xo = xb + ((wave ^ 1) * 64 + lane) * 16 * NK;
#pragma unroll
        for (int k = 0; k < NK; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q) st4(xo + 16 * k + 4 * ((q + lane) & 3), yp[(1 - H2) * NK + k][q >> 1][q & 1]);
        __syncthreads();
        const float* xi = xb + (wave * 64 + lane) * 16 * NK;
        f4 got[NK][4];
#pragma unroll
        for (int k = 0; k < NK; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q) got[k][q] = ld4(xi + 16 * k + 4 * ((q + lane) & 3));
        __syncthreads();
        if (w.y0 < 0) return;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int co = w.co0 + (H2 * NK + k) * 16 + lg * 4;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int a0 = q >> 1, b = q & 1;
                const int y = w.y0 + 2 * tr + a0, x = w.x0 + 2 * tc + b;
                if (y >= a.H || x >= a.W) continue;
                f4 v = yp[H2 * NK + k][a0][b] + got[k][q];
                float* o = a.out + (long(y) * W + x) * a.ldo + co;
                if constexpr (RELU) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = fmaxf(v[e], 0.0f);
                    st4(o, v);
                } else {
                    st4(o, ld4(o) + v);
                }
            }
        }
    };

    int u = blockIdx.x;
    if (u >= units) return;
    Unit cur = unit_at(u);
    int hcur[2], hnxt[2];
    halo_offsets(cur, hcur);
    load(cur, hcur, 0);
    stash(lds);
    __syncthreads();
    int kb = 0;
    for (;;) {
        const int un = u + int(gridDim.x);
        const Unit nxt = unit_at(un < units ? un : u);
        halo_offsets(nxt, hnxt);
        for (int c = 0; c < nch; ++c) {
            const bool more = c + 1 < nch || un < units;
            if (c + 1 < nch) load(cur, hcur, c + 1);
            else if (un < units) load(nxt, hnxt, 0);
            const float* buf = lds + kb * BSZ;
            using I0 = std::integral_constant<int, 0>;
            using I1 = std::integral_constant<int, 1>;
            using T1 = std::integral_constant<bool, true>;
            using T0 = std::integral_constant<bool, false>;
            if (c == 0) {
                if (hh == 0) slice(I0{}, T1{}, buf);
                else slice(I1{}, T1{}, buf);
            } else {
                if (hh == 0) slice(I0{}, T0{}, buf);
                else slice(I1{}, T0{}, buf);
            }
            if (more) stash(lds + (kb ^ 1) * BSZ);
            __syncthreads();
            kb ^= 1;
        }
        // The last slice's buffer (kb ^ 1) is free: its filter part takes the exchange.
        float* xb = lds + (kb ^ 1) * BSZ + HSZ;
        if (hh == 0) finish(std::integral_constant<int, 0>{}, cur, xb);
        else finish(std::integral_constant<int, 1>{}, cur, xb);
        if (un >= units) break;
        u = un;
        cur = nxt;
        hcur[0] = hnxt[0];
        hcur[1] = hnxt[1];
    }
}

template <bool BATCH>
static bool launch_wino(const Conv3Args& a, bool relu, bool wide, bool ures, hipStream_t s, const char** why) {
    static std::atomic<int> cus_c[8] = {}, pc_c[8] = {};
    auto occ = [&](int v, void (*kern)(Conv3Args, long, long), int threads, Occ* oc) {
        if (query_occ(kern, threads, cus_c[v], pc_c[v], oc)) return true;
        *why = "conv3x3_winograd: device query failed";
        return false;
    };
    const int nb = a.cout / (wide ? 32 : 16);
    const long tiles = long((a.W + 15) / 16) * ((a.H + 15) / 16);
    // Units are numbered 8 j + xcd with j < ceil(tiles / 8) * nb; numbers whose tile is
    // past the end (the last partial group of 8) carry y0 = -1 and do no loads or stores.
    const long units = ((tiles + 7) / 8) * 8 * nb;
    if (!ures && !wide) {
        // 16-channel units: 16 x 16 tiles, or pairs of 8 x 16 half-tiles when those take
        // fewer rounds of the persistent grid (or when a.pair asks for them).
        Occ o16, op;
        if (!occ(relu ? 1 : 0, relu ? k_wino<true, BATCH, false> : k_wino<false, BATCH, false>, 256, &o16) ||
            !occ(relu ? 7 : 6, relu ? k_wino<true, BATCH, true> : k_wino<false, BATCH, true>, 256, &op))
            return false;
        const long pairs = (long((a.W + 15) / 16) * ((a.H + 7) / 8) + 1) / 2;
        const long punits = ((pairs + 7) / 8) * 8 * nb;
        const long g16 = std::min<long>(units, long(o16.cus) * o16.per_cu);
        const long gp = std::min<long>(punits, long(op.cus) * op.per_cu);
        const bool pair = a.pair == 1 || (punits + gp - 1) / gp < (units + g16 - 1) / g16;
        dim3 g{unsigned(pair ? gp : g16), 1u, 1u}, block{256u, 1u, 1u};
        if (pair) {
            if (relu) hipLaunchKernelGGL((k_wino<true, BATCH, true>), g, block, 0, s, a, pairs, punits);
            else hipLaunchKernelGGL((k_wino<false, BATCH, true>), g, block, 0, s, a, pairs, punits);
        } else {
            if (relu) hipLaunchKernelGGL((k_wino<true, BATCH, false>), g, block, 0, s, a, tiles, units);
            else hipLaunchKernelGGL((k_wino<false, BATCH, false>), g, block, 0, s, a, tiles, units);
        }
        return true;
    }
    const int v = (relu ? 1 : 0) + (ures ? 4 : 2);
    Occ oc;
    if (!occ(v, ures ? (relu ? k_wino2<true, true, BATCH> : k_wino2<false, true, BATCH>)
                     : (relu ? k_wino2<true, false, BATCH> : k_wino2<false, false, BATCH>),
             512, &oc))
        return false;
    const long grid = std::min<long>(units, long(oc.cus) * oc.per_cu);
    dim3 g{unsigned(grid), 1u, 1u}, block{512u, 1u, 1u};
    if (ures) {
        if (relu) hipLaunchKernelGGL((k_wino2<true, true, BATCH>), g, block, 0, s, a, tiles, units);
        else hipLaunchKernelGGL((k_wino2<false, true, BATCH>), g, block, 0, s, a, tiles, units);
    } else {
        if (relu) hipLaunchKernelGGL((k_wino2<true, false, BATCH>), g, block, 0, s, a, tiles, units);
        else hipLaunchKernelGGL((k_wino2<false, false, BATCH>), g, block, 0, s, a, tiles, units);
    }
    return true;
}

template <int CB, bool BATCH>
static bool launch_wino3(const Conv3Args& a, bool relu, hipStream_t s, const char** why) {
    static std::atomic<int> cus_c[2] = {}, pc_c[2] = {};
    const int tx = (a.W + 15) / 16, ty = (a.H + 7) / 8;
    const long spatial = long(tx) * ty, nb = a.cout / CB;
    const long units = ((spatial + 7) / 8) * 8 * nb;
    if (units >= (1L << 31)) {
        *why = "conv3x3_winograd: more than 2^31 units";
        return false;
    }
    Occ oc;
    if (!query_occ(relu ? k_wino3<CB, true, BATCH> : k_wino3<CB, false, BATCH>, 256, cus_c[relu ? 1 : 0],
                   pc_c[relu ? 1 : 0], &oc)) {
        *why = "conv3x3_winograd: device query failed";
        return false;
    }
    const unsigned grid = unsigned(std::min<long>(units, long(oc.cus) * oc.per_cu));
    if (relu)
        hipLaunchKernelGGL((k_wino3<CB, true, BATCH>), dim3(grid), dim3(256), 0, s, a, tx, int(nb), int(spatial),
                           int(units));
    else
        hipLaunchKernelGGL((k_wino3<CB, false, BATCH>), dim3(grid), dim3(256), 0, s, a, tx, int(nb), int(spatial),
                           int(units));
    return true;
}

// The Winograd kernel a convolution runs on (none: the plane is too large for every form).
//   - k_wino3 (64-bit unit bases, 32-bit in-unit byte offsets: 10 halo rows of the plane must
//     span less than 2^31 bytes; stacked images in units of 8 rows) at 64 or more output
//     channels, where it is the fastest form: 64-channel units above 64 input channels,
//     32-channel units at 64 (level 1: 212 -> 208 us, twice the units at three workgroups
//     per CU) and for planes past 2^32 elements;
//   - k_wino6 (split-operand products) at cin = cout = 32 when the arguments ask for them;
//   - k_wino2 / k_wino (32-bit element offsets) elsewhere.
enum class WinoForm { k3_64, k3_32, split32, other, none };
static WinoForm wino_form(const Conv3Args& a, bool batch) {
    const bool fits32 = double(a.H) * a.W * a.ldi < 4294967296.0 && double(a.H) * a.W * a.ldo < 4294967296.0 &&
                        double(a.cout) * a.cin * 16 < 4294967296.0;
    const bool k3 = a.w8 && a.cblock == 0 && a.cin % 8 == 0 && a.cout % 32 == 0 &&
                    10.0 * a.W * a.ldi * 4 < 2147483648.0 && (!batch || a.img_h % 8 == 0);
    if (k3 && a.wino3 && ((a.cin >= 64 && a.cout % 64 == 0) || a.wino3 == 2))
        return a.cout % 64 == 0 && a.cin > 64 ? WinoForm::k3_64 : WinoForm::k3_32;
    if (!fits32) return !k3 ? WinoForm::none : a.cout % 64 == 0 ? WinoForm::k3_64 : WinoForm::k3_32;
    const bool ures = a.cout == 32 && a.cin == 32 && a.cblock != 16;
    return ures && a.split ? WinoForm::split32 : WinoForm::other;
}

bool conv3x3_winograd_split(const Conv3Args& a) {
    return wino_form(a, a.img_h > 0 && a.img_h < a.H) == WinoForm::split32;
}

bool conv3x3_winograd(const Conv3Args& a, bool relu, hipStream_t s, const char** why) {
    if (a.cin % 16 != 0 || a.cout % 16 != 0 || (a.H & 1) || (a.W & 1)) {
        *why = "conv3x3_winograd: cin and cout must be multiples of 16 and the plane even";
        return false;
    }
    const bool batch = a.img_h > 0 && a.img_h < a.H;
    if (batch && ((a.img_h & 1) || a.H % a.img_h != 0)) {
        *why = "conv3x3_winograd: stacked images must have an even height that divides the plane";
        return false;
    }
    switch (wino_form(a, batch)) {
    case WinoForm::k3_64:
        return batch ? launch_wino3<64, true>(a, relu, s, why) : launch_wino3<64, false>(a, relu, s, why);
    case WinoForm::k3_32:
        return batch ? launch_wino3<32, true>(a, relu, s, why) : launch_wino3<32, false>(a, relu, s, why);
    case WinoForm::split32:
        return batch ? launch_wino6<true>(a, relu, s, why) : launch_wino6<false>(a, relu, s, why);
    case WinoForm::none:
        *why = "conv3x3_winograd: plane too large for 32-bit element offsets";
        return false;
    case WinoForm::other:
        break;
    }
    // 32 output channels per unit, except at cin >= 256 (level 3 of the forward), where the
    // 16-channel kernel measured faster (238 against 247 us per launch at 1080p).
    const bool wide = a.cout % 32 == 0 && a.cin >= 32 && a.cin < 256 && a.cblock != 16;
    const bool ures = wide && a.cin == 32 && a.cout == 32;
    return batch ? launch_wino<true>(a, relu, wide, ures, s, why) : launch_wino<false>(a, relu, wide, ures, s, why);
}

// ---------------------------------------------------------------------------
// The fp16-operand 3x3 convolution (cin = cout = C), a direct implicit GEMM:
// out^T[co][px] = sum over taps (ky, kx) and ci of W[ky*3+kx][co][ci] in[px + (ky-1, kx-1)][ci].
// With fp16 products 16x cheaper than fp32 ones, the transforms of the Winograd form would
// cost more than the multiplications they save, so this form does 2.25x the products and
// no transforms.
//   - A workgroup owns an R-row x TW-column output tile. Its (R+2) x (TW+2) halo, all C
//     channels, is staged once into LDS as fp16: each 16-byte slot q = 4b + g of a pixel
//     packs channels 32b + 4g .. + 3 and 32b + 16 + 4g .. + 3, the k order of the f16
//     product, so a thread's two float4 loads convert straight into one slot. Pixels are
//     SP + 2 slots apart (SP = C / 8): 16 consecutive pixels x 2 slots land on distinct
//     16-byte slots mod 32, so operand reads are conflict-free, and every read is a fixed
//     per-lane base plus a compile-time offset.
//   - Wave w computes 32 output channels (co-group w % (C/32)) of a 16-pixel-wide strip
//     (w / (C/32)) for all R rows. Each halo-row fragment (16 pixels x 32 channels) read
//     for horizontal tap kx serves the output rows it is the ky = 0, 1, 2 tap of: 3 rows x
//     2 channel tiles of products per read.
//   - The k-permuted fp16 filters come from global memory: all of them held in registers
//     for C <= 64, else one 32-channel block at a time with the next block's loads in
//     flight during the current block's products.
// ---------------------------------------------------------------------------
template <int C, int R, int NWV, bool RELU>
__global__ __launch_bounds__(NWV * 64) void k_conv3h(Conv3Args a, int tiles_x, long tiles) {
    constexpr int CG = C / 32, KK = C / 32;
    static_assert(NWV % CG == 0, "the waves split into whole co-groups");
    constexpr int STRIPS = NWV / CG, TW = 16 * STRIPS, RP = TW + 2;
    constexpr int SP = C / 8, SPP = SP + 2;
    constexpr bool WRES = KK <= 2;                 // every filter block resident
    constexpr int NA = WRES ? KK : 2;              // filter blocks held (resident, or double buffer)
    __shared__ __align__(16) _Float16 halo[(R + 2) * RP * SPP * 8];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int cog = wave % CG, strip = wave / CG;
    const long ti = xcd_swizzle(blockIdx.x, gridDim.x);
    if (ti >= tiles) return;   // no barrier is reached by any wave of this workgroup
    const int ty = int(ti / tiles_x), tx = int(ti - long(ty) * tiles_x);
    const int y0 = ty * R, x0 = tx * TW;
    // The rows of this tile's image (R divides the image height: a tile never straddles).
    const int ih = a.img_h > 0 ? a.img_h : a.H;
    const int ylo = (y0 / ih) * ih, yhi = ylo + ih;

    // Filter fragments: A[tap][j] = W[tap][cog*32 + 16j + li][32kk + 8lg .. (k-permuted)].
    h8 wa[NA][9][2];
    auto wload = [&](int kk, h8 (&dst)[9][2]) {
#pragma unroll
        for (int tap = 0; tap < 9; ++tap)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                dst[tap][j] = ldh8(a.w16 + (long(tap * C + cog * 32 + j * 16 + li) * C + kk * 32 + lg * 8));
    };
#pragma unroll
    for (int k = 0; k < NA; ++k) wload(k, wa[k]);

    // Stage the halo (zero outside the plane: the convolution's zero padding), four passes
    // of the workgroup at a time (two above 32 channels, where the filters hold more
    // registers): their reads come from clamped addresses and are issued
    // together, and the zeros are selected at the LDS store (a read under the bounds test
    // was waited for in its own pass, one L2 round trip each).
    constexpr int NSLOT = (R + 2) * RP * SP, NTH = NWV * 64, NPASS = (NSLOT + NTH - 1) / NTH, PB = C <= 32 ? 4 : 2;
#pragma unroll
    for (int i0 = 0; i0 < NPASS; i0 += PB) {
        f4 va[PB], vb[PB];
        bool ok[PB];
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            const int f = tid + (i0 + j) * NTH, fc = f < NSLOT ? f : NSLOT - 1;
            const int q = fc % SP, p = fc / SP;
            const int hr = p / RP, hc = p - hr * RP;
            const int gy = y0 - 1 + hr, gx = x0 - 1 + hc;
            ok[j] = i0 + j < NPASS && f < NSLOT && gy >= ylo && gy < yhi && gx >= 0 && gx < a.W;
            const int cy = min(max(gy, ylo), yhi - 1), cx = min(max(gx, 0), a.W - 1);
            const float* src = a.in + (long(cy) * a.W + cx) * a.ldi + 32 * (q >> 2) + 4 * (q & 3);
            va[j] = ld4(src);
            vb[j] = ld4(src + 16);
        }
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            const int f = tid + (i0 + j) * NTH;
            if (i0 + j < NPASS && f < NSLOT)
                sth8(halo + ((f / SP) * SPP + f % SP) * 8, ok[j] ? pack8(va[j], vb[j]) : h8{0, 0, 0, 0, 0, 0, 0, 0});
        }
    }
    __syncthreads();

    f4 acc[R][2];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r][0] = acc[r][1] = f4{0.f, 0.f, 0.f, 0.f};
    const _Float16* hb = halo + ((strip * 16 + li) * SPP + lg) * 8;
    auto block = [&](int kk, const h8 (&w)[9][2]) {
#pragma unroll
        for (int dx = 0; dx < 3; ++dx)
#pragma unroll
            for (int hr = 0; hr < R + 2; ++hr) {
                const h8 b = ldh8(hb + ((hr * RP + dx) * SPP + kk * 4) * 8);
#pragma unroll
                for (int dy = 0; dy < 3; ++dy) {
                    const int r = hr - dy;
                    if (r < 0 || r >= R) continue;
#pragma unroll
                    for (int j = 0; j < 2; ++j) acc[r][j] = mfma16(w[dy * 3 + dx][j], b, acc[r][j]);
                }
            }
    };
    if constexpr (WRES) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) block(kk, wa[kk]);
    } else {
#pragma unroll 1
        for (int kk = 0; kk < KK; kk += 2) {
            block(kk, wa[0]);
            if (kk + 2 < KK) wload(kk + 2, wa[0]);
            block(kk + 1, wa[1]);
            if (kk + 3 < KK) wload(kk + 3, wa[1]);
        }
    }

    // Lanes hold output channels cog*32 + 16j + 4lg .. + 3 of pixel (y0 + r, x0 + 16 strip + li).
    const int x = x0 + strip * 16 + li;
    if (x >= a.W) return;
    // Accumulate form: the residual reads of all R rows are issued together, from clamped
    // rows, before the first store (one at a time under the row test, each was waited for).
    f4 res[RELU ? 1 : R][2];
    if constexpr (!RELU) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int yc = min(y0 + r, a.H - 1);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                res[r][j] = ld4(a.out + (long(yc) * a.W + x) * a.ldo + cog * 32 + j * 16 + lg * 4);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int y = y0 + r;
        if (y >= a.H) break;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float* o = a.out + (long(y) * a.W + x) * a.ldo + cog * 32 + j * 16 + lg * 4;
            if constexpr (RELU) {
                const f4 v = acc[r][j];
                st4(o, f4{fmaxf(v.x, 0.f), fmaxf(v.y, 0.f), fmaxf(v.z, 0.f), fmaxf(v.w, 0.f)});
            } else {
                st4(o, res[r][j] + acc[r][j]);
            }
        }
    }
}

template <int C, int R, int NWV>
static void launch_conv3h(const Conv3Args& a, bool relu, hipStream_t s) {
    constexpr int TW = 16 * (NWV / (C / 32));
    const int tiles_x = (a.W + TW - 1) / TW;
    const long tiles = long(tiles_x) * ((a.H + R - 1) / R);
    dim3 grid{unsigned(tiles), 1u, 1u}, block{unsigned(NWV * 64), 1u, 1u};
    if (relu) hipLaunchKernelGGL((k_conv3h<C, R, NWV, true>), grid, block, 0, s, a, tiles_x, tiles);
    else hipLaunchKernelGGL((k_conv3h<C, R, NWV, false>), grid, block, 0, s, a, tiles_x, tiles);
}

bool conv3x3_h16(const Conv3Args& a, bool relu, hipStream_t s, const char** why) {
    if (!a.w16 || a.cin != a.cout) {
        *why = "conv3x3_h16: needs the k-permuted fp16 filters and cin == cout";
        return false;
    }
    if (a.img_h > 0 && (a.img_h % 8 != 0 || a.H % a.img_h != 0)) {
        *why = "conv3x3_h16: stacked images must be a multiple of 8 rows high";
        return false;
    }
    if (a.H <= 0 || a.W <= 0) return true;
    // 256 channels: 8-row tiles, so each streamed filter block feeds twice the pixels (level 3
    // of the 1080p forward: 87 -> 59 us per launch).
    switch (a.cin) {
        case 32: launch_conv3h<32, 8, 4>(a, relu, s); break;
        case 64: launch_conv3h<64, 8, 4>(a, relu, s); break;
        case 128: launch_conv3h<128, 8, 4>(a, relu, s); break;
        case 256: launch_conv3h<256, 8, 8>(a, relu, s); break;
        default: *why = "conv3x3_h16: channels must be 32, 64, 128 or 256"; return false;
    }
    return true;
}

void winograd_filter(const float* g, int cout, int cin, float* u) {
    static const double G[4][3] = {{1, 0, 0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0, 0, 1}};
    for (int o = 0; o < cout; ++o)
        for (int c = 0; c < cin; ++c) {
            const float* k = g + (long(o) * cin + c) * 9;
            double t[4][3];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 3; ++j) t[i][j] = G[i][0] * k[j] + G[i][1] * k[3 + j] + G[i][2] * k[6 + j];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j)
                    u[(long(i * 4 + j) * cout + o) * cin + c] =
                        float(t[i][0] * G[j][0] + t[i][1] * G[j][1] + t[i][2] * G[j][2]);
        }
}

void build_gelu_table(float* tab) {
    // Abramowitz & Stegun 7.1.26, the erf of cpu.rs:318-332, in double.
    auto erf_as = [](double x) {
        const double t = 1.0 / (1.0 + 0.3275911 * std::fabs(x));
        const double y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t +
                                0.254829592) * t * std::exp(-x * x);
        return x >= 0 ? y : -y;
    };
    auto phi = [&](double v) { return 0.5 * (1.0 + erf_as(v / std::sqrt(2.0))); };
    for (int i = 0; i < GELU_PIECES; ++i) {
        // The cubic through f = 0, 1/3, 2/3, 1 of the piece [x0, x0 + 1/16): forward
        // differences in s = 3 f, expanded into powers of f.
        const double x0 = -6.0 + i / 16.0, h = 1.0 / 16.0;
        const double y0 = phi(x0), y1 = phi(x0 + h / 3), y2 = phi(x0 + 2 * h / 3), y3 = phi(x0 + h);
        const double d1 = y1 - y0, d2 = y2 - 2 * y1 + y0, d3 = y3 - 3 * y2 + 3 * y1 - y0;
        tab[4 * i + 0] = float(y0);
        tab[4 * i + 1] = float(3.0 * (d1 - d2 / 2 + d3 / 3));
        tab[4 * i + 2] = float(9.0 * (d2 / 2 - d3 / 2));
        tab[4 * i + 3] = float(4.5 * d3);
    }
}

void winograd_filter_slices(const float* u, int cout, int cin, float* u8) {
    for (int xi = 0; xi < 16; ++xi)
        for (int o = 0; o < cout; ++o)
            for (int c = 0; c < cin; ++c)
                u8[((long(c / 8) * 16 + xi) * cout + o) * 8 + c % 8] = u[(long(xi) * cout + o) * cin + c];
}

// ---------------------------------------------------------------------------
// Window attention, 8x8 windows (64 tokens), head_dim 32. One wave per (window, head).
//   S^T = K Q^T on MFMA (keys are the M rows, queries the N columns), so after the
//   product each lane holds, for ONE query, 16 of its 64 key logits; the other 48
//   are in the lanes 16, 32 and 48 away. Softmax: max and sum over the 16 values and a
//   two-step xor shuffle. The exponentials are then exactly the B operand of
//   O^T = V^T P^T (lane = query, registers = 4 consecutive keys of the lane's key group),
//   so no data moves between the two products and nothing goes through LDS; the 1/sum
//   normalisation is applied to the 8 outputs rather than the 16 weights.
// Logits are kept in log2 units, l = (q.k) * scale * log2(e) + log2(e) * bias, so a logit is
// one FMA and softmax uses 2^(l - max); masked logits are -FLT_MAX/4 (cpu.rs:365-370,
// 681-683). The per-head 15x15 bias tables sit in LDS; each lane reads the entries its 64
// logits use where the logits are formed. V is read transposed straight from memory (4-byte
// loads, 64 contiguous bytes per key), so the only LDS is the 7.2 KB of tables and the
// kernel fits in 128 VGPRs: four waves per SIMD, 4 096 (window, head) units in flight. The
// split-operand form (X6) holds K and V in split form, ~165 VGPRs: three waves per SIMD.
// ---------------------------------------------------------------------------
template <bool WIDE, int QS, bool X6 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(X6 ? 3 : 4, X6 ? 3 : 4))) void k_attention(AttnArgs a, long units) {
    // Element offsets: 32-bit (WIDE = false) unless the qkv plane reaches 2^32 elements.
    using U = typename std::conditional<WIDE, unsigned long, unsigned>::type;
    __shared__ float rps[8 * 225];                // log2(e) * rel-pos tables, all heads
    for (int i = threadIdx.x; i < a.heads * 225; i += 256) rps[i] = a.tab[i];
    __syncthreads();                              // the only barrier
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long u = long(blockIdx.x) * 4 + wave;
    if (u >= units) return;                      // whole wave exits together
    const int li = lane & 15, lg = lane >> 4;
    // A unit is (window, head, query part): QS parts of NQ = 4 / QS query tiles each. Unit
    // and window indices fit 32 bits (the launch grid is 32-bit).
    constexpr int NQ = 4 / QS;
    const unsigned wh_u = unsigned(u) / unsigned(QS);
    const int part = int(unsigned(u) - wh_u * unsigned(QS));
    const unsigned wi = wh_u / unsigned(a.heads);
    const int h = int(wh_u - wi * unsigned(a.heads));
    const int wh = int(wi / unsigned(a.nww)), ww = int(wi - unsigned(wh) * unsigned(a.nww));
    const int hoff = h * 32;

    // Element offsets of the rows of tokens 16m + li (Q and K: 16-byte row loads), and the
    // row and column parts of tokens 16kt + 4lg + r (V, read transposed: lane li takes dim
    // 16nd + li of those 4 keys with 4-byte loads, 64 contiguous bytes per key and
    // instruction). In pixel mode token (ty, tx) of window (wh, ww) is pixel
    // ((8wh + ty + shift) mod H, (8ww + tx + shift) mod W) (cpu.rs:648-652's cyclic shift
    // folded into the addressing).
    U off[4], offq[NQ], vy[4], vx[4];
    if (a.pixel_mode) {
        auto wy = [&](int ty) { int y = wh * 8 + ty + a.shift; return U(y >= a.H ? y - a.H : y); };
        auto wx = [&](int tx) { int x = ww * 8 + tx + a.shift; return U(x >= a.W ? x - a.W : x); };
        const U xq = wx(li & 7);
#pragma unroll
        for (int m = 0; m < 4; ++m) off[m] = (wy(2 * m + (li >> 3)) * U(a.W) + xq) * U(a.ldq);
#pragma unroll
        for (int j = 0; j < NQ; ++j) offq[j] = (wy(2 * (part * NQ + j) + (li >> 3)) * U(a.W) + xq) * U(a.ldq);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) vy[kt] = wy(2 * kt + (lg >> 1)) * U(a.W);
#pragma unroll
        for (int r = 0; r < 4; ++r) vx[r] = wx(4 * (lg & 1) + r);
    } else {
#pragma unroll
        for (int m = 0; m < 4; ++m) off[m] = (U(wi) * 64u + 16u * m + li) * U(a.ldq);
#pragma unroll
        for (int j = 0; j < NQ; ++j) offq[j] = (U(wi) * 64u + 16u * (part * NQ + j) + li) * U(a.ldq);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) vy[kt] = U(wi) * 64u + 16u * kt + 4u * lg;
#pragma unroll
        for (int r = 0; r < 4; ++r) vx[r] = r;
    }
    // Row (pixel or window-major token) of token 16m + li, recomputed where the outputs
    // are stored so that no register holds it through the products.
    auto row_of = [&](int m) -> U {
        if (a.pixel_mode) {
            int y = wh * 8 + 2 * m + (li >> 3) + a.shift, x = ww * 8 + (li & 7) + a.shift;
            y = y >= a.H ? y - a.H : y;
            x = x >= a.W ? x - a.W : x;
            return U(y) * U(a.W) + U(x);
        }
        return U(wi) * 64u + 16u * m + li;
    };
    const float* q_base = a.qkv + hoff;
    const float* k_base = a.qkv + a.C + hoff;
    const float* v_base = a.qkv + 2 * a.C + hoff + li;

    // All of the window-head's operands are requested before the first product.
    // kf / qf: token 16m + li, dims 16G + 4lg .. +3. vv: the A operand of O^T = V^T P^T,
    // dim 16nd + li against keys 16kt + 4lg + r.
    // X6 (split-operand products): K and V go to split form once (the 16-bit operand layout:
    // key block kk of V^T is key tiles 2kk, 2kk + 1), each query tile before its product.
    f4 kf[4][2], qf[NQ][2], vv[4][2];
    x8 kx[X6 ? 4 : 1], vsx[X6 ? 2 : 1][2];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int G = 0; G < 2; ++G) kf[m][G] = ld4(k_base + off[m] + G * 16 + lg * 4);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
        for (int G = 0; G < 2; ++G) qf[j][G] = ld4(q_base + offq[j] + G * 16 + lg * 4);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int nd = 0; nd < 2; ++nd)
#pragma unroll
            for (int r = 0; r < 4; ++r) vv[kt][nd][r] = v_base[(vy[kt] + vx[r]) * U(a.ldq) + 16 * nd];
    if constexpr (X6) {
#pragma unroll
        for (int m = 0; m < 4; ++m) kx[m] = split8(kf[m][0], kf[m][1]);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int nd = 0; nd < 2; ++nd) vsx[kk][nd] = split8(vv[2 * kk][nd], vv[2 * kk + 1][nd]);
    }
    // Bias: query p = 16nt + li and key q = 16mt + 4lg + r give table entry
    // (p/8 - q/8 + 7) * 15 + (p%8 - q%8 + 7) = base + 30 (nt - mt) - r (cpu.rs:532-546);
    // read from LDS where each logit is formed.
    const int base = h * 225 + 15 * ((li >> 3) - (lg >> 1)) + (li & 7) - 4 * (lg & 1) + 112;

    // Shifted-window mask (cpu.rs:548-589, 681-683): in the last window row, query and key
    // on different sides of the row split; in the last window column, on different sides of
    // the column split. The row part depends on (nt, mt) only, the column part on the lane.
    const bool row_edge = a.shift > 0 && wh == a.nwh - 1;
    const bool col_edge = a.shift > 0 && ww == a.nww - 1;
    const bool col_hit = col_edge && (((li & 7) < 4) != ((lg & 1) == 0));
    const float SENT = -3.4028234663852886e38f / 4.0f;
    const float sc = a.scale * 1.4426950408889634f;   // logits in log2 units: p = 2^(l - max)

#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        const int nt = part * NQ + j;
        f4 S[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) S[mt] = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (X6) {
            const x8 qx = split8(qf[j][0], qf[j][1]);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) S[mt] = mfma6(kx[mt], qx, S[mt]);
        } else {
#pragma unroll
            for (int G = 0; G < 2; ++G)
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) S[mt] = mfma4(kf[mt][G][s4], qf[j][G][s4], S[mt]);
        }
        // Logits for query 16nt + li against keys 16mt + 4lg + r.
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) S[mt][r] = fmaf(S[mt][r], sc, rps[base + 30 * (nt - mt) - r]);
        if (row_edge || col_edge) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const bool hit = (row_edge && ((nt < 2) != (mt < 2))) || col_hit;
#pragma unroll
                for (int r = 0; r < 4; ++r) S[mt][r] = hit ? SENT : S[mt][r];
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, S[mt][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        float sum = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(S[mt][r] - mx);
                S[mt][r] = e;
                sum += e;
            }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        // O^T = V^T P^T with the unnormalised weights (lane = query, registers = 4
        // consecutive keys: the B operand as they stand), then O / sum: each lane ends with
        // dims 16nd + 4lg .. +3 of query 16nt + li.
        f4 O[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
        if constexpr (X6) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const x8 px = split8(S[2 * kk], S[2 * kk + 1]);
#pragma unroll
                for (int nd = 0; nd < 2; ++nd) O[nd] = mfma6(vsx[kk][nd], px, O[nd]);
            }
        } else {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int nd = 0; nd < 2; ++nd) O[nd] = mfma4(vv[kt][nd][r], S[kt][r], O[nd]);
        }
        const float inv = 1.0f / sum;
        float* o = a.out + long(row_of(nt)) * a.ldo + hoff + lg * 4;
        st4(o, O[0] * inv);
        st4(o + 16, O[1] * inv);
    }
}

bool attention(const AttnArgs& a, hipStream_t s, const char** why) {
    if (a.C != a.heads * 32) { *why = "attention: head_dim must be 32"; return false; }
    const double rows = a.pixel_mode ? double(a.H) * a.W : double(a.nwh) * a.nww * 64.0;
    // 32-bit element offsets while the qkv and output planes allow (the measured form), else 64-bit.
    const bool wide = a.wide || rows * double(a.ldq) >= 4294967296.0 || rows * double(a.ldo) >= 4294967296.0;
    if (a.shift != 0 && a.shift != 4) { *why = "attention: the shifted-window mask assumes shift 4"; return false; }
    if (a.heads > 8) { *why = "attention: at most 8 heads"; return false; }
    const long wheads = long(a.nwh) * a.nww * a.heads;
    if (wheads == 0) return true;
    // fp32 products: two query parts per (window, head) when the (window, head) units alone
    // would not give the chip two rounds of waves, so that loads, products and stores of
    // different waves overlap (the key and value rows are then read by both parts, from L2
    // the second time). The split-operand form (three waves per SIMD) measured faster
    // without the split at every level (C = 256: 31.4 -> 28.8 us).
    const int qs = a.qsplit ? a.qsplit : (!a.split && wheads <= 4096 ? 2 : 1);
    const long units = wheads * qs;
    dim3 grid(unsigned((units + 3) / 4));
    if (a.split) {
        if (qs == 2) {
            if (wide) hipLaunchKernelGGL((k_attention<true, 2, true>), grid, dim3(256), 0, s, a, units);
            else hipLaunchKernelGGL((k_attention<false, 2, true>), grid, dim3(256), 0, s, a, units);
        } else {
            if (wide) hipLaunchKernelGGL((k_attention<true, 1, true>), grid, dim3(256), 0, s, a, units);
            else hipLaunchKernelGGL((k_attention<false, 1, true>), grid, dim3(256), 0, s, a, units);
        }
    } else if (qs == 2) {
        if (wide) hipLaunchKernelGGL((k_attention<true, 2>), grid, dim3(256), 0, s, a, units);
        else hipLaunchKernelGGL((k_attention<false, 2>), grid, dim3(256), 0, s, a, units);
    } else {
        if (wide) hipLaunchKernelGGL((k_attention<true, 1>), grid, dim3(256), 0, s, a, units);
        else hipLaunchKernelGGL((k_attention<false, 1>), grid, dim3(256), 0, s, a, units);
    }
    return true;
}

// ---------------------------------------------------------------------------
// Fused window attention half: one wave per 8x8 window, all heads.
//   1. the window's 64 token rows are read through the shifted index map, LayerNormed in
//      registers and parked in this wave's LDS slice;
//   2. per head: Q^T = Wq Xn^T and K^T = Wk Xn^T (head dims as the MFMA rows) land with
//      each lane holding 4 consecutive dims of one token - the operand layout of
//      S^T = K Q^T - and V = Xn Wv^T (tokens as rows) lands in the operand layout of
//      O^T = V^T P^T; softmax as in k_attention; O^T is then already the B operand of the
//      projection out^T += Wp_h O^T, accumulated over heads in registers;
//   3. x += out + bias, written back through the same index map (a permutation, so each
//      window owns its 64 rows).
// ---------------------------------------------------------------------------
template <int T, bool MLP, bool H16, bool X6 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(T == 32 ? 2 : 1, 2))) void k_msa(MsaArgs a, long nw) {
    constexpr int HEADS = T / 32, KG = T / 16, OT = T / 16;
    // X6 (split-operand products, t = 32): the normalised tokens stay in registers in split
    // form (at t = 32 a lane's LayerNorm output is exactly its operand of the q/k/v
    // products), so the LDS holds only the MLP weights, as three bf16 planes each.
    static_assert(!X6 || (!H16 && T == 32), "split products: t = 32, fp32 rows");
    constexpr bool L16 = H16 || X6;   // 16-bit operand layout and pitches
    // Normalised tokens per wave: fp32 rows of T + 4 floats, or fp16 rows of T + 16 halves
    // in the k-permuted order of the f16 products.
    constexpr int LDX = H16 ? T + 16 : T + 4;
    constexpr int XSF = X6 ? 0 : 4 * 64 * LDX;
    // MLP weights, resident for the whole workgroup: W0 [4T][T] and W2 [T][4T] with row
    // pitches T + 8 and 4T + 8 floats (16-bit: T + 16 and 4T + 16 halves, k-permuted), both
    // conflict-free for 128-bit operand reads.
    constexpr int HID = 4 * T, P0 = L16 ? T + 16 : T + 8, P2 = L16 ? HID + 16 : HID + 8;
    constexpr int NP = X6 ? 3 : 1;
    constexpr int MLPF = MLP ? NP * (HID * P0 + T * P2) : 0;
    using ET = std::conditional_t<X6, __bf16, std::conditional_t<H16, _Float16, float>>;
    __shared__ __align__(16) ET xs[XSF + MLPF + (XSF + MLPF == 0 ? 8 : 0)];
    __shared__ __align__(16) float gtab[MLP ? GELU_TABLE : 4];
    // The hidden bias too: read where each hidden chunk's products end, from global memory
    // its wait came right after them.
    __shared__ __align__(16) float b0s[MLP ? HID : 4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    ET* const wm0 = xs + XSF;
    ET* const wm2 = wm0 + NP * HID * P0;
    const int li = lane & 15, lg = lane >> 4;
    const long wi = long(blockIdx.x) * 4 + wave;
    const bool valid = wi < nw;
    // Window wi = (image, window row, window column); the roll wraps within the image.
    // Window counts fit 32 bits (the launch grid is 32-bit), so the divisions are 32-bit.
    const unsigned wpi = unsigned(a.nwh) * unsigned(a.nww);
    const int img = valid ? int(unsigned(wi) / wpi) : 0;
    const int wr = valid ? int(unsigned(wi) - unsigned(img) * wpi) : 0;
    const int wh = int(unsigned(wr) / unsigned(a.nww)), ww = wr - wh * a.nww;
    const long ybase = long(img) * a.H;
    ET* xw = xs + (X6 ? 0 : wave * 64 * LDX);
    auto rowof = [&](int t) -> long {
        int y = wh * 8 + (t >> 3) + a.shift;
        int x = ww * 8 + (t & 7) + a.shift;
        if (y >= a.H) y -= a.H;
        if (x >= a.W) x -= a.W;
        return (ybase + y) * a.W + x;
    };
    // The window's token rows are requested first (invalid waves read window 0's rows and
    // discard them), so they are in flight with the staging reads below.
    f4 xin[4][KG];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const long row = rowof(mt * 16 + li);
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) xin[mt][kg] = ld4(a.x + row * a.ldx + kg * 16 + lg * 4);
    }
    f4 ln1g[KG], ln1b[KG];
#pragma unroll
    for (int kg = 0; kg < KG; ++kg) {
        ln1g[kg] = ld4(a.ln_g + kg * 16 + lg * 4);
        ln1b[kg] = ld4(a.ln_b + kg * 16 + lg * 4);
    }
    // The staging of the GELU table, the hidden bias and the MLP weights issues all of a
    // thread's reads before its LDS stores, so they are in flight together (a load-store
    // loop waits a full L2 round trip per pass, at the start of every workgroup).
    f4 gtv = f4{0.f, 0.f, 0.f, 0.f};
    float b0v = 0.f;
    if constexpr (MLP) {
        static_assert(GELU_TABLE / 4 <= 256 && HID <= 256, "one table chunk and one bias per thread");
        gtv = ld4(a.gelu + 4 * min(int(threadIdx.x), GELU_TABLE / 4 - 1));
        b0v = a.b0[min(int(threadIdx.x), HID - 1)];
    }
    if constexpr (MLP && X6) {
        constexpr int NV = NP * HID * T / 8 / 256;   // 16-byte chunks per thread, each matrix
        static_assert(NV * 256 == NP * HID * T / 8, "weight staging must split evenly");
        b8 v0[NV], v2[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int f = threadIdx.x + 256 * j;
            const int p = f / (HID * T / 8), g = f % (HID * T / 8);
            v0[j] = ldb8(a.x0 + long(p) * HID * T + long(g / (T / 8)) * T + (g % (T / 8)) * 8);
            v2[j] = ldb8(a.x2 + long(p) * HID * T + long(g / (HID / 8)) * HID + (g % (HID / 8)) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);   // every read above, every store below
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int f = threadIdx.x + 256 * j;
            const int p = f / (HID * T / 8), g = f % (HID * T / 8);
            stb8(wm0 + p * HID * P0 + (g / (T / 8)) * P0 + (g % (T / 8)) * 8, v0[j]);
            stb8(wm2 + p * T * P2 + (g / (HID / 8)) * P2 + (g % (HID / 8)) * 8, v2[j]);
        }
    } else if constexpr (MLP) {
        constexpr int EV = H16 ? 8 : 4;   // elements per 16-byte chunk
        constexpr int NV = HID * T / EV / 256;
        static_assert(NV * 256 == HID * T / EV, "weight staging must split evenly");
        const ET* g0 = H16 ? reinterpret_cast<const ET*>(a.h0) : reinterpret_cast<const ET*>(a.w0);
        const ET* g2 = H16 ? reinterpret_cast<const ET*>(a.h2) : reinterpret_cast<const ET*>(a.w2);
        f4 v0[NV], v2[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int f = threadIdx.x + 256 * j;
            v0[j] = ld4(reinterpret_cast<const float*>(g0 + long(f / (T / EV)) * T + (f % (T / EV)) * EV));
            v2[j] = ld4(reinterpret_cast<const float*>(g2 + long(f / (HID / EV)) * HID + (f % (HID / EV)) * EV));
        }
        __builtin_amdgcn_sched_barrier(0);   // every read above, every store below
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int f = threadIdx.x + 256 * j;
            st4(reinterpret_cast<float*>(wm0 + (f / (T / EV)) * P0 + (f % (T / EV)) * EV), v0[j]);
            st4(reinterpret_cast<float*>(wm2 + (f / (HID / EV)) * P2 + (f % (HID / EV)) * EV), v2[j]);
        }
    }
    if constexpr (MLP) {
        if (threadIdx.x < GELU_TABLE / 4) st4(gtab + 4 * threadIdx.x, gtv);
        if (threadIdx.x < HID) b0s[threadIdx.x] = b0v;
    }

    // 1. LN1 of the window's tokens into LDS. The raw rows stay in registers for the
    // attention residual (the wave is register-limited to two per SIMD either way).
    x8 xbx[X6 ? 4 : 1][X6 ? KG / 2 : 1];
    if (valid) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f4 v[KG];
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) v[kg] = xin[mt][kg];
            float sm = 0.f;
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) sm += (v[kg].x + v[kg].y) + (v[kg].z + v[kg].w);
            sm += __shfl_xor(sm, 16);
            sm += __shfl_xor(sm, 32);
            const float mu = sm / float(T);
            float q = 0.f;
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                f4 d = v[kg] - mu;
                q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            }
            q += __shfl_xor(q, 16);
            q += __shfl_xor(q, 32);
            const float rs = __builtin_amdgcn_rsqf(q * (1.0f / float(T)) + 1e-5f);
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                v[kg] = (v[kg] - mu) * rs * ln1g[kg] + ln1b[kg];
            }
            if constexpr (X6) {
#pragma unroll
                for (int kk = 0; kk < KG / 2; ++kk) xbx[mt][kk] = split8(v[2 * kk], v[2 * kk + 1]);
            } else if constexpr (H16) {
#pragma unroll
                for (int kk = 0; kk < KG / 2; ++kk)
                    sth8(xw + (mt * 16 + li) * LDX + kk * 32 + lg * 8, pack8(v[2 * kk], v[2 * kk + 1]));
            } else {
#pragma unroll
                for (int kg = 0; kg < KG; ++kg) st4(xw + (mt * 16 + li) * LDX + kg * 16 + lg * 4, v[kg]);
            }
        }
    }
    __syncthreads();
    if (!valid) return;   // no barrier follows

    const bool row_edge = a.shift > 0 && wh == a.nwh - 1;
    const bool col_edge = a.shift > 0 && ww == a.nww - 1;
    const float SENT = -3.4028234663852886e38f / 4.0f;
    const float sc2 = a.scale * 1.4426950408889634f;   // logits in log2 units: p = 2^(l - max)
    f4 acc[4][OT];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int ot = 0; ot < OT; ++ot) acc[nt][ot] = f4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
    for (int h = 0; h < HEADS; ++h) {
        f4 qf[4][2], kf[4][2], vf[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int d = 0; d < 2; ++d) qf[mt][d] = kf[mt][d] = vf[mt][d] = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (X6) {
            constexpr long PS = 3L * T * T;
            const __bf16* wq = a.xqkv + long(h * 32) * T;
            const __bf16* wk = a.xqkv + long(T + h * 32) * T;
            const __bf16* wv = a.xqkv + long(2 * T + h * 32) * T;
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) {
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const x8 fq = ldx8(wq + (d * 16 + li) * T + kk * 32 + lg * 8, PS);
                    const x8 fk = ldx8(wk + (d * 16 + li) * T + kk * 32 + lg * 8, PS);
                    const x8 fv = ldx8(wv + (d * 16 + li) * T + kk * 32 + lg * 8, PS);
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        qf[mt][d] = mfma6(fq, xbx[mt][kk], qf[mt][d]);
                        kf[mt][d] = mfma6(fk, xbx[mt][kk], kf[mt][d]);
                        vf[mt][d] = mfma6(xbx[mt][kk], fv, vf[mt][d]);
                    }
                }
            }
        } else if constexpr (H16) {
            const _Float16* wq = a.hqkv + long(h * 32) * T;
            const _Float16* wk = a.hqkv + long(T + h * 32) * T;
            const _Float16* wv = a.hqkv + long(2 * T + h * 32) * T;
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) {
                h8 xb[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) xb[mt] = ldh8(xw + (mt * 16 + li) * LDX + kk * 32 + lg * 8);
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const h8 fq = ldh8(wq + (d * 16 + li) * T + kk * 32 + lg * 8);
                    const h8 fk = ldh8(wk + (d * 16 + li) * T + kk * 32 + lg * 8);
                    const h8 fv = ldh8(wv + (d * 16 + li) * T + kk * 32 + lg * 8);
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        qf[mt][d] = mfma16(fq, xb[mt], qf[mt][d]);
                        kf[mt][d] = mfma16(fk, xb[mt], kf[mt][d]);
                        vf[mt][d] = mfma16(xb[mt], fv, vf[mt][d]);
                    }
                }
            }
        } else {
            const float* wq = a.wqkv + long(h * 32) * T;
            const float* wk = a.wqkv + long(T + h * 32) * T;
            const float* wv = a.wqkv + long(2 * T + h * 32) * T;
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                f4 xb[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) xb[mt] = ld4(xw + (mt * 16 + li) * LDX + kg * 16 + lg * 4);
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const f4 fq = ld4(wq + (d * 16 + li) * T + kg * 16 + lg * 4);
                    const f4 fk = ld4(wk + (d * 16 + li) * T + kg * 16 + lg * 4);
                    const f4 fv = ld4(wv + (d * 16 + li) * T + kg * 16 + lg * 4);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) {
                            qf[mt][d] = mfma4(fq[s], xb[mt][s], qf[mt][d]);
                            kf[mt][d] = mfma4(fk[s], xb[mt][s], kf[mt][d]);
                            vf[mt][d] = mfma4(xb[mt][s], fv[s], vf[mt][d]);
                        }
                }
            }
        }
        // Biases: qf/kf lanes hold dims 16d + 4lg .. +3 of token 16mt + li; vf lanes hold
        // dim 16d + li of tokens 16mt + 4lg .. +3.
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const f4 bq = ld4(a.bqkv + h * 32 + d * 16 + lg * 4);
            const f4 bk = ld4(a.bqkv + T + h * 32 + d * 16 + lg * 4);
            const float bv = a.bqkv[2 * T + h * 32 + d * 16 + li];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                qf[mt][d] += bq;
                kf[mt][d] += bk;
                vf[mt][d] += bv;
            }
        }
        const float* tab = a.tab + (long(h) * 64 + lane) * 64;
        // fp16 operands of S^T = K Q^T (the head's 32 dims are one k block) and of
        // O^T = V^T P^T (keys 32kk .. 32kk + 31 are k block kk).
        h8 kh[H16 ? 4 : 1], qh[H16 ? 4 : 1], vh[H16 ? 2 : 1][2];
        x8 kx[X6 ? 4 : 1], vx[X6 ? 2 : 1][2];
        if constexpr (X6) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) kx[mt] = split8(kf[mt][0], kf[mt][1]);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int nd = 0; nd < 2; ++nd) vx[kk][nd] = split8(vf[2 * kk][nd], vf[2 * kk + 1][nd]);
        } else if constexpr (H16) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                kh[mt] = pack8(kf[mt][0], kf[mt][1]);
                qh[mt] = pack8(qf[mt][0], qf[mt][1]);
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int nd = 0; nd < 2; ++nd) vh[kk][nd] = pack8(vf[2 * kk][nd], vf[2 * kk + 1][nd]);
        }
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            f4 S[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) S[mt] = f4{0.f, 0.f, 0.f, 0.f};
            if constexpr (X6) {
                const x8 qx = split8(qf[nt][0], qf[nt][1]);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) S[mt] = mfma6(kx[mt], qx, S[mt]);
            } else if constexpr (H16) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) S[mt] = mfma16(kh[mt], qh[nt], S[mt]);
            } else {
#pragma unroll
                for (int G = 0; G < 2; ++G)
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) S[mt] = mfma4(kf[mt][G][s], qf[nt][G][s], S[mt]);
            }
            const bool q_row_lo = nt < 2;
            const bool q_col_lo = (li & 7) < 4;
            const bool k_col_lo = (lg & 1) == 0;
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const f4 b = ld4(tab + nt * 16 + mt * 4);
                const bool hit = (row_edge && (q_row_lo != (mt < 2))) || (col_edge && (q_col_lo != k_col_lo));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = fmaf(S[mt][r], sc2, b[r]);
                    if (hit) v = SENT;
                    S[mt][r] = v;
                    mx = fmaxf(mx, v);
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            float sum = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f(S[mt][r] - mx);
                    S[mt][r] = e;
                    sum += e;
                }
            sum += __shfl_xor(sum, 16);
            sum += __shfl_xor(sum, 32);
            const float inv = __builtin_amdgcn_rcpf(sum);
            f4 O[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
            if constexpr (X6) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const x8 px = split8(S[2 * kk], S[2 * kk + 1]);
#pragma unroll
                    for (int nd = 0; nd < 2; ++nd) O[nd] = mfma6(vx[kk][nd], px, O[nd]);
                }
                O[0] = O[0] * inv;
                O[1] = O[1] * inv;
                const x8 ox = split8(O[0], O[1]);
#pragma unroll
                for (int ot = 0; ot < OT; ++ot)
                    acc[nt][ot] = mfma6(ldx8(a.xp + long(ot * 16 + li) * T + h * 32 + lg * 8, long(T) * T), ox, acc[nt][ot]);
            } else if constexpr (H16) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const h8 ph = pack8(S[2 * kk], S[2 * kk + 1]);
#pragma unroll
                    for (int nd = 0; nd < 2; ++nd) O[nd] = mfma16(vh[kk][nd], ph, O[nd]);
                }
                O[0] = O[0] * inv;
                O[1] = O[1] * inv;
                // out^T += Wp[:, head dims] O^T: the head's dims are k block h of Wp.
                const h8 oh = pack8(O[0], O[1]);
#pragma unroll
                for (int ot = 0; ot < OT; ++ot)
                    acc[nt][ot] = mfma16(ldh8(a.hp + long(ot * 16 + li) * T + h * 32 + lg * 8), oh, acc[nt][ot]);
            } else {
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
#pragma unroll
                        for (int nd = 0; nd < 2; ++nd) O[nd] = mfma4(vf[kt][nd][r], S[kt][r], O[nd]);
                    }
                O[0] = O[0] * inv;
                O[1] = O[1] * inv;
                // out^T += Wp[:, head dims] O^T.
#pragma unroll
                for (int ot = 0; ot < OT; ++ot)
#pragma unroll
                    for (int nd = 0; nd < 2; ++nd) {
                        const f4 fw = ld4(a.wp + long(ot * 16 + li) * T + h * 32 + nd * 16 + lg * 4);
#pragma unroll
                        for (int s = 0; s < 4; ++s) acc[nt][ot] = mfma4(fw[s], O[nd][s], acc[nt][ot]);
                    }
            }
        }
    }
    // 3. Residual: lanes hold outputs 16ot + 4lg .. +3 of token 16nt + li.
    f4 xr[4][OT];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int ot = 0; ot < OT; ++ot) xr[nt][ot] = xin[nt][ot] + (acc[nt][ot] + ld4(a.bp + ot * 16 + lg * 4));
    if constexpr (MLP) {
        // 4. The MLP on the window's tokens (cpu.rs:800-860), exactly as k_mlp computes it:
        // LN2 in registers, the hidden layer produced 32 units at a time transposed (so it
        // is directly the second product's operand), GELU, and the second residual.
        constexpr int HC = 32, HT = HC / 16;
        f4 xn[4][OT];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            float sm = 0.f;
#pragma unroll
            for (int kg = 0; kg < OT; ++kg) sm += (xr[mt][kg].x + xr[mt][kg].y) + (xr[mt][kg].z + xr[mt][kg].w);
            sm += __shfl_xor(sm, 16);
            sm += __shfl_xor(sm, 32);
            const float mu = sm / float(T);
            float q = 0.f;
#pragma unroll
            for (int kg = 0; kg < OT; ++kg) {
                f4 d = xr[mt][kg] - mu;
                q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            }
            q += __shfl_xor(q, 16);
            q += __shfl_xor(q, 32);
            const float rs = __builtin_amdgcn_rsqf(q * (1.0f / float(T)) + 1e-5f);
#pragma unroll
            for (int kg = 0; kg < OT; ++kg) {
                f4 gg = ld4(a.ln2_g + kg * 16 + lg * 4), bb = ld4(a.ln2_b + kg * 16 + lg * 4);
                xn[mt][kg] = (xr[mt][kg] - mu) * rs * gg + bb;
            }
        }
        f4 acc2[4][OT];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < OT; ++nt) acc2[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
        h8 xnh[H16 ? 4 : 1][H16 ? OT / 2 : 1];
        x8 xnx[X6 ? 4 : 1][X6 ? OT / 2 : 1];
        if constexpr (X6) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int kk = 0; kk < OT / 2; ++kk) xnx[mt][kk] = split8(xn[mt][2 * kk], xn[mt][2 * kk + 1]);
        } else if constexpr (H16) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int kk = 0; kk < OT / 2; ++kk) xnh[mt][kk] = pack8(xn[mt][2 * kk], xn[mt][2 * kk + 1]);
        }
#pragma unroll 1
        for (int ch = 0; ch < HID / HC; ++ch) {
            f4 acc1[HT][4];
#pragma unroll
            for (int ht = 0; ht < HT; ++ht)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) acc1[ht][mt] = f4{0.f, 0.f, 0.f, 0.f};
            if constexpr (X6) {
#pragma unroll
                for (int kk = 0; kk < OT / 2; ++kk)
#pragma unroll
                    for (int ht = 0; ht < HT; ++ht) {
                        const x8 wv = ldx8(wm0 + (ch * HC + ht * 16 + li) * P0 + kk * 32 + lg * 8, HID * P0);
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) acc1[ht][mt] = mfma6(wv, xnx[mt][kk], acc1[ht][mt]);
                    }
            } else if constexpr (H16) {
#pragma unroll
                for (int kk = 0; kk < OT / 2; ++kk)
#pragma unroll
                    for (int ht = 0; ht < HT; ++ht) {
                        const h8 wv = ldh8(wm0 + (ch * HC + ht * 16 + li) * P0 + kk * 32 + lg * 8);
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) acc1[ht][mt] = mfma16(wv, xnh[mt][kk], acc1[ht][mt]);
                    }
            } else {
#pragma unroll
                for (int kg = 0; kg < OT; ++kg)
#pragma unroll
                    for (int ht = 0; ht < HT; ++ht) {
                        const f4 wv = ld4(wm0 + (ch * HC + ht * 16 + li) * P0 + kg * 16 + lg * 4);
#pragma unroll
                        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                            for (int mt = 0; mt < 4; ++mt) acc1[ht][mt] = mfma4(wv[s4], xn[mt][kg][s4], acc1[ht][mt]);
                    }
            }
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) {
                const f4 bb = ld4(b0s + ch * HC + ht * 16 + lg * 4);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc1[ht][mt][r] = gelu_lut(gtab, acc1[ht][mt][r] + bb[r]);
            }
            if constexpr (X6) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    const x8 hv = split8(acc1[0][mt], acc1[1][mt]);
#pragma unroll
                    for (int nt = 0; nt < OT; ++nt)
                        acc2[mt][nt] = mfma6(ldx8(wm2 + (nt * 16 + li) * P2 + ch * 32 + lg * 8, T * P2), hv, acc2[mt][nt]);
                }
            } else if constexpr (H16) {
                // HC = 32 hidden units: k block ch of W2.
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    const h8 hv = pack8(acc1[0][mt], acc1[1][mt]);
#pragma unroll
                    for (int nt = 0; nt < OT; ++nt)
                        acc2[mt][nt] = mfma16(ldh8(wm2 + (nt * 16 + li) * P2 + ch * 32 + lg * 8), hv, acc2[mt][nt]);
                }
            } else {
#pragma unroll
                for (int ht = 0; ht < HT; ++ht)
#pragma unroll
                    for (int nt = 0; nt < OT; ++nt) {
                        const f4 wv = ld4(wm2 + (nt * 16 + li) * P2 + ch * HC + ht * 16 + lg * 4);
#pragma unroll
                        for (int r = 0; r < 4; ++r)
#pragma unroll
                            for (int mt = 0; mt < 4; ++mt) acc2[mt][nt] = mfma4(wv[r], acc1[ht][mt][r], acc2[mt][nt]);
                    }
            }
        }
#pragma unroll
        for (int nt = 0; nt < OT; ++nt) {
            const f4 bv = ld4(a.b2 + nt * 16 + lg * 4);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) xr[mt][nt] = xr[mt][nt] + (acc2[mt][nt] + bv);
        }
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const long row = rowof(nt * 16 + li);
#pragma unroll
        for (int ot = 0; ot < OT; ++ot) st4(a.x + row * a.ldx + ot * 16 + lg * 4, xr[nt][ot]);
    }
}

// ---------------------------------------------------------------------------
// The window-attention half at t = 64, 128 and 256 (cpu.rs:791-799), one workgroup per
// window and one wave per head (t / 32 waves):
//   1. the waves LayerNorm the window's 64 token rows (read through the shifted index
//      map) into LDS;
//   2. each wave computes its head's q, k, v from the normalised rows (weights from L2,
//      operand layouts as in k_msa), the attention, and parks its 64 x 32 output in LDS;
//   3. after a barrier each wave computes 32 of the t projection outputs of all 64 tokens
//      from the parked head outputs (out^T = Wp O^T), adds bias and residual and writes the
//      rows back through the same index map.
// The qkv rows and the attention output never reach HBM; the projection of all heads needs
// no cross-wave accumulation in registers. With the MLP option (t = 64) the rows after the
// attention residual stay in LDS and 4. the MLP runs on whole token tiles (two per wave,
// weights from L2) before the single write-back. (At t = 128 a wave would own one tile, a
// weight load would feed a quarter as many products, and the separate MLP kernel, which
// shares LDS-staged weights over 64 rows, measured faster.)
// ---------------------------------------------------------------------------
template <int T, bool MLP, bool H16, bool X6 = false>
__global__ __launch_bounds__(T * 2) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_wmsa(MsaArgs a, long nw) {
    // X6: split-operand products. The normalised tokens are split once, by the wave that
    // normalises them, into three bf16 planes of k-permuted rows (pitch PH); after the q/k/v
    // products have read them, the same region takes the head outputs, split by the wave
    // that forms them. (Without the MLP option: the split mode runs the t = 64 MLP as k_mlp.)
    static_assert(!(X6 && (H16 || MLP)), "split products: fp32 rows, no fused MLP");
    constexpr int HEADS = T / 32, KG = T / 16, LDX = T + 8;
    // fp16 mode keeps the normalised tokens and the head outputs as k-permuted halves,
    // rows of PH = T + 16 (conflict-free 128-bit reads), inside the same arrays.
    constexpr int PH = T + 16;
    static_assert(PH <= 2 * LDX, "fp16 rows fit the fp32 rows");
    constexpr int XPS = 64 * PH;   // X6: one plane of the split rows
    __shared__ __align__(16) float lds[X6 ? 3 * XPS / 2 : 2 * 64 * LDX];
    float* const xs = lds;                  // normalised tokens [token][channel]
    float* const os = lds + 64 * LDX;       // head outputs [token][head * 32 + dim]
    __bf16* const sx = reinterpret_cast<__bf16*>(lds);
    __shared__ __align__(16) float gtab[MLP ? GELU_TABLE : 4];
    _Float16* const xsh = reinterpret_cast<_Float16*>(xs);
    _Float16* const osh = reinterpret_cast<_Float16*>(os);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane & 15, lg = lane >> 4;
    if constexpr (MLP) load_gelu_table(gtab, a.gelu, threadIdx.x, T * 2);
    const long wi = blockIdx.x;
    // Window wi = (image, window row, window column); the roll wraps within the image.
    // Window counts fit 32 bits (the launch grid is 32-bit), so the divisions are 32-bit.
    const unsigned wpi = unsigned(a.nwh) * unsigned(a.nww);
    const int img = int(unsigned(wi) / wpi);
    const int wr = int(unsigned(wi) - unsigned(img) * wpi);
    const int wh = int(unsigned(wr) / unsigned(a.nww)), ww = wr - wh * a.nww;
    const long ybase = long(img) * a.H;
    auto rowof = [&](int t) -> long {
        int y = wh * 8 + (t >> 3) + a.shift;
        int x = ww * 8 + (t & 7) + a.shift;
        if (y >= a.H) y -= a.H;
        if (x >= a.W) x -= a.W;
        return (ybase + y) * a.W + x;
    };

    // 1. LN1 (cpu.rs:338-357) of token tiles 16m .. 16m + 15, m = wave, wave + HEADS, ...
    for (int m = wave; m < 4; m += HEADS) {
        const long row = rowof(m * 16 + li);
        f4 v[KG];
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) v[kg] = ld4(a.x + row * a.ldx + kg * 16 + lg * 4);
        float sm = 0.f;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) sm += (v[kg].x + v[kg].y) + (v[kg].z + v[kg].w);
        sm += __shfl_xor(sm, 16);
        sm += __shfl_xor(sm, 32);
        const float mu = sm / float(T);
        float q = 0.f;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) {
            f4 d = v[kg] - mu;
            q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
        q += __shfl_xor(q, 16);
        q += __shfl_xor(q, 32);
        const float rs = __builtin_amdgcn_rsqf(q * (1.0f / float(T)) + 1e-5f);
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) {
            f4 gg = ld4(a.ln_g + kg * 16 + lg * 4), bb = ld4(a.ln_b + kg * 16 + lg * 4);
            v[kg] = (v[kg] - mu) * rs * gg + bb;
        }
        if constexpr (X6) {
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk) {
                const x8 p = split8(v[2 * kk], v[2 * kk + 1]);
                __bf16* d = sx + (m * 16 + li) * PH + kk * 32 + lg * 8;
                stb8(d, p.h);
                stb8(d + XPS, p.m);
                stb8(d + 2 * XPS, p.l);
            }
        } else if constexpr (H16) {
#pragma unroll
            for (int kk = 0; kk < KG / 2; ++kk)
                sth8(xsh + (m * 16 + li) * PH + kk * 32 + lg * 8, pack8(v[2 * kk], v[2 * kk + 1]));
        } else {
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) st4(xs + (m * 16 + li) * LDX + kg * 16 + lg * 4, v[kg]);
        }
    }
    __syncthreads();

    // 2. Head h = wave.
    const int h = wave;
    {
        f4 qf[4][2], kf[4][2], vf[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int d = 0; d < 2; ++d) qf[mt][d] = kf[mt][d] = vf[mt][d] = f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (X6) {
            constexpr long PS = 3L * T * T;   // plane stride of the qkv weight
            const __bf16* wq = a.xqkv + long(h * 32) * T;
            const __bf16* wk = a.xqkv + long(T + h * 32) * T;
            const __bf16* wv = a.xqkv + long(2 * T + h * 32) * T;
#pragma unroll 1
            for (int kk = 0; kk < KG / 2; ++kk) {
                x8 xb[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) xb[mt] = ldx8(sx + (mt * 16 + li) * PH + kk * 32 + lg * 8, XPS);
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const x8 fq = ldx8(wq + (d * 16 + li) * T + kk * 32 + lg * 8, PS);
                    const x8 fk = ldx8(wk + (d * 16 + li) * T + kk * 32 + lg * 8, PS);
                    const x8 fv = ldx8(wv + (d * 16 + li) * T + kk * 32 + lg * 8, PS);
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        qf[mt][d] = mfma6(fq, xb[mt], qf[mt][d]);
                        kf[mt][d] = mfma6(fk, xb[mt], kf[mt][d]);
                        vf[mt][d] = mfma6(xb[mt], fv, vf[mt][d]);
                    }
                }
            }
        } else if constexpr (H16) {
            const _Float16* wq = a.hqkv + long(h * 32) * T;
            const _Float16* wk = a.hqkv + long(T + h * 32) * T;
            const _Float16* wv = a.hqkv + long(2 * T + h * 32) * T;
#pragma unroll 2
            for (int kk = 0; kk < KG / 2; ++kk) {
                h8 xb[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) xb[mt] = ldh8(xsh + (mt * 16 + li) * PH + kk * 32 + lg * 8);
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const h8 fq = ldh8(wq + (d * 16 + li) * T + kk * 32 + lg * 8);
                    const h8 fk = ldh8(wk + (d * 16 + li) * T + kk * 32 + lg * 8);
                    const h8 fv = ldh8(wv + (d * 16 + li) * T + kk * 32 + lg * 8);
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        qf[mt][d] = mfma16(fq, xb[mt], qf[mt][d]);
                        kf[mt][d] = mfma16(fk, xb[mt], kf[mt][d]);
                        vf[mt][d] = mfma16(xb[mt], fv, vf[mt][d]);
                    }
                }
            }
        } else {
            const float* wq = a.wqkv + long(h * 32) * T;
            const float* wk = a.wqkv + long(T + h * 32) * T;
            const float* wv = a.wqkv + long(2 * T + h * 32) * T;
#pragma unroll 2
            for (int kg = 0; kg < KG; ++kg) {
                f4 xb[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) xb[mt] = ld4(xs + (mt * 16 + li) * LDX + kg * 16 + lg * 4);
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                    const f4 fq = ld4(wq + (d * 16 + li) * T + kg * 16 + lg * 4);
                    const f4 fk = ld4(wk + (d * 16 + li) * T + kg * 16 + lg * 4);
                    const f4 fv = ld4(wv + (d * 16 + li) * T + kg * 16 + lg * 4);
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) {
                            qf[mt][d] = mfma4(fq[s4], xb[mt][s4], qf[mt][d]);
                            kf[mt][d] = mfma4(fk[s4], xb[mt][s4], kf[mt][d]);
                            vf[mt][d] = mfma4(xb[mt][s4], fv[s4], vf[mt][d]);
                        }
                }
            }
        }
        // qf/kf lanes hold dims 16d + 4lg .. +3 of token 16mt + li; vf lanes hold dim
        // 16d + li of tokens 16mt + 4lg .. +3.
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const f4 bq = ld4(a.bqkv + h * 32 + d * 16 + lg * 4);
            const f4 bk = ld4(a.bqkv + T + h * 32 + d * 16 + lg * 4);
            const float bv = a.bqkv[2 * T + h * 32 + d * 16 + li];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                qf[mt][d] += bq;
                kf[mt][d] += bk;
                vf[mt][d] += bv;
            }
        }
        // X6: every wave has read the split rows; the region now takes the head outputs.
        if constexpr (X6) __syncthreads();
        const bool row_edge = a.shift > 0 && wh == a.nwh - 1;
        const bool col_edge = a.shift > 0 && ww == a.nww - 1;
        const float SENT = -3.4028234663852886e38f / 4.0f;
        const float sc2 = a.scale * 1.4426950408889634f;   // logits in log2 units: p = 2^(l - max)
        const float* tab = a.tab + (long(h) * 64 + lane) * 64;
        h8 kh[H16 ? 4 : 1], qh[H16 ? 4 : 1], vh[H16 ? 2 : 1][2];
        x8 kx[X6 ? 4 : 1], vx[X6 ? 2 : 1][2];
        if constexpr (X6) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) kx[mt] = split8(kf[mt][0], kf[mt][1]);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int nd = 0; nd < 2; ++nd) vx[kk][nd] = split8(vf[2 * kk][nd], vf[2 * kk + 1][nd]);
        } else if constexpr (H16) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                kh[mt] = pack8(kf[mt][0], kf[mt][1]);
                qh[mt] = pack8(qf[mt][0], qf[mt][1]);
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int nd = 0; nd < 2; ++nd) vh[kk][nd] = pack8(vf[2 * kk][nd], vf[2 * kk + 1][nd]);
        }
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            f4 S[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) S[mt] = f4{0.f, 0.f, 0.f, 0.f};
            if constexpr (X6) {
                const x8 qx = split8(qf[nt][0], qf[nt][1]);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) S[mt] = mfma6(kx[mt], qx, S[mt]);
            } else if constexpr (H16) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) S[mt] = mfma16(kh[mt], qh[nt], S[mt]);
            } else {
#pragma unroll
                for (int G = 0; G < 2; ++G)
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) S[mt] = mfma4(kf[mt][G][s4], qf[nt][G][s4], S[mt]);
            }
            const bool q_row_lo = nt < 2;
            const bool q_col_lo = (li & 7) < 4;
            const bool k_col_lo = (lg & 1) == 0;
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const f4 b = ld4(tab + nt * 16 + mt * 4);
                const bool hit = (row_edge && (q_row_lo != (mt < 2))) || (col_edge && (q_col_lo != k_col_lo));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = fmaf(S[mt][r], sc2, b[r]);
                    if (hit) v = SENT;
                    S[mt][r] = v;
                    mx = fmaxf(mx, v);
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            float sum = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f(S[mt][r] - mx);
                    S[mt][r] = e;
                    sum += e;
                }
            sum += __shfl_xor(sum, 16);
            sum += __shfl_xor(sum, 32);
            const float inv = __builtin_amdgcn_rcpf(sum);
            f4 O[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
            if constexpr (X6) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const x8 px = split8(S[2 * kk], S[2 * kk + 1]);
#pragma unroll
                    for (int nd = 0; nd < 2; ++nd) O[nd] = mfma6(vx[kk][nd], px, O[nd]);
                }
                O[0] = O[0] * inv;
                O[1] = O[1] * inv;
                // The head's dims are k block h of the projection.
                const x8 p = split8(O[0], O[1]);
                __bf16* d = sx + (nt * 16 + li) * PH + h * 32 + lg * 8;
                stb8(d, p.h);
                stb8(d + XPS, p.m);
                stb8(d + 2 * XPS, p.l);
            } else if constexpr (H16) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const h8 ph = pack8(S[2 * kk], S[2 * kk + 1]);
#pragma unroll
                    for (int nd = 0; nd < 2; ++nd) O[nd] = mfma16(vh[kk][nd], ph, O[nd]);
                }
                O[0] = O[0] * inv;
                O[1] = O[1] * inv;
                // The head's dims are k block h of the projection.
                sth8(osh + (nt * 16 + li) * PH + h * 32 + lg * 8, pack8(O[0], O[1]));
            } else {
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
#pragma unroll
                        for (int nd = 0; nd < 2; ++nd) O[nd] = mfma4(vf[kt][nd][r], S[kt][r], O[nd]);
                    }
                O[0] = O[0] * inv;
                O[1] = O[1] * inv;
                // Lanes hold dims 16nd + 4lg .. +3 of query 16nt + li.
#pragma unroll
                for (int nd = 0; nd < 2; ++nd) st4(os + (nt * 16 + li) * LDX + h * 32 + nd * 16 + lg * 4, O[nd]);
            }
        }
    }
    __syncthreads();

    // 3. Projection columns c0 .. c0 + 31 of all tokens, bias and residual.
    const int c0 = wave * 32;
    f4 acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt][0] = acc[mt][1] = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (X6) {
#pragma unroll 2
        for (int kk = 0; kk < KG / 2; ++kk) {
            x8 ob[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) ob[mt] = ldx8(sx + (mt * 16 + li) * PH + kk * 32 + lg * 8, XPS);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const x8 fw = ldx8(a.xp + long(c0 + ct * 16 + li) * T + kk * 32 + lg * 8, long(T) * T);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) acc[mt][ct] = mfma6(fw, ob[mt], acc[mt][ct]);
            }
        }
    } else if constexpr (H16) {
#pragma unroll 4
        for (int kk = 0; kk < KG / 2; ++kk) {
            h8 ob[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) ob[mt] = ldh8(osh + (mt * 16 + li) * PH + kk * 32 + lg * 8);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const h8 fw = ldh8(a.hp + long(c0 + ct * 16 + li) * T + kk * 32 + lg * 8);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) acc[mt][ct] = mfma16(fw, ob[mt], acc[mt][ct]);
            }
        }
    } else {
#pragma unroll 4
        for (int kg = 0; kg < KG; ++kg) {
            f4 ob[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) ob[mt] = ld4(os + (mt * 16 + li) * LDX + kg * 16 + lg * 4);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const f4 fw = ld4(a.wp + long(c0 + ct * 16 + li) * T + kg * 16 + lg * 4);
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) acc[mt][ct] = mfma4(fw[s4], ob[mt][s4], acc[mt][ct]);
            }
        }
    }
    // The residual rows and the projection bias are all read before the first store (read
    // per store, each read was waited for between the stores).
    f4 rres[4][2], bpv[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) bpv[ct] = ld4(a.bp + c0 + ct * 16 + lg * 4);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const long row = rowof(mt * 16 + li);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) rres[mt][ct] = ld4(a.x + row * a.ldx + c0 + ct * 16 + lg * 4);
    }
    if constexpr (!MLP) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const long row = rowof(mt * 16 + li);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                st4(a.x + row * a.ldx + c0 + ct * 16 + lg * 4, rres[mt][ct] + (acc[mt][ct] + bpv[ct]));
        }
        return;
    } else {
        // The block's rows after the attention residual go to LDS (xs is free: phase 2 is
        // over), so that phase 4 sees whole rows.
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                st4(xs + (mt * 16 + li) * LDX + c0 + ct * 16 + lg * 4, rres[mt][ct] + (acc[mt][ct] + bpv[ct]));
        __syncthreads();
        // 4. The MLP (cpu.rs:800-860) on whole token tiles: wave w takes tiles w, w + HEADS,
        // ... (MT of them); LN2 in registers, the hidden layer 32 units at a time, transposed
        // (H^T = W0c Xn^T is directly the second product's operand), GELU, the residual.
        constexpr int MT = 4 / HEADS, HID = 4 * T, HC = 32, HT = HC / 16;
        f4 xr[MT][KG], xn[MT][KG];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int m = wave + i * HEADS;
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) xr[i][kg] = ld4(xs + (m * 16 + li) * LDX + kg * 16 + lg * 4);
            float sm = 0.f;
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) sm += (xr[i][kg].x + xr[i][kg].y) + (xr[i][kg].z + xr[i][kg].w);
            sm += __shfl_xor(sm, 16);
            sm += __shfl_xor(sm, 32);
            const float mu = sm / float(T);
            float q = 0.f;
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                f4 d = xr[i][kg] - mu;
                q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
            }
            q += __shfl_xor(q, 16);
            q += __shfl_xor(q, 32);
            const float rs = __builtin_amdgcn_rsqf(q * (1.0f / float(T)) + 1e-5f);
#pragma unroll
            for (int kg = 0; kg < KG; ++kg) {
                f4 gg = ld4(a.ln2_g + kg * 16 + lg * 4), bb = ld4(a.ln2_b + kg * 16 + lg * 4);
                xn[i][kg] = (xr[i][kg] - mu) * rs * gg + bb;
            }
        }
        f4 acc2[MT][KG];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int nt = 0; nt < KG; ++nt) acc2[i][nt] = f4{0.f, 0.f, 0.f, 0.f};
        h8 xnh[H16 ? MT : 1][H16 ? KG / 2 : 1];
        x8 xnx[X6 ? MT : 1][X6 ? KG / 2 : 1];
        if constexpr (X6) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int kk = 0; kk < KG / 2; ++kk) xnx[i][kk] = split8(xn[i][2 * kk], xn[i][2 * kk + 1]);
        } else if constexpr (H16) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int kk = 0; kk < KG / 2; ++kk) xnh[i][kk] = pack8(xn[i][2 * kk], xn[i][2 * kk + 1]);
        }
#pragma unroll 1
        for (int ch = 0; ch < HID / HC; ++ch) {
            f4 acc1[HT][MT];
#pragma unroll
            for (int ht = 0; ht < HT; ++ht)
#pragma unroll
                for (int i = 0; i < MT; ++i) acc1[ht][i] = f4{0.f, 0.f, 0.f, 0.f};
            if constexpr (X6) {
#pragma unroll
                for (int kk = 0; kk < KG / 2; ++kk)
#pragma unroll
                    for (int ht = 0; ht < HT; ++ht) {
                        const x8 wv = ldx8(a.x0 + long(ch * HC + ht * 16 + li) * T + kk * 32 + lg * 8, 4L * T * T);
#pragma unroll
                        for (int i = 0; i < MT; ++i) acc1[ht][i] = mfma6(wv, xnx[i][kk], acc1[ht][i]);
                    }
            } else if constexpr (H16) {
#pragma unroll
                for (int kk = 0; kk < KG / 2; ++kk)
#pragma unroll
                    for (int ht = 0; ht < HT; ++ht) {
                        const h8 wv = ldh8(a.h0 + long(ch * HC + ht * 16 + li) * T + kk * 32 + lg * 8);
#pragma unroll
                        for (int i = 0; i < MT; ++i) acc1[ht][i] = mfma16(wv, xnh[i][kk], acc1[ht][i]);
                    }
            } else {
#pragma unroll
                for (int kg = 0; kg < KG; ++kg)
#pragma unroll
                    for (int ht = 0; ht < HT; ++ht) {
                        const f4 wv = ld4(a.w0 + long(ch * HC + ht * 16 + li) * T + kg * 16 + lg * 4);
#pragma unroll
                        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                            for (int i = 0; i < MT; ++i) acc1[ht][i] = mfma4(wv[s4], xn[i][kg][s4], acc1[ht][i]);
                    }
            }
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) {
                const f4 bb = ld4(a.b0 + ch * HC + ht * 16 + lg * 4);
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc1[ht][i][r] = gelu_lut(gtab, acc1[ht][i][r] + bb[r]);
            }
            if constexpr (X6) {
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const x8 hv = split8(acc1[0][i], acc1[1][i]);
#pragma unroll
                    for (int nt = 0; nt < KG; ++nt)
                        acc2[i][nt] = mfma6(ldx8(a.x2 + long(nt * 16 + li) * HID + ch * 32 + lg * 8, 4L * T * T), hv, acc2[i][nt]);
                }
            } else if constexpr (H16) {
                // HC = 32 hidden units: k block ch of W2.
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const h8 hv = pack8(acc1[0][i], acc1[1][i]);
#pragma unroll
                    for (int nt = 0; nt < KG; ++nt)
                        acc2[i][nt] = mfma16(ldh8(a.h2 + long(nt * 16 + li) * HID + ch * 32 + lg * 8), hv, acc2[i][nt]);
                }
            } else {
#pragma unroll
                for (int ht = 0; ht < HT; ++ht)
#pragma unroll
                    for (int nt = 0; nt < KG; ++nt) {
                        const f4 wv = ld4(a.w2 + long(nt * 16 + li) * HID + ch * HC + ht * 16 + lg * 4);
#pragma unroll
                        for (int r = 0; r < 4; ++r)
#pragma unroll
                            for (int i = 0; i < MT; ++i) acc2[i][nt] = mfma4(wv[r], acc1[ht][i][r], acc2[i][nt]);
                    }
            }
        }
        // The output bias is read once, ahead of the stores (read per store, each read was
        // waited for between them).
        f4 b2v[KG];
#pragma unroll
        for (int nt = 0; nt < KG; ++nt) b2v[nt] = ld4(a.b2 + nt * 16 + lg * 4);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const long row = rowof((wave + i * HEADS) * 16 + li);
#pragma unroll
            for (int nt = 0; nt < KG; ++nt)
                st4(a.x + row * a.ldx + nt * 16 + lg * 4, xr[i][nt] + (acc2[i][nt] + b2v[nt]));
        }
    }
}

template <bool H16>
static bool launch_msa(const MsaArgs& a, long nw, hipStream_t s, const char** why) {
    dim3 grid{unsigned((nw + 3) / 4), 1u, 1u}, block{256u, 1u, 1u};
    dim3 wgrid{unsigned(nw), 1u, 1u}, wblock{unsigned(a.t * 2), 1u, 1u};
    if (!H16 && a.xqkv && a.xp && (!a.w0 || (a.x0 && a.x2))) {
        if (a.t == 32 && a.w0) hipLaunchKernelGGL((k_msa<32, true, false, true>), grid, block, 0, s, a, nw);
        else if (a.t == 32) hipLaunchKernelGGL((k_msa<32, false, false, true>), grid, block, 0, s, a, nw);
        else if (a.w0) {
            *why = "msa_fused: the split-operand form runs the MLP at t >= 64 as its own kernel";
            return false;
        } else if (a.t == 64) hipLaunchKernelGGL((k_wmsa<64, false, false, true>), wgrid, wblock, 0, s, a, nw);
        else if (a.t == 128) hipLaunchKernelGGL((k_wmsa<128, false, false, true>), wgrid, wblock, 0, s, a, nw);
        else if (a.t == 256) hipLaunchKernelGGL((k_wmsa<256, false, false, true>), wgrid, wblock, 0, s, a, nw);
        else {
            *why = "msa_fused: t must be 32, 64, 128 or 256";
            return false;
        }
        return true;
    }
    if (a.t == 32 && a.w0) hipLaunchKernelGGL((k_msa<32, true, H16>), grid, block, 0, s, a, nw);
    else if (a.t == 32) hipLaunchKernelGGL((k_msa<32, false, H16>), grid, block, 0, s, a, nw);
    else if (a.t == 64 && a.w0) hipLaunchKernelGGL((k_wmsa<64, true, H16>), wgrid, wblock, 0, s, a, nw);
    else if (a.t == 64) hipLaunchKernelGGL((k_wmsa<64, false, H16>), wgrid, wblock, 0, s, a, nw);
    else if (a.t == 128) hipLaunchKernelGGL((k_wmsa<128, false, H16>), wgrid, wblock, 0, s, a, nw);
    else if (a.t == 256) hipLaunchKernelGGL((k_wmsa<256, false, H16>), wgrid, wblock, 0, s, a, nw);
    else {
        *why = "msa_fused: t must be 32, 64, 128 or 256";
        return false;
    }
    return true;
}

bool msa_fused(const MsaArgs& a, hipStream_t s, const char** why) {
    const long nw = long(a.nwh) * a.nww * a.nimg;
    if (nw == 0) return true;
    if (a.w0 && a.t != 32 && a.t != 64) {
        *why = "msa_fused: the fused MLP is available at t = 32, 64";
        return false;
    }
    if (a.w0 && !a.gelu) {
        *why = "msa_fused: no GELU table";
        return false;
    }
    if (a.hqkv) {
        if (!a.hp || (a.w0 && (!a.h0 || !a.h2))) {
            *why = "msa_fused: the fp16 path needs every k-permuted weight it uses";
            return false;
        }
        return launch_msa<true>(a, nw, s, why);
    }
    return launch_msa<false>(a, nw, s, why);
}

void build_bias_table(const float* rp, int heads, float* tab) {
    // tab[h][lane][nt][mt][r] = log2(e) B_h[query 16nt + lane%16][key 16mt + 4(lane/16) + r],
    // B_h[p][q] = rp[h][(p/8 - q/8 + 7)][(p%8 - q%8 + 7)]   (cpu.rs:532-546); the window
    // kernels keep logits in log2 units (softmax as 2^(l - max)).
    for (int h = 0; h < heads; ++h)
        for (int lane = 0; lane < 64; ++lane)
            for (int nt = 0; nt < 4; ++nt)
                for (int mt = 0; mt < 4; ++mt)
                    for (int r = 0; r < 4; ++r) {
                        int p = nt * 16 + (lane & 15);
                        int q = mt * 16 + (lane >> 4) * 4 + r;
                        int dy = p / 8 - q / 8 + 7, dx = p % 8 - q % 8 + 7;
                        tab[((long(h) * 64 + lane) * 4 + nt) * 16 + mt * 4 + r] =
                            float(double(rp[h * 225 + dy * 15 + dx]) * 1.4426950408889634);
                    }
}

void build_attn_table(const float* rp, int heads, float* tab) {
    // tab[h][dy][dx] = log2(e) * rp[h][dy][dx]: the attention kernel keeps logits in log2
    // units (softmax as 2^(l - max)).
    for (long i = 0; i < long(heads) * 225; ++i) tab[i] = float(double(rp[i]) * 1.4426950408889634);
}

// ---------------------------------------------------------------------------
// m_head: in_nc -> 64, 3x3, as a small implicit GEMM on the matrix cores. K = in_nc*9
// (channel, ky, kx) padded to 32; out^T = W A^T so each lane ends with 4 consecutive
// output channels of one pixel. The input is the NCHW image of size hh x ww, replicate-
// padded on the fly to the H x W plane (plan.rs:67-82) and zero-padded outside it
// (cpu.rs:66-71). Each wave computes 16 pixels x 64 channels per step, 4 steps.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_head(const float* __restrict__ x, int cin, int hh, int ww, int H,
                                              int W, const float* __restrict__ w, float* __restrict__ out,
                                              int add, long P) {
    // P = nimg H W: image b is rows [b H, (b + 1) H) of the output plane and x + b cin hh ww.
    constexpr int LDW = 36;
    __shared__ float sw[64 * LDW];            // W[co][k], k = ci*9 + tap, zero beyond cin*9
    const int K = cin * 9;
    {
        // All eight reads of a thread in flight together (clamped k, zero selected at the
        // store): one at a time, each waited for, they were a chain of L2 round trips at the
        // start of every workgroup.
        float wv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = threadIdx.x + 256 * j, co = i >> 5, k = i & 31;
            wv[j] = w[co * K + (k < K ? k : K - 1)];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = threadIdx.x + 256 * j, co = i >> 5, k = i & 31;
            sw[co * LDW + k] = k < K ? wv[j] : 0.0f;
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane & 15, lg = lane >> 4;
    f4 wf[4][2];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) wf[nt][kg] = ld4(&sw[(nt * 16 + li) * LDW + kg * 16 + lg * 4]);
    // The 4 pixel groups of this wave, software-pipelined: the next group's input taps are
    // requested before the current group's products and stores (and, when accumulating, the
    // current group's output rows before its products).
    // Every tap is loaded (from a clamped, valid address) and then selected: taps past K,
    // pixels past P and taps in the zero padding read as 0. With no load under a branch the
    // wait before a group's products can leave the next group's loads in flight.
    auto gather = [&](int step, f4 (&av)[2]) {
        const long pr = (long(blockIdx.x) * 16 + wave * 4 + step) * 16 + li;
        const long p = pr < P ? pr : P - 1;
        const int yy = int(p / W), xx = int(p - long(yy) * W);
        const int b = yy / H, y = yy - b * H;
        const float* xb = x + long(b) * cin * hh * ww;
#pragma unroll
        for (int kg = 0; kg < 2; ++kg)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int kr = kg * 16 + lg * 4 + s, k = kr < K ? kr : K - 1;
                const int ci = k / 9, tap = k - ci * 9;
                const int sy = y + tap / 3 - 1, sx = xx + tap % 3 - 1;
                const bool ok = kr < K && pr < P && sy >= 0 && sy < H && sx >= 0 && sx < W;
                const int cy = min(max(sy, 0), hh - 1), cx = min(max(sx, 0), ww - 1);
                const float v = xb[(long(ci) * hh + cy) * ww + cx];
                av[kg][s] = ok ? v : 0.0f;
            }
    };
    if (!add) {
        // Plain form: the taps of all four pixel groups are requested before the first
        // product (one round trip per wave instead of one per group).
        f4 av[4][2];
#pragma unroll
        for (int step = 0; step < 4; ++step) gather(step, av[step]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int step = 0; step < 4; ++step) {
            const long p = (long(blockIdx.x) * 16 + wave * 4 + step) * 16 + li;
            f4 acc[4];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma4(wf[nt][kg][s], av[step][kg][s], acc[nt]);
            if (p < P) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) st4(out + p * 64 + lg * 4 + nt * 16, acc[nt]);
            }
        }
        return;
    }
    f4 cur[2], nxt[2];
    gather(0, cur);
#pragma unroll
    for (int step = 0; step < 4; ++step) {
        const long p = (long(blockIdx.x) * 16 + wave * 4 + step) * 16 + li;
        float* o = out + p * 64 + lg * 4;
        f4 prev[4];
        if (add) {
            const float* oc = out + (p < P ? p : P - 1) * 64 + lg * 4;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) prev[nt] = ld4(oc + nt * 16);
        }
        if (step + 1 < 4) gather(step + 1, nxt);
        f4 acc[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[nt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kg = 0; kg < 2; ++kg)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma4(wf[nt][kg][s], cur[kg][s], acc[nt]);
        if (p < P) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) st4(o + nt * 16, add ? prev[nt] + acc[nt] : acc[nt]);
        }
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) cur[kg] = nxt[kg];
    }
}

bool head_conv(const float* x, int cin, int hh, int ww, int H, int W, const float* w, int dim,
               float* out, bool add, hipStream_t s, int nimg) {
    if (dim != 64 || cin * 9 > 32 || nimg < 1) return false;
    const long P = long(H) * W * nimg;
    hipLaunchKernelGGL(k_head, dim3(unsigned((P + 255) / 256)), dim3(256), 0, s, x, cin, hh, ww, H, W, w, out,
                       add ? 1 : 0, P);
    return true;
}

// ---------------------------------------------------------------------------
// m_tail: 64 -> cout (1 or 3), 3x3, from the pixel-major plane into NCHW, cropped to
// oh x ow (plan.rs:85-94). One thread per output pixel of a 16x16 tile; 16-channel slices
// of the 18x18 halo go through LDS as float4; the weights are wave-uniform, so they are
// read through the scalar cache and used as scalar operands of the FMAs.
// Sum order per output: channel, ky, kx ascending (cpu.rs:99-127).
// ---------------------------------------------------------------------------
template <int COUT>
__global__ __launch_bounds__(256) void k_tail(const float* __restrict__ in, int H, int W,
                                              const float* __restrict__ w, float* __restrict__ out, int oh,
                                              int ow) {
    constexpr int HW = 18, CH = 16, LDC = CH + 4, DIM = 64;
    __shared__ float hs[HW * HW * LDC];
    // Stacked images: tile rows y0 .. y0 + 15 of the plane lie in image b (16 divides H).
    const int tx = (W + 15) / 16;
    const int ys = int(blockIdx.x / tx) * 16, x0 = int(blockIdx.x % tx) * 16;
    const int b = ys / H, y0 = ys - b * H;
    in += long(b) * H * W * DIM;
    out += long(b) * COUT * oh * ow;
    const int ly = threadIdx.x >> 4, lx = threadIdx.x & 15;
    float acc[COUT];
#pragma unroll
    for (int o = 0; o < COUT; ++o) acc[o] = 0.f;
    // The halo slice for channels c0 .. c0 + 15 (at most 6 float4 per thread), loaded one slice
    // ahead into registers: slice c0 + 16 reads the other halves of the 128-byte lines slice c0
    // read, so it is requested while they are still in the caches, and its latency overlaps
    // the current slice's arithmetic.
    constexpr int NV = (HW * HW * 4 + 255) / 256;
    f4 hv[NV];
    auto hload = [&](int c0) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = threadIdx.x + i * 256;
            const int px = f >> 2, c4 = f & 3;
            const int gy = y0 - 1 + px / HW, gx = x0 - 1 + px % HW;
            hv[i] = (f < HW * HW * 4 && gy >= 0 && gy < H && gx >= 0 && gx < W)
                        ? ld4(in + (long(gy) * W + gx) * DIM + c0 + c4 * 4)
                        : f4{0.f, 0.f, 0.f, 0.f};
        }
    };
    hload(0);
    for (int c0 = 0; c0 < DIM; c0 += CH) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int f = threadIdx.x + i * 256;
            if (f < HW * HW * 4) st4(&hs[(f >> 2) * LDC + (f & 3) * 4], hv[i]);
        }
        __syncthreads();
        if (c0 + CH < DIM) hload(c0 + CH);
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            f4 v[9];
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) v[tap] = ld4(&hs[((ly + tap / 3) * HW + lx + tap % 3) * LDC + c4 * 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = c0 + c4 * 4 + e;
#pragma unroll
                for (int tap = 0; tap < 9; ++tap)
#pragma unroll
                    for (int o = 0; o < COUT; ++o) acc[o] += w[(o * DIM + c) * 9 + tap] * v[tap][e];
            }
        }
    }
    const int y = y0 + ly, x = x0 + lx;
    if (y < oh && x < ow)
#pragma unroll
        for (int o = 0; o < COUT; ++o) out[(long(o) * oh + y) * ow + x] = acc[o];
}

// ---------------------------------------------------------------------------
// m_tail with split-operand products (the default fp32 mode). For every pixel p of a tile's
// halo the 9 x COUT partial sums Z[p][tap * COUT + o] = sum_ci in[p][ci] W[o][ci][tap] are one
// 64 -> 16 MT product on the bf16 matrix cores (weights as the MFMA rows, split once per
// workgroup; pixel rows split in registers) and go to LDS; each output is then the sum of
// its nine taps' values at the shifted pixels, out[o][y][x] = sum_tap Z[(y + dy, x + dx)]
// [tap * COUT + o], taps in (ky, kx) order. Zero padding: halo pixels outside the image read
// as zero rows, so their Z is zero. Tiles of 16 x 32 output pixels (halo 18 x 34), one output
// pixel per thread, 8 waves, persistent over the tiles.
// ---------------------------------------------------------------------------
template <int COUT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_tail6(const float* __restrict__ in, int H, int W, const float* __restrict__ w,
                                               float* __restrict__ out, int oh, int ow, int tiles) {
    constexpr int DIM = 64, TH = 16, TW = 32, HWD = TW + 2, HP = (TH + 2) * HWD;   // 612 halo pixels
    constexpr int NJ = 9 * COUT, MT = (NJ + 15) / 16;
    constexpr int ZP = (NJ + 3) / 4 * 4;            // Z row pitch: the NJ values, 16-byte aligned
    constexpr int NG = (HP + 15) / 16, GPW = (NG + 7) / 8;
    __shared__ __align__(16) float zs[HP * ZP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
    // Weight fragments: row j = 16 mt + li (tap j / COUT, output o = j % COUT), k block kb holds
    // ci 32 kb + 4 lg .. + 3 and 32 kb + 16 + 4 lg .. + 3, the order of the pixel operand.
    x8 wf[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int j = mt * 16 + li;
            f4 a0, a1;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c0 = 32 * kb + 4 * lg + e;
                a0[e] = j < NJ ? w[((j % COUT) * DIM + c0) * 9 + j / COUT] : 0.0f;
                a1[e] = j < NJ ? w[((j % COUT) * DIM + c0 + 16) * 9 + j / COUT] : 0.0f;
            }
            wf[mt][kb] = split8(a0, a1);
        }
    const int tx = (W + TW - 1) / TW, tpi = tx * ((H + TH - 1) / TH);
    for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
        const int b = t / tpi, r = t - b * tpi;
        const int y0 = (r / tx) * TH, x0 = (r - (r / tx) * tx) * TW;
        const float* const inb = in + long(b) * H * W * DIM;
        // The wave's halo pixel groups, one at a time with the next group's rows in flight:
        // every row is loaded (clamped address) and selected. (With the rows of all five
        // groups in registers at once, two workgroups would not fit a CU.)
        auto loadg = [&](int gi, f4 (&dst)[4]) {
            const int p = 16 * (wave + 8 * gi) + li;
            const int gy = y0 - 1 + p / HWD, gx = x0 - 1 + p % HWD;
            const bool ok = p < HP && gy >= 0 && gy < H && gx >= 0 && gx < W;
            const int cy = min(max(gy, 0), H - 1), cx = min(max(gx, 0), W - 1);
            const float* src = inb + (long(cy) * W + cx) * DIM + lg * 4;
#pragma unroll
            for (int kg = 0; kg < 4; ++kg) {
                const f4 v = ld4(src + kg * 16);
                dst[kg] = ok ? v : f4{0.f, 0.f, 0.f, 0.f};
            }
        };
        f4 xv[2][4];
        loadg(0, xv[0]);
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            if (gi + 1 < GPW) loadg(gi + 1, xv[(gi + 1) & 1]);
            const int g = wave + 8 * gi;
            if (g < NG) {   // wave-uniform
                const f4 (&xc)[4] = xv[gi & 1];
                const x8 p0 = split8(xc[0], xc[1]), p1 = split8(xc[2], xc[3]);
                const int p = 16 * g + li;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    f4 d = mfma6(wf[mt][0], p0, f4{0.f, 0.f, 0.f, 0.f});
                    d = mfma6(wf[mt][1], p1, d);
                    if (p < HP && mt * 16 + lg * 4 < ZP) st4(zs + p * ZP + mt * 16 + lg * 4, d);
                }
            }
        }
        __syncthreads();
        const int ly = tid / TW, lx = tid % TW;
        float acc[COUT];
#pragma unroll
        for (int o = 0; o < COUT; ++o) acc[o] = 0.f;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const float* z = zs + ((ly + tap / 3) * HWD + lx + tap % 3) * ZP + tap * COUT;
#pragma unroll
            for (int o = 0; o < COUT; ++o) acc[o] += z[o];
        }
        const int y = y0 + ly, x = x0 + lx;
        if (y < oh && x < ow) {
            float* ob = out + long(b) * COUT * oh * ow;
#pragma unroll
            for (int o = 0; o < COUT; ++o) ob[(long(o) * oh + y) * ow + x] = acc[o];
        }
        __syncthreads();   // the next tile's Z overwrites this one's
    }
}

bool tail_conv(const float* in, int dim, int H, int W, const float* w, int cout, float* out, int oh,
               int ow, hipStream_t s, int nimg, bool split) {
    if (dim != 64 || nimg < 1 || (nimg > 1 && H % 16 != 0)) return false;
    if (split && (cout == 3 || cout == 1)) {
        const long t6 = long((W + 31) / 32) * ((H + 15) / 16) * nimg;
        if (t6 >= (1L << 31)) return false;
        static std::atomic<int> cus_c[2] = {}, pc_c[2] = {};
        Occ oc;
        const int v = cout == 3 ? 1 : 0;
        if (!query_occ(cout == 3 ? k_tail6<3> : k_tail6<1>, 512, cus_c[v], pc_c[v], &oc)) return false;
        const unsigned grid = unsigned(std::min<long>(t6, long(oc.cus) * oc.per_cu));
        if (cout == 3) hipLaunchKernelGGL(k_tail6<3>, dim3(grid), dim3(512), 0, s, in, H, W, w, out, oh, ow, int(t6));
        else hipLaunchKernelGGL(k_tail6<1>, dim3(grid), dim3(512), 0, s, in, H, W, w, out, oh, ow, int(t6));
        return true;
    }
    const unsigned tiles = unsigned(((W + 15) / 16) * ((H + 15) / 16) * nimg);
    if (cout == 3) hipLaunchKernelGGL(k_tail<3>, dim3(tiles), dim3(256), 0, s, in, H, W, w, out, oh, ow);
    else if (cout == 1) hipLaunchKernelGGL(k_tail<1>, dim3(tiles), dim3(256), 0, s, in, H, W, w, out, oh, ow);
    else return false;
    return true;
}

// ---------------------------------------------------------------------------
// Layout changes: 32x32 tiles through LDS.
// ---------------------------------------------------------------------------
__global__ void k_nchw_to_nhwc(const float* __restrict__ src, float* __restrict__ dst, int c, long P, long ld) {
    __shared__ float t[32][33];
    long p0 = long(blockIdx.x) * 32;
    int c0 = blockIdx.y * 32;
    int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 8 rows of 32
    for (int i = ty; i < 32; i += 8) {
        int cc = c0 + i;
        long p = p0 + tx;
        t[i][tx] = (cc < c && p < P) ? src[long(cc) * P + p] : 0.f;
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        long p = p0 + i;
        int cc = c0 + tx;
        if (cc < c && p < P) dst[p * ld + cc] = t[tx][i];
    }
}

__global__ void k_nhwc_to_nchw(const float* __restrict__ src, float* __restrict__ dst, int c, long P, long ld) {
    __shared__ float t[32][33];
    long p0 = long(blockIdx.x) * 32;
    int c0 = blockIdx.y * 32;
    int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8) {
        long p = p0 + i;
        int cc = c0 + tx;
        t[i][tx] = (cc < c && p < P) ? src[p * ld + cc] : 0.f;
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        int cc = c0 + i;
        long p = p0 + tx;
        if (cc < c && p < P) dst[long(cc) * P + p] = t[tx][i];
    }
}

void nchw_to_nhwc(const float* src, float* dst, int c, long P, long ld, hipStream_t s) {
    dim3 grid(unsigned((P + 31) / 32), unsigned((c + 31) / 32));
    hipLaunchKernelGGL(k_nchw_to_nhwc, grid, dim3(256), 0, s, src, dst, c, P, ld);
}
void nhwc_to_nchw(const float* src, float* dst, int c, long P, long ld, hipStream_t s) {
    dim3 grid(unsigned((P + 31) / 32), unsigned((c + 31) / 32));
    hipLaunchKernelGGL(k_nhwc_to_nchw, grid, dim3(256), 0, s, src, dst, c, P, ld);
}

// The k-permuted fp16 copy of a weight matrix [rows][K] (K % 32 == 0): output chunk
// q = 4 b + g of a row (8 halves) packs k = 32 b + 4 g .. + 3 and 32 b + 16 + 4 g .. + 3.
__global__ void k_h16_permute(const float* __restrict__ src, _Float16* __restrict__ dst, long rows, int K) {
    const long n = rows * (K / 8);
    for (long i = long(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += long(gridDim.x) * blockDim.x) {
        const long row = i / (K / 8);
        const int q = int(i - row * (K / 8));
        const float* p = src + row * K + 32 * (q >> 2) + 4 * (q & 3);
        sth8(dst + row * K + q * 8, pack8(ld4(p), ld4(p + 16)));
    }
}

void h16_permute(const float* src, half_t* dst, long rows, int K, hipStream_t s) {
    const long n = rows * (K / 8);
    if (n <= 0) return;
    dim3 grid{unsigned(std::min<long>((n + 255) / 256, 4096)), 1u, 1u}, block{256u, 1u, 1u};
    hipLaunchKernelGGL(k_h16_permute, grid, block, 0, s, src, dst, rows, K);
}

// The split weight planes: the same chunk order as k_h16_permute, parts h, m, l of every
// element in planes rows * K elements apart (split8).
__global__ void k_x6_permute(const float* __restrict__ src, __bf16* __restrict__ dst, long rows, int K) {
    const long n = rows * (K / 8), ps = rows * long(K);
    for (long i = long(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += long(gridDim.x) * blockDim.x) {
        const long row = i / (K / 8);
        const int q = int(i - row * (K / 8));
        const float* p = src + row * K + 32 * (q >> 2) + 4 * (q & 3);
        const x8 v = split8(ld4(p), ld4(p + 16));
        __bf16* d = dst + row * K + q * 8;
        stb8(d, v.h);
        stb8(d + ps, v.m);
        stb8(d + 2 * ps, v.l);
    }
}

void x6_permute(const float* src, bf16_t* dst, long rows, int K, hipStream_t s) {
    const long n = rows * (K / 8);
    if (n <= 0) return;
    dim3 grid{unsigned(std::min<long>((n + 255) / 256, 4096)), 1u, 1u}, block{256u, 1u, 1u};
    hipLaunchKernelGGL(k_x6_permute, grid, block, 0, s, src, dst, rows, K);
}

__global__ void k_copy_f4(const f4* __restrict__ src, f4* __restrict__ dst, long n) {
    for (long i = long(blockIdx.x) * 256 + threadIdx.x; i < n; i += long(gridDim.x) * 256) dst[i] = src[i];
}

void copy_f4(const void* src, void* dst, long n, hipStream_t s) {
    const unsigned blocks = unsigned(std::min<long>((n + 255) / 256, 256L * 64));
    hipLaunchKernelGGL(k_copy_f4, dim3(blocks), dim3(256), 0, s, static_cast<const f4*>(src), static_cast<f4*>(dst), n);
}

// The window map of the attention kernel (win_row, pixel mode), as a copy.
__global__ void k_window_map(const float* __restrict__ src, float* __restrict__ dst, int c, int H, int W,
                             int shift, int gather, long total) {
    long gid = long(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= total) return;
    int ch = int(gid % c);
    long tokn = gid / c;
    long wi = tokn >> 6;
    int t = int(tokn & 63);
    int nww = W / 8;
    int wh = int(wi / nww), ww = int(wi % nww);
    int y = wh * 8 + (t >> 3) + shift, x = ww * 8 + (t & 7) + shift;
    if (y >= H) y -= H;
    if (x >= W) x -= W;
    long p = long(y) * W + x;
    if (gather) dst[tokn * c + ch] = src[p * c + ch];
    else dst[p * c + ch] = src[tokn * c + ch];
}

void window_gather(const float* x, float* tok, int c, int H, int W, int shift, hipStream_t s) {
    long total = long(H) * W * c;
    hipLaunchKernelGGL(k_window_map, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, x, tok, c, H, W,
                       shift, 1, total);
}
void window_scatter(const float* tok, float* x, int c, int H, int W, int shift, hipStream_t s) {
    long total = long(H) * W * c;
    hipLaunchKernelGGL(k_window_map, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, tok, x, c, H, W,
                       shift, 0, total);
}

}  // namespace scunet
