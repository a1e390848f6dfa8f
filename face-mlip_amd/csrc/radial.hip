// Radial MLP of a factorised pass on the fp32 matrix cores (face/model.py:465-469):
//   u1  = rb W_in^T + b_in + pair_tab[pair]     hid = silu(u1)        (E, H)
//   u2  = hid W1^T + b1                         h2  = silu(u2)        (E, H)
//   phi = (h2 W_phi^T + b_phi) * env                                  (E, B)
// rb already carries the envelope (face/model.py:676). The last layer's 4C CP columns are an
// edge-linear launch on h2 (linear.hip).
//
// Work: one wave per tile of 16 edges, all layers in the transposed orientation (features x
// edges): each layer is D = W . X^T with M = output features, N = edges, K = input features,
// so the D layout of one v_mfma_f32_16x16x4f32 chain (feature 4q + r, edge j in register r of
// lane j + 16q) is directly the B operand of the next chain, whose K index q of instruction r
// is input feature 4q + r of the block. Weights, biases and the pair table sit in LDS.
#include "common.h"

#include <mutex>

namespace face {

constexpr int kRadWaves = 4;                           // waves per workgroup

struct RadialWeights {
    const float *w_in, *b_in, *pair_tab, *w1, *b1, *w_phi, *b_phi;
};

// The passes of one launch: each set is one pass's weights and its outputs (forward) or upstream
// and input gradients (backward) over the same edges (rb, pair, env shared); workgroups
// [k * blocks_per_set, (k + 1) * blocks_per_set) serve set k, so independent passes share a
// launch (at small edge counts one pass fills about one wave per SIMD).
constexpr int kRadMaxSets = 4;
struct RadialSets {
    RadialWeights W[kRadMaxSets];
    float* h2[kRadMaxSets];
    float* phi[kRadMaxSets];
    const float* gh2[kRadMaxSets];
    const float* gphi[kRadMaxSets];
    const float* gphi2[kRadMaxSets];
    float* grb[kRadMaxSets];
    float* genv[kRadMaxSets];
    int n, blocks_per_set;
};

// sigmoid with the hardware exp2 and reciprocal (about 1 ulp each): the IEEE expf and divide
// sequences dominated the instruction count of the radial kernels
__device__ __forceinline__ float sigmoidf_(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.44269504088896341f * x));
}
// silu(u) = u s with s = sigmoid(u), kept for the derivative
__device__ __forceinline__ v4f silu4_s(v4f u, v4f& s) {
    v4f o;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s[r] = sigmoidf_(u[r]);
        o[r] = u[r] * s[r];
    }
    return o;
}
// d silu(u) / du = s (1 + u (1 - s)) = s + h (1 - s) from s = sigmoid(u) and h = silu(u)
__device__ __forceinline__ v4f dsilu4_sh(v4f s, v4f h) { return s + h * (1.f - s); }

// LDS image of the weights (floats): w_in [H][SI] (zero beyond n_basis), b_in [H],
// pair_tab [n_pair][H], w1 [H][S1], b1 [H], w_phi [16 BB][S1] (zero rows >= B), b_phi [16 BB].
struct RadialLds {
    int SI, S1, o_bin, o_pt, o_w1, o_b1, o_wp, o_bp, total;
    __host__ __device__ RadialLds(int H, int BB, int n_pair) {
        // w_in rows at a stride of 20 floats: the forward's read (row j, column 4kb+q) and the
        // backward's (row 4q+r, column j) each touch 64 distinct banks; at 16 the backward's was 4-way
        SI = 20;
        S1 = H + 4;
        o_bin = H * SI;
        o_pt = o_bin + H;
        o_w1 = o_pt + n_pair * H;
        o_b1 = o_w1 + H * S1;
        o_wp = o_b1 + H;
        o_bp = o_wp + 16 * BB * S1;
        total = o_bp + 16 * BB;
    }
};

// dst[v] = src(v) for v < n over the workgroup, 8 loads per thread in flight per batch.
template <typename Src>
__device__ __forceinline__ void stage_lds(float* dst, int n, Src src) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    for (int v0 = 0; v0 < n; v0 += 8 * nthr) {
        float b[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int v = v0 + u * nthr + tid;
            b[u] = v < n ? src(v) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int v = v0 + u * nthr + tid;
            if (v < n) dst[v] = b[u];
        }
    }
}

__device__ void radial_stage(float* lds, const RadialLds& L, const RadialWeights& W, int H, int BB, int nbasis,
                             int n_pair, int B) {
    stage_lds(lds, H * L.SI, [&](int v) {
        const int h = v / L.SI, k = v - h * L.SI;
        return k < nbasis ? W.w_in[h * nbasis + k] : 0.f;
    });
    stage_lds(lds + L.o_bin, H, [&](int v) { return W.b_in[v]; });
    stage_lds(lds + L.o_b1, H, [&](int v) { return W.b1[v]; });
    stage_lds(lds + L.o_pt, n_pair * H, [&](int v) { return W.pair_tab[v]; });
    stage_lds(lds + L.o_w1, H * L.S1, [&](int v) {
        const int h = v / L.S1, k = v - h * L.S1;
        return k < H ? W.w1[h * H + k] : 0.f;
    });
    stage_lds(lds + L.o_wp, 16 * BB * L.S1, [&](int v) {
        const int b = v / L.S1, k = v - b * L.S1;
        return (b < B && k < H) ? W.w_phi[b * H + k] : 0.f;
    });
    stage_lds(lds + L.o_bp, 16 * BB, [&](int v) { return v < B ? W.b_phi[v] : 0.f; });
}

__device__ __forceinline__ v4f lds4(const float* p) { return *reinterpret_cast<const v4f*>(p); }

// Forward chain of one tile (D layout): the two hidden activations hid, hh, their sigmoids s1, s2
// (for the backward's SiLU derivative) and phi before the envelope.
template <int HB, int BB>
__device__ __forceinline__ void radial_chain(const float* lds, const RadialLds& L, const float* xb, int nkb, int p,
                                             int j, int q, v4f (&s1)[HB], v4f (&hid)[HB], v4f (&s2)[HB],
                                             v4f (&hh)[HB], v4f (&pl)[BB]) {
    constexpr int H = 16 * HB;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
        v4f acc = z4;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            if (kb < nkb) acc = mfma_16x16x4(lds[(16 * hb + j) * L.SI + 4 * kb + q], xb[kb], acc);
        const v4f u1 = acc + lds4(lds + L.o_bin + 16 * hb + 4 * q) + lds4(lds + L.o_pt + p * H + 16 * hb + 4 * q);
        hid[hb] = silu4_s(u1, s1[hb]);
    }
#pragma unroll
    for (int h2b = 0; h2b < HB; ++h2b) {
        v4f acc = z4;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            const v4f a = lds4(lds + L.o_w1 + (16 * h2b + j) * L.S1 + 16 * hb + 4 * q);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc = mfma_16x16x4(a[r], hid[hb][r], acc);
        }
        hh[h2b] = silu4_s(acc + lds4(lds + L.o_b1 + 16 * h2b + 4 * q), s2[h2b]);
    }
#pragma unroll
    for (int bb = 0; bb < BB; ++bb) {
        v4f acc = z4;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            const v4f a = lds4(lds + L.o_wp + (16 * bb + j) * L.S1 + 16 * hb + 4 * q);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc = mfma_16x16x4(a[r], hh[hb][r], acc);
        }
        pl[bb] = acc + lds4(lds + L.o_bp + 16 * bb + 4 * q);
    }
}

// Row e, columns c0 .. c0+3 (those < n) of a row-major (*, ld) array.
__device__ __forceinline__ void store_cols(float* row, int c0, int n, v4f v) {
    if (c0 + 3 < n && ((reinterpret_cast<uintptr_t>(row + c0) & 15) == 0)) {
        st4(row + c0, v);
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (c0 + r < n) row[c0 + r] = v[r];
    }
}
__device__ __forceinline__ v4f load_cols(const float* row, int c0, int n) {
    if (c0 + 3 < n && ((reinterpret_cast<uintptr_t>(row + c0) & 15) == 0)) return ld4(row + c0);
    v4f v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (c0 + r < n) v[r] = row[c0 + r];
    return v;
}

template <int HB, int BB>
__global__ __launch_bounds__(kRadWaves * kWave) void radial_fwd_kernel(
    const float* __restrict__ rb, int ld_rb, int nbasis, const int32_t* __restrict__ pair,
    const float* __restrict__ env, int64_t E, RadialSets S, int n_pair, int B, int ld_h2, int ld_phi,
    int tiles_per_wave) {
    extern __shared__ float lds[];
    constexpr int H = 16 * HB;
    const int set = blockIdx.x / S.blocks_per_set;
    const int64_t bx = blockIdx.x - (int64_t)set * S.blocks_per_set;
    float* __restrict__ h2 = S.h2[set];
    float* __restrict__ phi = S.phi[set];
    const RadialLds L(H, BB, n_pair);
    radial_stage(lds, L, S.W[set], H, BB, nbasis, n_pair, B);
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int j = lane & 15, q = lane >> 4;
    const int nkb = (nbasis + 3) >> 2;
    const int64_t wave = bx * kRadWaves + threadIdx.x / kWave;
    for (int s = 0; s < tiles_per_wave; ++s) {
        const int64_t t0 = (wave * tiles_per_wave + s) * 16;
        if (t0 >= E) break;                            // uniform per wave
        const int64_t e = t0 + j;
        const bool ok = e < E;
        float xb[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) xb[kb] = (ok && 4 * kb + q < nbasis) ? rb[e * ld_rb + 4 * kb + q] : 0.f;
        int p = ok ? pair[e] : 0;
        p = p < 0 ? 0 : (p >= n_pair ? n_pair - 1 : p);
        v4f s1[HB], hid[HB], s2[HB], hh[HB], pl[BB];
        radial_chain<HB, BB>(lds, L, xb, nkb, p, j, q, s1, hid, s2, hh, pl);
        if (ok) {
            if (h2) {
#pragma unroll
                for (int hb = 0; hb < HB; ++hb) st4(h2 + e * ld_h2 + 16 * hb + 4 * q, hh[hb]);
            }
            const float ev = env ? env[e] : 1.f;
#pragma unroll
            for (int bb = 0; bb < BB; ++bb) store_cols(phi + e * ld_phi, 16 * bb + 4 * q, B, pl[bb] * ev);
        }
    }
}

template <int HB, int BB>
__global__ __launch_bounds__(kRadWaves * kWave) __attribute__((amdgpu_waves_per_eu(3))) void radial_bwd_kernel(
    const float* __restrict__ rb, int ld_rb, int nbasis, const int32_t* __restrict__ pair,
    const float* __restrict__ env, int64_t E, RadialSets S, int n_pair, int B, int ld_gh2, int ld_gphi, int ld_grb,
    int tiles_per_wave) {
    extern __shared__ float lds[];
    constexpr int H = 16 * HB;
    const int set = blockIdx.x / S.blocks_per_set;
    const int64_t bx = blockIdx.x - (int64_t)set * S.blocks_per_set;
    const float* __restrict__ gh2 = S.gh2[set];
    const float* __restrict__ gphi = S.gphi[set];
    const float* __restrict__ gphi2 = S.gphi2[set];
    float* __restrict__ grb = S.grb[set];
    float* __restrict__ genv = S.genv[set];
    const RadialLds L(H, BB, n_pair);
    radial_stage(lds, L, S.W[set], H, BB, nbasis, n_pair, B);
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int j = lane & 15, q = lane >> 4;
    const int nkb = (nbasis + 3) >> 2;
    const int64_t wave = bx * kRadWaves + threadIdx.x / kWave;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < tiles_per_wave; ++s) {
        const int64_t t0 = (wave * tiles_per_wave + s) * 16;
        if (t0 >= E) break;                            // uniform per wave
        const int64_t e = t0 + j;
        const bool ok = e < E;
        float xb[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) xb[kb] = (ok && 4 * kb + q < nbasis) ? rb[e * ld_rb + 4 * kb + q] : 0.f;
        int p = ok ? pair[e] : 0;
        p = p < 0 ? 0 : (p >= n_pair ? n_pair - 1 : p);
        v4f s1[HB], hid[HB], s2[HB], hh[HB], pl[BB];
        radial_chain<HB, BB>(lds, L, xb, nkb, p, j, q, s1, hid, s2, hh, pl);
        const float ev = ok ? (env ? env[e] : 1.f) : 0.f;
        // phi = pl * env: d env = sum_b gphi pl; d pl = gphi * env
        v4f gp[BB];
        float sden = 0.f;
#pragma unroll
        for (int bb = 0; bb < BB; ++bb) {
            gp[bb] = ok ? load_cols(gphi + e * ld_gphi, 16 * bb + 4 * q, B) : z4;
            if (gphi2 && ok) gp[bb] += load_cols(gphi2 + e * ld_gphi, 16 * bb + 4 * q, B);
            sden += gp[bb][0] * pl[bb][0] + gp[bb][1] * pl[bb][1] + gp[bb][2] * pl[bb][2] + gp[bb][3] * pl[bb][3];
            gp[bb] = gp[bb] * ev;
        }
        sden += __shfl_xor(sden, 16, kWave);
        sden += __shfl_xor(sden, 32, kWave);
        if (ok && genv && q == 0) genv[e] = sden;
        // d h2 = gh2 + W_phi^T d pl;  d u2 = d h2 * silu'(u2)
        v4f du2[HB];
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            v4f acc = (ok && gh2) ? ld4(gh2 + e * ld_gh2 + 16 * hb + 4 * q) : z4;
#pragma unroll
            for (int bb = 0; bb < BB; ++bb) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc = mfma_16x16x4(lds[L.o_wp + (16 * bb + 4 * q + r) * L.S1 + 16 * hb + j], gp[bb][r], acc);
            }
            du2[hb] = acc * dsilu4_sh(s2[hb], hh[hb]);
        }
        // d hid = W1^T d u2;  d u1 = d hid * silu'(u1)
        v4f du1[HB];
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
            v4f acc = z4;
#pragma unroll
            for (int h2b = 0; h2b < HB; ++h2b) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc = mfma_16x16x4(lds[L.o_w1 + (16 * h2b + 4 * q + r) * L.S1 + 16 * hb + j], du2[h2b][r], acc);
            }
            du1[hb] = acc * dsilu4_sh(s1[hb], hid[hb]);
        }
        // d rb = W_in^T d u1 (M = basis functions, one block of 16)
        v4f acc = z4;
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc = mfma_16x16x4(lds[(16 * hb + 4 * q + r) * L.SI + j], du1[hb][r], acc);
        }
        if (ok && grb) store_cols(grb + e * ld_grb, 4 * q, nbasis, acc);
    }
}

static size_t radial_lds_bytes(int H, int B, int n_pair) {
    return (size_t)RadialLds(H, (B + 15) / 16, n_pair).total * sizeof(float);
}

static int radial_tiles_per_wave(int64_t E) {
    const int64_t tiles = (E + 15) / 16;
    int64_t t = tiles / (256 * kRadWaves * 2);
    return (int)(t < 1 ? 1 : (t > 8 ? 8 : t));
}

static bool radial_args_ok(const float* rb, int ld_rb, int nbasis, const int32_t* pair, int64_t E,
                           const RadialWeights& W, int n_pair, int H, int B) {
    if (E < 0 || nbasis < 1 || nbasis > 16 || ld_rb < nbasis || n_pair < 1 || H < 16 || H > 64 || H % 16 ||
        B < 1 || B > 64)
        return false;
    if (E > 0 && (!rb || !pair)) return false;
    return W.w_in && W.b_in && W.pair_tab && W.w1 && W.b1 && W.w_phi && W.b_phi;
}


// ------------------------------------------------------------------ compiled radial (splines)
// phi(r; pair) from a table on a uniform grid r_g = g dr (face/model.py:383-418): values T and
// exact derivatives dT, (P pairs, G points, F columns) row-major; cubic Hermite (C1) between
// grid points, x = clamp(r / dr, 0, G - 1), i = min(floor x, G - 2), t = x - i:
//   S = h00 T[i] + h10 dr dT[i] + h01 T[i+1] + h11 dr dT[i+1]
//   h00 = 2t^3 - 3t^2 + 1, h10 = t^3 - 2t^2 + t, h01 = -2t^3 + 3t^2, h11 = t^3 - t^2,
// evaluated as T[i] + h01 (T[i+1] - T[i]) + ... (h00 = 1 - h01): neighbouring table values differ
// by ~dr |dS/dr|, and their fp32 difference is exact, whereas h00 T[i] + h01 T[i+1] rounds both
// products before they cancel -- in the r-derivative 6t(1-t) (T[i+1] - T[i]) / dr that round-off
// would be ~1e-4 of the slope at 4096 points.
// Columns f < nb go to phi[e][f] times env[e], columns f >= nb to R[e][f - nb] as they are
// (the CP columns: the pooling kernels apply the envelope). L lanes per edge (a power of two,
// about the row width) walk the columns, so every table row is read coalesced; the backward
// sums its column terms over those lanes.
struct SplineTab {
    const float *T, *dT;
    int P, G, F;
    float dr;
};

struct SplineCell {
    int64_t row;                                       // offset of T[pair][i][0]
    float t;
    bool inside;                                       // r / dr within [0, G - 1] (clamp passes d/dr)
};

__device__ __forceinline__ SplineCell spline_cell(float r, int32_t pair, const SplineTab& S) {
    SplineCell c;
    const float x0 = r / S.dr, hi = (float)(S.G - 1);
    c.inside = x0 >= 0.f && x0 <= hi;
    const float x = fminf(fmaxf(x0, 0.f), hi);        // NaN -> 0: the cell stays inside the table
    const int i = min((int)floorf(x), S.G - 2);
    c.t = x - (float)i;
    const int p = min(max((int)pair, 0), S.P - 1);
    c.row = ((int64_t)p * S.G + i) * S.F;
    return c;
}

// W columns per lane and load (1, or 4 when the rows are float4-aligned and nb % 4 == 0)
template <int W>
struct SplineVec;
template <>
struct SplineVec<1> {
    typedef float T;
    static __device__ __forceinline__ float ld(const float* p) { return *p; }
    static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
    static __device__ __forceinline__ float sum(float v) { return v; }
};
template <>
struct SplineVec<4> {
    typedef v4f T;
    static __device__ __forceinline__ v4f ld(const float* p) { return ld4(p); }
    static __device__ __forceinline__ void st(float* p, v4f v) { st4(p, v); }
    static __device__ __forceinline__ float sum(v4f v) { return (v[0] + v[1]) + (v[2] + v[3]); }
};

// The Hermite terms with their products fused in one fixed order (every kernel evaluating a spline
// rounds the same way):  herm = a dp + (b m0 + c m1),  with dp = p1 - p0 the table difference.
__device__ __forceinline__ float herm(float a, float dp, float b, float m0, float c, float m1) {
    return __builtin_fmaf(a, dp, __builtin_fmaf(b, m0, c * m1));
}
__device__ __forceinline__ v4f herm(float a, v4f dp, float b, v4f m0, float c, v4f m1) {
    v4f o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = herm(a, dp[k], b, m0[k], c, m1[k]);
    return o;
}
// acc + x y, fused per component
__device__ __forceinline__ float fma_acc(float acc, float x, float y) { return __builtin_fmaf(x, y, acc); }
__device__ __forceinline__ v4f fma_acc(v4f acc, v4f x, v4f y) {
    v4f o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = __builtin_fmaf(x[k], y[k], acc[k]);
    return o;
}

template <int L, int W>
__global__ __launch_bounds__(256) void radial_spline_fwd_kernel(const float* __restrict__ r,
                                                                const int32_t* __restrict__ pair, int64_t E,
                                                                SplineTab S, const float* __restrict__ env, int nb,
                                                                const int32_t* __restrict__ order,
                                                                float* __restrict__ phi, int ld_phi,
                                                                float* __restrict__ R, int ld_R) {
    typedef SplineVec<W> V;
    const int64_t tid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t q = tid / L;
    const int l = (int)(tid % L);
    if (q >= E) return;
    const int64_t e = order ? (int64_t)order[q] : q;
    const SplineCell c = spline_cell(r[e], pair[e], S);
    const float t = c.t, t2 = t * t, t3 = t2 * t;
    const float h10 = t3 - 2.f * t2 + t, h01 = -2.f * t3 + 3.f * t2, h11 = t3 - t2;
    const float ev = env ? env[e] : 1.f;
    const float* T0 = S.T + c.row;
    const float* D0 = S.dT + c.row;
    for (int f = W * l; f < S.F; f += W * L) {
        const typename V::T p0 = V::ld(T0 + f), p1 = V::ld(T0 + S.F + f);
        const typename V::T m0 = V::ld(D0 + f) * S.dr, m1 = V::ld(D0 + S.F + f) * S.dr;
        const typename V::T v = p0 + herm(h01, p1 - p0, h10, m0, h11, m1);
        if (f < nb)
            V::st(phi + e * ld_phi + f, v * ev);
        else
            V::st(R + e * ld_R + f - nb, v);
    }
}

template <int L, int W>
__global__ __launch_bounds__(256) void radial_spline_bwd_kernel(const float* __restrict__ r,
                                                                const int32_t* __restrict__ pair, int64_t E,
                                                                SplineTab S, const float* __restrict__ env, int nb,
                                                                const int32_t* __restrict__ order,
                                                                const float* __restrict__ gphi, int ld_gphi,
                                                                const float* __restrict__ gR, int ld_gR,
                                                                float* __restrict__ gr, float* __restrict__ genv) {
    typedef SplineVec<W> V;
    const int64_t tid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t q = tid / L;
    const int l = (int)(tid % L);
    if (q >= E) return;                                // whole groups of L lanes share q
    const int64_t e = order ? (int64_t)order[q] : q;
    const SplineCell c = spline_cell(r[e], pair[e], S);
    const float t = c.t, t2 = t * t, t3 = t2 * t;
    const float h10 = t3 - 2.f * t2 + t, h01 = -2.f * t3 + 3.f * t2, h11 = t3 - t2;
    const float d10 = 3.f * t2 - 4.f * t + 1.f, d01 = -6.f * t2 + 6.f * t, d11 = 3.f * t2 - 2.f * t;
    const float ev = env ? env[e] : 1.f;
    const float* T0 = S.T + c.row;
    const float* D0 = S.dT + c.row;
    typename V::T sr = {}, se = {};                    // d/dt and d/denv partial sums
    for (int f = W * l; f < S.F; f += W * L) {
        const bool lo = f < nb;
        const float* gp = lo ? gphi : gR;
        const typename V::T zero = {};
        const typename V::T gv = gp ? V::ld(lo ? gphi + e * ld_gphi + f : gR + e * ld_gR + f - nb) : zero;
        const typename V::T p0 = V::ld(T0 + f), p1 = V::ld(T0 + S.F + f);
        const typename V::T m0 = V::ld(D0 + f) * S.dr, m1 = V::ld(D0 + S.F + f) * S.dr;
        const typename V::T dp = p1 - p0;
        const typename V::T dv = herm(d01, dp, d10, m0, d11, m1);
        if (lo) {
            se = fma_acc(se, gv, p0 + herm(h01, dp, h10, m0, h11, m1));
            sr = fma_acc(sr, gv * ev, dv);
        } else {
            sr = fma_acc(sr, gv, dv);
        }
    }
    float srs = group_sum(V::sum(sr), L);
    float ses = group_sum(V::sum(se), L);
    if (l == 0) {
        gr[e] = c.inside ? srs / S.dr : 0.f;
        if (genv) genv[e] = ses;
    }
}

// Cell-run form of the two kernels above, for edges visited in table-cell order (`order` from
// the counting sort below; ~E / (P G) consecutive edges share one cell): a wave walks 64
// consecutive positions of the order, lane l owning column quads l + 64 s (s < NS, rows
// float4-aligned), and keeps the current cell's four table rows (T, dT at grid points i, i + 1)
// in registers, reloading them only where the cell changes. Each edge's phi / R row (forward) or
// upstream-gradient row (backward) is one coalesced row access; the per-edge quantities (edge,
// cell, t, env) are loaded once per wave and read back with v_readlane. Lane l's columns and the
// order of its partial sums are those of the L = 64 kernels above, so the results are the same.
constexpr int kRunLen = 64;                            // positions of the order per wave

struct RunEdges {                                      // this lane's edge of the wave's run
    int32_t e, cell;
    float t, ev;
    int inside;
};

__device__ __forceinline__ RunEdges run_edges(const float* __restrict__ r, const int32_t* __restrict__ pair,
                                              const float* __restrict__ env, const int32_t* __restrict__ order,
                                              int64_t q0, int n, int lane, const SplineTab& S) {
    RunEdges u{0, 0, 0.f, 0.f, 0};
    if (lane < n) {
        u.e = order[q0 + lane];
        const SplineCell c = spline_cell(r[u.e], pair[u.e], S);
        u.cell = (int32_t)(c.row / S.F);
        u.t = c.t;
        u.inside = c.inside;
        u.ev = env ? env[u.e] : 1.f;
    }
    return u;
}

template <int NS>
__global__ __launch_bounds__(256) void radial_spline_run_fwd_kernel(const float* __restrict__ r,
                                                                    const int32_t* __restrict__ pair, int64_t E,
                                                                    SplineTab S, const float* __restrict__ env, int nb,
                                                                    const int32_t* __restrict__ order,
                                                                    float* __restrict__ phi, int ld_phi,
                                                                    float* __restrict__ R, int ld_R) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t q0 = ((int64_t)blockIdx.x * (blockDim.x / kWave) +
                        __builtin_amdgcn_readfirstlane(threadIdx.x / kWave)) * kRunLen;
    if (q0 >= E) return;                               // uniform per wave
    const int n = (int)min((int64_t)kRunLen, E - q0);
    const RunEdges u = run_edges(r, pair, env, order, q0, n, lane, S);
    v4f p0[NS], p1[NS], m0[NS], m1[NS];
    int32_t cur = -1;
    for (int k = 0; k < n; ++k) {
        const int32_t cell = __builtin_amdgcn_readlane(u.cell, k);
        const int64_t e = __builtin_amdgcn_readlane(u.e, k);
        if (cell != cur) {                             // uniform: reload the cell's rows
            cur = cell;
            const float* T0 = S.T + (int64_t)cell * S.F;
            const float* D0 = S.dT + (int64_t)cell * S.F;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int f = 4 * (lane + kWave * s);
                if (f < S.F) {
                    p0[s] = ld4(T0 + f), p1[s] = ld4(T0 + S.F + f);
                    m0[s] = ld4(D0 + f) * S.dr, m1[s] = ld4(D0 + S.F + f) * S.dr;
                }
            }
        }
        const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(u.t), k));
        const float ev = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(u.ev), k));
        const float t2 = t * t, t3 = t2 * t;
        const float h10 = t3 - 2.f * t2 + t, h01 = -2.f * t3 + 3.f * t2, h11 = t3 - t2;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int f = 4 * (lane + kWave * s);
            if (f < S.F) {
                const v4f v = p0[s] + herm(h01, p1[s] - p0[s], h10, m0[s], h11, m1[s]);
                if (f < nb)
                    st4(phi + e * ld_phi + f, v * ev);
                else
                    st4(R + e * ld_R + f - nb, v);
            }
        }
    }
}

template <int NS>
__global__ __launch_bounds__(256) void radial_spline_run_bwd_kernel(const float* __restrict__ r,
                                                                    const int32_t* __restrict__ pair, int64_t E,
                                                                    SplineTab S, const float* __restrict__ env, int nb,
                                                                    const int32_t* __restrict__ order,
                                                                    const float* __restrict__ gphi, int ld_gphi,
                                                                    const float* __restrict__ gR, int ld_gR,
                                                                    float* __restrict__ gr, float* __restrict__ genv) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t q0 = ((int64_t)blockIdx.x * (blockDim.x / kWave) +
                        __builtin_amdgcn_readfirstlane(threadIdx.x / kWave)) * kRunLen;
    if (q0 >= E) return;                               // uniform per wave
    const int n = (int)min((int64_t)kRunLen, E - q0);
    const RunEdges u = run_edges(r, pair, env, order, q0, n, lane, S);
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    // upstream gradient of column quad s of edge e (zero where its operand is absent)
    auto load_g = [&](int64_t e, v4f (&g)[NS]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int f = 4 * (lane + kWave * s);
            g[s] = z4;
            if (f < S.F) {
                if (f < nb) {
                    if (gphi) g[s] = ld4(gphi + e * ld_gphi + f);
                } else if (gR) {
                    g[s] = ld4(gR + e * ld_gR + f - nb);
                }
            }
        }
    };
    v4f p0[NS], p1[NS], m0[NS], m1[NS], g[NS], gn[NS];
    load_g(__builtin_amdgcn_readlane(u.e, 0), gn);
    int32_t cur = -1;
    for (int k = 0; k < n; ++k) {
        const int32_t cell = __builtin_amdgcn_readlane(u.cell, k);
        const int64_t e = __builtin_amdgcn_readlane(u.e, k);
#pragma unroll
        for (int s = 0; s < NS; ++s) g[s] = gn[s];
        if (k + 1 < n) load_g(__builtin_amdgcn_readlane(u.e, k + 1), gn);   // next edge's row in flight
        if (cell != cur) {
            cur = cell;
            const float* T0 = S.T + (int64_t)cell * S.F;
            const float* D0 = S.dT + (int64_t)cell * S.F;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int f = 4 * (lane + kWave * s);
                if (f < S.F) {
                    p0[s] = ld4(T0 + f), p1[s] = ld4(T0 + S.F + f);
                    m0[s] = ld4(D0 + f) * S.dr, m1[s] = ld4(D0 + S.F + f) * S.dr;
                }
            }
        }
        const float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(u.t), k));
        const float ev = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(u.ev), k));
        const int inside = __builtin_amdgcn_readlane(u.inside, k);
        const float t2 = t * t, t3 = t2 * t;
        const float h10 = t3 - 2.f * t2 + t, h01 = -2.f * t3 + 3.f * t2, h11 = t3 - t2;
        const float d10 = 3.f * t2 - 4.f * t + 1.f, d01 = -6.f * t2 + 6.f * t, d11 = 3.f * t2 - 2.f * t;
        v4f sr = z4, se = z4;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int f = 4 * (lane + kWave * s);
            if (f < S.F) {
                const v4f dp = p1[s] - p0[s];
                const v4f dv = herm(d01, dp, d10, m0[s], d11, m1[s]);
                if (f < nb) {
                    se = fma_acc(se, g[s], p0[s] + herm(h01, dp, h10, m0[s], h11, m1[s]));
                    sr = fma_acc(sr, g[s] * ev, dv);
                } else {
                    sr = fma_acc(sr, g[s], dv);
                }
            }
        }
        const float srs = group_sum(SplineVec<4>::sum(sr), kWave);
        const float ses = group_sum(SplineVec<4>::sum(se), kWave);
        if (lane == 0) {
            gr[e] = inside ? srs / S.dr : 0.f;
            if (genv) genv[e] = ses;
        }
    }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// column-quad slots per lane of the cell-run kernels (edges given in table-cell order, float4
// rows, up to 5 x 64 quads), or 0 for the per-edge kernels
static int run_slots(const int32_t* order, bool vec, int F) {
    const int ns = (F / 4 + kWave - 1) / kWave;
    return (order && vec && ns <= 5) ? ns : 0;
}

// lanes per edge: a power of two about the number of column groups (W columns each), at most 64
static int spline_lanes(int F, int W) {
    const int g = (F + W - 1) / W;
    return g <= 4 ? 4 : (g <= 8 ? 8 : (g <= 16 ? 16 : (g <= 32 ? 32 : 64)));
}

// Edge order by table cell (pair, grid interval): a counting sort, so that consecutive
// workgroups of the spline kernels read the same table rows (from L2) instead of each edge
// gathering its rows from HBM. Order within a cell is arbitrary (atomic cursors): every edge's
// outputs are its own, so the results do not depend on it.
__global__ __launch_bounds__(256) void spline_zero_kernel(int32_t* __restrict__ a, int64_t n) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t < n) a[t] = 0;
}

__global__ __launch_bounds__(256) void spline_count_kernel(const float* __restrict__ r,
                                                           const int32_t* __restrict__ pair, int64_t E, SplineTab S,
                                                           int32_t* __restrict__ cnt) {
    const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (e >= E) return;
    const SplineCell c = spline_cell(r[e], pair[e], S);
    atomicAdd(cnt + c.row / S.F, 1);
}

// exclusive scan of n counts in place, one workgroup of 1024 threads (n = P * G, tens of
// thousands): per-thread chunk sums, a workgroup scan of the 1024 partials in LDS, then each
// thread rewrites its chunk
__global__ __launch_bounds__(1024) void spline_scan_kernel(int32_t* __restrict__ cnt, int n) {
    __shared__ int32_t part[1024];
    const int t = threadIdx.x, chunk = (n + 1023) / 1024;
    const int b = min(n, t * chunk), e = min(n, b + chunk);
    int32_t s = 0;
    for (int k = b; k < e; ++k) s += cnt[k];
    part[t] = s;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {              // Hillis-Steele inclusive scan
        const int32_t v = t >= o ? part[t - o] : 0;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    int32_t run = t > 0 ? part[t - 1] : 0;
    for (int k = b; k < e; ++k) {
        const int32_t c = cnt[k];
        cnt[k] = run;
        run += c;
    }
}

__global__ __launch_bounds__(256) void spline_place_kernel(const float* __restrict__ r,
                                                           const int32_t* __restrict__ pair, int64_t E, SplineTab S,
                                                           int32_t* __restrict__ cursor,
                                                           int32_t* __restrict__ order) {
    const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (e >= E) return;
    const SplineCell c = spline_cell(r[e], pair[e], S);
    order[atomicAdd(cursor + c.row / S.F, 1)] = (int32_t)e;
}

static bool spline_args_ok(const float* r, const int32_t* pair, int64_t E, const float* T, const float* dT, int P,
                           int G, int F, float dr, int nb) {
    if (E < 0 || P < 1 || G < 2 || F < 1 || !(dr > 0.f) || nb < 0 || nb > F) return false;
    return E == 0 || (r && pair && T && dT);
}

}  // namespace face

using namespace face;

#define FACE_RADIAL_DISPATCH(KERNEL, ...)                                                               \
    do {                                                                                                \
        const int hb_ = H / 16, bb_ = (B + 15) / 16;                                                    \
        const int64_t waves_ = ((E + 15) / 16 + tpw - 1) / tpw;                                         \
        S.blocks_per_set = (int)((waves_ + kRadWaves - 1) / kRadWaves);                                 \
        const dim3 grid_((unsigned)((int64_t)S.blocks_per_set * S.n)), block_(kRadWaves * kWave);        \
        const hipStream_t st_ = (hipStream_t)stream;                                                    \
        switch (hb_ * 10 + bb_) {                                                                       \
            case 11: hipLaunchKernelGGL((KERNEL<1, 1>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 12: hipLaunchKernelGGL((KERNEL<1, 2>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 21: hipLaunchKernelGGL((KERNEL<2, 1>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 22: hipLaunchKernelGGL((KERNEL<2, 2>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 31: hipLaunchKernelGGL((KERNEL<3, 1>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 32: hipLaunchKernelGGL((KERNEL<3, 2>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 41: hipLaunchKernelGGL((KERNEL<4, 1>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 42: hipLaunchKernelGGL((KERNEL<4, 2>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 43: hipLaunchKernelGGL((KERNEL<4, 3>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            case 44: hipLaunchKernelGGL((KERNEL<4, 4>), grid_, block_, lds, st_, __VA_ARGS__); break;   \
            default: return FACE_ERR_UNSUPPORTED;                                                       \
        }                                                                                               \
    } while (0)

static bool radial_sets_ok(const float* rb, int ld_rb, int nbasis, const int32_t* pair, int64_t E, int n_sets,
                           const RadialSets& S, int n_pair, int H, int B) {
    if (n_sets < 1 || n_sets > kRadMaxSets) return false;
    for (int k = 0; k < n_sets; ++k)
        if (!radial_args_ok(rb, ld_rb, nbasis, pair, E, S.W[k], n_pair, H, B)) return false;
    return true;
}

static int radial_fwd_launch(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair, const float* env,
                             int64_t E, RadialSets& S, int32_t n_pair, int32_t H, int32_t B, int32_t ld_h2,
                             int32_t ld_phi, void* stream) {
    if (!radial_sets_ok(rb, ld_rb, n_basis, pair, E, S.n, S, n_pair, H, B) || ld_phi < B) return FACE_ERR_ARG;
    for (int k = 0; k < S.n; ++k)
        if ((E > 0 && !S.phi[k]) || (S.h2[k] && (ld_h2 < H || ld_h2 % 4 || ((uintptr_t)S.h2[k] & 15))))
            return FACE_ERR_ARG;
    if (E == 0) return 0;
    const size_t lds = radial_lds_bytes(H, B, n_pair);
    if (lds > 65536) return FACE_ERR_UNSUPPORTED;
    const int tpw = radial_tiles_per_wave(E);
    FACE_RADIAL_DISPATCH(radial_fwd_kernel, rb, ld_rb, n_basis, pair, env, E, S, n_pair, B, ld_h2, ld_phi, tpw);
    FACE_LAUNCH_CHECK();
    return 0;
}

static int radial_bwd_launch(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair, const float* env,
                             int64_t E, RadialSets& S, int32_t n_pair, int32_t H, int32_t B, int32_t ld_gh2,
                             int32_t ld_gphi, int32_t ld_grb, void* stream) {
    if (!radial_sets_ok(rb, ld_rb, n_basis, pair, E, S.n, S, n_pair, H, B) || ld_gphi < B) return FACE_ERR_ARG;
    for (int k = 0; k < S.n; ++k)
        if ((E > 0 && !S.gphi[k]) || (S.gh2[k] && (ld_gh2 < H || ld_gh2 % 4 || ((uintptr_t)S.gh2[k] & 15))) ||
            (S.grb[k] && ld_grb < n_basis))
            return FACE_ERR_ARG;
    if (E == 0) return 0;
    const size_t lds = radial_lds_bytes(H, B, n_pair);
    if (lds > 65536) return FACE_ERR_UNSUPPORTED;
    const int tpw = radial_tiles_per_wave(E);
    FACE_RADIAL_DISPATCH(radial_bwd_kernel, rb, ld_rb, n_basis, pair, env, E, S, n_pair, B, ld_gh2, ld_gphi, ld_grb,
                         tpw);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_radial_fwd(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair,
                               const float* env, int64_t E, const float* w_in, const float* b_in,
                               const float* pair_tab, int32_t n_pair, int32_t H, const float* w1, const float* b1,
                               const float* w_phi, const float* b_phi, int32_t B, float* h2, int32_t ld_h2,
                               float* phi, int32_t ld_phi, void* stream) {
    RadialSets S{};
    S.n = 1;
    S.W[0] = RadialWeights{w_in, b_in, pair_tab, w1, b1, w_phi, b_phi};
    S.h2[0] = h2;
    S.phi[0] = phi;
    return radial_fwd_launch(rb, ld_rb, n_basis, pair, env, E, S, n_pair, H, B, ld_h2, ld_phi, stream);
}

extern "C" int face_radial_bwd(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair,
                               const float* env, int64_t E, const float* w_in, const float* b_in,
                               const float* pair_tab, int32_t n_pair, int32_t H, const float* w1, const float* b1,
                               const float* w_phi, const float* b_phi, int32_t B, const float* gh2, int32_t ld_gh2,
                               const float* gphi, const float* gphi2, int32_t ld_gphi, float* grb, int32_t ld_grb,
                               float* genv, void* stream) {
    RadialSets S{};
    S.n = 1;
    S.W[0] = RadialWeights{w_in, b_in, pair_tab, w1, b1, w_phi, b_phi};
    S.gh2[0] = gh2;
    S.gphi[0] = gphi;
    S.gphi2[0] = gphi2;
    S.grb[0] = grb;
    S.genv[0] = genv;
    return radial_bwd_launch(rb, ld_rb, n_basis, pair, env, E, S, n_pair, H, B, ld_gh2, ld_gphi, ld_grb, stream);
}

// weights of set k from the host arrays (w[k * 7 + 0..6] = w_in, b_in, pair_tab, w1, b1, w_phi, b_phi)
static bool radial_sets_from(int32_t n_sets, const float* const* w, RadialSets& S) {
    if (n_sets < 1 || n_sets > kRadMaxSets || !w) return false;
    S.n = n_sets;
    for (int k = 0; k < n_sets; ++k)
        S.W[k] = RadialWeights{w[7 * k], w[7 * k + 1], w[7 * k + 2], w[7 * k + 3], w[7 * k + 4], w[7 * k + 5],
                               w[7 * k + 6]};
    return true;
}

extern "C" int face_radial_fwd_sets(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair,
                                    const float* env, int64_t E, int32_t n_sets, const float* const* weights,
                                    int32_t n_pair, int32_t H, int32_t B, float* const* h2, int32_t ld_h2,
                                    float* const* phi, int32_t ld_phi, void* stream) {
    RadialSets S{};
    if (!radial_sets_from(n_sets, weights, S) || !phi) return FACE_ERR_ARG;
    for (int k = 0; k < n_sets; ++k) {
        S.h2[k] = h2 ? h2[k] : nullptr;
        S.phi[k] = phi[k];
    }
    return radial_fwd_launch(rb, ld_rb, n_basis, pair, env, E, S, n_pair, H, B, ld_h2, ld_phi, stream);
}

extern "C" int face_radial_bwd_sets(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair,
                                    const float* env, int64_t E, int32_t n_sets, const float* const* weights,
                                    int32_t n_pair, int32_t H, int32_t B, const float* const* gh2, int32_t ld_gh2,
                                    const float* const* gphi, const float* const* gphi2, int32_t ld_gphi,
                                    float* const* grb, int32_t ld_grb, float* const* genv, void* stream) {
    RadialSets S{};
    if (!radial_sets_from(n_sets, weights, S) || !gphi) return FACE_ERR_ARG;
    for (int k = 0; k < n_sets; ++k) {
        S.gh2[k] = gh2 ? gh2[k] : nullptr;
        S.gphi[k] = gphi[k];
        S.gphi2[k] = gphi2 ? gphi2[k] : nullptr;
        S.grb[k] = grb ? grb[k] : nullptr;
        S.genv[k] = genv ? genv[k] : nullptr;
    }
    return radial_bwd_launch(rb, ld_rb, n_basis, pair, env, E, S, n_pair, H, B, ld_gh2, ld_gphi, ld_grb, stream);
}

extern "C" int face_radial_spline_fwd(const float* r, const int32_t* pair, int64_t E, const float* T, const float* dT,
                                      int32_t P, int32_t G, int32_t F, float dr, const float* env, int32_t nb,
                                      const int32_t* order, float* phi, int32_t ld_phi, float* R, int32_t ld_R,
                                      void* stream) {
    if (!spline_args_ok(r, pair, E, T, dT, P, G, F, dr, nb) || (nb > 0 && (ld_phi < nb || (E > 0 && !phi))) ||
        (nb < F && (ld_R < F - nb || (E > 0 && !R))))
        return FACE_ERR_ARG;
    if (E == 0) return 0;
    const SplineTab tab{T, dT, P, G, F, dr};
    const bool vec = F % 4 == 0 && nb % 4 == 0 && al16(T) && al16(dT) && (nb == 0 || (ld_phi % 4 == 0 && al16(phi))) &&
                     (nb == F || (ld_R % 4 == 0 && al16(R)));
    const int W = vec ? 4 : 1, L = spline_lanes(F, W);
    const dim3 grid((unsigned)((E * L + 255) / 256)), block(256);
    const hipStream_t st = (hipStream_t)stream;
#define FACE_SPLINE(K_, L_, W_) \
    hipLaunchKernelGGL((K_<L_, W_>), grid, block, 0, st, r, pair, E, tab, env, nb, order, ARGS_)
#define FACE_SPLINE_RUN(K_, NS_)                                                               \
    do {                                                                                       \
        const dim3 rgrid((unsigned)(((E + kRunLen - 1) / kRunLen + 3) / 4)), rblock(4 * kWave); \
        switch (NS_) {                                                                         \
            case 1: hipLaunchKernelGGL((K_<1>), rgrid, rblock, 0, st, r, pair, E, tab, env, nb, order, ARGS_); break; \
            case 2: hipLaunchKernelGGL((K_<2>), rgrid, rblock, 0, st, r, pair, E, tab, env, nb, order, ARGS_); break; \
            case 3: hipLaunchKernelGGL((K_<3>), rgrid, rblock, 0, st, r, pair, E, tab, env, nb, order, ARGS_); break; \
            case 4: hipLaunchKernelGGL((K_<4>), rgrid, rblock, 0, st, r, pair, E, tab, env, nb, order, ARGS_); break; \
            default: hipLaunchKernelGGL((K_<5>), rgrid, rblock, 0, st, r, pair, E, tab, env, nb, order, ARGS_); break; \
        }                                                                                      \
    } while (0)
#define FACE_SPLINE_L(K_, W_)                           \
    switch (L) {                                        \
        case 4: FACE_SPLINE(K_, 4, W_); break;          \
        case 8: FACE_SPLINE(K_, 8, W_); break;          \
        case 16: FACE_SPLINE(K_, 16, W_); break;        \
        case 32: FACE_SPLINE(K_, 32, W_); break;        \
        default: FACE_SPLINE(K_, 64, W_); break;        \
    }
#define ARGS_ phi, ld_phi, R, ld_R
    const int ns = run_slots(order, vec, F);
    if (ns > 0) {
        FACE_SPLINE_RUN(radial_spline_run_fwd_kernel, ns);
    } else if (vec) {
        FACE_SPLINE_L(radial_spline_fwd_kernel, 4)
    } else {
        FACE_SPLINE_L(radial_spline_fwd_kernel, 1)
    }
#undef ARGS_
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_radial_spline_bwd(const float* r, const int32_t* pair, int64_t E, const float* T, const float* dT,
                                      int32_t P, int32_t G, int32_t F, float dr, const float* env, int32_t nb,
                                      const int32_t* order, const float* gphi, int32_t ld_gphi, const float* gR,
                                      int32_t ld_gR, float* gr, float* genv, void* stream) {
    if (!spline_args_ok(r, pair, E, T, dT, P, G, F, dr, nb) || (gphi && ld_gphi < nb) || (gR && ld_gR < F - nb) ||
        (E > 0 && !gr))
        return FACE_ERR_ARG;
    if (E == 0) return 0;
    const SplineTab tab{T, dT, P, G, F, dr};
    const bool vec = F % 4 == 0 && nb % 4 == 0 && al16(T) && al16(dT) &&
                     (!gphi || (ld_gphi % 4 == 0 && al16(gphi))) && (!gR || (ld_gR % 4 == 0 && al16(gR)));
    const int W = vec ? 4 : 1, L = spline_lanes(F, W);
    const dim3 grid((unsigned)((E * L + 255) / 256)), block(256);
    const hipStream_t st = (hipStream_t)stream;
#define ARGS_ gphi, ld_gphi, gR, ld_gR, gr, genv
    const int ns = run_slots(order, vec, F);
    if (ns > 0) {
        FACE_SPLINE_RUN(radial_spline_run_bwd_kernel, ns);
    } else if (vec) {
        FACE_SPLINE_L(radial_spline_bwd_kernel, 4)
    } else {
        FACE_SPLINE_L(radial_spline_bwd_kernel, 1)
    }
#undef ARGS_
#undef FACE_SPLINE_L
#undef FACE_SPLINE_RUN
#undef FACE_SPLINE
    FACE_LAUNCH_CHECK();
    return 0;
}

// ---------------------------------------------------------------- allocation-free edge order
// face_radial_spline_order with its counting-sort counters in a file-scope device array instead of a
// caller workspace, for callers that cannot allocate. Each GPU the library runs on holds its own copy
// of the array (4 MiB) until the process ends. In host code `spline_order_scratch` names a host-side
// stand-in, not device memory: its device address is taken once per device with
// hipGetSymbolAddress (that device current) and only that address is passed to kernels.
static __device__ __align__(256) int32_t spline_order_scratch[FACE_SPLINE_ORDER_SCRATCH];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's copy of spline_order_scratch (looked up on the first call on the
// device, with that device current); nullptr and the HIP status on failure.
int32_t* spline_scratch_for(int dev, int* status) {
    *status = 0;
    if (dev < 0 || dev >= kMaxDevices) {
        *status = FACE_ERR_ARG;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void* p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(spline_order_scratch));
        if (cur >= 0 && cur != dev) {
            const hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess || !p) {
            *status = e != hipSuccess ? (int)e : FACE_ERR_ARG;
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<int32_t*>(p);
    }
    return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int face_radial_spline_order_noalloc(const float* r, const int32_t* pair, int64_t E, int32_t P, int32_t G,
                                                float dr, int32_t* order, void* stream) {
    if (E < 0 || P < 1 || G < 2 || !(dr > 0.f) || E > 0x7fffffff) return FACE_ERR_ARG;
    if ((int64_t)P * G > FACE_SPLINE_ORDER_SCRATCH) return FACE_ERR_SCRATCH;
    if (E == 0) return 0;
    if (!r || !pair || !order) return FACE_ERR_ARG;
    int dev = -1;
    hipError_t e = stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    int status = 0;
    int32_t* work = spline_scratch_for(dev, &status);
    if (!work) return status;
    return face_radial_spline_order(r, pair, E, P, G, dr, work, order, stream);
}

extern "C" int face_radial_spline_order(const float* r, const int32_t* pair, int64_t E, int32_t P, int32_t G,
                                        float dr, int32_t* work, int32_t* order, void* stream) {
    if (E < 0 || P < 1 || G < 2 || !(dr > 0.f) || (int64_t)P * G > 0x7fffffff || E > 0x7fffffff) return FACE_ERR_ARG;
    if (E == 0) return 0;
    if (!r || !pair || !work || !order) return FACE_ERR_ARG;
    const SplineTab tab{nullptr, nullptr, P, G, 1, dr};
    const int64_t n = (int64_t)P * G;
    const hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(spline_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, work, n);
    hipLaunchKernelGGL(spline_count_kernel, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, st, r, pair, E, tab,
                       work);
    hipLaunchKernelGGL(spline_scan_kernel, dim3(1), dim3(1024), 0, st, work, (int)n);
    hipLaunchKernelGGL(spline_place_kernel, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, st, r, pair, E, tab,
                       work, order);
    FACE_LAUNCH_CHECK();
    return 0;
}
