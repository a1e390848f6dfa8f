// Per-(atom, channel) invariant algebra of FACE's symmetric Cartesian moments (gfx950).
//
// Forward and hand-derived backward of face/node_kernel.py:212-228 (= face/model.py:252-264,
// 288-291). One thread per (atom, channel); every operand is read through explicit
// (atom, channel, component) strides, so the kernels consume the projection GEMM output
// (atom, component, 3C) in place and write the invariant families straight into the
// (atom, 9C) feature row the readout consumes.
#include "common.h"

namespace face {

// Symmetric component of a rank-2 / rank-3 full index (component order xx,yy,zz,xy,xz,yz and
// xxx,yyy,zzz,xxy,xxz,xyy,yyz,xzz,yzz,xyz; face/cartesian.py:11-17).
__host__ __device__ constexpr int sym2(int a, int b) {
    return a == b ? a : (a + b == 1 ? 3 : (a + b == 2 ? 4 : 5));
}
__host__ __device__ constexpr int sym3(int a, int b, int c) {
    // sort (a,b,c) then map the multiset to its component
    int lo = a < b ? a : b, hi = a < b ? b : a;
    int x = c < lo ? c : lo, z = c > hi ? c : hi, y = a + b + c - x - z;
    if (x == y && y == z) return x;
    if (x == y) return z == 1 ? 3 : (x == 0 ? 4 : 6);     // (0,0,1) (0,0,2) (1,1,2)
    if (y == z) return x == 0 ? (y == 1 ? 5 : 7) : 8;     // (0,1,1) (0,2,2) (1,2,2)
    return 9;                                             // (0,1,2)
}

struct Strided8 {
    const float* p[8];
    int64_t sn[8], sc[8], sk[8];
};
struct StridedOut8 {
    float* p[8];
    int64_t sn[8], sc[8], sk[8];
};
struct Str3 {
    int64_t sn, sc, sk;
};

struct NodeRegs {
    float p1[3], q1[3], s1[3], p2[9], q2[9], s2[9], p3[27], q3[27];
};

__device__ __forceinline__ void load_node(const Strided8& in, int64_t n, int c, NodeRegs& r) {
#define LD(T, a) (in.p[T][n * in.sn[T] + (int64_t)c * in.sc[T] + (int64_t)(a)*in.sk[T]])
    float t2p[6], t2q[6], t2s[6], t3p[10], t3q[10];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        r.p1[a] = LD(0, a);
        r.q1[a] = LD(1, a);
        r.s1[a] = LD(2, a);
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        t2p[k] = LD(3, k);
        t2q[k] = LD(4, k);
        t2s[k] = LD(5, k);
    }
#pragma unroll
    for (int k = 0; k < 10; ++k) {
        t3p[k] = LD(6, k);
        t3q[k] = LD(7, k);
    }
#undef LD
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            r.p2[a * 3 + b] = t2p[sym2(a, b)];
            r.q2[a * 3 + b] = t2q[sym2(a, b)];
            r.s2[a * 3 + b] = t2s[sym2(a, b)];
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                r.p3[a * 9 + b * 3 + d] = t3p[sym3(a, b, d)];
                r.q3[a * 9 + b * 3 + d] = t3q[sym3(a, b, d)];
            }
        }
}

// Intermediate contractions shared by forward and backward.
struct NodeMid {
    float q2s1[3], p2q1[3], p3q2[3], pq2[9], p3s1[9];
};

__device__ __forceinline__ void node_mid(const NodeRegs& r, NodeMid& m) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        float x = 0.f, y = 0.f, z = 0.f;
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            x = fmaf(r.q2[a * 3 + b], r.s1[b], x);
            y = fmaf(r.p2[a * 3 + b], r.q1[b], y);
#pragma unroll
            for (int d = 0; d < 3; ++d) z = fmaf(r.p3[a * 9 + b * 3 + d], r.q2[b * 3 + d], z);
        }
        m.q2s1[a] = x;
        m.p2q1[a] = y;
        m.p3q2[a] = z;
    }
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            float x = 0.f, y = 0.f;
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                x = fmaf(r.p2[a * 3 + b], r.q2[b * 3 + d], x);
                y = fmaf(r.p3[a * 9 + d * 3 + b], r.s1[b], y);
            }
            m.pq2[a * 3 + d] = x;
            m.p3s1[a * 3 + d] = y;
        }
}

// The eight invariant families of one (atom, channel) (face/node_kernel.py:18-64).
__device__ __forceinline__ void node_invariants(const NodeRegs& r, const NodeMid& m, float (&f)[8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = 0.f;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        f[0] = fmaf(r.p1[a], r.q1[a], f[0]);
        f[3] = fmaf(r.p1[a], m.q2s1[a], f[3]);
        f[5] = fmaf(m.p3q2[a], r.s1[a], f[5]);
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) f[1] = fmaf(r.p2[k], r.q2[k], f[1]);
#pragma unroll
    for (int k = 0; k < 27; ++k) f[2] = fmaf(r.p3[k], r.q3[k], f[2]);
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            f[4] = fmaf(m.pq2[a * 3 + d], r.s2[d * 3 + a], f[4]);
            f[7] = fmaf(r.q1[a] * m.p3s1[a * 3 + d], r.q1[d], f[7]);
            float x = 0.f;
#pragma unroll
            for (int b = 0; b < 3; ++b)
#pragma unroll
                for (int e = 0; e < 3; ++e) x = fmaf(r.p3[e * 9 + b * 3 + a], r.q3[e * 9 + b * 3 + d], x);
            f[6] = fmaf(x, r.s2[a * 3 + d], f[6]);
        }
}

// V (3) and Mf (9 full or 6 symmetrised) of one (atom, channel), written at vo / mo with the
// component strides vsk / msk.
__device__ __forceinline__ void node_eq_outputs(const NodeRegs& r, const NodeMid& m, const float* __restrict__ av,
                                                const float* __restrict__ bv, int c, int C, float* vo, int64_t vsk,
                                                float* mo, int64_t msk, int mf_mode) {
    const float a0 = av[c], a1 = av[C + c], a2 = av[2 * C + c], a3 = av[3 * C + c];
    const float b0 = bv[c], b1 = bv[C + c], b2 = bv[2 * C + c], b3 = bv[3 * C + c];
#pragma unroll
    for (int a = 0; a < 3; ++a) vo[a * vsk] = a0 * r.p1[a] + a1 * m.q2s1[a] + a2 * m.p3q2[a] + a3 * m.p2q1[a];
    float mf[9];
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int d = 0; d < 3; ++d)
            mf[a * 3 + d] = b0 * r.p2[a * 3 + d] + b1 * r.p1[a] * r.q1[d] + b2 * m.pq2[a * 3 + d] +
                            b3 * m.p3s1[a * 3 + d];
    if (mf_mode == 0) {
#pragma unroll
        for (int k = 0; k < 9; ++k) mo[k * msk] = mf[k];
    } else {
#pragma unroll
        for (int a = 0; a < 3; ++a) mo[a * msk] = mf[a * 4];
        mo[3 * msk] = 0.5f * (mf[1] + mf[3]);
        mo[4 * msk] = 0.5f * (mf[2] + mf[6]);
        mo[5 * msk] = 0.5f * (mf[5] + mf[7]);
    }
}

// Input gradients of one (atom, channel) from the invariant-family gradients g, gV, gM (full
// 3x3) and the V / Mf coefficients: the full tensors' gradients formed entry by entry and folded
// into the symmetric components they were expanded from; the coefficient partials when dap.
__device__ __forceinline__ void node_bwd_core(const NodeRegs& r, const NodeMid& m, const float (&g)[8],
                                              const float (&gv)[3], const float (&gm)[9], float a0, float a1,
                                              float a2, float a3, float b0, float b1, float b2, float b3,
                                              const StridedOut8& out, int64_t n, int c, float* dap,
                                              float* dbp) {
    // ---- rank 1
    float dp1[3], dq1[3], ds1[3];
#pragma unroll
    for (int z = 0; z < 3; ++z) {
        float gmq = 0.f, gmp = 0.f, gvp2 = 0.f, gvq2 = 0.f, p1q2 = 0.f, t8 = 0.f, qp3s1 = 0.f, gmp3 = 0.f;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            gmq = fmaf(gm[z * 3 + a], r.q1[a], gmq);           // sum_d gM[z,d] Q1[d]
            gmp = fmaf(gm[a * 3 + z], r.p1[a], gmp);           // sum_a gM[a,z] P1[a]
            gvp2 = fmaf(gv[a], r.p2[a * 3 + z], gvp2);         // sum_a gV[a] P2[a,z]
            gvq2 = fmaf(gv[a], r.q2[a * 3 + z], gvq2);         // sum_a gV[a] Q2[a,z]
            p1q2 = fmaf(r.p1[a], r.q2[a * 3 + z], p1q2);       // sum_a P1[a] Q2[a,z]
            qp3s1 = fmaf(m.p3s1[z * 3 + a], r.q1[a], qp3s1);   // sum_d P3[z,b,d] S1[b] Q1[d]
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                t8 = fmaf(r.p3[z * 9 + a * 3 + d] * r.q1[a], r.q1[d], t8);   // sum P3[z,a,d] Q1 Q1
                gmp3 = fmaf(gm[a * 3 + d], r.p3[a * 9 + d * 3 + z], gmp3);   // sum gM[a,d] P3[a,d,z]
            }
        }
        dp1[z] = g[0] * r.q1[z] + g[3] * m.q2s1[z] + a0 * gv[z] + b1 * gmq;
        dq1[z] = g[0] * r.p1[z] + 2.f * g[7] * qp3s1 + a3 * gvp2 + b1 * gmp;
        ds1[z] = g[3] * p1q2 + g[5] * m.p3q2[z] + g[7] * t8 + a1 * gvq2 + b3 * gmp3;
    }
    // ---- rank 2 (full entries folded into 6 components)
    float dp2[6] = {0, 0, 0, 0, 0, 0}, dq2[6] = {0, 0, 0, 0, 0, 0}, ds2[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int x = 0; x < 3; ++x)
#pragma unroll
        for (int y = 0; y < 3; ++y) {
            float q2s2 = 0.f, s2p2 = 0.f, gmq2 = 0.f, gmp2 = 0.f, p3s1v = 0.f, gvp3 = 0.f, x33 = 0.f;
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                q2s2 = fmaf(r.q2[y * 3 + d], r.s2[d * 3 + x], q2s2);   // (Q2 S2)[y,x]
                s2p2 = fmaf(r.s2[y * 3 + d], r.p2[d * 3 + x], s2p2);   // (S2 P2)[y,x]
                gmq2 = fmaf(gm[x * 3 + d], r.q2[y * 3 + d], gmq2);     // sum_d gM[x,d] Q2[y,d]
                gmp2 = fmaf(gm[d * 3 + y], r.p2[d * 3 + x], gmp2);     // sum_a gM[a,y] P2[a,x]
                p3s1v = fmaf(r.p3[d * 9 + x * 3 + y], r.s1[d], p3s1v);
                gvp3 = fmaf(gv[d], r.p3[d * 9 + x * 3 + y], gvp3);
#pragma unroll
                for (int b = 0; b < 3; ++b) x33 = fmaf(r.p3[d * 9 + b * 3 + x], r.q3[d * 9 + b * 3 + y], x33);
            }
            const int k = sym2(x, y);
            dp2[k] += g[1] * r.q2[x * 3 + y] + g[4] * q2s2 + a3 * gv[x] * r.q1[y] + b0 * gm[x * 3 + y] + b2 * gmq2;
            dq2[k] += g[1] * r.p2[x * 3 + y] + g[3] * r.p1[x] * r.s1[y] + g[4] * s2p2 + g[5] * p3s1v +
                      a1 * gv[x] * r.s1[y] + a2 * gvp3 + b2 * gmp2;
            ds2[k] += g[4] * m.pq2[y * 3 + x] + g[6] * x33;
        }
    // ---- rank 3 (27 entries folded into 10 components)
    float dp3[10], dq3[10];
#pragma unroll
    for (int k = 0; k < 10; ++k) dp3[k] = dq3[k] = 0.f;
#pragma unroll
    for (int x = 0; x < 3; ++x)
#pragma unroll
        for (int y = 0; y < 3; ++y)
#pragma unroll
            for (int z = 0; z < 3; ++z) {
                float q3s2 = 0.f, p3s2 = 0.f;
#pragma unroll
                for (int e = 0; e < 3; ++e) {
                    q3s2 = fmaf(r.q3[x * 9 + y * 3 + e], r.s2[z * 3 + e], q3s2);
                    p3s2 = fmaf(r.p3[x * 9 + y * 3 + e], r.s2[e * 3 + z], p3s2);
                }
                const int k = sym3(x, y, z);
                dp3[k] += g[2] * r.q3[x * 9 + y * 3 + z] + g[5] * r.q2[y * 3 + z] * r.s1[x] + g[6] * q3s2 +
                          g[7] * r.q1[x] * r.s1[y] * r.q1[z] + a2 * gv[x] * r.q2[y * 3 + z] +
                          b3 * gm[x * 3 + y] * r.s1[z];
                dq3[k] += g[2] * r.p3[x * 9 + y * 3 + z] + g[6] * p3s2;
            }
#define ST(T, a, v) (out.p[T][n * out.sn[T] + (int64_t)c * out.sc[T] + (int64_t)(a)*out.sk[T]] = (v))
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        ST(0, a, dp1[a]);
        ST(1, a, dq1[a]);
        ST(2, a, ds1[a]);
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        ST(3, k, dp2[k]);
        ST(4, k, dq2[k]);
        ST(5, k, ds2[k]);
    }
#pragma unroll
    for (int k = 0; k < 10; ++k) {
        ST(6, k, dp3[k]);
        ST(7, k, dq3[k]);
    }
#undef ST
    if (dap) {
        float d0 = 0, d1 = 0, d2 = 0, d3 = 0, e0 = 0, e1 = 0, e2 = 0, e3 = 0;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            d0 = fmaf(gv[a], r.p1[a], d0);
            d1 = fmaf(gv[a], m.q2s1[a], d1);
            d2 = fmaf(gv[a], m.p3q2[a], d2);
            d3 = fmaf(gv[a], m.p2q1[a], d3);
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                const float w = gm[a * 3 + d];
                e0 = fmaf(w, r.p2[a * 3 + d], e0);
                e1 = fmaf(w, r.p1[a] * r.q1[d], e1);
                e2 = fmaf(w, m.pq2[a * 3 + d], e2);
                e3 = fmaf(w, m.p3s1[a * 3 + d], e3);
            }
        }
        dap[0] = d0; dap[1] = d1; dap[2] = d2; dap[3] = d3;
        dbp[0] = e0; dbp[1] = e1; dbp[2] = e2; dbp[3] = e3;
    }
}

__global__ __launch_bounds__(256) void node_fwd_kernel(Strided8 in, const float* __restrict__ av,
                                                       const float* __restrict__ bv, float* __restrict__ inv,
                                                       Str3 si, float* __restrict__ V, Str3 sv,
                                                       float* __restrict__ Mf, Str3 sm, int mf_mode, int64_t N,
                                                       int C, int eq) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= N * C) return;
    const int64_t n = t / C;
    const int c = (int)(t - n * C);
    NodeRegs r;
    load_node(in, n, c, r);
    NodeMid m;
    node_mid(r, m);
    float f[8];
    node_invariants(r, m, f);
    float* o = inv + n * si.sn + (int64_t)c * si.sc;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k * si.sk] = f[k];
    if (!eq) return;
    node_eq_outputs(r, m, av, bv, c, C, V + n * sv.sn + (int64_t)c * sv.sc, sv.sk,
                    Mf + n * sm.sn + (int64_t)c * sm.sc, sm.sk, mf_mode);
}

// Gradients with respect to the FULL tensors are formed entry by entry and folded into the
// symmetric components they were expanded from (sum over the entries of a component).
__global__ __launch_bounds__(256) void node_bwd_kernel(Strided8 in, const float* __restrict__ av,
                                                       const float* __restrict__ bv, const float* __restrict__ gI,
                                                       Str3 sgi, const float* __restrict__ gV, Str3 sgv,
                                                       const float* __restrict__ gM, Str3 sgm, int mf_mode,
                                                       StridedOut8 out, float* __restrict__ da,
                                                       float* __restrict__ db, int64_t N, int C, int eq) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= N * C) return;
    const int64_t n = t / C;
    const int c = (int)(t - n * C);
    NodeRegs r;
    load_node(in, n, c, r);
    NodeMid m;
    node_mid(r, m);
    float g[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) g[k] = gI ? gI[n * sgi.sn + (int64_t)c * sgi.sc + k * sgi.sk] : 0.f;
    float a0 = 0, a1 = 0, a2 = 0, a3 = 0, b0 = 0, b1 = 0, b2 = 0, b3 = 0;
    float gv[3] = {0, 0, 0}, gm[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (eq) {
        a0 = av[c]; a1 = av[C + c]; a2 = av[2 * C + c]; a3 = av[3 * C + c];
        b0 = bv[c]; b1 = bv[C + c]; b2 = bv[2 * C + c]; b3 = bv[3 * C + c];
        if (gV) {
#pragma unroll
            for (int a = 0; a < 3; ++a) gv[a] = gV[n * sgv.sn + (int64_t)c * sgv.sc + a * sgv.sk];
        }
        if (gM) {
            const float* gp = gM + n * sgm.sn + (int64_t)c * sgm.sc;
            if (mf_mode == 0) {
#pragma unroll
                for (int k = 0; k < 9; ++k) gm[k] = gp[k * sgm.sk];
            } else {
#pragma unroll
                for (int a = 0; a < 3; ++a)
#pragma unroll
                    for (int d = 0; d < 3; ++d)
                        gm[a * 3 + d] = (a == d ? 1.f : 0.5f) * gp[sym2(a, d) * sgm.sk];
            }
        }
    }
    node_bwd_core(r, m, g, gv, gm, a0, a1, a2, a3, b0, b1, b2, b3, out, n, c,
                  (eq && da && db) ? da + t * 4 : nullptr, (eq && da && db) ? db + t * 4 : nullptr);
}

// ------------------------------------------------------------------ node algebra + readout LayerNorm
// The readout row x = [P0 | inv_1 .. inv_8] (9C, family-major, face/model.py:244-249) normalised
// by the readout LayerNorm (face/model.py:140, :332) in the kernel that forms it: one workgroup per
// atom, thread = channel (C <= 256; the workgroup is C rounded up to whole waves), each thread
// holding its 9 row entries; the row's mean and biased variance are two workgroup sums (mean
// first, then the centred squares). The row itself is never written: the backward recomputes it
// from the projection outputs, then applies the LayerNorm backward and the node-algebra backward
// to the same registers.
__device__ __forceinline__ float wg_sum(float v, float* sh) {
    v = group_sum(v, kWave);
    __syncthreads();                                   // sh is free again (an earlier sum read it)
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x / kWave); ++i) t += sh[i];
    return t;
}

__global__ __launch_bounds__(256) void node_ln_fwd_kernel(Strided8 in, const float* __restrict__ p0, int64_t p0_sn,
                                                          const float* __restrict__ av, const float* __restrict__ bv,
                                                          const float* __restrict__ lw, const float* __restrict__ lb,
                                                          float eps, float* __restrict__ y, int64_t ld_y,
                                                          float* __restrict__ stats, float* __restrict__ V, Str3 sv,
                                                          float* __restrict__ Mf, Str3 sm, int mf_mode, int C,
                                                          int eq) {
    __shared__ float sh[256 / kWave];
    const int64_t n = blockIdx.x;
    const int c = threadIdx.x;
    const bool act = c < C;
    float x[9];
    NodeRegs r;
    NodeMid m;
    if (act) {
        load_node(in, n, c, r);
        node_mid(r, m);
        float f[8];
        node_invariants(r, m, f);
        x[0] = p0[n * p0_sn + c];
#pragma unroll
        for (int k = 0; k < 8; ++k) x[1 + k] = f[k];
    } else {
#pragma unroll
        for (int k = 0; k < 9; ++k) x[k] = 0.f;
    }
    const float F = 9.f * (float)C;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 9; ++k) s += x[k];
    const float mu = wg_sum(s, sh) / F;
    float ss = 0.f;
    if (act) {
#pragma unroll
        for (int k = 0; k < 9; ++k) ss = fmaf(x[k] - mu, x[k] - mu, ss);
    }
    const float rs = 1.f / sqrtf(wg_sum(ss, sh) / F + eps);
    if (act) {
        float* yr = y + n * ld_y + c;
#pragma unroll
        for (int k = 0; k < 9; ++k) yr[k * C] = (x[k] - mu) * rs * lw[k * C + c] + lb[k * C + c];
        if (eq)
            node_eq_outputs(r, m, av, bv, c, C, V + n * sv.sn + (int64_t)c * sv.sc, sv.sk,
                            Mf + n * sm.sn + (int64_t)c * sm.sc, sm.sk, mf_mode);
    }
    if (c == 0) {
        stats[2 * n] = mu;
        stats[2 * n + 1] = rs;
    }
}

// dx = rstd (g - mean(g) - xh mean(g xh)) with g = dy w, xh = (x - mean) rstd, then dx[0] -> dP0 and
// dx[1..8] as the invariant-family gradients of the node-algebra backward.
__global__ __launch_bounds__(256) void node_ln_bwd_kernel(Strided8 in, const float* __restrict__ p0, int64_t p0_sn,
                                                          const float* __restrict__ av, const float* __restrict__ bv,
                                                          const float* __restrict__ lw, const float* __restrict__ gy,
                                                          int64_t ld_gy, const float* __restrict__ stats,
                                                          const float* __restrict__ gV, Str3 sgv,
                                                          const float* __restrict__ gM, Str3 sgm, int mf_mode,
                                                          StridedOut8 out, float* __restrict__ dp0, int64_t dp0_sn,
                                                          float* __restrict__ da, float* __restrict__ db, int C,
                                                          int eq) {
    __shared__ float sh[256 / kWave];
    const int64_t n = blockIdx.x;
    const int c = threadIdx.x;
    const bool act = c < C;
    const float mu = stats[2 * n], rs = stats[2 * n + 1];
    NodeRegs r;
    NodeMid m;
    float xh[9], g[9];
    float sg = 0.f, sgx = 0.f;
    if (act) {
        load_node(in, n, c, r);
        node_mid(r, m);
        float f[8];
        node_invariants(r, m, f);
        xh[0] = (p0[n * p0_sn + c] - mu) * rs;
#pragma unroll
        for (int k = 0; k < 8; ++k) xh[1 + k] = (f[k] - mu) * rs;
        const float* gr = gy + n * ld_gy + c;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            g[k] = gr[k * C] * lw[k * C + c];
            sg += g[k];
            sgx = fmaf(g[k], xh[k], sgx);
        }
    }
    const float F = 9.f * (float)C;
    const float ag = wg_sum(sg, sh) / F, agx = wg_sum(sgx, sh) / F;
    if (!act) return;                                  // every barrier is behind
    dp0[n * dp0_sn + c] = rs * (g[0] - ag - xh[0] * agx);
    float gi[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) gi[k] = rs * (g[1 + k] - ag - xh[1 + k] * agx);
    float a0 = 0, a1 = 0, a2 = 0, a3 = 0, b0 = 0, b1 = 0, b2 = 0, b3 = 0;
    float gv[3] = {0, 0, 0}, gm[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    if (eq) {
        a0 = av[c]; a1 = av[C + c]; a2 = av[2 * C + c]; a3 = av[3 * C + c];
        b0 = bv[c]; b1 = bv[C + c]; b2 = bv[2 * C + c]; b3 = bv[3 * C + c];
        if (gV) {
#pragma unroll
            for (int a = 0; a < 3; ++a) gv[a] = gV[n * sgv.sn + (int64_t)c * sgv.sc + a * sgv.sk];
        }
        if (gM) {
            const float* gp = gM + n * sgm.sn + (int64_t)c * sgm.sc;
            if (mf_mode == 0) {
#pragma unroll
                for (int k = 0; k < 9; ++k) gm[k] = gp[k * sgm.sk];
            } else {
#pragma unroll
                for (int a = 0; a < 3; ++a)
#pragma unroll
                    for (int d = 0; d < 3; ++d)
                        gm[a * 3 + d] = (a == d ? 1.f : 0.5f) * gp[sym2(a, d) * sgm.sk];
            }
        }
    }
    const int64_t t = n * C + c;
    node_bwd_core(r, m, gi, gv, gm, a0, a1, a2, a3, b0, b1, b2, b3, out, n, c,
                  (eq && da && db) ? da + t * 4 : nullptr, (eq && da && db) ? db + t * 4 : nullptr);
}

static bool fill_in(const float* const* ins, const int64_t* st, Strided8& s) {
    for (int k = 0; k < 8; ++k) {
        if (!ins[k]) return false;
        s.p[k] = ins[k];
        s.sn[k] = st[3 * k];
        s.sc[k] = st[3 * k + 1];
        s.sk[k] = st[3 * k + 2];
    }
    return true;
}

}  // namespace face

using namespace face;

extern "C" int face_node_fwd(const float* const* ins, const int64_t* in_strides, const float* a, const float* b,
                             float* inv, const int64_t* inv_strides, float* V, const int64_t* V_strides, float* Mf,
                             const int64_t* Mf_strides, int32_t mf_mode, int64_t N, int32_t C, int32_t eq,
                             void* stream) {
    if (N < 0 || C <= 0 || !ins || !in_strides || !inv || !inv_strides) return FACE_ERR_ARG;
    if (eq && (!a || !b || !V || !V_strides || !Mf || !Mf_strides || (mf_mode != 0 && mf_mode != 1)))
        return FACE_ERR_ARG;
    if (N == 0) return 0;
    Strided8 s;
    if (!fill_in(ins, in_strides, s)) return FACE_ERR_ARG;
    Str3 si{inv_strides[0], inv_strides[1], inv_strides[2]};
    Str3 sv{0, 0, 0}, sm{0, 0, 0};
    if (eq) {
        sv = Str3{V_strides[0], V_strides[1], V_strides[2]};
        sm = Str3{Mf_strides[0], Mf_strides[1], Mf_strides[2]};
    }
    const int64_t total = N * (int64_t)C;
    hipLaunchKernelGGL(node_fwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, s,
                       a, b, inv, si, V, sv, Mf, sm, mf_mode, N, C, eq);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_node_bwd(const float* const* ins, const int64_t* in_strides, const float* a, const float* b,
                             const float* gI, const int64_t* gI_strides, const float* gV, const int64_t* gV_strides,
                             const float* gM, const int64_t* gM_strides, int32_t mf_mode, float* const* outs,
                             const int64_t* out_strides, float* da, float* db, int64_t N, int32_t C, int32_t eq,
                             void* stream) {
    if (N < 0 || C <= 0 || !ins || !in_strides || !outs || !out_strides) return FACE_ERR_ARG;
    if (eq && (!a || !b || (mf_mode != 0 && mf_mode != 1))) return FACE_ERR_ARG;
    if ((gI && !gI_strides) || (gV && !gV_strides) || (gM && !gM_strides)) return FACE_ERR_ARG;
    if (N == 0) return 0;
    Strided8 s;
    if (!fill_in(ins, in_strides, s)) return FACE_ERR_ARG;
    StridedOut8 o;
    for (int k = 0; k < 8; ++k) {
        if (!outs[k]) return FACE_ERR_ARG;
        o.p[k] = outs[k];
        o.sn[k] = out_strides[3 * k];
        o.sc[k] = out_strides[3 * k + 1];
        o.sk[k] = out_strides[3 * k + 2];
    }
    Str3 sgi{0, 0, 0}, sgv{0, 0, 0}, sgm{0, 0, 0};
    if (gI) sgi = Str3{gI_strides[0], gI_strides[1], gI_strides[2]};
    if (gV) sgv = Str3{gV_strides[0], gV_strides[1], gV_strides[2]};
    if (gM) sgm = Str3{gM_strides[0], gM_strides[1], gM_strides[2]};
    const int64_t total = N * (int64_t)C;
    hipLaunchKernelGGL(node_bwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, s,
                       a, b, gI, sgi, gV, sgv, gM, sgm, mf_mode, o, da, db, N, C, eq);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_node_ln_fwd(const float* const* ins, const int64_t* in_strides, const float* p0, int64_t p0_sn,
                                const float* a, const float* b, const float* ln_w, const float* ln_b, float eps,
                                float* y, int64_t ld_y, float* stats, float* V, const int64_t* V_strides, float* Mf,
                                const int64_t* Mf_strides, int32_t mf_mode, int64_t N, int32_t C, int32_t eq,
                                void* stream) {
    if (N < 0 || C <= 0 || C > 256 || !ins || !in_strides || !p0 || p0_sn < C || !ln_w || !ln_b || !y ||
        ld_y < 9 * (int64_t)C || !stats)
        return FACE_ERR_ARG;
    if (eq && (!a || !b || !V || !V_strides || !Mf || !Mf_strides || (mf_mode != 0 && mf_mode != 1)))
        return FACE_ERR_ARG;
    if (N == 0) return 0;
    Strided8 s;
    if (!fill_in(ins, in_strides, s)) return FACE_ERR_ARG;
    Str3 sv{0, 0, 0}, sm{0, 0, 0};
    if (eq) {
        sv = Str3{V_strides[0], V_strides[1], V_strides[2]};
        sm = Str3{Mf_strides[0], Mf_strides[1], Mf_strides[2]};
    }
    const int block = (C + kWave - 1) / kWave * kWave;
    hipLaunchKernelGGL(node_ln_fwd_kernel, dim3((unsigned)N), dim3(block), 0, (hipStream_t)stream, s, p0, p0_sn, a,
                       b, ln_w, ln_b, eps, y, ld_y, stats, V, sv, Mf, sm, mf_mode, C, eq);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_node_ln_bwd(const float* const* ins, const int64_t* in_strides, const float* p0, int64_t p0_sn,
                                const float* a, const float* b, const float* ln_w, const float* gy, int64_t ld_gy,
                                const float* stats, const float* gV, const int64_t* gV_strides, const float* gM,
                                const int64_t* gM_strides, int32_t mf_mode, float* const* outs,
                                const int64_t* out_strides, float* dp0, int64_t dp0_sn, float* da, float* db,
                                int64_t N, int32_t C, int32_t eq, void* stream) {
    if (N < 0 || C <= 0 || C > 256 || !ins || !in_strides || !p0 || p0_sn < C || !ln_w || !gy ||
        ld_gy < 9 * (int64_t)C || !stats || !outs || !out_strides || !dp0 || dp0_sn < C)
        return FACE_ERR_ARG;
    if (eq && (!a || !b || (mf_mode != 0 && mf_mode != 1))) return FACE_ERR_ARG;
    if ((gV && !gV_strides) || (gM && !gM_strides)) return FACE_ERR_ARG;
    if (N == 0) return 0;
    Strided8 s;
    if (!fill_in(ins, in_strides, s)) return FACE_ERR_ARG;
    StridedOut8 o;
    for (int k = 0; k < 8; ++k) {
        if (!outs[k]) return FACE_ERR_ARG;
        o.p[k] = outs[k];
        o.sn[k] = out_strides[3 * k];
        o.sc[k] = out_strides[3 * k + 1];
        o.sk[k] = out_strides[3 * k + 2];
    }
    Str3 sgv{0, 0, 0}, sgm{0, 0, 0};
    if (gV) sgv = Str3{gV_strides[0], gV_strides[1], gV_strides[2]};
    if (gM) sgm = Str3{gM_strides[0], gM_strides[1], gM_strides[2]};
    const int block = (C + kWave - 1) / kWave * kWave;
    hipLaunchKernelGGL(node_ln_bwd_kernel, dim3((unsigned)N), dim3(block), 0, (hipStream_t)stream, s, p0, p0_sn, a,
                       b, ln_w, gy, ld_gy, stats, gV, sgv, gM, sgm, mf_mode, o, dp0, dp0_sn, da, db, C, eq);
    FACE_LAUNCH_CHECK();
    return 0;
}

namespace face {

// ------------------------------------------------------------------ gated equivariant outputs
// Vo[a, n, c] = V[a, n, c] gv[n, c], Mo[k, n, c] = Ms[k, n, c] gm[n, c] with gvm = [gv | gm]
// (N, 2C) the gate row (face/model.py:286-296); V (3, N, C), Ms (6, N, C) contiguous. Thread =
// (atom, channel quad), float4 throughout (C % 4 == 0, 16-byte aligned arrays).
__global__ __launch_bounds__(256) void eq_gate_fwd_kernel(const float* __restrict__ V, const float* __restrict__ Ms,
                                                          const float* __restrict__ gvm, int64_t N, int C,
                                                          float* __restrict__ Vo, float* __restrict__ Mo) {
    const int C4 = C / 4;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= N * C4) return;
    const int64_t n = t / C4;
    const int c = 4 * (int)(t - n * C4);
    const int64_t NC = N * C, o = n * C + c;
    const v4f gv = ld4(gvm + n * 2 * C + c), gm = ld4(gvm + n * 2 * C + C + c);
#pragma unroll
    for (int a = 0; a < 3; ++a) st4(Vo + a * NC + o, ld4(V + a * NC + o) * gv);
#pragma unroll
    for (int k = 0; k < 6; ++k) st4(Mo + k * NC + o, ld4(Ms + k * NC + o) * gm);
}

// Backward: dV = gVo gv, dMs = gMo gm, dgv = sum_a gVo[a] V[a], dgm = sum_k gMo[k] Ms[k].
__global__ __launch_bounds__(256) void eq_gate_bwd_kernel(const float* __restrict__ V, const float* __restrict__ Ms,
                                                          const float* __restrict__ gvm, const float* __restrict__ gVo,
                                                          const float* __restrict__ gMo, int64_t N, int C,
                                                          float* __restrict__ dV, float* __restrict__ dMs,
                                                          float* __restrict__ dgvm) {
    const int C4 = C / 4;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= N * C4) return;
    const int64_t n = t / C4;
    const int c = 4 * (int)(t - n * C4);
    const int64_t NC = N * C, o = n * C + c;
    const v4f gv = ld4(gvm + n * 2 * C + c), gm = ld4(gvm + n * 2 * C + C + c);
    v4f sv = {0.f, 0.f, 0.f, 0.f}, sm = sv;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const v4f g = ld4(gVo + a * NC + o);
        sv += g * ld4(V + a * NC + o);
        st4(dV + a * NC + o, g * gv);
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const v4f g = ld4(gMo + k * NC + o);
        sm += g * ld4(Ms + k * NC + o);
        st4(dMs + k * NC + o, g * gm);
    }
    st4(dgvm + n * 2 * C + c, sv);
    st4(dgvm + n * 2 * C + C + c, sm);
}

static bool eq_gate_ok(int64_t N, int C, std::initializer_list<const void*> ps) {
    if (N < 0 || C <= 0) return false;
    for (const void* p : ps)
        if (!p) return false;
    return true;
}
static bool vec4_ok(int C, std::initializer_list<const void*> ps) {
    if (C % 4) return false;
    for (const void* p : ps)
        if ((uintptr_t)p & 15) return false;
    return true;
}

}  // namespace face

extern "C" int face_eq_gate_fwd(const float* V, const float* Ms, const float* gvm, int64_t N, int32_t C, float* Vo,
                                float* Mo, void* stream) {
    if (!eq_gate_ok(N, C, {V, Ms, gvm, Vo, Mo})) return FACE_ERR_ARG;
    if (!vec4_ok(C, {V, Ms, gvm, Vo, Mo})) return FACE_ERR_UNSUPPORTED;
    if (N == 0) return 0;
    const int64_t total = N * (C / 4);
    hipLaunchKernelGGL(eq_gate_fwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       V, Ms, gvm, N, C, Vo, Mo);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_eq_gate_bwd(const float* V, const float* Ms, const float* gvm, const float* gVo,
                                const float* gMo, int64_t N, int32_t C, float* dV, float* dMs, float* dgvm,
                                void* stream) {
    if (!eq_gate_ok(N, C, {V, Ms, gvm, gVo, gMo, dV, dMs, dgvm})) return FACE_ERR_ARG;
    if (!vec4_ok(C, {V, Ms, gvm, gVo, gMo, dV, dMs, dgvm})) return FACE_ERR_UNSUPPORTED;
    if (N == 0) return 0;
    const int64_t total = N * (C / 4);
    hipLaunchKernelGGL(eq_gate_bwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       V, Ms, gvm, gVo, gMo, N, C, dV, dMs, dgvm);
    FACE_LAUNCH_CHECK();
    return 0;
}

namespace face {

// ------------------------------------------------------------------ readout LayerNorm
// y = (x - mean) rstd w + b over rows of F features (face/model.py:140, :332: nn.LayerNorm of the
// invariant row, biased variance, rstd = 1 / sqrt(var + eps)). One wave per row, the row held in
// registers as float4 (F % 4 == 0, F <= 2048); mean and rstd are kept for the backward.
constexpr int kLnMaxU = 8;                            // float4 per lane: F <= 64 * 4 * 8

template <int U>
__global__ __launch_bounds__(256) void layer_norm_fwd_kernel(const float* __restrict__ x, int64_t N, int F,
                                                             const float* __restrict__ w, const float* __restrict__ b,
                                                             float eps, float* __restrict__ y,
                                                             float* __restrict__ mean, float* __restrict__ rstd) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t n = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
    if (n >= N) return;
    const int F4 = F / 4;
    const float* xr = x + n * F;
    v4f v[U];
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c4 = lane + kWave * u;
        v[u] = c4 < F4 ? ld4(xr + 4 * c4) : (v4f){0.f, 0.f, 0.f, 0.f};
        s += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
    }
    const float mu = group_sum(s, kWave) / (float)F;
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c4 = lane + kWave * u;
        if (c4 < F4) {
            const v4f d = v[u] - mu;
            ss += (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]);
        }
    }
    const float rs = 1.f / sqrtf(group_sum(ss, kWave) / (float)F + eps);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c4 = lane + kWave * u;
        if (c4 < F4) st4(y + n * F + 4 * c4, (v[u] - mu) * rs * ld4(w + 4 * c4) + ld4(b + 4 * c4));
    }
    if (lane == 0) {
        mean[n] = mu;
        rstd[n] = rs;
    }
}

// dx = rstd (g - mean(g) - xh mean(g xh)), g = dy w, xh = (x - mean) rstd (no weight gradients).
template <int U>
__global__ __launch_bounds__(256) void layer_norm_bwd_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ dy, int64_t N, int F,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ mean,
                                                             const float* __restrict__ rstd, float* __restrict__ dx) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t n = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
    if (n >= N) return;
    const int F4 = F / 4;
    const float mu = mean[n], rs = rstd[n];
    v4f g[U], xh[U];
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c4 = lane + kWave * u;
        const v4f z = {0.f, 0.f, 0.f, 0.f};
        g[u] = c4 < F4 ? ld4(dy + n * F + 4 * c4) * ld4(w + 4 * c4) : z;
        xh[u] = c4 < F4 ? (ld4(x + n * F + 4 * c4) - mu) * rs : z;
        sg += (g[u][0] + g[u][1]) + (g[u][2] + g[u][3]);
        const v4f p = g[u] * xh[u];
        sgx += (p[0] + p[1]) + (p[2] + p[3]);
    }
    const float a = group_sum(sg, kWave) / (float)F, c = group_sum(sgx, kWave) / (float)F;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c4 = lane + kWave * u;
        if (c4 < F4) st4(dx + n * F + 4 * c4, rs * (g[u] - a - xh[u] * c));
    }
}

static int ln_units(int F) { return (F / 4 + kWave - 1) / kWave; }

}  // namespace face

extern "C" int face_layer_norm_fwd(const float* x, int64_t N, int32_t F, const float* w, const float* b, float eps,
                                   float* y, float* mean, float* rstd, void* stream) {
    if (N < 0 || F <= 0 || !x || !w || !b || !y || !mean || !rstd) return FACE_ERR_ARG;
    if (F % 4 || ln_units(F) > kLnMaxU || !vec4_ok(F, {x, w, b, y})) return FACE_ERR_UNSUPPORTED;
    if (N == 0) return 0;
    const dim3 grid((unsigned)((N + 3) / 4)), block(256);
    const hipStream_t st = (hipStream_t)stream;
    switch (ln_units(F)) {
#define FACE_LNF(U_) \
    case U_: hipLaunchKernelGGL(layer_norm_fwd_kernel<U_>, grid, block, 0, st, x, N, F, w, b, eps, y, mean, rstd); break
        FACE_LNF(1); FACE_LNF(2); FACE_LNF(3); FACE_LNF(4); FACE_LNF(5); FACE_LNF(6); FACE_LNF(7); FACE_LNF(8);
#undef FACE_LNF
        default: return FACE_ERR_UNSUPPORTED;
    }
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_layer_norm_bwd(const float* x, const float* dy, int64_t N, int32_t F, const float* w,
                                   const float* mean, const float* rstd, float* dx, void* stream) {
    if (N < 0 || F <= 0 || !x || !dy || !w || !mean || !rstd || !dx) return FACE_ERR_ARG;
    if (F % 4 || ln_units(F) > kLnMaxU || !vec4_ok(F, {x, dy, w, dx})) return FACE_ERR_UNSUPPORTED;
    if (N == 0) return 0;
    const dim3 grid((unsigned)((N + 3) / 4)), block(256);
    const hipStream_t st = (hipStream_t)stream;
    switch (ln_units(F)) {
#define FACE_LNB(U_) \
    case U_: hipLaunchKernelGGL(layer_norm_bwd_kernel<U_>, grid, block, 0, st, x, dy, N, F, w, mean, rstd, dx); break
        FACE_LNB(1); FACE_LNB(2); FACE_LNB(3); FACE_LNB(4); FACE_LNB(5); FACE_LNB(6); FACE_LNB(7); FACE_LNB(8);
#undef FACE_LNB
        default: return FACE_ERR_UNSUPPORTED;
    }
    FACE_LAUNCH_CHECK();
    return 0;
}
