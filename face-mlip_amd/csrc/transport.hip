// Transport moments of FACE's directional passes (gfx950), face/model.py:514-533.
//
// For receiver i and radial channel b, with the neighbour's transport tables V_j (3) and
// M_j (6, sym storage) of channel kd and the bond direction u:
//   D[i, b, kd, :] = scale * sum_{e in row i} phi[e, b] F(u_e, V_j[kd], M_j[kd])
//   F = [V (3) | M u (3) | M (6) | sym(u (x) V) (6)]                      (18 features)
// which equals the reference's monomial sums [1, u] (x) phi (x) [V | M] followed by its (36,18)
// transport map (face/model.py:342-362, :515-526), formed here per edge so only 18 of the 36
// columns are accumulated. The outputs are written straight in the layout the channel mixers
// read: D1 (3, N, B*2*Kd) = [V | M u], D2 (6, N, B*2*Kd) = [M | sym(u V)], channel
// b*2*Kd + t*Kd + kd (t = first or second half), face/model.py:527-528.
//
// Tables: V element (component a, atom n, channel kd) at V[a*v_sq + n*v_sn + kd], M likewise.
#include "common.h"

namespace face {

constexpr int kTT = 16;   // edges per LDS tile
constexpr int kFP = 20;   // 18 features padded to a float4 multiple

__device__ __forceinline__ int s2(int a, int b) { return a == b ? a : (a + b == 1 ? 3 : (a + b == 2 ? 4 : 5)); }

__device__ __forceinline__ void transport_features(const float* u, const float* V, const float* M, float* F) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        F[a] = V[a];
        float mu = 0.f;
#pragma unroll
        for (int c = 0; c < 3; ++c) mu = fmaf(M[s2(a, c)], u[c], mu);
        F[3 + a] = mu;
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) F[6 + k] = M[k];
    F[12] = u[0] * V[0];
    F[13] = u[1] * V[1];
    F[14] = u[2] * V[2];
    F[15] = 0.5f * (u[0] * V[1] + u[1] * V[0]);
    F[16] = 0.5f * (u[0] * V[2] + u[2] * V[0]);
    F[17] = 0.5f * (u[1] * V[2] + u[2] * V[1]);
}

struct Tables {
    const float* V;
    const float* M;
    int64_t v_sn, v_sq, m_sn, m_sq;
};

__device__ __forceinline__ void load_tables(const Tables& T, int64_t n, int kd, float* V, float* M) {
#pragma unroll
    for (int a = 0; a < 3; ++a) V[a] = T.V[a * T.v_sq + n * T.v_sn + kd];
#pragma unroll
    for (int k = 0; k < 6; ++k) M[k] = T.M[k * T.m_sq + n * T.m_sn + kd];
}

// Workgroup = atom i; thread = (b, kd) with kd fastest, 18 accumulators. Per edge tile the
// features F[t, kd, :] are formed once in LDS and broadcast over the B radial channels.
__global__ __launch_bounds__(1024) void transport_fwd_kernel(const float* __restrict__ phi, int ld_phi, int B,
                                                              Tables T, int Kd, const float* __restrict__ Y, int ld_Y,
                                                              const int32_t* __restrict__ col,
                                                              const int32_t* __restrict__ row_ptr, int64_t N,
                                                              float scale, float* __restrict__ D1,
                                                              float* __restrict__ D2) {
    extern __shared__ float lds[];
    float* s_F = lds;                       // kTT * Kd * kFP
    float* s_phi = s_F + kTT * Kd * kFP;    // kTT * B
    const int64_t i = blockIdx.x;
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int kd = tid % Kd, b = tid / Kd;
    const bool ok = b < B;
    float acc[18];
#pragma unroll
    for (int o = 0; o < 18; ++o) acc[o] = 0.f;
    const int64_t e0 = row_ptr[i], e1 = row_ptr[i + 1];
    for (int64_t t0 = e0; t0 < e1; t0 += kTT) {
        const int nt = (int)min((int64_t)kTT, e1 - t0);
        for (int q = tid; q < nt * Kd; q += nthr) {
            const int t = q / Kd, k = q - t * Kd;
            const int64_t e = t0 + t;
            const float* y = Y + e * ld_Y;
            const float u[3] = {y[1], y[2], y[3]};
            float V[3], M[6], F[18];
            load_tables(T, col[e], k, V, M);
            transport_features(u, V, M, F);
            float* dst = s_F + (t * Kd + k) * kFP;
#pragma unroll
            for (int o = 0; o < 18; ++o) dst[o] = F[o];
        }
        for (int q = tid; q < nt * B; q += nthr) {
            const int t = q / B;
            s_phi[q] = phi[(t0 + t) * ld_phi + (q - t * B)];
        }
        __syncthreads();
        if (ok) {
            for (int t = 0; t < nt; ++t) {
                const float p = s_phi[t * B + b];
                const float4* f = reinterpret_cast<const float4*>(s_F + (t * Kd + kd) * kFP);
#pragma unroll
                for (int o4 = 0; o4 < 5; ++o4) {
                    const float4 v = f[o4];
                    acc[o4 * 4 + 0] = fmaf(p, v.x, acc[o4 * 4 + 0]);
                    acc[o4 * 4 + 1] = fmaf(p, v.y, acc[o4 * 4 + 1]);
                    if (o4 < 4) {
                        acc[o4 * 4 + 2] = fmaf(p, v.z, acc[o4 * 4 + 2]);
                        acc[o4 * 4 + 3] = fmaf(p, v.w, acc[o4 * 4 + 3]);
                    }
                }
            }
        }
        __syncthreads();
    }
    if (!ok) return;
    const int64_t W = (int64_t)B * 2 * Kd;
    const int64_t ch0 = (int64_t)b * 2 * Kd + kd;          // first half (t = 0)
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        D1[(a * N + i) * W + ch0] = scale * acc[a];
        D1[(a * N + i) * W + ch0 + Kd] = scale * acc[3 + a];
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        D2[(k * N + i) * W + ch0] = scale * acc[6 + k];
        D2[(k * N + i) * W + ch0 + Kd] = scale * acc[12 + k];
    }
}

// Matrix-core forward for B == 16, Kd == 16 (the flagship widths): per atom the sums are the
// product D_o[b][kd] = sum_e phi[e][b] F_o[e][kd] with the row's edges as K. One wave per atom
// row; per step of 4 edges (edge e0 + 4s + q in K slot q), lane (j, q) forms the 18 features of
// its edge at channel kd = j from u and the neighbour's table row, and each feature o is one
// v_mfma_f32_16x16x4f32 with A = phi^T (lane (j, q): phi[e][b = j]) and B = F_o (lane (j, q):
// F_o[e][kd = j]); tile o holds b = 4q + r of channel j in register r of lane (j, q). Edges past
// the row carry phi = 0. The next step's operands are loaded while the current one multiplies,
// and the neighbour indices one step earlier still, so no gather waits on its index.
constexpr int kTfWaves = 4;

__global__ __launch_bounds__(kTfWaves * kWave) void transport_fwd_mfma_kernel(
    const float* __restrict__ phi, int ld_phi, Tables T, const float* __restrict__ Y, int ld_Y,
    const int32_t* __restrict__ col, const int32_t* __restrict__ row_ptr, int64_t N, float scale,
    float* __restrict__ D1, float* __restrict__ D2) {
    constexpr int Kd = 16, B = 16, W = 2 * B * Kd;
    const int lane = threadIdx.x & (kWave - 1);
    const int j = lane & 15, q = lane >> 4;
    const int64_t i = (int64_t)blockIdx.x * kTfWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (i >= N) return;
    const int64_t e0 = row_ptr[i], e1 = row_ptr[i + 1];
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    v4f acc[18];
#pragma unroll
    for (int o = 0; o < 18; ++o) acc[o] = z4;
    if (e1 > e0) {
        const int64_t ns = (e1 - e0 + 3) / 4;
        auto edge = [&](int64_t s) { return min(e0 + 4 * s + q, e1 - 1); };
        struct Op {
            float p, u[3], V[3], M[6];
        };
        auto load = [&](int64_t s, int32_t c, Op& o) __attribute__((always_inline)) {
            const int64_t e = e0 + 4 * s + q;
            const int64_t ec = min(e, e1 - 1);
            o.p = e < e1 ? phi[ec * ld_phi + j] : 0.f;
            const float* y = Y + ec * ld_Y;
            o.u[0] = y[1];
            o.u[1] = y[2];
            o.u[2] = y[3];
            load_tables(T, c, j, o.V, o.M);
        };
        Op cur, nxt;
        int32_t cn = col[edge(ns > 1 ? 1 : 0)];          // neighbour of step 1
        load(0, col[edge(0)], cur);
        for (int64_t s = 0; s < ns; ++s) {
            const int32_t cnn = col[edge(s + 2 < ns ? s + 2 : s)];
            if (s + 1 < ns) load(s + 1, cn, nxt);
            float F[18];
            transport_features(cur.u, cur.V, cur.M, F);
#pragma unroll
            for (int o = 0; o < 18; ++o) acc[o] = mfma_16x16x4(cur.p, F[o], acc[o]);
            cur = nxt;
            cn = cnn;
        }
    }
    // feature o -> (table, component, half): D1 = [V | M u], D2 = [M | sym(u V)]
#pragma unroll
    for (int o = 0; o < 18; ++o) {
        float* const base = o < 6 ? D1 : D2;
        const int comp = o < 6 ? o % 3 : (o - 6) % 6;
        const int half = o < 6 ? o / 3 : (o - 6) / 6;
        float* const dst = base + (comp * N + i) * W + half * Kd + j;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[(4 * q + r) * 2 * Kd] = scale * acc[o][r];
    }
}

// Workgroup = atom i; gD (B x Kd x 18, scaled) staged in LDS. Lane = (edge slot, kd), KP lanes
// per edge (Kd rounded up to a power of two). Per edge and channel kd:
//   dphi[b] = sum_{kd,o} gD[b,kd,o] F[kd,o]   (summed over the KP lanes)
//   dF[o]   = sum_b phi[b] gD[b,kd,o]         -> dV, dM (per-edge table gradient), du (summed)
__global__ __launch_bounds__(256) void transport_bwd_kernel(const float* __restrict__ phi, int ld_phi, int B,
                                                             Tables T, int Kd, int KP,
                                                             const float* __restrict__ Y, int ld_Y,
                                                             const int32_t* __restrict__ col,
                                                             const int32_t* __restrict__ row_ptr, int64_t N,
                                                             float scale, const float* __restrict__ gD1,
                                                             const float* __restrict__ gD2,
                                                             float* __restrict__ dphi, int ld_dphi,
                                                             float* __restrict__ dT_edge, float* __restrict__ gY) {
    extern __shared__ float lds[];
    float* s_g = lds;                        // B * Kd * kFP
    const int64_t i = blockIdx.x;
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int64_t W = (int64_t)B * 2 * Kd;
    // (channel fastest: each wave reads contiguous runs of the nine upstream component rows)
    for (int q = tid; q < B * Kd * kFP; q += nthr) {
        const int r = q % (B * Kd), o = q / (B * Kd);
        const int k = r % Kd, bb = r / Kd;
        const int64_t ch0 = (int64_t)bb * 2 * Kd + k;
        float v = 0.f;
        if (o < 3) v = gD1[(o * N + i) * W + ch0];
        else if (o < 6) v = gD1[((o - 3) * N + i) * W + ch0 + Kd];
        else if (o < 12) v = gD2[((o - 6) * N + i) * W + ch0];
        else if (o < 18) v = gD2[((o - 12) * N + i) * W + ch0 + Kd];
        s_g[r * kFP + o] = scale * v;
    }
    __syncthreads();
    const int kd = tid & (KP - 1);
    const int slot = tid / KP;
    const int nslots = nthr / KP;
    const int64_t e0 = row_ptr[i], e1 = row_ptr[i + 1];
    for (int64_t base = e0; base < e1; base += nslots) {   // same trip count for every lane
        const int64_t e = base + slot;
        const bool valid = e < e1 && kd < Kd;
        float u[3] = {0.f, 0.f, 0.f}, V[3] = {0.f, 0.f, 0.f}, M[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, F[18];
        if (valid) {
            const float* y = Y + e * ld_Y;
            u[0] = y[1]; u[1] = y[2]; u[2] = y[3];
            load_tables(T, col[e], kd, V, M);
        }
        transport_features(u, V, M, F);
        float dF[18];
#pragma unroll
        for (int o = 0; o < 18; ++o) dF[o] = 0.f;
        for (int bb = 0; bb < B; ++bb) {                 // same trip count for every lane
            const float p = valid ? phi[e * ld_phi + bb] : 0.f;
            const float4* g = reinterpret_cast<const float4*>(s_g + (bb * Kd + (valid ? kd : 0)) * kFP);
            float s = 0.f;
#pragma unroll
            for (int o4 = 0; o4 < 5; ++o4) {
                const float4 v = g[o4];
                const float gv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int o = o4 * 4 + j;
                    if (o < 18) {
                        s = fmaf(gv[j], F[o], s);
                        dF[o] = fmaf(p, gv[j], dF[o]);
                    }
                }
            }
            // dphi[b]: sum over the KP lanes of this edge, written by one of them
            const float v = group_sum(valid ? s : 0.f, KP);
            if (dphi && e < e1 && kd == (bb & (KP - 1))) dphi[e * ld_dphi + bb] = v;
        }
        // table and direction gradients from dF
        float dV[3] = {dF[0], dF[1], dF[2]}, dM[6], du[3] = {0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 6; ++k) dM[k] = dF[6 + k];
#pragma unroll
        for (int a = 0; a < 3; ++a)
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                dM[s2(a, c)] = fmaf(u[c], dF[3 + a], dM[s2(a, c)]);
                du[c] = fmaf(M[s2(a, c)], dF[3 + a], du[c]);
            }
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            du[a] = fmaf(V[a], dF[12 + a], du[a]);
            dV[a] = fmaf(u[a], dF[12 + a], dV[a]);
        }
        {
            const int pa[3] = {0, 0, 1}, pb[3] = {1, 2, 2};
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                const float h = 0.5f * dF[15 + k];
                const int a = pa[k], c = pb[k];
                du[a] = fmaf(V[c], h, du[a]);
                du[c] = fmaf(V[a], h, du[c]);
                dV[c] = fmaf(u[a], h, dV[c]);
                dV[a] = fmaf(u[c], h, dV[a]);
            }
        }
        if (valid && dT_edge) {
            float* o = dT_edge + e * 9 * Kd + kd;
#pragma unroll
            for (int a = 0; a < 3; ++a) o[a * Kd] = dV[a];
#pragma unroll
            for (int k = 0; k < 6; ++k) o[(3 + k) * Kd] = dM[k];
        }
#pragma unroll
        for (int a = 0; a < 3; ++a) du[a] = group_sum(valid ? du[a] : 0.f, KP);
        if (e < e1 && kd == 0 && gY) {
            float* gy = gY + e * 20;
            gy[1] += du[0];
            gy[2] += du[1];
            gy[3] += du[2];
        }
    }
}

// Matrix-core backward for B == 16, Kd == 16 (the flagship widths). One wave per atom row;
// the row's upstream gradient G[o][b][kd] = scale * gD (18 x 16 x 16) sits in the wave's LDS
// slice. Per tile of 16 edges, lane (j, q) owns edge j and channels kd = 4q + r (r = 0..3):
//   dphi[b, e]   = sum_{o, kd} G[o][b][kd] F[e][kd][o]   M = b, N = e, K = kd (one o per chain step)
//   dF[o][kd, e] = sum_b G[o][b][kd] phi[e][b]          M = kd, N = e, K = b
// With v_mfma_f32_16x16x4f32 (A[i][k] in lane i + 16k, B[k][n] in lane n + 16k, D[4q + r][n] in
// register r of lane n + 16q) the F operand of lane (j, q) for K index q is its own channel
// 4q + kc, and the dF block of o lands in register r = kd - 4q of lane (j, q): every lane ends
// with all 18 dF[o] of its 4 channels and forms the table and direction gradients locally.
__global__ __launch_bounds__(2 * kWave) void transport_bwd_mfma_kernel(
    const float* __restrict__ phi, int ld_phi, Tables T, const float* __restrict__ Y, int ld_Y,
    const int32_t* __restrict__ col, const int32_t* __restrict__ row_ptr, int64_t N, float scale,
    const float* __restrict__ gD1, const float* __restrict__ gD2, float* __restrict__ dphi, int ld_dphi,
    float* __restrict__ dT_edge, float* __restrict__ gY) {
    constexpr int Kd = 16, B = 16, W = 2 * B * Kd;
    extern __shared__ float lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int w = threadIdx.x / kWave;
    const int64_t i = (int64_t)blockIdx.x * 2 + w;
    if (i >= N) return;                               // uniform per wave
    float* sG = lds + (size_t)w * 18 * B * Kd;
    // channel (b, kd) fastest: contiguous reads; all 18 component rows of a lane in flight at once
    for (int c0 = 0; c0 < B * Kd; c0 += kWave) {
        const int r = c0 + lane;
        const int kd = r % Kd, b = r / Kd;
        const int64_t ch = (int64_t)b * 2 * Kd + kd;
        float g[18];
#pragma unroll
        for (int o = 0; o < 18; ++o) {
            if (o < 3) g[o] = gD1[(o * N + i) * W + ch];
            else if (o < 6) g[o] = gD1[((o - 3) * N + i) * W + ch + Kd];
            else if (o < 12) g[o] = gD2[((o - 6) * N + i) * W + ch];
            else g[o] = gD2[((o - 12) * N + i) * W + ch + Kd];
        }
#pragma unroll
        for (int o = 0; o < 18; ++o) sG[o * B * Kd + r] = scale * g[o];
    }
    __builtin_amdgcn_wave_barrier();
    const int j = lane & 15, q = lane >> 4;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    const int64_t e0 = row_ptr[i], e1 = row_ptr[i + 1];
    for (int64_t t0 = e0; t0 < e1; t0 += 16) {
        const int64_t e = t0 + j;
        const bool ok = e < e1;
        float u[3] = {0.f, 0.f, 0.f}, ph[4] = {0.f, 0.f, 0.f, 0.f};
        v4f V[3], Mt[6];
        if (ok) {
            const float* y = Y + e * ld_Y;
            u[0] = y[1]; u[1] = y[2]; u[2] = y[3];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) ph[kb] = phi[e * ld_phi + 4 * kb + q];
            const int64_t n = col[e];
#pragma unroll
            for (int a = 0; a < 3; ++a) V[a] = ld4(T.V + a * T.v_sq + n * T.v_sn + 4 * q);
#pragma unroll
            for (int k = 0; k < 6; ++k) Mt[k] = ld4(T.M + k * T.m_sq + n * T.m_sn + 4 * q);
        } else {
#pragma unroll
            for (int a = 0; a < 3; ++a) V[a] = z4;
#pragma unroll
            for (int k = 0; k < 6; ++k) Mt[k] = z4;
        }
        v4f acc_phi = z4;
        v4f dV[3] = {z4, z4, z4}, dM[6] = {z4, z4, z4, z4, z4, z4};
        float du[3] = {0.f, 0.f, 0.f};
#pragma unroll
        for (int o = 0; o < 18; ++o) {
            // features F[o] of this lane's 4 channels
            v4f F;
            if (o < 3) {
                F = V[o];
            } else if (o < 6) {
                const int a = o - 3;
                F = Mt[s2(a, 0)] * u[0] + Mt[s2(a, 1)] * u[1] + Mt[s2(a, 2)] * u[2];
            } else if (o < 12) {
                F = Mt[o - 6];
            } else if (o < 15) {
                F = V[o - 12] * u[o - 12];
            } else {
                const int a = o == 17 ? 1 : 0, c = o == 15 ? 1 : 2;
                F = 0.5f * (V[c] * u[a] + V[a] * u[c]);
            }
            const float* g = sG + o * B * Kd;
            // dphi: K index q <-> channel 4q + kc; A = G[o][b = j][4q .. 4q + 3]
            const v4f ga = *reinterpret_cast<const v4f*>(g + j * Kd + 4 * q);
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) acc_phi = mfma_16x16x4(ga[kc], F[kc], acc_phi);
            // dF[o]: register r <-> channel 4q + r; A = G[o][b = 4kb + q][kd = j]
            v4f d = z4;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) d = mfma_16x16x4(g[(4 * kb + q) * Kd + j], ph[kb], d);
            if (o < 3) {
                dV[o] += d;
            } else if (o < 6) {
                const int a = o - 3;
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    dM[s2(a, c)] += u[c] * d;
                    const v4f pm = Mt[s2(a, c)] * d;
                    du[c] += pm[0] + pm[1] + pm[2] + pm[3];
                }
            } else if (o < 12) {
                dM[o - 6] += d;
            } else if (o < 15) {
                const int a = o - 12;
                const v4f pv = V[a] * d;
                du[a] += pv[0] + pv[1] + pv[2] + pv[3];
                dV[a] += u[a] * d;
            } else {
                const int a = o == 17 ? 1 : 0, c = o == 15 ? 1 : 2;
                const v4f h = 0.5f * d;
                const v4f pc = V[c] * h, pa = V[a] * h;
                du[a] += pc[0] + pc[1] + pc[2] + pc[3];
                du[c] += pa[0] + pa[1] + pa[2] + pa[3];
                dV[c] += u[a] * h;
                dV[a] += u[c] * h;
            }
            __builtin_amdgcn_sched_barrier(0);        // keep each o step's operands local
        }
        if (ok) {
            if (dphi) st4(dphi + e * ld_dphi + 4 * q, acc_phi);       // register r <-> b = 4q + r
            if (dT_edge) {
                float* o = dT_edge + e * 9 * Kd + 4 * q;
#pragma unroll
                for (int a = 0; a < 3; ++a) st4(o + a * Kd, dV[a]);
#pragma unroll
                for (int k = 0; k < 6; ++k) st4(o + (3 + k) * Kd, dM[k]);
            }
        }
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            du[a] += __shfl_xor(du[a], 16, kWave);
            du[a] += __shfl_xor(du[a], 32, kWave);
        }
        if (ok && q == 0 && gY) {
            float* gy = gY + e * 20;
            gy[1] += du[0];
            gy[2] += du[1];
            gy[3] += du[2];
        }
    }
}

// Node-table gradient of the transport tables: gV[a, n, kd] = sum_{e in row n} dT_edge[rev e, a, kd]
// (the edges whose neighbour is n are the reverses of row n); same for gM. Eight edges per
// round, their gathers issued together (one dependent load after another per edge would leave
// each thread a memory latency per edge), summed in row order.
__global__ __launch_bounds__(256) void transport_table_grad_kernel(const float* __restrict__ dT_edge, int Kd,
                                                                    const int32_t* __restrict__ row_ptr,
                                                                    const int32_t* __restrict__ rev, int64_t N,
                                                                    float* __restrict__ gV, int64_t v_sn,
                                                                    int64_t v_sq, float* __restrict__ gM,
                                                                    int64_t m_sn, int64_t m_sq) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= N * 9 * Kd) return;
    const int64_t n = t / (9 * Kd);
    const int r = (int)(t - n * 9 * Kd);
    const int q = r / Kd, kd = r - q * Kd;
    const int64_t e1 = row_ptr[n + 1];
    const int64_t st = 9 * (int64_t)Kd;
    float s = 0.f;
    int64_t e = row_ptr[n];
    for (; e + 8 <= e1; e += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = dT_edge[(int64_t)rev[e + u] * st + r];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; e < e1; ++e) s += dT_edge[(int64_t)rev[e] * st + r];
    if (q < 3) gV[q * v_sq + n * v_sn + kd] = s;
    else gM[(q - 3) * m_sq + n * m_sn + kd] = s;
}

}  // namespace face

using namespace face;

extern "C" int face_transport_fwd(const float* phi, int32_t ld_phi, int32_t B, const float* V, int64_t v_sn,
                                  int64_t v_sq, const float* M, int64_t m_sn, int64_t m_sq, int32_t Kd,
                                  const float* Y, int32_t ld_Y, const int32_t* col, const int32_t* row_ptr, int64_t N,
                                  float scale, float* D1, float* D2, void* stream) {
    if (N < 0 || B <= 0 || Kd <= 0 || ld_phi < B || ld_Y < 4 || B * Kd > 1024) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!phi || !V || !M || !Y || !col || !row_ptr || !D1 || !D2) return FACE_ERR_ARG;
    const int nthr = ((B * Kd + kWave - 1) / kWave) * kWave;
    const size_t lds = ((size_t)kTT * Kd * kFP + kTT * B) * sizeof(float);
    if (lds > 65536) return FACE_ERR_UNSUPPORTED;
    Tables T{V, M, v_sn, v_sq, m_sn, m_sq};
    if (B == 16 && Kd == 16) {
        hipLaunchKernelGGL(transport_fwd_mfma_kernel, dim3((unsigned)((N + kTfWaves - 1) / kTfWaves)),
                           dim3(kTfWaves * kWave), 0, (hipStream_t)stream, phi, ld_phi, T, Y, ld_Y, col, row_ptr, N,
                           scale, D1, D2);
        FACE_LAUNCH_CHECK();
        return 0;
    }
    hipLaunchKernelGGL(transport_fwd_kernel, dim3((unsigned)N), dim3(nthr), lds, (hipStream_t)stream, phi, ld_phi, B,
                       T, Kd, Y, ld_Y, col, row_ptr, N, scale, D1, D2);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_transport_bwd(const float* phi, int32_t ld_phi, int32_t B, const float* V, int64_t v_sn,
                                  int64_t v_sq, const float* M, int64_t m_sn, int64_t m_sq, int32_t Kd,
                                  const float* Y, int32_t ld_Y, const int32_t* col, const int32_t* row_ptr,
                                  const int32_t* rev, int64_t N, int32_t max_row, float scale, const float* gD1,
                                  const float* gD2, float* dphi, int32_t ld_dphi, float* dT_edge, float* gV,
                                  float* gM, float* gY, void* stream) {
    if (N < 0 || B <= 0 || B > 32 || Kd <= 0 || Kd > 64 || ld_phi < B || ld_Y < 4 || max_row < 0) return FACE_ERR_ARG;
    if (dphi && ld_dphi < B) return FACE_ERR_ARG;
    if ((gV || gM) && (!gV || !gM || !dT_edge || !rev)) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!phi || !V || !M || !Y || !col || !row_ptr || !gD1 || !gD2) return FACE_ERR_ARG;
    int KP = 1;
    while (KP < Kd) KP <<= 1;
    const int per_wave = kWave / KP;
    int nw = (max_row + per_wave - 1) / per_wave;
    nw = nw < 1 ? 1 : (nw > 4 ? 4 : nw);
    const size_t lds = (size_t)B * Kd * kFP * sizeof(float);
    if (lds > 65536) return FACE_ERR_UNSUPPORTED;
    Tables T{V, M, v_sn, v_sq, m_sn, m_sq};
    hipStream_t st = (hipStream_t)stream;
    const bool a16 = !(((uintptr_t)V | (uintptr_t)M | (uintptr_t)(dphi ? dphi : V) | (uintptr_t)(dT_edge ? dT_edge : V)) & 15);
    if (B == 16 && Kd == 16 && a16 && v_sn % 4 == 0 && v_sq % 4 == 0 && m_sn % 4 == 0 && m_sq % 4 == 0 &&
        (!dphi || ld_dphi % 4 == 0)) {
        const size_t lds2 = (size_t)2 * 18 * 16 * 16 * sizeof(float);
        hipLaunchKernelGGL(transport_bwd_mfma_kernel, dim3((unsigned)((N + 1) / 2)), dim3(2 * kWave), lds2, st, phi,
                           ld_phi, T, Y, ld_Y, col, row_ptr, N, scale, gD1, gD2, dphi, ld_dphi, dT_edge, gY);
    } else {
        hipLaunchKernelGGL(transport_bwd_kernel, dim3((unsigned)N), dim3(nw * kWave), lds, st, phi, ld_phi, B, T, Kd,
                           KP, Y, ld_Y, col, row_ptr, N, scale, gD1, gD2, dphi, ld_dphi, dT_edge, gY);
    }
    if (gV) {
        const int64_t total = N * 9 * Kd;
        hipLaunchKernelGGL(transport_table_grad_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                           dT_edge, Kd, row_ptr, rev, N, gV, v_sn, v_sq, gM, m_sn, m_sq);
    }
    FACE_LAUNCH_CHECK();
    return 0;
}
