// Receiver-segmented density reductions for FACE (gfx950).
//
// Factor density  D[i,x,b*K+k] = sum_{e in row i} phi[e,b] msg[m(e),k] Y[e,x]            (face/kernels.py:3,170-178)
// CP density      A[i,x,c]     = sum_{e in row i} env[e] R[e,l(x),c] msg[m(e),c] Y[e,x]   (face/model.py:496-502)
//
// Every output row belongs to exactly one workgroup, so the reductions run in registers and
// LDS with no global atomics; results are bitwise reproducible run to run.
//
// Outputs (and upstream gradients) are addressed per rank block: element (atom i, monomial x,
// column c) lives at p[l(x)] + i*sa + (x - x0(l))*sx + c. The reference layout (N, NX, W) is
// p[l] = base + x0(l)*W, sa = NX*W, sx = W; the model keeps each rank as its own (k_l, N, W)
// tensor (p[l] = D_l, sa = W, sx = N*W) so the channel-mixing GEMMs read contiguous blocks.
#include "common.h"

#include <algorithm>
#include <cstdlib>

namespace face {

constexpr int kBlock = 256;
constexpr int kTileE = 32;   // edges staged per LDS tile (factor forward)

__host__ __device__ constexpr int rank_start(int l) { return l == 0 ? 0 : (l == 1 ? 1 : (l == 2 ? 4 : 10)); }

struct RankOut {
    float* p[4];
    int64_t sa, sx;
    __device__ __forceinline__ float* at(int64_t i, int x) const {
        float* b = x < 1 ? p[0] : (x < 4 ? p[1] : (x < 10 ? p[2] : p[3]));
        return b + i * sa + (int64_t)(x - rank_start(rank_of(x))) * sx;
    }
};
struct RankIn {
    const float* p[4];
    int64_t sa, sx;
    __device__ __forceinline__ const float* at(int64_t i, int x) const {
        const float* b = x < 1 ? p[0] : (x < 4 ? p[1] : (x < 10 ? p[2] : p[3]));
        return b + i * sa + (int64_t)(x - rank_start(rank_of(x))) * sx;
    }
};

// ------------------------------------------------------------------ factor forward
// Workgroup = (atom i, column chunk). Thread owns CPT columns (b,k) and NX accumulators
// per column; the edge tile (phi, msg, Y) is staged in LDS and read as broadcasts.
template <int NX, int CPT>
__global__ __launch_bounds__(kBlock) void density_fwd_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int M, int B, int K, RankOut D) {
    extern __shared__ float lds[];
    float* s_phi = lds;                    // kTileE * B
    float* s_msg = s_phi + kTileE * B;     // kTileE * K
    float* s_Y = s_msg + kTileE * K;       // kTileE * NX
    const int64_t i = blockIdx.x;
    const int BK = B * K;
    const int tid = threadIdx.x;
    int bcol[CPT], kcol[CPT];
    bool ok[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = blockIdx.y * (kBlock * CPT) + j * kBlock + tid;
        ok[j] = c < BK;
        bcol[j] = ok[j] ? c / K : 0;
        kcol[j] = ok[j] ? c - bcol[j] * K : 0;
    }
    float acc[CPT][NX];
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
        for (int x = 0; x < NX; ++x) acc[j][x] = 0.f;

    int64_t e0, e1;
    row_range(row_ptr, i, M, e0, e1);
    for (int64_t t0 = e0; t0 < e1; t0 += kTileE) {
        const int nt = (int)min((int64_t)kTileE, e1 - t0);
        for (int q = tid; q < nt * B; q += kBlock) {
            const int t = q / B;
            s_phi[q] = phi[(t0 + t) * ld_phi + (q - t * B)];
        }
        for (int q = tid; q < nt * K; q += kBlock) {
            const int t = q / K;
            const int64_t row = msg_row ? (int64_t)msg_row[t0 + t] : t0 + t;
            s_msg[q] = msg[row * ld_msg + (q - t * K)];
        }
        for (int q = tid; q < nt * NX; q += kBlock) {
            const int t = q / NX;
            s_Y[q] = Y[(t0 + t) * ld_Y + (q - t * NX)];
        }
        __syncthreads();
        for (int t = 0; t < nt; ++t) {
            float p[CPT];
#pragma unroll
            for (int j = 0; j < CPT; ++j) p[j] = s_phi[t * B + bcol[j]] * s_msg[t * K + kcol[j]];
            const float* y = s_Y + t * NX;
#pragma unroll
            for (int x = 0; x < NX; ++x) {
                const float yx = y[x];
#pragma unroll
                for (int j = 0; j < CPT; ++j) acc[j][x] = fmaf(p[j], yx, acc[j][x]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        if (!ok[j]) continue;
        const int c = blockIdx.y * (kBlock * CPT) + j * kBlock + tid;
#pragma unroll
        for (int x = 0; x < NX; ++x) D.at(i, x)[c] = acc[j][x];
    }
}

// ------------------------------------------------------------------ factor forward on MFMA
// B = 16, NX = 20, K = 16 KB: for monomial x, D[x] (16 b x K) = sum_e U_x[e, :]^T msg[e, :] with
// U_x[e, b] = Y[e, x] phi[e, b], a v_mfma_f32_16x16x4f32 chain per (monomial, 16-channel block):
// A = U_x^T (basis j, K index q), B = msg rows, basis 4q + r and channel j in register r of lane
// j + 16q. One atom per workgroup, its 4 waves own 5 monomials each (no cross-wave sums). The
// row is walked in chunks of 32 edges held in registers; instruction r of a chunk takes edges
// 4r .. 4r + 3 (K index q = edge 4r + q), so a chunk of ne edges issues ceil(ne / 4)
// instructions per chain instead of whole 16-edge tiles (an 18-edge row: 5 instead of 8). Every
// load of a chunk is issued before its first product (one memory latency per chunk), and in the
// row's last chunk (the only one for rows of <= 32 edges) each monomial's D_x is stored as soon
// as its chain ends, while the next monomial's products run. Against 16-edge tiles with the next
// tile prefetched and all stores at the end (the same products, summed in another order): 864-atom FCC
// 14.0 -> 13.4 us, 64 molecules 16.5 -> 16.3 us, 100,000 atoms at K = 64 4453 -> 4168 us.
// Measured and not kept: 5 or 10 waves per atom (each reloads the chunk's phi and message rows:
// 864 atoms 15.2 / 16.9 us); a workgroup whose computing waves hand finished tiles through LDS to
// a storing wave so that no product waits behind a store (864 atoms 14.4 us); persistent
// workgroups streaming several atoms each, the next atom's chunk staged through a double-buffered
// LDS tile while the current one is multiplied and stored (one, two or four workgroups per CU:
// 864 atoms 18.2 / 13.4 / 14.3 us, 64 molecules 24.7 / 17.2 / 16.3 us, 100,000 atoms 7.2 / 4.9 /
// 4.9 ms).
constexpr int kDrWaves = 4;
constexpr int kDrCh = 32;                                // edges per register chunk

template <int KB>
__global__ __launch_bounds__(kDrWaves * kWave) void density_fwd_row_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int M, RankOut D) {
    constexpr int K = 16 * KB, NXW = 20 / kDrWaves, NI = kDrCh / 4;
    const int lane = threadIdx.x & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int x0 = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave) * NXW;
    const int64_t n = blockIdx.x;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    v4f acc[NXW][KB];
#pragma unroll
    for (int xx = 0; xx < NXW; ++xx)
#pragma unroll
        for (int c = 0; c < KB; ++c) acc[xx][c] = z4;
    int64_t a, bnd;
    row_range(row_ptr, n, M, a, bnd);
    auto store = [&](int xx) {
        float* dx = D.at(n, x0 + xx);
#pragma unroll
        for (int c = 0; c < KB; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) dx[(4 * q + r) * K + 16 * c + j] = acc[xx][c][r];
    };
    if (a >= bnd) {                                      // empty row: zeros
#pragma unroll
        for (int xx = 0; xx < NXW; ++xx) store(xx);
        return;
    }
    for (int64_t c0 = a; c0 < bnd; c0 += kDrCh) {
        const int ne = (int)min((int64_t)kDrCh, bnd - c0);
        const int ni = (ne + 3) >> 2;                    // uniform over the workgroup
        const bool last = c0 + kDrCh >= bnd;
        // every slot loads (edges past the row end clamped to its last edge, phi zeroed there): no
        // branches between the loads, so the gathered rows' indices all issue before one wait
        float ph[NI], yv[NXW][NI], mb[KB][NI];
        int64_t ev[NI], rw[NI];
#pragma unroll
        for (int r = 0; r < NI; ++r) ev[r] = c0 + min(4 * r + q, ne - 1);
        if (msg_row) {                                   // one uniform branch around all slots
#pragma unroll
            for (int r = 0; r < NI; ++r) rw[r] = msg_row[ev[r]];
        } else {
#pragma unroll
            for (int r = 0; r < NI; ++r) rw[r] = ev[r];
        }
#pragma unroll
        for (int r = 0; r < NI; ++r) {
            const float p = phi[ev[r] * ld_phi + j];
            ph[r] = 4 * r + q < ne ? p : 0.f;
#pragma unroll
            for (int c = 0; c < KB; ++c) mb[c][r] = msg[rw[r] * ld_msg + 16 * c + j];
#pragma unroll
            for (int xx = 0; xx < NXW; ++xx) yv[xx][r] = Y[ev[r] * ld_Y + x0 + xx];
        }
        // keep every load here, ahead of the products (the compiler would otherwise sink each slot's
        // loads into its conditional block: a memory latency per slot)
#pragma unroll
        for (int r = 0; r < NI; ++r) {
            asm volatile("" ::"v"(ph[r]));
#pragma unroll
            for (int c = 0; c < KB; ++c) asm volatile("" ::"v"(mb[c][r]));
#pragma unroll
            for (int xx = 0; xx < NXW; ++xx) asm volatile("" ::"v"(yv[xx][r]));
        }
#pragma unroll
        for (int xx = 0; xx < NXW; ++xx) {
#pragma unroll
            for (int r = 0; r < NI; ++r) {
                if (r < ni) {
                    const float u = yv[xx][r] * ph[r];
#pragma unroll
                    for (int c = 0; c < KB; ++c) acc[xx][c] = mfma_16x16x4(u, mb[c][r], acc[xx][c]);
                }
            }
            if (last) store(xx);
        }
    }
}

// ------------------------------------------------------------------ factor backward
// Workgroup = atom i; G[i] (NX x B x K) is staged in LDS, split in GN k-slices of KS
// columns (slice stride KSP, 16-byte aligned). A lane is (edge slot, k-slice g): it keeps
// phi[e,:], its msg slice and their gradients in registers and walks every (x, b):
//   s = sum_k G[x,b,k] msg[k]          -> dphi[b] += s Y[x],  dY[x] += s phi[b]
//   dmsg[k] += G[x,b,k] Y[x] phi[b]
// dY and dphi are then summed over the GN lanes of the edge (butterfly shuffles).
template <int NX, int B, int KS>
__global__ __launch_bounds__(kBlock) void density_bwd_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int M, int K, int glog, RankIn G, float* __restrict__ dphi, int ld_dphi, float* __restrict__ dmsg, int ld_dmsg,
    float* __restrict__ dY, int ld_dY) {
    constexpr int KSP = (KS + 3) & ~3;
    extern __shared__ float lds[];
    const int GN = 1 << glog;
    const int64_t i = blockIdx.x;
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int nslot = NX * B * GN * KSP;
    for (int p = tid; p < nslot; p += nthr) {
        const int kk = p % KSP;
        int r = p / KSP;
        const int g = r % GN;
        r /= GN;
        const int b = r % B, x = r / B;
        const int k = g * KS + kk;
        lds[p] = (kk < KS && k < K) ? G.at(i, x)[b * K + k] : 0.f;
    }
    __syncthreads();

    const int g = tid & (GN - 1);
    const int slot = tid >> glog;
    const int nslots = nthr >> glog;
    int64_t e0, e1;
    row_range(row_ptr, i, M, e0, e1);
    for (int64_t base = e0; base < e1; base += nslots) {   // same trip count for every lane
        const int64_t e = base + slot;
        const bool valid = e < e1;
        float ph[B], dph[B], mg[KS], dmg[KS];
        const int64_t row = valid ? (msg_row ? (int64_t)msg_row[e] : e) : 0;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            ph[b] = valid ? phi[e * ld_phi + b] : 0.f;
            dph[b] = 0.f;
        }
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            const int k = g * KS + kk;
            mg[kk] = (valid && k < K) ? msg[row * ld_msg + k] : 0.f;
            dmg[kk] = 0.f;
        }
#pragma unroll 1
        for (int x = 0; x < NX; ++x) {
            const float y = valid ? Y[e * ld_Y + x] : 0.f;
            const float* gx = lds + ((x * B) * GN + g) * KSP;
            float dy = 0.f;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float* gp = gx + b * GN * KSP;
                const float yp = y * ph[b];
                float s = 0.f;
#pragma unroll
                for (int kk = 0; kk < KS; ++kk) {
                    const float gv = gp[kk];
                    s = fmaf(gv, mg[kk], s);
                    dmg[kk] = fmaf(gv, yp, dmg[kk]);
                }
                dph[b] = fmaf(s, y, dph[b]);
                dy = fmaf(s, ph[b], dy);
            }
            dy = group_sum(dy, GN);
            if (dY && valid && g == 0) dY[e * ld_dY + x] = dy;
        }
#pragma unroll
        for (int b = 0; b < B; ++b) dph[b] = group_sum(dph[b], GN);
        if (valid) {
            if (dphi) {
#pragma unroll
                for (int b = 0; b < B; ++b)
                    if ((b & (GN - 1)) == g) dphi[e * ld_dphi + b] = dph[b];
            }
            if (dmsg) {
#pragma unroll
                for (int kk = 0; kk < KS; ++kk) {
                    const int k = g * KS + kk;
                    if (k < K) dmsg[e * ld_dmsg + k] = dmg[kk];
                }
            }
        }
    }
}

// ------------------------------------------------------------------ factor backward on MFMA
// B = 16 basis functions, NX = 20 monomials, K = 16 KB message channels: with the columns of
// G[i] flattened as (x, b), the 16-column block x is monomial x. Tiles of 16 edges; per monomial
// x two v_mfma_f32_16x16x4f32 chains:
//   S[e, b]  = sum_k msg[e, k] G[x, b, k]       (A = msg rows, K index q of instruction r of chunk
//                                                c = channel 16 c + 4q + r; B = G rows)
//   dmsg[e, k] += sum_b Y[e, x] phi[e, b] G[x, b, k]   (A = Y[e, x] phi[e, :], K index q of
//                                                instruction r = basis 4q + r; B = G columns)
// both with edge 4q + r in register r of lane j + 16q (column j = basis b, resp. channel k).
// From S: dphi[e, b] += S Y[e, x], and dY[e, x] = sum_b S phi[e, b], a sum over the 16 lanes
// of a row group. WPA = 1: one wave per atom (kDbWaves atoms per workgroup). WPA > 1: one atom
// per workgroup, its WPA waves split the monomials and sum their dphi / dmsg partials in LDS
// (small systems, where one wave per atom leaves the SIMDs idle).
constexpr int kDbWaves = 8;
constexpr int kDbYS = 21;                                // Y tile row stride (floats)

template <int KB, int WPA>
__global__ __launch_bounds__((WPA > 1 ? WPA : kDbWaves) * kWave) void density_bwd_mfma_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int64_t N, int M, RankIn G, float* __restrict__ dphi, int ld_dphi, float* __restrict__ dmsg, int ld_dmsg,
    float* __restrict__ dY, int ld_dY) {
    constexpr int K = 16 * KB, NXW = 20 / WPA, NSLOT = (NXW + 15) / 16;
    constexpr int YW = WPA > 1 ? 1 : kDbWaves;           // Y tiles: one per atom of the workgroup
    constexpr int PW = WPA > 1 ? WPA : 1;
    __shared__ float sY[YW][16 * kDbYS];
    __shared__ float sP[PW][16 * (16 + K)];               // dphi | dmsg partials (WPA > 1)
    const int lane = threadIdx.x & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int64_t n = WPA > 1 ? (int64_t)blockIdx.x : (int64_t)blockIdx.x * kDbWaves + wv;
    if (n >= N) return;                                  // WPA = 1 only: no workgroup barrier there
    const int x0 = WPA > 1 ? wv * NXW : 0;
    float* ys = sY[WPA > 1 ? 0 : wv];
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    int64_t a, bnd;
    row_range(row_ptr, n, M, a, bnd);
    for (int64_t e0 = a; e0 < bnd; e0 += 16) {
        const int ne = (int)min((int64_t)16, bnd - e0);
        // the tile's Y (16 x 20) into LDS, zero past the row end
        if (WPA > 1) {
            __syncthreads();                             // previous tile's Y and partials consumed
            for (int v = threadIdx.x; v < 320; v += WPA * kWave) {
                const int t = v / 20, x = v - t * 20;
                ys[t * kDbYS + x] = t < ne ? Y[(e0 + t) * ld_Y + x] : 0.f;
            }
            __syncthreads();
        } else {
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int u = 0; u < 5; ++u) {
                const int v = u * kWave + lane, t = v / 20, x = v - t * 20;
                ys[t * kDbYS + x] = t < ne ? Y[(e0 + t) * ld_Y + x] : 0.f;
            }
            __builtin_amdgcn_wave_barrier();
        }
        // edge e0 + j: message row and phi[4q .. 4q + 3] (A operands), zero past the row end
        const bool oki = j < ne;
        const int64_t ei = e0 + min(j, ne - 1);
        const int64_t rowi = msg_row ? (int64_t)msg_row[ei] : ei;
        v4f mA[KB];
#pragma unroll
        for (int c = 0; c < KB; ++c) mA[c] = oki ? ld4(msg + rowi * ld_msg + 16 * c + 4 * q) : z4;
        const v4f ph4 = oki ? ld4(phi + ei * ld_phi + 4 * q) : z4;
        // edges e0 + 4q + r at basis j (for dY)
        float phT[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) phT[r] = phi[(e0 + min(4 * q + r, ne - 1)) * ld_phi + j];
        v4f dph = z4, dm[KB];
#pragma unroll
        for (int c = 0; c < KB; ++c) dm[c] = z4;
        float dyk[4][NSLOT];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int sl = 0; sl < NSLOT; ++sl) dyk[r][sl] = 0.f;
#pragma unroll 2
        for (int xx = 0; xx < NXW; ++xx) {
            const int x = x0 + xx;
            const float* gx = G.at(n, x);                // (16 b) x K
            v4f sv = z4;
#pragma unroll
            for (int c = 0; c < KB; ++c) {
                const v4f gv = ld4(gx + j * K + 16 * c + 4 * q);
#pragma unroll
                for (int r = 0; r < 4; ++r) sv = mfma_16x16x4(mA[c][r], gv[r], sv);
            }
            const float yi = ys[j * kDbYS + x];
#pragma unroll
            for (int c = 0; c < KB; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) dm[c] = mfma_16x16x4(yi * ph4[r], gx[(4 * q + r) * K + 16 * c + j], dm[c]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                dph[r] = fmaf(sv[r], ys[(4 * q + r) * kDbYS + x], dph[r]);
                float v = sv[r] * phT[r];
                v = row16_sum(v);
                if (j == (xx & 15)) dyk[r][xx >> 4] = v;
            }
        }
        // dY of this wave's monomials
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 4 * q + r;
            if (dY && t < ne) {
#pragma unroll
                for (int sl = 0; sl < NSLOT; ++sl)
                    if (16 * sl + j < NXW) dY[(e0 + t) * ld_dY + x0 + 16 * sl + j] = dyk[r][sl];
            }
        }
        if (WPA > 1) {
            // partials of the WPA waves summed by wave 0
            float* mine = sP[wv];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                mine[(4 * q + r) * 16 + j] = dph[r];
#pragma unroll
                for (int c = 0; c < KB; ++c) mine[256 + (4 * q + r) * K + 16 * c + j] = dm[c][r];
            }
            __syncthreads();
            if (wv == 0) {
#pragma unroll
                for (int w = 1; w < WPA; ++w) {
                    const float* o = sP[w];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        dph[r] += o[(4 * q + r) * 16 + j];
#pragma unroll
                        for (int c = 0; c < KB; ++c) dm[c][r] += o[256 + (4 * q + r) * K + 16 * c + j];
                    }
                }
            }
        }
        if (WPA == 1 || wv == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 4 * q + r;
                if (t < ne) {
                    const int64_t e = e0 + t;
                    if (dphi) dphi[e * ld_dphi + j] = dph[r];
                    if (dmsg) {
#pragma unroll
                        for (int c = 0; c < KB; ++c) dmsg[e * ld_dmsg + 16 * c + j] = dm[c][r];
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------ factor backward, small systems
// One atom per workgroup of 4 waves, wave w on monomials 5w .. 5w + 4 (the per-monomial MFMA
// chains of density_bwd_mfma_kernel), for K <= 32. The wave's G operands (5 monomials x 16 b x K,
// both operand layouts: 80 registers at K = 32) are read once per atom, while the first tile's
// rows load, and stay in registers over the atom's tiles; per 16-edge tile the Y tile, the message
// rows and phi are issued together before the workgroup barrier. A tile then costs one memory
// latency instead of one per pair of monomials (the G reads of density_bwd_mfma_kernel). The
// four waves' dphi / dmsg partials are summed through LDS by all four. At K = 32 the kernel holds
// ~230 registers (two waves per SIMD); capped at four waves per SIMD it spills 312 bytes and runs
// 1.8x slower. Measured against density_bwd_mfma_kernel<2, 4>: 35.5 -> 27.3 us (864-atom FCC),
// 37.6 -> 32.3 us (1,344 atoms), 153 -> 113 us (2,000 atoms of 70 neighbours), same bits.
constexpr int kDsWaves = 4;

template <int KB>
__global__ __launch_bounds__(kDsWaves * kWave) void density_bwd_split_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int M, RankIn G, float* __restrict__ dphi, int ld_dphi, float* __restrict__ dmsg, int ld_dmsg,
    float* __restrict__ dY, int ld_dY) {
    constexpr int K = 16 * KB, NXW = 20 / kDsWaves;
    __shared__ float sY[16 * kDbYS];
    __shared__ float sP[kDsWaves][16 * (16 + K)];        // dphi | dmsg partials
    const int tid = threadIdx.x, lane = tid & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int64_t n = blockIdx.x;
    const int x0 = wv * NXW;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    // G_x operands: gv = G[x][b = j][16c + 4q .. + 3] (S chain), gs = G[x][b = 4q + r][16c + j] (dmsg chain)
    v4f gv[NXW][KB];
    float gs[NXW][KB][4];
#pragma unroll
    for (int xx = 0; xx < NXW; ++xx) {
        const float* gx = G.at(n, x0 + xx);
#pragma unroll
        for (int c = 0; c < KB; ++c) {
            gv[xx][c] = ld4(gx + j * K + 16 * c + 4 * q);
#pragma unroll
            for (int r = 0; r < 4; ++r) gs[xx][c][r] = gx[(4 * q + r) * K + 16 * c + j];
        }
    }
    int64_t a, bnd;
    row_range(row_ptr, n, M, a, bnd);
    for (int64_t e0 = a; e0 < bnd; e0 += 16) {
        const int ne = (int)min((int64_t)16, bnd - e0);
        // this tile's loads, all issued before the barrier: the Y tile (16 x 20, zero past the row
        // end; 320 values over 256 threads), the message row and phi of edge e0 + j, phi of edges
        // e0 + 4q + r at basis j
        float yl[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int v = u * kDsWaves * kWave + tid, t = v / 20, x = v - t * 20;
            yl[u] = (v < 320 && t < ne) ? Y[(e0 + t) * ld_Y + x] : 0.f;
        }
        const bool oki = j < ne;
        const int64_t ei = e0 + min(j, ne - 1);
        const int64_t rowi = msg_row ? (int64_t)msg_row[ei] : ei;
        v4f mA[KB];
#pragma unroll
        for (int c = 0; c < KB; ++c) mA[c] = oki ? ld4(msg + rowi * ld_msg + 16 * c + 4 * q) : z4;
        const v4f ph4 = oki ? ld4(phi + ei * ld_phi + 4 * q) : z4;
        float phT[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) phT[r] = phi[(e0 + min(4 * q + r, ne - 1)) * ld_phi + j];
        __syncthreads();                                 // previous tile's Y and partials consumed
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int v = u * kDsWaves * kWave + tid, t = v / 20, x = v - t * 20;
            if (v < 320) sY[t * kDbYS + x] = yl[u];
        }
        __syncthreads();
        v4f dph = z4, dm[KB];
#pragma unroll
        for (int c = 0; c < KB; ++c) dm[c] = z4;
        float dyk[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) dyk[r] = 0.f;
#pragma unroll
        for (int xx = 0; xx < NXW; ++xx) {
            const int x = x0 + xx;
            v4f sv = z4;
#pragma unroll
            for (int c = 0; c < KB; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) sv = mfma_16x16x4(mA[c][r], gv[xx][c][r], sv);
            const float yi = sY[j * kDbYS + x];
#pragma unroll
            for (int c = 0; c < KB; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) dm[c] = mfma_16x16x4(yi * ph4[r], gs[xx][c][r], dm[c]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                dph[r] = fmaf(sv[r], sY[(4 * q + r) * kDbYS + x], dph[r]);
                float v = sv[r] * phT[r];
                v = row16_sum(v);
                if (j == xx) dyk[r] = v;
            }
        }
        // dY of this wave's monomials: lane j < 5 holds monomial x0 + j of edge e0 + 4q + r
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 4 * q + r;
            if (dY && t < ne && j < NXW) dY[(e0 + t) * ld_dY + x0 + j] = dyk[r];
        }
        // partials of the four waves, summed by all four: thread tid takes values tid, tid + 256, ...
        // of the block (dphi | dmsg), adding the waves' partials in wave order (one wave doing all
        // the sums and stores left the other three waiting at the next tile's barrier: 864 atoms
        // 27.6 -> 27.0 us, 64 molecules 32.1 -> 31.0 us)
        float* mine = sP[wv];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            mine[(4 * q + r) * 16 + j] = dph[r];
#pragma unroll
            for (int c = 0; c < KB; ++c) mine[256 + (4 * q + r) * K + 16 * c + j] = dm[c][r];
        }
        __syncthreads();
        constexpr int NV = 16 * (16 + K), NU = (NV + kDsWaves * kWave - 1) / (kDsWaves * kWave);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int v = u * kDsWaves * kWave + tid;
            if (v < NV) {
                float sum = sP[0][v];
#pragma unroll
                for (int w = 1; w < kDsWaves; ++w) sum += sP[w][v];
                if (v < 256) {
                    const int t = v >> 4, b = v & 15;
                    if (dphi && t < ne) dphi[(e0 + t) * ld_dphi + b] = sum;
                } else {
                    const int t = (v - 256) / K, k = (v - 256) - t * K;
                    if (dmsg && t < ne) dmsg[(e0 + t) * ld_dmsg + k] = sum;
                }
            }
        }
    }
}

// ------------------------------------------------------------------ factor backward, G in LDS
// Large systems (long rows, K up to 64): one workgroup of 4 waves per atom stages the atom's G
// (20 x 16 x K) in LDS in two halves of 10 monomials (row stride K + 4: the 16 rows one
// instruction reads sit on distinct banks), so that G is read from memory once per group of 4
// edge tiles of the atom instead of once per tile and monomial. Wave w takes tile w of each
// group and keeps its operands (msg, phi) and accumulators (dphi, dmsg) in registers over both
// halves; per monomial the two MFMA chains of density_bwd_mfma_kernel run against the LDS copy,
// and dY[e, x] is complete per monomial.
constexpr int kDbLWaves = 4;

template <int KB>
__global__ __launch_bounds__(kDbLWaves * kWave) void density_bwd_lds_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    RankIn G, float* __restrict__ dphi, int ld_dphi, float* __restrict__ dmsg, int ld_dmsg, float* __restrict__ dY,
    int ld_dY) {
    constexpr int K = 16 * KB, GS = K + 4, XH = 10;
    __shared__ float sG[XH * 16 * GS];
    __shared__ float sY[kDbLWaves][16 * kDbYS];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int64_t n = blockIdx.x;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    const int64_t a = row_ptr[n], bnd = row_ptr[n + 1];
    const int ntile = (int)((bnd - a + 15) / 16);
    float* ys = sY[wv];
#pragma unroll 1
    for (int g0 = 0; g0 < ntile; g0 += kDbLWaves) {
        // this wave's tile of the group: operands and accumulators
        const int t = g0 + wv;
        const int64_t e0 = a + 16 * (int64_t)t;
        const int ne = t < ntile ? (int)min((int64_t)16, bnd - e0) : 0;
        v4f mA[KB], ph4 = z4, dph = z4, dm[KB];
        float phT[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < KB; ++c) dm[c] = mA[c] = z4;
        if (ne > 0) {
#pragma unroll
            for (int u = 0; u < 5; ++u) {
                const int v = u * kWave + lane, tt = v / 20, x = v - tt * 20;
                ys[tt * kDbYS + x] = tt < ne ? Y[(e0 + tt) * ld_Y + x] : 0.f;
            }
            const bool oki = j < ne;
            const int64_t ei = e0 + min(j, ne - 1);
            const int64_t rowi = msg_row ? (int64_t)msg_row[ei] : ei;
#pragma unroll
            for (int c = 0; c < KB; ++c) mA[c] = oki ? ld4(msg + rowi * ld_msg + 16 * c + 4 * q) : z4;
            ph4 = oki ? ld4(phi + ei * ld_phi + 4 * q) : z4;
#pragma unroll
            for (int r = 0; r < 4; ++r) phT[r] = phi[(e0 + min(4 * q + r, ne - 1)) * ld_phi + j];
        }
#pragma unroll 1
        for (int h = 0; h < 2; ++h) {
            // stage G[x0 .. x0 + 9] of the atom: 16 rows of K per monomial, row stride GS
            __syncthreads();                                   // previous half (or group) consumed
            const int x0 = XH * h;
            constexpr int NV = XH * 16 * K / 4;
            for (int v0 = 0; v0 < NV; v0 += 4 * kDbLWaves * kWave) {
                v4f b4[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int v = v0 + u * kDbLWaves * kWave + tid;
                    if (v < NV) {
                        const int xl = v / (4 * K), rem = v - xl * 4 * K;        // rem: float4 index in (16, K)
                        b4[u] = ld4(G.at(n, x0 + xl) + 4 * rem);
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int v = v0 + u * kDbLWaves * kWave + tid;
                    if (v < NV) {
                        const int xl = v / (4 * K), rem = v - xl * 4 * K, b = rem / (K / 4), k4 = rem - b * (K / 4);
                        st4(sG + (xl * 16 + b) * GS + 4 * k4, b4[u]);
                    }
                }
            }
            __syncthreads();
            if (ne > 0) {
                float dyk[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
                for (int xl = 0; xl < XH; ++xl) {
                    const int x = x0 + xl;
                    const float* gx = sG + xl * 16 * GS;
                    v4f sv = z4;
#pragma unroll
                    for (int c = 0; c < KB; ++c) {
                        const v4f gv = *reinterpret_cast<const v4f*>(gx + j * GS + 16 * c + 4 * q);
#pragma unroll
                        for (int r = 0; r < 4; ++r) sv = mfma_16x16x4(mA[c][r], gv[r], sv);
                    }
                    const float yi = ys[j * kDbYS + x];
#pragma unroll
                    for (int c = 0; c < KB; ++c)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            dm[c] = mfma_16x16x4(yi * ph4[r], gx[(4 * q + r) * GS + 16 * c + j], dm[c]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        dph[r] = fmaf(sv[r], ys[(4 * q + r) * kDbYS + x], dph[r]);
                        float v = sv[r] * phT[r];
                        v = row16_sum(v);
                        if (j == xl) dyk[r] = v;
                    }
                }
                if (dY && j < XH) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int te = 4 * q + r;
                        if (te < ne) dY[(e0 + te) * ld_dY + x0 + j] = dyk[r];
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int te = 4 * q + r;
            if (te < ne) {
                const int64_t e = e0 + te;
                if (dphi) dphi[e * ld_dphi + j] = dph[r];
                if (dmsg) {
#pragma unroll
                    for (int c = 0; c < KB; ++c) dmsg[e * ld_dmsg + 16 * c + j] = dm[c][r];
                }
            }
        }
    }
}

// ------------------------------------------------------------------ CP forward
// Workgroup = (atom i, channel chunk); thread = channel c with 20 accumulators. Per edge it
// streams R[e,0..3,c] and msg[m(e),c] (coalesced over c); Y and env are staged in LDS.
constexpr int kTileCP = 16;

__global__ __launch_bounds__(kBlock) void cp_density_fwd_kernel(
    const float* __restrict__ R, int ld_R, const float* __restrict__ env, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int M, int C, RankOut A) {
    __shared__ float s_Y[kTileCP * 20];
    __shared__ float s_env[kTileCP];
    const int64_t i = blockIdx.x;
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int c = blockIdx.y * nthr + tid;
    const bool ok = c < C;
    float acc[20];
#pragma unroll
    for (int x = 0; x < 20; ++x) acc[x] = 0.f;
    int64_t e0, e1;
    row_range(row_ptr, i, M, e0, e1);
    for (int64_t t0 = e0; t0 < e1; t0 += kTileCP) {
        const int nt = (int)min((int64_t)kTileCP, e1 - t0);
        for (int q = tid; q < nt * 20; q += nthr) {
            const int t = q / 20;
            s_Y[q] = Y[(t0 + t) * ld_Y + (q - t * 20)];
        }
        if (tid < nt) s_env[tid] = env ? env[t0 + tid] : 1.f;
        __syncthreads();
        if (ok) {
#pragma unroll 4
            for (int t = 0; t < nt; ++t) {
                const int64_t e = t0 + t;
                const int64_t row = msg_row ? (int64_t)msg_row[e] : e;
                const float m = msg[row * ld_msg + c] * s_env[t];
                const float* Re = R + e * ld_R + c;
                const float w0 = Re[0] * m, w1 = Re[C] * m, w2 = Re[2 * C] * m, w3 = Re[3 * C] * m;
                const float* y = s_Y + t * 20;
                acc[0] = fmaf(w0, y[0], acc[0]);
#pragma unroll
                for (int x = 1; x < 4; ++x) acc[x] = fmaf(w1, y[x], acc[x]);
#pragma unroll
                for (int x = 4; x < 10; ++x) acc[x] = fmaf(w2, y[x], acc[x]);
#pragma unroll
                for (int x = 10; x < 20; ++x) acc[x] = fmaf(w3, y[x], acc[x]);
            }
        }
        __syncthreads();
    }
    if (ok) {
#pragma unroll
        for (int x = 0; x < 20; ++x) A.at(i, x)[c] = acc[x];
    }
}

// One wave per atom row, lane L owning channels 4L .. 4L + 3 (C <= 256): float4 loads of R and
// the messages, the edge's Y row, envelope and message row through scalar loads (wave-uniform
// addresses), no LDS and no barrier; the next edge's vector loads are issued before the current
// edge's products.
constexpr int kCpfWaves = 4;

__global__ __launch_bounds__(kCpfWaves * kWave) void cp_density_fwd_wave_kernel(
    const float* __restrict__ R, int ld_R, const float* __restrict__ env, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int64_t N, int M, int C, RankOut A) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t i = (int64_t)blockIdx.x * kCpfWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (i >= N) return;
    const int c = 4 * (lane < C / 4 ? lane : C / 4 - 1);    // lanes past C / 4 repeat the last quad
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    v4f acc[20];
#pragma unroll
    for (int x = 0; x < 20; ++x) acc[x] = z4;
    int64_t e0, e1;
    row_range(row_ptr, i, M, e0, e1);
    if (e1 > e0) {
        auto load = [&](int64_t e, v4f (&r)[4], v4f& m) __attribute__((always_inline)) {
            const float* Re = R + e * ld_R + c;
#pragma unroll
            for (int l = 0; l < 4; ++l) r[l] = ld4(Re + l * C);
            const int64_t row = msg_row ? (int64_t)msg_row[e] : e;
            m = ld4(msg + row * ld_msg + c);
        };
        v4f r[4], m, rn[4], mn;
        load(e0, r, m);
        for (int64_t e = e0; e < e1; ++e) {
            load(e + 1 < e1 ? e + 1 : e, rn, mn);
            float y[20];
#pragma unroll
            for (int x = 0; x < 20; ++x) y[x] = Y[e * ld_Y + x];
            const float ev = env ? env[e] : 1.f;
            const v4f me = m * ev;
            const v4f w0 = r[0] * me, w1 = r[1] * me, w2 = r[2] * me, w3 = r[3] * me;
            acc[0] += w0 * y[0];
#pragma unroll
            for (int x = 1; x < 4; ++x) acc[x] += w1 * y[x];
#pragma unroll
            for (int x = 4; x < 10; ++x) acc[x] += w2 * y[x];
#pragma unroll
            for (int x = 10; x < 20; ++x) acc[x] += w3 * y[x];
#pragma unroll
            for (int l = 0; l < 4; ++l) r[l] = rn[l];
            m = mn;
        }
    }
    if (lane < C / 4) {
#pragma unroll
        for (int x = 0; x < 20; ++x) st4(A.at(i, x) + c, acc[x]);
    }
}

// ------------------------------------------------------------------ CP backward
// Workgroup = atom i, one thread per channel (C <= 256); gA[i] sits in registers (channel
// view) and in LDS (monomial view). Per tile of edges:
//   channel phase:  t_l = sum_{x in l} gA[x,c] Y[e,x];   dR[e,l,c] = env m t_l;
//                   dmsg[e,c] = env sum_l R[e,l,c] t_l;   w[e,l,c] = R m -> LDS
//   monomial phase: P[e,x] = sum_c gA[x,c] w[e,l(x),c]   (lane = (edge pair, x), float4 walks)
//                   dY[e,x] = env P[e,x];  denv[e] = sum_x Y[e,x] P[e,x]
constexpr int kTileCPB = 8;

__global__ __launch_bounds__(kBlock) void cp_density_bwd_kernel(
    const float* __restrict__ R, int ld_R, const float* __restrict__ env, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int M, int C, RankIn gA, float* __restrict__ dR, int ld_dR, float* __restrict__ dmsg, int ld_dmsg,
    float* __restrict__ dY, int ld_dY, float* __restrict__ denv) {
    extern __shared__ float lds[];
    const int CS = ((C + 3) & ~3) + 4;           // row stride: float4-aligned, staggered banks
    float* s_g = lds;                            // 20 x CS
    float* s_w = s_g + 20 * CS;                  // kTileCPB*4 x CS
    float* s_Y = s_w + kTileCPB * 4 * CS;        // kTileCPB x 20
    float* s_P = s_Y + kTileCPB * 20;            // kTileCPB x 20
    float* s_env = s_P + kTileCPB * 20;          // kTileCPB
    const int64_t i = blockIdx.x;
    const int tid = threadIdx.x, nthr = blockDim.x;
    for (int q = tid; q < 20 * CS; q += nthr) {
        const int x = q / CS, c = q - x * CS;
        s_g[q] = c < C ? gA.at(i, x)[c] : 0.f;
    }
    for (int q = tid; q < kTileCPB * 4 * CS; q += nthr) s_w[q] = 0.f;   // padding columns stay zero
    const int c = tid;
    const bool ok = c < C;
    float g[20];
#pragma unroll
    for (int x = 0; x < 20; ++x) g[x] = ok ? gA.at(i, x)[c] : 0.f;
    const int nc4 = (C + 3) >> 2;
    int64_t e0, e1;
    row_range(row_ptr, i, M, e0, e1);
    for (int64_t t0 = e0; t0 < e1; t0 += kTileCPB) {
        const int nt = (int)min((int64_t)kTileCPB, e1 - t0);
        for (int q = tid; q < nt * 20; q += nthr) {
            const int t = q / 20;
            s_Y[q] = Y[(t0 + t) * ld_Y + (q - t * 20)];
        }
        if (tid < nt) s_env[tid] = env ? env[t0 + tid] : 1.f;
        __syncthreads();
        if (ok) {
            float rv[kTileCPB][4], mv[kTileCPB];
#pragma unroll
            for (int t = 0; t < kTileCPB; ++t) {        // every load of the tile in flight at once
                if (t < nt) {
                    const int64_t e = t0 + t;
                    const int64_t row = msg_row ? (int64_t)msg_row[e] : e;
                    mv[t] = msg[row * ld_msg + c];
                    const float* Re = R + e * ld_R + c;
                    rv[t][0] = Re[0];
                    rv[t][1] = Re[C];
                    rv[t][2] = Re[2 * C];
                    rv[t][3] = Re[3 * C];
                }
            }
#pragma unroll
            for (int t = 0; t < kTileCPB; ++t) {
                if (t >= nt) break;
                const int64_t e = t0 + t;
                const float m = mv[t];
                const float ev = s_env[t];
                const float r0 = rv[t][0], r1 = rv[t][1], r2 = rv[t][2], r3 = rv[t][3];
                const float* y = s_Y + t * 20;
                float t0v = g[0] * y[0], t1v = 0.f, t2v = 0.f, t3v = 0.f;
#pragma unroll
                for (int x = 1; x < 4; ++x) t1v = fmaf(g[x], y[x], t1v);
#pragma unroll
                for (int x = 4; x < 10; ++x) t2v = fmaf(g[x], y[x], t2v);
#pragma unroll
                for (int x = 10; x < 20; ++x) t3v = fmaf(g[x], y[x], t3v);
                if (dR) {
                    const float em = ev * m;
                    float* dRe = dR + e * ld_dR + c;
                    dRe[0] = em * t0v;
                    dRe[C] = em * t1v;
                    dRe[2 * C] = em * t2v;
                    dRe[3 * C] = em * t3v;
                }
                if (dmsg) dmsg[e * ld_dmsg + c] = ev * (r0 * t0v + r1 * t1v + r2 * t2v + r3 * t3v);
                float* w = s_w + (t * 4) * CS + c;
                w[0] = r0 * m;
                w[CS] = r1 * m;
                w[2 * CS] = r2 * m;
                w[3 * CS] = r3 * m;
            }
        }
        __syncthreads();
        if (dY || denv) {
            const int npair = (nt + 1) >> 1;
            for (int q = tid; q < npair * 20; q += nthr) {
                const int tp = q / 20, x = q - tp * 20;
                const int ta = 2 * tp, tb = ta + 1;
                const int l = rank_of(x);
                const float4* gx = reinterpret_cast<const float4*>(s_g + x * CS);
                const float4* wa = reinterpret_cast<const float4*>(s_w + (ta * 4 + l) * CS);
                const float4* wb = reinterpret_cast<const float4*>(s_w + ((tb < nt ? tb : ta) * 4 + l) * CS);
                float sa = 0.f, sb = 0.f;
                for (int c4 = 0; c4 < nc4; ++c4) {
                    const float4 gv = gx[c4], av = wa[c4], bv = wb[c4];
                    sa = fmaf(gv.x, av.x, sa); sa = fmaf(gv.y, av.y, sa); sa = fmaf(gv.z, av.z, sa); sa = fmaf(gv.w, av.w, sa);
                    sb = fmaf(gv.x, bv.x, sb); sb = fmaf(gv.y, bv.y, sb); sb = fmaf(gv.z, bv.z, sb); sb = fmaf(gv.w, bv.w, sb);
                }
                s_P[ta * 20 + x] = sa;
                if (dY) dY[(t0 + ta) * ld_dY + x] = s_env[ta] * sa;
                if (tb < nt) {
                    s_P[tb * 20 + x] = sb;
                    if (dY) dY[(t0 + tb) * ld_dY + x] = s_env[tb] * sb;
                }
            }
            __syncthreads();
            if (denv && tid < nt) {
                float s = 0.f;
#pragma unroll
                for (int x = 0; x < 20; ++x) s = fmaf(s_Y[tid * 20 + x], s_P[tid * 20 + x], s);
                denv[t0 + tid] = s;
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------ CP backward on MFMA
// One wave per atom row, no workgroup barriers. The row is walked in tiles of 16 edges and,
// inside a tile, in steps of 32 channels (two 16-channel MFMA blocks h); both contractions
// run on v_mfma_f32_16x16x4f32:
//   t_l[c, e] = sum_{x in l} gA[x, c] Y[e, x]         (M = channels, N = edges, K = monomials)
//   P[x, e]   = sum_c gA[x, c] R[e, l(x), c] msg[e, c] (M = monomials, N = edges, K = channels)
// Operand layouts of the 16x16x4 f32 instruction: A[i][k] in lane i + 16k, B[k][j] in lane
// j + 16k, D[4q + r][j] in register r of lane j + 16q. Lane (j, q) therefore holds t for edge
// j and channels 16h + 4q + r, which is where it loads R / msg as float4 and writes dR / dmsg
// (each wave-wide access covers 64 contiguous bytes per edge), and register r of R*msg is the
// B operand of the P chain with K index = channel 16h + 4q + r.
// P rows: accumulator lo holds x = 0..3 (rank 0 in row 0, rank 1 in rows 1-3), hi holds
// x = 4..19 (rank 2 in rows 0-5, rank 3 in rows 6-15); each chain alternates the two ranks it
// serves, with the A operand zeroed outside the rank's rows. The atom's gA (20 x C) is staged
// in the wave's own LDS slice.
// Monomial chunks of the t contraction (K = 4 per instruction): chunk k covers
// x = kChunkX0[k] + q for q < kChunkLen[k], rank kChunkRank[k]; rank l owns chunks
// [kRankChunk0[l], kRankChunk1[l]).
__device__ constexpr int kChunkX0[7] = {0, 1, 4, 8, 10, 14, 18};
__device__ constexpr int kChunkLen[7] = {1, 3, 4, 2, 4, 4, 2};
__device__ constexpr int kRankChunk0[4] = {0, 1, 2, 4};
__device__ constexpr int kRankChunk1[4] = {1, 2, 4, 7};

constexpr int kCpStep = 32;                           // channels per step (C % kCpStep == 0)
constexpr int kCpRowsPerBlock = 2;                    // waves (= atom rows) per workgroup
// LDS row stride of the staged gA (floats).
__host__ __device__ constexpr int cp_mfma_stride(int C) { return C + 4; }

__global__ __launch_bounds__(kCpRowsPerBlock * kWave) __attribute__((amdgpu_waves_per_eu(2))) void cp_density_bwd_mfma_kernel(
    const float* __restrict__ R, int ld_R, const float* __restrict__ env, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int64_t N, int M, int C, RankIn gA, float* __restrict__ dR, int ld_dR, float* __restrict__ dmsg, int ld_dmsg,
    float* __restrict__ dY, int ld_dY, float* __restrict__ denv) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int w = threadIdx.x / kWave;
    const int64_t i = (int64_t)blockIdx.x * kCpRowsPerBlock + w;
    if (i >= N) return;                               // uniform per wave
    const int GS = cp_mfma_stride(C);
    float* sg = lds + (size_t)w * 20 * GS;
    const int j = lane & 15, q = lane >> 4;
    const int nc4 = C >> 2;
    // stage gA[i]: up to 4 float4 per lane in flight per batch
    for (int v0 = 0; v0 < 20 * nc4; v0 += 4 * kWave) {
        v4f buf[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int v = v0 + u * kWave + lane;
            if (v < 20 * nc4) {
                const int x = v / nc4, c4 = v - x * nc4;
                buf[u] = ld4(gA.at(i, x) + 4 * c4);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int v = v0 + u * kWave + lane;
            if (v < 20 * nc4) {
                const int x = v / nc4, c4 = v - x * nc4;
                *reinterpret_cast<v4f*>(sg + x * GS + 4 * c4) = buf[u];
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    const int t_off = q * GS + j;                     // + kChunkX0[k] * GS + channel block start
    const int own = 4 * q;                            // + channel block start
    const int plo_off = (j < 4 ? j : 0) * GS + own, phi_off = (4 + j) * GS + own;
    const float sel0 = j == 0 ? 1.f : 0.f, sel1 = (j >= 1 && j < 4) ? 1.f : 0.f;
    const float sel2 = j < 6 ? 1.f : 0.f, sel3 = j >= 6 ? 1.f : 0.f;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    int64_t e0, e1;
    row_range(row_ptr, i, M, e0, e1);
    for (int64_t t0 = e0; t0 < e1; t0 += 16) {
        const int64_t e = t0 + j;
        const bool ok = e < e1;
        float yq[7];
#pragma unroll
        for (int k = 0; k < 7; ++k) yq[k] = (ok && q < kChunkLen[k]) ? Y[e * ld_Y + kChunkX0[k] + q] : 0.f;
        const float ev = ok ? (env ? env[e] : 1.f) : 0.f;
        const int64_t mrow = ok ? (msg_row ? (int64_t)msg_row[e] : e) : 0;
        const float* Re = R + e * ld_R + own;
        const float* me = msg + mrow * ld_msg + own;
        v4f plo = z4, phi = z4;
#pragma unroll 1
        for (int cs = 0; cs < C; cs += kCpStep) {
            v4f r[2][4], m[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int l = 0; l < 4; ++l) r[h][l] = ok ? ld4(Re + l * C + cs + 16 * h) : z4;
                m[h] = ok ? ld4(me + cs + 16 * h) : z4;
            }
            v4f dm[2] = {z4, z4};
#pragma unroll
            for (int l = 0; l < 4; ++l) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    v4f t = z4;
#pragma unroll
                    for (int k = kRankChunk0[l]; k < kRankChunk1[l]; ++k) {
                        const float a = q < kChunkLen[k] ? sg[t_off + kChunkX0[k] * GS + cs + 16 * h] : 0.f;
                        t = mfma_16x16x4(a, yq[k], t);
                    }
                    if (ok && dR) st4(dR + e * ld_dR + l * C + cs + own + 16 * h, (ev * m[h]) * t);
                    dm[h] += r[h][l] * t;
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (ok && dmsg) st4(dmsg + e * ld_dmsg + cs + own + 16 * h, ev * dm[h]);
                const v4f alo = *reinterpret_cast<const v4f*>(sg + plo_off + cs + 16 * h);
                const v4f ahi = *reinterpret_cast<const v4f*>(sg + phi_off + cs + 16 * h);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const float mm = m[h][rr];
                    plo = mfma_16x16x4(sel0 * alo[rr], r[h][0][rr] * mm, plo);
                    phi = mfma_16x16x4(sel2 * ahi[rr], r[h][2][rr] * mm, phi);
                    plo = mfma_16x16x4(sel1 * alo[rr], r[h][1][rr] * mm, plo);
                    phi = mfma_16x16x4(sel3 * ahi[rr], r[h][3][rr] * mm, phi);
                }
            }
        }
        // lane (j, q) holds P[x, e] for x = 4 + 4q + r (hi) and, in lanes q == 0, x = r (lo)
        float s = 0.f;
        if (ok) {
            const v4f yhi = ld4(Y + e * ld_Y + 4 + 4 * q);
            s = yhi[0] * phi[0] + yhi[1] * phi[1] + yhi[2] * phi[2] + yhi[3] * phi[3];
            if (dY) st4(dY + e * ld_dY + 4 + 4 * q, ev * phi);
            if (q == 0) {
                const v4f ylo = ld4(Y + e * ld_Y);
                s += ylo[0] * plo[0] + ylo[1] * plo[1] + ylo[2] * plo[2] + ylo[3] * plo[3];
                if (dY) st4(dY + e * ld_dY, ev * plo);
            }
        }
        s += __shfl_xor(s, 16, kWave);
        s += __shfl_xor(s, 32, kWave);
        if (denv && ok && q == 0) denv[e] = s;
    }
}

// ------------------------------------------------------------------ CP radial backward, shared W
// The pooling backward of cp_density_bwd_mfma_kernel fused with the CP columns of the last radial
// layer: instead of writing dR, multiply it by W on the matrix cores, dh2[e, h] = sum_{l,c}
// dR[e, l, c] W[l C + c, h] for 16 HB hidden units, w_t = W^T (16 HB, 4C) row-major (M = edges,
// N = hidden units, K = (rank, channel): the t registers scaled to dR are the A operand and D
// rows are edges 4q + r). W is read from LDS:
// persistent workgroups of kLdsWaves waves, each wave walking the 16-edge tiles of its own rows
// (rows gw, gw + waves, ...), one tile per round; all waves of a workgroup step through the
// 32-channel steps of their tiles in lockstep, and the step's slab of W^T (all hidden units x
// 4 ranks x 32 channels, row stride 132 floats so that the float4 operand reads of 8
// consecutive lanes hit distinct banks) is staged once per workgroup, the next slab being
// fetched into registers while the current step computes. Every wave runs the workgroup's
// largest round count, so every barrier is reached by all waves.
constexpr int kLdsWaves = 8;
constexpr int kSlabRS = 4 * kCpStep + 4;              // slab row stride (floats) per hidden unit

template <int HB>
__global__ __launch_bounds__(kLdsWaves * kWave) void cp_radial_bwd_lds_kernel(
    const float* __restrict__ R, int ld_R, const float* __restrict__ env, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int64_t N, int M, int C, RankIn gA, float* __restrict__ dmsg, int ld_dmsg, float* __restrict__ dY, int ld_dY,
    float* __restrict__ denv, const float* __restrict__ w_t, float* __restrict__ dh2, int ld_dh2) {
    constexpr int H = 16 * HB;
    extern __shared__ float lds[];
    const int GS = cp_mfma_stride(C);
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    float* sW = lds;                                                  // H x kSlabRS
    float* sg = lds + H * kSlabRS + (size_t)w * 20 * GS;             // this wave's gA row
    int* s_cnt = reinterpret_cast<int*>(lds + H * kSlabRS + (size_t)kLdsWaves * 20 * GS);
    const int64_t stride = (int64_t)gridDim.x * kLdsWaves;
    const int64_t gw = (int64_t)blockIdx.x * kLdsWaves + w;
    // rounds = the largest tile count over the workgroup's waves
    int my_tiles = 0;
    for (int64_t i = gw; i < N; i += stride) {
        int64_t a, b;
        row_range(row_ptr, i, M, a, b);
        my_tiles += (int)((b - a + 15) / 16);
    }
    if (lane == 0) s_cnt[w] = my_tiles;
    __syncthreads();
    int rounds = 0;
#pragma unroll
    for (int k = 0; k < kLdsWaves; ++k) rounds = max(rounds, s_cnt[k]);
    const int nsteps = C / kCpStep;
    // W slab fetch: the slab is H x 4 ranks x 8 float4; thread tid owns float4 u * blockDim + tid
    static_assert(HB * 16 * 4 * (kCpStep / 4) == HB * kLdsWaves * kWave, "slab float4s = HB per thread");
    auto slab_load = [&](int cs, v4f (&buf)[HB]) {
#pragma unroll
        for (int u = 0; u < HB; ++u) {
            const int f = u * kLdsWaves * kWave + tid;
            const int h = f >> 5, l = (f >> 3) & 3, c4 = f & 7;
            buf[u] = ld4(w_t + (int64_t)h * 4 * C + l * C + cs + 4 * c4);
        }
    };
    auto slab_store = [&](const v4f (&buf)[HB]) {
#pragma unroll
        for (int u = 0; u < HB; ++u) {
            const int f = u * kLdsWaves * kWave + tid;
            const int h = f >> 5, l = (f >> 3) & 3, c4 = f & 7;
            *reinterpret_cast<v4f*>(sW + h * kSlabRS + l * kCpStep + 4 * c4) = buf[u];
        }
    };
    v4f wbuf[HB];
    slab_load(0, wbuf);
    const int j = lane & 15, q = lane >> 4;
    const int nc4 = C >> 2;
    const int t_off = q * GS + j, own = 4 * q;
    const int plo_off = (j < 4 ? j : 0) * GS + own, phi_off = (4 + j) * GS + own;
    const float sel0 = j == 0 ? 1.f : 0.f, sel1 = (j >= 1 && j < 4) ? 1.f : 0.f;
    const float sel2 = j < 6 ? 1.f : 0.f, sel3 = j >= 6 ? 1.f : 0.f;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    int64_t row = gw - stride, t_next = 0, e_end = 0;   // tile cursor of this wave
    for (int rd = 0; rd < rounds; ++rd) {
        const bool active = rd < my_tiles;
        int64_t t0 = 0, e1 = 0;
        if (active) {
            if (t_next >= e_end) {                        // next row with edges; stage its gA
                int64_t a, b;
                do {
                    row += stride;
                    row_range(row_ptr, row, M, a, b);
                } while (b <= a);
                t_next = a;
                e_end = b;
                for (int v0 = 0; v0 < 20 * nc4; v0 += 4 * kWave) {
                    v4f buf[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int v = v0 + u * kWave + lane;
                        if (v < 20 * nc4) {
                            const int x = v / nc4, c4 = v - x * nc4;
                            buf[u] = ld4(gA.at(row, x) + 4 * c4);
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int v = v0 + u * kWave + lane;
                        if (v < 20 * nc4) {
                            const int x = v / nc4, c4 = v - x * nc4;
                            *reinterpret_cast<v4f*>(sg + x * GS + 4 * c4) = buf[u];
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            t0 = t_next;
            e1 = e_end;
            t_next += 16;
        }
        const int64_t e = t0 + j;
        const bool ok = active && e < e1;
        float yq[7];
#pragma unroll
        for (int k = 0; k < 7; ++k) yq[k] = (ok && q < kChunkLen[k]) ? Y[e * ld_Y + kChunkX0[k] + q] : 0.f;
        const float ev = ok ? (env ? env[e] : 1.f) : 0.f;
        const int64_t mrow = ok ? (msg_row ? (int64_t)msg_row[e] : e) : 0;
        const float* Re = R + (ok ? e : 0) * ld_R + own;
        const float* me = msg + mrow * ld_msg + own;
        v4f plo = z4, phi = z4;
        v4f dacc[HB];
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) dacc[hb] = z4;
        v4f rn[2][4], mn[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int l = 0; l < 4; ++l) rn[h][l] = ok ? ld4(Re + l * C + 16 * h) : z4;
            mn[h] = ok ? ld4(me + 16 * h) : z4;
        }
#pragma unroll 1
        for (int st = 0; st < nsteps; ++st) {
            const int cs = st * kCpStep;
            __syncthreads();                              // every wave is done with the previous slab
            slab_store(wbuf);
            __syncthreads();
            const bool more = st + 1 < nsteps || rd + 1 < rounds;
            if (more) slab_load(st + 1 < nsteps ? cs + kCpStep : 0, wbuf);
            v4f r[2][4], m[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                m[h] = mn[h];
#pragma unroll
                for (int l = 0; l < 4; ++l) r[h][l] = rn[h][l];
            }
            if (st + 1 < nsteps) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int l = 0; l < 4; ++l) rn[h][l] = ok ? ld4(Re + l * C + cs + kCpStep + 16 * h) : z4;
                    mn[h] = ok ? ld4(me + cs + kCpStep + 16 * h) : z4;
                }
            }
            if (active) {
                // t for every (rank, half) first, so no MFMA result is read right after its issue;
                // the chunk operands are read unmasked: yq is 0 on the lanes past a chunk's length
                // (only the last chunk's rows run past monomial 19 and are clamped to it)
                v4f tt[4][2];
#pragma unroll
                for (int l = 0; l < 4; ++l)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        v4f t = z4;
#pragma unroll
                        for (int k = kRankChunk0[l]; k < kRankChunk1[l]; ++k) {
                            const int xr = kChunkX0[k] + 3 < 20 ? t_off + kChunkX0[k] * GS
                                                                 : min(kChunkX0[k] + q, 19) * GS + j;
                            t = mfma_16x16x4(sg[xr + cs + 16 * h], yq[k], t);
                        }
                        tt[l][h] = t;
                    }
                v4f dm[2] = {z4, z4};
#pragma unroll
                for (int l = 0; l < 4; ++l) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const v4f t = tt[l][h];
                        const v4f g = (ev * m[h]) * t;
                        const float* wl = sW + j * kSlabRS + l * kCpStep + 16 * h + own;
#pragma unroll
                        for (int hb = 0; hb < HB; ++hb) {
                            const v4f wv = *reinterpret_cast<const v4f*>(wl + hb * 16 * kSlabRS);
#pragma unroll
                            for (int rr = 0; rr < 4; ++rr) dacc[hb] = mfma_16x16x4(g[rr], wv[rr], dacc[hb]);
                        }
                        dm[h] += r[h][l] * t;
                    }
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    if (ok && dmsg) st4(dmsg + e * ld_dmsg + cs + own + 16 * h, ev * dm[h]);
                    const v4f alo = *reinterpret_cast<const v4f*>(sg + plo_off + cs + 16 * h);
                    const v4f ahi = *reinterpret_cast<const v4f*>(sg + phi_off + cs + 16 * h);
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const float mm = m[h][rr];
                        plo = mfma_16x16x4(sel0 * alo[rr], r[h][0][rr] * mm, plo);
                        phi = mfma_16x16x4(sel2 * ahi[rr], r[h][2][rr] * mm, phi);
                        plo = mfma_16x16x4(sel1 * alo[rr], r[h][1][rr] * mm, plo);
                        phi = mfma_16x16x4(sel3 * ahi[rr], r[h][3][rr] * mm, phi);
                    }
                }
            }
        }
        if (active) {
            // lane (j, q) holds P[x, e] for x = 4 + 4q + r (hi) and, in lanes q == 0, x = r (lo)
            float s = 0.f;
            if (ok) {
                const v4f yhi = ld4(Y + e * ld_Y + 4 + 4 * q);
                s = yhi[0] * phi[0] + yhi[1] * phi[1] + yhi[2] * phi[2] + yhi[3] * phi[3];
                if (dY) st4(dY + e * ld_dY + 4 + 4 * q, ev * phi);
                if (q == 0) {
                    const v4f ylo = ld4(Y + e * ld_Y);
                    s += ylo[0] * plo[0] + ylo[1] * plo[1] + ylo[2] * plo[2] + ylo[3] * plo[3];
                    if (dY) st4(dY + e * ld_dY, ev * plo);
                }
            }
            s += __shfl_xor(s, 16, kWave);
            s += __shfl_xor(s, 32, kWave);
            if (denv && ok && q == 0) denv[e] = s;
            // dacc[hb] register r of lane (j, q): edge t0 + 4q + r, hidden unit 16 hb + j
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int64_t er = t0 + 4 * q + rr;
                if (er < e1) {
#pragma unroll
                    for (int hb = 0; hb < HB; ++hb) dh2[er * ld_dh2 + 16 * hb + j] = dacc[hb][rr];
                }
            }
        }
    }
}

// ------------------------------------------------------------------ CP radial backward, resident W
// The product of cp_radial_bwd_lds_kernel when all of W^T (H x 4C) fits in LDS: W^T is staged
// once per workgroup (rows unpadded, float4 chunk c of row h stored at chunk c ^ (h & 15), so the
// 16 rows read by one instruction fall on distinct banks) and every wave then works alone, with
// no workgroup barrier: wave w owns the atom rows whose first edge lies in the w-th equal share
// of the edges, walks their 16-edge tiles in 16-channel steps, reads gA straight from memory and
// loads the next step's operands while the current step computes. Lane (j, q) holds channels
// c0 + 4q .. c0 + 4q + 3 of edge j of the tile for R, m, t and dR; the dh2 accumulator D rows
// are edges 4q + r, columns hidden units 16 hb + j.
constexpr int kResStep = 16;                          // channels per step (C % kResStep == 0)
// rank of the monomials of chunk k (kChunkX0 / kChunkLen)
__device__ constexpr int kChunkRank[7] = {0, 1, 2, 2, 3, 3, 3};

// Smallest r in [0, n] with a[r] >= target (a nondecreasing, a[n] >= target), the 64 lanes of
// the wave probing 64 points per pass; the result is wave-uniform.
__device__ __forceinline__ int64_t wave_lower_bound(const int32_t* __restrict__ a, int64_t n, int64_t target,
                                                    int lane) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t step = (hi - lo + kWave - 1) / kWave;
        const int64_t p = min(lo + (int64_t)lane * step, hi);
        const uint64_t m = __ballot(a[p] >= target);      // a[hi] >= target: clamped probes are true
        if (m == 0) {
            lo += (int64_t)(kWave - 1) * step + 1;
        } else {
            const int f = __ffsll((unsigned long long)m) - 1;
            const int64_t pf = min(lo + (int64_t)f * step, hi);
            if (f > 0) lo += (int64_t)(f - 1) * step + 1;
            hi = pf;
        }
    }
    return lo < n ? lo : n;
}

// A wave-uniform 64-bit value held in scalar registers.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <int HB, int NW>
__global__ __launch_bounds__(NW * kWave) void cp_radial_bwd_res_kernel(
    const float* __restrict__ R, int ld_R, const float* __restrict__ env, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int64_t N, int M, int C, RankIn gA, float* __restrict__ dmsg, int ld_dmsg, float* __restrict__ dY, int ld_dY,
    float* __restrict__ denv, const float* __restrict__ w_t, float* __restrict__ dh2, int ld_dh2) {
    constexpr int H = 16 * HB;
    extern __shared__ float lds[];                    // W^T image, H rows of 4C floats
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int j = lane & 15, q = lane >> 4;
    const int RS = 4 * C, nch = C;
    stage4<8>(
        H * nch, [&](int f) { return ld4(w_t + 4 * (int64_t)f); },
        [&](int f, v4f x) {
            const int h = f / nch, c = f - h * nch;
            st4(lds + h * RS + 4 * (c ^ (h & 15)), x);
        });
    __syncthreads();
    // this wave's rows: those whose first edge lies in its share of the edges
    const int64_t W = (int64_t)gridDim.x * NW;
    const int64_t gw = (int64_t)blockIdx.x * NW + __builtin_amdgcn_readfirstlane(tid / kWave);
    int64_t row, row_end;
    if (row_ptr) {
        const int64_t E = row_ptr[N];
        row = wave_lower_bound(row_ptr, N, E * gw / W, lane);
        row_end = wave_lower_bound(row_ptr, N, E * (gw + 1) / W, lane);
    } else {
        row = N * gw / W;
        row_end = N * (gw + 1) / W;
    }
    row = uniform64(row);
    row_end = uniform64(row_end);
    const int nsteps = C / kResStep;
    // per-lane monomial offsets (within the rank's block) of the t operands of the 7 chunks
    // (lanes past a chunk's length read its first monomial; their Y factor is 0) and of the
    // dY product rows x = j (j < 4, else 0) and x = 4 + j
    // (32-bit element offsets from the rank block's row start: the host checks 19 sx + C < 2^31)
    int toff[7];
#pragma unroll
    for (int k = 0; k < 7; ++k)
        toff[k] = ((q < kChunkLen[k] ? q : 0) + kChunkX0[k] - rank_start(kChunkRank[k])) * (int)gA.sx + j;
    const int xlo = j < 4 ? j : 0, xhi = 4 + j;
    const float sel0 = j == 0 ? 1.f : 0.f, sel1 = (j >= 1 && j < 4) ? 1.f : 0.f;
    const float sel2 = j < 6 ? 1.f : 0.f, sel3 = j >= 6 ? 1.f : 0.f;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    const int own = 4 * q;

    // operands of one (tile, step): R of the 4 ranks, m, the 7 t operands, the dY product rows
    struct Slot {
        v4f r[4], m, alo, ahi;
        float ta[7];
    };
    auto load_slot = [&](int64_t rw, int64_t eld, int64_t mr, int st, Slot& s) {
        const int c0 = st * kResStep;
        const float* Re = R + eld * ld_R + c0 + own;
#pragma unroll
        for (int l = 0; l < 4; ++l) s.r[l] = ld4(Re + l * C);
        s.m = ld4(msg + mr * ld_msg + c0 + own);
#pragma unroll
        for (int k = 0; k < 7; ++k) s.ta[k] = (gA.p[kChunkRank[k]] + rw * gA.sa + c0)[toff[k]];
        s.alo = ld4(gA.at(rw, xlo) + c0 + own);
        s.ahi = ld4(gA.at(rw, xhi) + c0 + own);
    };
    // per-tile values: Y factors of the chunks, Y rows x = 4 + 4q .. and x = 0 .. 3 for the dY
    // product, envelope, message row
    struct Head {
        float yq[7], ev;
        v4f yhi, ylo;
        int64_t eld, mr;
        bool ok;
    };
    auto load_head = [&](int64_t t0, int64_t e1, Head& h) {
        const int64_t e = t0 + j;
        h.ok = e < e1;
        h.eld = h.ok ? e : e1 - 1;
#pragma unroll
        for (int k = 0; k < 7; ++k) h.yq[k] = (h.ok && q < kChunkLen[k]) ? Y[h.eld * ld_Y + kChunkX0[k] + q] : 0.f;
        h.ev = h.ok ? (env ? env[h.eld] : 1.f) : 0.f;
        h.mr = msg_row ? (int64_t)msg_row[h.eld] : h.eld;
        h.yhi = ld4(Y + h.eld * ld_Y + 4 + 4 * q);
        h.ylo = ld4(Y + h.eld * ld_Y);
    };
    // tile cursor: (rw, t0, e1) -> the next tile of this wave's rows; false when none is left
    auto next_tile = [&](int64_t& rw, int64_t& t0, int64_t& e1) -> bool {
        if (t0 + 16 < e1) {
            t0 += 16;
            return true;
        }
        while (++rw < row_end) {
            int64_t a, b;
            row_range(row_ptr, rw, M, a, b);
            if (b > a) {
                t0 = a;
                e1 = b;
                return true;
            }
        }
        return false;
    };

    int64_t rw = row - 1, t0 = 0, e1 = 0;
    if (!next_tile(rw, t0, e1)) return;
    Head hd, hn;
    load_head(t0, e1, hd);
    Slot sa, sb;
    load_slot(rw, hd.eld, hd.mr, 0, sa);
    int64_t nrw = rw, nt0 = t0, ne1 = e1;             // the tile after the current one
    bool more = next_tile(nrw, nt0, ne1);
    if (more)
        load_head(nt0, ne1, hn);
    else
        hn = hd;
    v4f dacc[HB];
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) dacc[hb] = z4;
    v4f plo = z4, phi = z4;
    int st = 0;
    // One (tile, step) computed on `cu` while the following one is loaded into `nx`: the next
    // step of this tile, else step 0 of the next tile (this tile's step 0 again, unused, when
    // none is left), so that the loads are issued on every path and the two buffers alternate
    // without copies. False when this wave's last tile is done.
    auto step = [&](Slot& cu, Slot& nx) __attribute__((always_inline)) -> bool {
        const bool last = st + 1 == nsteps;
        const bool to_next = last && more;
        load_slot(to_next ? nrw : rw, to_next ? hn.eld : hd.eld, to_next ? hn.mr : hd.mr, last ? 0 : st + 1, nx);
        __builtin_amdgcn_sched_barrier(0);           // keep the loads ahead of this step's work
        const int c0 = st * kResStep;
        const int64_t e = t0 + j;
        // P[x, e] = sum_c gA[x, c] R_{l(x)}[e, c] m[e, c] for the dY rows (first: it needs only
        // loaded operands, and covers the latency of the t products below)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float mm = cu.m[rr];
            plo = mfma_16x16x4(sel0 * cu.alo[rr], cu.r[0][rr] * mm, plo);
            phi = mfma_16x16x4(sel2 * cu.ahi[rr], cu.r[2][rr] * mm, phi);
            plo = mfma_16x16x4(sel1 * cu.alo[rr], cu.r[1][rr] * mm, plo);
            phi = mfma_16x16x4(sel3 * cu.ahi[rr], cu.r[3][rr] * mm, phi);
        }
        // t_l[c, e] = sum_{x in rank l} gA[x, c] Y[e, x]
        v4f tt[4];
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            v4f t = z4;
#pragma unroll
            for (int k = kRankChunk0[l]; k < kRankChunk1[l]; ++k) t = mfma_16x16x4(cu.ta[k], hd.yq[k], t);
            tt[l] = t;
        }
        // dR_l = ev m t_l; dh2 += dR_l W_l^T; dm = sum_l R_l t_l (the W^T operands of rank l + 1
        // are read while rank l's products issue)
        v4f dm = z4;
        v4f wv[2][HB];
        auto read_w = [&](int l, v4f (&w)[HB]) __attribute__((always_inline)) {
            const int c4 = ((l * C + c0) >> 2) + q;
#pragma unroll
            for (int hb = 0; hb < HB; ++hb) w[hb] = ld4(lds + (16 * hb + j) * RS + 4 * (c4 ^ j));
        };
        read_w(0, wv[0]);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            if (l < 3) read_w(l + 1, wv[(l + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            const v4f g = (hd.ev * cu.m) * tt[l];
#pragma unroll
            for (int hb = 0; hb < HB; ++hb)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) dacc[hb] = mfma_16x16x4(g[rr], wv[l & 1][hb][rr], dacc[hb]);
            dm += cu.r[l] * tt[l];
        }
        if (hd.ok && dmsg) st4(dmsg + e * ld_dmsg + c0 + own, hd.ev * dm);
        if (!last) {
            ++st;
            return true;
        }
        // tile done: lane (j, q) holds P[x, e] for x = 4 + 4q + r (hi) and, in lanes q == 0,
        // x = r (lo)
        float s = 0.f;
        if (hd.ok) {
            const v4f yhi = hd.yhi, ylo = hd.ylo;
            s = yhi[0] * phi[0] + yhi[1] * phi[1] + yhi[2] * phi[2] + yhi[3] * phi[3];
            if (dY) st4(dY + e * ld_dY + 4 + 4 * q, hd.ev * phi);
            if (q == 0) {
                s += ylo[0] * plo[0] + ylo[1] * plo[1] + ylo[2] * plo[2] + ylo[3] * plo[3];
                if (dY) st4(dY + e * ld_dY, hd.ev * plo);
            }
        }
        s += __shfl_xor(s, 16, kWave);
        s += __shfl_xor(s, 32, kWave);
        if (denv && hd.ok && q == 0) denv[e] = s;
        // dacc[hb] register r of lane (j, q): edge t0 + 4q + r, hidden unit 16 hb + j
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int64_t er = t0 + 4 * q + rr;
            if (er < e1) {
#pragma unroll
                for (int hb = 0; hb < HB; ++hb) dh2[er * ld_dh2 + 16 * hb + j] = dacc[hb][rr];
            }
        }
        if (!more) return false;
        rw = nrw, t0 = nt0, e1 = ne1;
        hd = hn;
        more = next_tile(nrw, nt0, ne1);
        if (more) load_head(nt0, ne1, hn);
#pragma unroll
        for (int hb = 0; hb < HB; ++hb) dacc[hb] = z4;
        plo = z4, phi = z4;
        st = 0;
        return true;
    };
    while (step(sa, sb) && step(sb, sa)) {
    }
}

// ------------------------------------------------------------------ CP radial forward, fused
// R = h2 W^T + b (the CP columns of the last radial layer) and the CP pooling of R in one launch:
// each 16-edge tile's R is computed on the matrix cores, written once (the backward reads it) and
// pooled from the same registers, so R is never read back. Orientation: D = h2 . W^T with the
// tile's edges as rows, so lane (j, q) holds R[edge 4q + r][column c0 + j] in register r — the B
// operand layout of the pooling product A_l[x, c] += sum_e Y[e, x] * w_l[e, c] (w_l = env m R_l)
// with edge 4q + r in K slot q of instruction r, whose A operand is Y^T (row x = lane j).
// Workgroup = (channel part, group of kCrfWaves edge shares): the part's W rows (4 ranks x NCB
// 16-channel blocks) sit in LDS for the whole launch; wave w walks the atom rows whose first
// edge lies in its equal share of the edges, in tiles of 16 consecutive edges that may span
// atom rows: the pooling of a tile runs once per atom segment it holds (Y masked to the
// segment), and an atom's accumulators are stored and cleared when its last edge is pooled.
// Rows with no edges get zero rows. Accumulation order: K slot then edge, so A differs from the
// edge-serial cp_density_fwd kernels in rounding only; R is bitwise the edge_linear_fwd product
// (same K split per instruction, same order). R goes out through non-temporal stores (read next
// by the backward, milliseconds later).
// Measured on the 24,000-atom liquid (C = 160, H = 64, 1.25 M edges, per-edge messages): 1.85 ms
// against 1.07 + 0.96 ms for the radial head and the pooling kernel; with node-table messages
// gathered through msg_row, 2.03 ms against 1.07 + 0.82: the model takes this launch for per-edge
// messages only. The kernel runs at two waves per SIMD (LDS: 80 KB of W per workgroup; about 250
// registers, of which 80 hold the pooling accumulators of 5 channel blocks) and is bound by
// latency rather than by its 0.86 ms of MFMA issue: without the R stores it takes 1.38 ms, as
// loads and stores share the in-order vmcnt counter and each channel block's loads wait for the
// previous block's stores. Measured and not kept: message and bias values issued a block ahead
// (1.93 ms), message rows issued a tile ahead (1.91 / 1.96 ms with gathered rows: spills; as
// 32-bit row indices with addresses formed per channel block, 1.89 / 1.94 ms against the
// two-launch 1.90 ms),
// ranks 0-2 sharing one accumulator tile through the K slots (2.24 ms: twelve dependent
// products per segment).
constexpr int kCrfWaves = 4;

// LDS row stride of the W image: H + 4 floats keeps the 16 rows one read touches on distinct banks;
// at H = 64 the rows are unpadded with float4 chunk c of row f stored at chunk (c + f) mod 16
// (lin_off), which does the same in 80 KB for 5 channel blocks: two workgroups per CU.
__host__ __device__ constexpr int crf_stride(int H) { return H == 64 ? 64 : H + 4; }

template <int HB, int NCB>
__global__ __launch_bounds__(kCrfWaves * kWave) __attribute__((amdgpu_waves_per_eu(2))) void cp_radial_fwd_kernel(
    const float* __restrict__ h2, int ld_h2, const float* __restrict__ w, const float* __restrict__ b,
    const float* __restrict__ env, const float* __restrict__ msg, int ld_msg, const int32_t* __restrict__ msg_row,
    const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr, int64_t N, int C, int nparts,
    RankOut A, float* __restrict__ R, int ld_R) {
    constexpr int H = 16 * HB, NCH = H / 4, ROWS = 4 * NCB * 16, S = crf_stride(H);
    constexpr bool rot = S == H;
    extern __shared__ float lds[];                    // W rows (l, cb, jj) of this part, lin_off image
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int j = lane & 15, q = lane >> 4;
    // blocks b and b + 8 run on the same XCD: both parts of an edge share read its h2 / Y rows
    // through one L2
    const int bid = blockIdx.x;
    const int part = (bid / 8) % nparts;
    const int64_t grp = (int64_t)(bid / (8 * nparts)) * 8 + (bid & 7);
    const int64_t ngrp = gridDim.x / nparts;
    const int cb0 = part * NCB;
    const int ncb = min(NCB, C / 16 - cb0);
    const int64_t E = row_ptr[N];
    // W and h2 may be NULL when there are no edges (then only zero rows are written); W is staged
    // only when there are edges to multiply
    if (E > 0 && (w == nullptr || h2 == nullptr)) return;
    if (E > 0) {
        stage4<8>(
            ROWS * NCH,
            [&](int f) {
                const int rr = f / NCH, c4 = f - rr * NCH;
                const int l = rr / (NCB * 16), cb = (rr >> 4) - l * NCB, jj = rr & 15;
                const v4f z = {0.f, 0.f, 0.f, 0.f};
                return cb < ncb ? ld4(w + (int64_t)(l * C + 16 * (cb0 + cb) + jj) * H + 4 * c4) : z;
            },
            [&](int f, v4f x) {
                const int rr = f / NCH, c4 = f - rr * NCH;
                st4(lds + lin_off(rr, c4, S, NCH, rot), x);
            });
    }
    __syncthreads();
    const int64_t W = ngrp * kCrfWaves;
    const int64_t gw = grp * kCrfWaves + __builtin_amdgcn_readfirstlane(tid / kWave);
    int64_t at = uniform64(wave_lower_bound(row_ptr, N, E * gw / W, lane));
    const int64_t a_end = gw + 1 == W ? N : uniform64(wave_lower_bound(row_ptr, N, E * (gw + 1) / W, lane));
    if (at >= a_end) return;
    const int64_t e_beg = row_ptr[at], e_end = row_ptr[a_end];
    // row_ptr[i] with i made wave-uniform: a scalar load (the segment walks below follow stores
    // in divergent branches, after which a vector load and a vmcnt(0) wait, i.e. a wait for every
    // store in flight, would otherwise be emitted)
    auto rp = [&](int64_t i) __attribute__((always_inline)) { return (int64_t)row_ptr[uniform64(i)]; };
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    const int sx = (int)A.sx;                         // the host checks 19 sx + C < 2^31
    // rows x = 4q + r of each rank block of one atom for the part's channel block cb; (jl, ql)
    // are the lane's (j, q) passed through an empty asm once per tile, so that the compiler
    // rebuilds these addresses per tile instead of holding one 64-bit address per (block, row)
    auto store_rank_rows = [&](int64_t atom, int cb, const v4f (&v)[4], int jl, int ql) __attribute__((always_inline)) {
        const int c = 16 * (cb0 + cb) + jl;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const int nl = l == 0 ? 1 : (l == 1 ? 3 : (l == 2 ? 6 : 10));
            float* base = A.p[l] + atom * A.sa;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (4 * ql + r < nl) base[(4 * ql + r) * sx + c] = v[l][r];
        }
    };
    const v4f zrow[4] = {z4, z4, z4, z4};
    // leading rows with no edges (and the whole share when it has none)
    while (at < a_end && rp(at + 1) == rp(at)) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
            if (cb < ncb) store_rank_rows(at, cb, zrow, j, q);
        ++at;
    }
    if (e_beg >= e_end) return;
    v4f pacc[NCB][4];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int l = 0; l < 4; ++l) pacc[cb][l] = z4;
    // h2 rows of a tile (A operand, K index q of instruction r of chunk kb = feature 16 kb + 4q + r)
    v4f hn[HB];
    auto load_h2 = [&](int64_t t0) __attribute__((always_inline)) {
        const int64_t e = min(t0 + j, e_end - 1);
#pragma unroll
        for (int kb = 0; kb < HB; ++kb) hn[kb] = ld4(h2 + e * ld_h2 + 16 * kb + 4 * q);
    };
    load_h2(e_beg);
    for (int64_t t0 = e_beg; t0 < e_end; t0 += 16) {
        const int64_t t1 = min(t0 + 16, e_end);
        int jl = j, ql = q;
        asm volatile("" : "+v"(jl), "+v"(ql));
        // lane part of the W reads of chunk kb (row j, float4 chunk 4 kb + q); the rows of rank l
        // and block cb add the constant (l NCB + cb) 16 S, an immediate offset of the read
        int lw[HB];
#pragma unroll
        for (int kb = 0; kb < HB; ++kb) lw[kb] = lin_off(jl, 4 * kb + ql, S, NCH, rot);
        v4f hv[HB];
#pragma unroll
        for (int kb = 0; kb < HB; ++kb) hv[kb] = hn[kb];
        if (t0 + 16 < e_end) load_h2(t0 + 16);
        // pooling-side values of edges t0 + 4q + r: Y rows of each rank (row x = lane j), envelope,
        // message row
        float yv[4][4], ev[4];
        const float* mp[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t e = min(t0 + 4 * ql + r, t1 - 1);
            ev[r] = env ? env[e] : 1.f;
            mp[r] = msg + (msg_row ? (int64_t)msg_row[e] : e) * ld_msg + 16 * cb0 + jl;
            const float* ye = Y + e * ld_Y + jl;
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const int nl = l == 0 ? 1 : (l == 1 ? 3 : (l == 2 ? 6 : 10));
                yv[l][r] = jl < nl ? ye[rank_start(l)] : 0.f;
            }
        }
        float* const Rt = R ? R + t0 * ld_R : nullptr;
        const float* const bt = b ? b + 16 * cb0 + jl : nullptr;
        int64_t nxt = at;
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            if (cb < ncb) {
                __builtin_amdgcn_sched_barrier(0);       // one channel block's operands live at a time
                const int c = 16 * (cb0 + cb) + jl;
                float mv[4], bias[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) mv[r] = mp[r][16 * cb];
#pragma unroll
                for (int l = 0; l < 4; ++l) bias[l] = bt ? bt[l * C + 16 * cb] : 0.f;
                v4f acc[4] = {z4, z4, z4, z4};
                // W operands of chunk kb + 1 read while chunk kb's products issue
                v4f wv[2][4];
                auto read_w = [&](int kb, v4f (&w4)[4]) __attribute__((always_inline)) {
#pragma unroll
                    for (int l = 0; l < 4; ++l)
                        w4[l] = lds4_at(lds, lw[kb] + (l * NCB + cb) * 16 * S);
                };
                read_w(0, wv[0]);
#pragma unroll
                for (int kb = 0; kb < HB; ++kb) {
                    if (kb + 1 < HB) read_w(kb + 1, wv[(kb + 1) & 1]);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int l = 0; l < 4; ++l) acc[l] = mfma_16x16x4(hv[kb][r], wv[kb & 1][l][r], acc[l]);
                }
                // R rows out, then w_l = env m R_l in place
#pragma unroll
                for (int l = 0; l < 4; ++l) acc[l] += bias[l];
                if (Rt) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (t0 + 4 * ql + r < t1) {
#pragma unroll
                            for (int l = 0; l < 4; ++l)
                                __builtin_nontemporal_store(acc[l][r], Rt + (4 * ql + r) * ld_R + l * C + c);
                        }
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float me = mv[r] * ev[r];
#pragma unroll
                    for (int l = 0; l < 4; ++l) acc[l][r] *= me;
                }
                // the tile's atom segments (row ends read through a wave-uniform index: scalar
                // loads, one per atom; atom a starts where atom a - 1 ends)
                int64_t a = at, lo = t0;
                int64_t a_hi = rp(a + 1);
                while (true) {
                    const int64_t hi = min(a_hi, t1);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t e = t0 + 4 * ql + r;
                        const bool in = e >= lo && e < hi;
#pragma unroll
                        for (int l = 0; l < 4; ++l)
                            pacc[cb][l] = mfma_16x16x4(in ? yv[l][r] : 0.f, acc[l][r], pacc[cb][l]);
                    }
                    if (a_hi > t1) break;             // the atom goes on into the next tile
                    store_rank_rows(a, cb, pacc[cb], jl, ql);
#pragma unroll
                    for (int l = 0; l < 4; ++l) pacc[cb][l] = z4;
                    const int64_t start = a_hi;       // where the next atom's edges begin
                    ++a;
                    while (a < a_end) {
                        a_hi = rp(a + 1);
                        if (a_hi != start) break;
                        store_rank_rows(a, cb, zrow, jl, ql);
                        ++a;
                    }
                    if (a >= a_end || start >= t1) break;
                    lo = start;
                }
                nxt = a;
            }
        }
        at = nxt;
    }
}

// ------------------------------------------------------------------ launch helpers

template <int NX>
static int launch_fwd_nx(int cpt, dim3 grid, size_t lds, hipStream_t st, const float* phi, int ld_phi,
                         const float* msg, int ld_msg, const int32_t* msg_row, const float* Y, int ld_Y,
                         const int32_t* row_ptr, int M, int B, int K, RankOut D) {
#define FACE_FWD(C_)                                                                                          \
    hipLaunchKernelGGL((density_fwd_kernel<NX, C_>), grid, dim3(kBlock), lds, st, phi, ld_phi, msg, ld_msg,  \
                       msg_row, Y, ld_Y, row_ptr, M, B, K, D)
    switch (cpt) {
        case 1: FACE_FWD(1); break;
        case 2: FACE_FWD(2); break;
        case 4: FACE_FWD(4); break;
        case 9: FACE_FWD(9); break;
        default: return FACE_ERR_UNSUPPORTED;
    }
#undef FACE_FWD
    FACE_LAUNCH_CHECK();
    return 0;
}

template <int NX, int B, int KS>
static int launch_bwd3(int glog, int nthr, int64_t N, hipStream_t st, const float* phi, int ld_phi,
                       const float* msg, int ld_msg, const int32_t* msg_row, const float* Y, int ld_Y,
                       const int32_t* row_ptr, int M, int K, RankIn G, float* dphi, int ld_dphi, float* dmsg,
                       int ld_dmsg, float* dY, int ld_dY) {
    constexpr int KSP = (KS + 3) & ~3;
    const size_t lds = (size_t)NX * B * (1 << glog) * KSP * sizeof(float);
    if ((int64_t)lds > device_max_lds()) return FACE_ERR_UNSUPPORTED;
    auto kern = density_bwd_kernel<NX, B, KS>;
    if (lds > 65536 &&
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return FACE_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(kern, dim3((unsigned)N), dim3(nthr), lds, st, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y,
                       row_ptr, M, K, glog, G, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY);
    FACE_LAUNCH_CHECK();
    return 0;
}

template <int NX, int B>
static int launch_bwd_b(int ks, int glog, int nthr, int64_t N, hipStream_t st, const float* phi, int ld_phi,
                        const float* msg, int ld_msg, const int32_t* msg_row, const float* Y, int ld_Y,
                        const int32_t* row_ptr, int M, int K, RankIn G, float* dphi, int ld_dphi, float* dmsg,
                        int ld_dmsg, float* dY, int ld_dY) {
#define FACE_BWD(KS_)                                                                                            \
    return launch_bwd3<NX, B, KS_>(glog, nthr, N, st, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, K, \
                                   G, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY)
    switch (ks) {
        case 4: FACE_BWD(4);
        case 8: FACE_BWD(8);
        case 9: FACE_BWD(9);
        default: return FACE_ERR_UNSUPPORTED;
    }
#undef FACE_BWD
}

template <int NX>
static int launch_bwd_nx(int B, int ks, int glog, int nthr, int64_t N, hipStream_t st, const float* phi,
                         int ld_phi, const float* msg, int ld_msg, const int32_t* msg_row, const float* Y, int ld_Y,
                         const int32_t* row_ptr, int M, int K, RankIn G, float* dphi, int ld_dphi, float* dmsg,
                         int ld_dmsg, float* dY, int ld_dY) {
#define FACE_BWDB(B_)                                                                                       \
    return launch_bwd_b<NX, B_>(ks, glog, nthr, N, st, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, \
                                M, K, G, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY)
    switch (B) {
        case 4: FACE_BWDB(4);
        case 8: FACE_BWDB(8);
        case 16: FACE_BWDB(16);
        case 32: FACE_BWDB(32);
        default: return FACE_ERR_UNSUPPORTED;
    }
#undef FACE_BWDB
}

// Chooses the k-slice split (GN lanes of KS columns per edge) and the workgroup size that
// waste the fewest lanes for rows of length max_row.
static bool plan_bwd(int K, int max_row, int& ks_out, int& glog_out, int& nthr_out) {
    const int ks_opts[3] = {4, 8, 9};
    double best = -1.0;
    for (int glog = 0; glog <= 5; ++glog) {
        const int GN = 1 << glog;
        for (int ks : ks_opts) {
            if (GN * ks < K || (GN > 1 && (GN / 2) * ks >= K)) continue;   // minimal GN for this ks
            const int per_wave = kWave / GN;
            int nw = (max_row + per_wave - 1) / per_wave;
            nw = nw < 1 ? 1 : (nw > 4 ? 4 : nw);
            const int slots = nw * per_wave;
            const int passes = (max_row + slots - 1) / slots;
            const double lane_eff = (double)max_row / (double)(passes * slots > 0 ? passes * slots : 1);
            const double k_eff = (double)K / (double)(GN * ks);
            const double score = lane_eff * k_eff + 1e-3 * ks;   // prefer fewer shuffles on ties
            if (score > best) {
                best = score;
                ks_out = ks;
                glog_out = glog;
                nthr_out = nw * kWave;
            }
        }
    }
    return best > 0.0;
}

// Rank-block descriptors from the C-ABI arguments; every rank the NX monomials touch needs a pointer.
static bool rank_out(float* const* p, int64_t sa, int64_t sx, int NX, RankOut& r) {
    const int nr = NX == 20 ? 4 : 2;
    for (int l = 0; l < 4; ++l) r.p[l] = (p && l < nr) ? p[l] : nullptr;
    r.sa = sa;
    r.sx = sx;
    for (int l = 0; l < nr; ++l)
        if (!r.p[l]) return false;
    return sa > 0 && sx > 0;
}
static bool rank_in(const float* const* p, int64_t sa, int64_t sx, int NX, RankIn& r) {
    const int nr = NX == 20 ? 4 : 2;
    for (int l = 0; l < 4; ++l) r.p[l] = (p && l < nr) ? p[l] : nullptr;
    r.sa = sa;
    r.sx = sx;
    for (int l = 0; l < nr; ++l)
        if (!r.p[l]) return false;
    return sa > 0 && sx > 0;
}

}  // namespace face

using namespace face;

extern "C" int face_density_fwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg,
                                const int32_t* msg_row, const float* Y, int32_t ld_Y, int32_t NX,
                                const int32_t* row_ptr, int64_t N, int32_t M, int32_t B, int32_t K,
                                float* const* D_ranks, int64_t atom_stride, int64_t x_stride, void* stream) {
    if (N < 0 || B <= 0 || K <= 0 || (NX != 4 && NX != 20)) return FACE_ERR_ARG;
    if (ld_phi < B || ld_msg < K || ld_Y < NX || (!row_ptr && M < 0)) return FACE_ERR_ARG;
    if (N == 0) return 0;
    RankOut D;
    if (!phi || !msg || !Y || !rank_out(D_ranks, atom_stride, x_stride, NX, D)) return FACE_ERR_ARG;
    if (NX == 20 && B == 16 && K % 16 == 0 && K <= 64) {          // matrix cores
#define FACE_DFR(KB_)                                                                                         \
    hipLaunchKernelGGL((density_fwd_row_kernel<KB_>), dim3((unsigned)N), dim3(kDrWaves * kWave), 0,              \
                       (hipStream_t)stream, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, D)
        switch (K / 16) {
            case 1: FACE_DFR(1); break;
            case 2: FACE_DFR(2); break;
            case 3: FACE_DFR(3); break;
            default: FACE_DFR(4); break;
        }
#undef FACE_DFR
        FACE_LAUNCH_CHECK();
        return 0;
    }
    const int BK = B * K;
    const int opts20[3] = {1, 2, 4}, opts4[4] = {1, 2, 4, 9};
    const int* opts = NX == 20 ? opts20 : opts4;
    const int nopt = NX == 20 ? 3 : 4;
    int cpt = opts[nopt - 1];
    for (int q = 0; q < nopt; ++q)
        if (kBlock * opts[q] >= BK) {
            cpt = opts[q];
            break;
        }
    const unsigned chunks = (unsigned)((BK + kBlock * cpt - 1) / (kBlock * cpt));
    const size_t lds = (size_t)kTileE * (B + K + NX) * sizeof(float);
    if ((int64_t)lds > 65536) return FACE_ERR_UNSUPPORTED;
    dim3 grid((unsigned)N, chunks);
    hipStream_t st = (hipStream_t)stream;
    if (NX == 20)
        return launch_fwd_nx<20>(cpt, grid, lds, st, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, B, K, D);
    return launch_fwd_nx<4>(cpt, grid, lds, st, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, B, K, D);
}

// Route of the factor backward for CSR rows: G staged in LDS per atom for systems of at least 64
// atoms per CU (density_bwd_lds_kernel), the per-wave kernel below that. FACE_DENSITY_BWD_LDS=0 / 1
// in the environment forces either (read on every call).
static bool use_lds_bwd(int64_t N) {
    const char* e = getenv("FACE_DENSITY_BWD_LDS");
    if (e && (e[0] == '0' || e[0] == '1')) return e[0] == '1';
    return N >= (int64_t)device_cu_count() * 64;
}

extern "C" int face_density_bwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg,
                                const int32_t* msg_row, const float* Y, int32_t ld_Y, int32_t NX,
                                const int32_t* row_ptr, int64_t N, int32_t M, int32_t max_row, int32_t B, int32_t K,
                                const float* const* G_ranks, int64_t atom_stride, int64_t x_stride, float* dphi,
                                int32_t ld_dphi, float* dmsg, int32_t ld_dmsg, float* dY, int32_t ld_dY,
                                void* stream) {
    if (N < 0 || B <= 0 || K <= 0 || (NX != 4 && NX != 20) || max_row < 0) return FACE_ERR_ARG;
    if (ld_phi < B || ld_msg < K || ld_Y < NX || (!row_ptr && M < 0)) return FACE_ERR_ARG;
    if ((dphi && ld_dphi < B) || (dmsg && ld_dmsg < K) || (dY && ld_dY < NX)) return FACE_ERR_ARG;
    if (N == 0 || max_row == 0) return 0;
    RankIn G;
    if (!phi || !msg || !Y || !rank_in(G_ranks, atom_stride, x_stride, NX, G)) return FACE_ERR_ARG;
    hipStream_t st = (hipStream_t)stream;
    // matrix cores: 20 monomials, B = 16, whole 16-channel blocks, 16-byte aligned rows
    if (NX == 20 && B == 16 && K % 16 == 0 && K <= 64 && ld_phi % 4 == 0 && ld_msg % 4 == 0 && G.sa % 4 == 0 &&
        G.sx % 4 == 0 && ((uintptr_t)phi & 15) == 0 && ((uintptr_t)msg & 15) == 0 && ((uintptr_t)G.p[0] & 15) == 0 &&
        ((uintptr_t)G.p[1] & 15) == 0 && ((uintptr_t)G.p[2] & 15) == 0 && ((uintptr_t)G.p[3] & 15) == 0) {
        // CSR rows of large systems: G staged in LDS per atom (read once), see density_bwd_lds_kernel
        if (row_ptr && use_lds_bwd(N)) {
#define FACE_DBL(KB_)                                                                                          \
    hipLaunchKernelGGL((density_bwd_lds_kernel<KB_>), dim3((unsigned)N), dim3(kDbLWaves * kWave), 0, st, phi,   \
                       ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, G, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY)
            switch (K / 16) {
                case 1: FACE_DBL(1); break;
                case 2: FACE_DBL(2); break;
                case 3: FACE_DBL(3); break;
                default: FACE_DBL(4); break;
            }
#undef FACE_DBL
            FACE_LAUNCH_CHECK();
            return 0;
        }
        // small systems: split each atom's monomials over 4 waves (one atom per workgroup)
        const bool split = N < (int64_t)device_cu_count() * 16;
        const dim3 grid(split ? (unsigned)N : (unsigned)((N + kDbWaves - 1) / kDbWaves));
        const dim3 block(split ? 4 * kWave : kDbWaves * kWave);
#define FACE_DBM(KB_)                                                                                           \
    do {                                                                                                        \
        if (split && KB_ <= 2)                                                                                  \
            hipLaunchKernelGGL((density_bwd_split_kernel<(KB_ <= 2 ? KB_ : 2)>), grid, block, 0, st, phi, ld_phi, \
                               msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, G, dphi, ld_dphi, dmsg, ld_dmsg, dY,   \
                               ld_dY);                                                                          \
        else if (split)                                                                                         \
            hipLaunchKernelGGL((density_bwd_mfma_kernel<KB_, 4>), grid, block, 0, st, phi, ld_phi, msg, ld_msg,  \
                               msg_row, Y, ld_Y, row_ptr, N, M, G, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY);     \
        else                                                                                                    \
            hipLaunchKernelGGL((density_bwd_mfma_kernel<KB_, 1>), grid, block, 0, st, phi, ld_phi, msg, ld_msg,  \
                               msg_row, Y, ld_Y, row_ptr, N, M, G, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY);     \
    } while (0)
        switch (K / 16) {
            case 1: FACE_DBM(1); break;
            case 2: FACE_DBM(2); break;
            case 3: FACE_DBM(3); break;
            default: FACE_DBM(4); break;
        }
#undef FACE_DBM
        FACE_LAUNCH_CHECK();
        return 0;
    }
    int ks = 8, glog = 2, nthr = 128;
    if (!plan_bwd(K, max_row, ks, glog, nthr)) return FACE_ERR_UNSUPPORTED;
    if (NX == 20)
        return launch_bwd_nx<20>(B, ks, glog, nthr, N, st, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, K,
                                 G, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY);
    return launch_bwd_nx<4>(B, ks, glog, nthr, N, st, phi, ld_phi, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, K, G,
                            dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY);
}

// The MFMA backward reads and writes float4s: whole channel steps, 16-byte aligned rows and
// rank blocks.
static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
static bool mfma_layout_ok(const float* R, int ld_R, const float* msg, int ld_msg, const float* Y, int ld_Y, int C,
                           const RankIn& gA, const float* dR, int ld_dR, const float* dmsg, int ld_dmsg,
                           const float* dY, int ld_dY, int step = kCpStep) {
    if (C % step || ld_R % 4 || ld_msg % 4 || ld_Y % 4 || gA.sa % 4 || gA.sx % 4) return false;
    if (!aligned16(R) || !aligned16(msg) || !aligned16(Y)) return false;
    for (int l = 0; l < 4; ++l)
        if (!aligned16(gA.p[l])) return false;
    if (dR && (ld_dR % 4 || !aligned16(dR))) return false;
    if (dmsg && (ld_dmsg % 4 || !aligned16(dmsg))) return false;
    if (dY && (ld_dY % 4 || !aligned16(dY))) return false;
    return true;
}

extern "C" int face_cp_density_fwd(const float* R, int32_t ld_R, const float* env, const float* msg, int32_t ld_msg,
                                   const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr,
                                   int64_t N, int32_t M, int32_t C, float* const* A_ranks, int64_t atom_stride,
                                   int64_t x_stride, void* stream) {
    if (N < 0 || C <= 0 || ld_R < 4 * C || ld_msg < C || ld_Y < 20 || (!row_ptr && M < 0)) return FACE_ERR_ARG;
    if (N == 0) return 0;
    RankOut A;
    if (!R || !msg || !Y || !rank_out(A_ranks, atom_stride, x_stride, 20, A)) return FACE_ERR_ARG;
    const bool a16 = aligned16(R) && aligned16(msg) && ld_R % 4 == 0 && ld_msg % 4 == 0 && A.sa % 4 == 0 &&
                     A.sx % 4 == 0 && aligned16(A.p[0]) && aligned16(A.p[1]) && aligned16(A.p[2]) && aligned16(A.p[3]);
    if (a16 && C % 4 == 0 && C <= 4 * kWave) {
        hipLaunchKernelGGL(cp_density_fwd_wave_kernel, dim3((unsigned)((N + kCpfWaves - 1) / kCpfWaves)),
                           dim3(kCpfWaves * kWave), 0, (hipStream_t)stream, R, ld_R, env, msg, ld_msg, msg_row, Y,
                           ld_Y, row_ptr, N, M, C, A);
        FACE_LAUNCH_CHECK();
        return 0;
    }
    int nthr = ((C + kWave - 1) / kWave) * kWave;
    if (nthr > kBlock) nthr = kBlock;
    dim3 grid((unsigned)N, (unsigned)((C + nthr - 1) / nthr));
    hipLaunchKernelGGL(cp_density_fwd_kernel, grid, dim3(nthr), 0, (hipStream_t)stream, R, ld_R, env, msg, ld_msg,
                       msg_row, Y, ld_Y, row_ptr, M, C, A);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_cp_density_bwd(const float* R, int32_t ld_R, const float* env, const float* msg, int32_t ld_msg,
                                   const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr,
                                   int64_t N, int32_t M, int32_t max_row, int32_t C, const float* const* gA_ranks,
                                   int64_t atom_stride, int64_t x_stride, float* dR, int32_t ld_dR, float* dmsg,
                                   int32_t ld_dmsg, float* dY, int32_t ld_dY, float* denv, void* stream) {
    if (N < 0 || C <= 0 || ld_R < 4 * C || ld_msg < C || ld_Y < 20 || (!row_ptr && M < 0)) return FACE_ERR_ARG;
    if ((dR && ld_dR < 4 * C) || (dmsg && ld_dmsg < C) || (dY && ld_dY < 20)) return FACE_ERR_ARG;
    if (N == 0 || max_row == 0) return 0;
    RankIn gA;
    if (!R || !msg || !Y || !rank_in(gA_ranks, atom_stride, x_stride, 20, gA)) return FACE_ERR_ARG;
    if (mfma_layout_ok(R, ld_R, msg, ld_msg, Y, ld_Y, C, gA, dR, ld_dR, dmsg, ld_dmsg, dY, ld_dY)) {
        // one atom row per wave, kCpRowsPerBlock rows per workgroup, each with its gA slice in LDS
        const size_t lds = (size_t)kCpRowsPerBlock * 20 * cp_mfma_stride(C) * sizeof(float);
        if (lds > 65536) return FACE_ERR_UNSUPPORTED;
        hipLaunchKernelGGL(cp_density_bwd_mfma_kernel, dim3((unsigned)((N + kCpRowsPerBlock - 1) / kCpRowsPerBlock)),
                           dim3(kCpRowsPerBlock * kWave), lds, (hipStream_t)stream, R, ld_R, env, msg, ld_msg, msg_row,
                           Y, ld_Y, row_ptr, N, M, C, gA, dR, ld_dR, dmsg, ld_dmsg, dY, ld_dY, denv);
        FACE_LAUNCH_CHECK();
        return 0;
    }
    if (C > kBlock) return FACE_ERR_UNSUPPORTED;
    const int nthr = ((C + kWave - 1) / kWave) * kWave;
    const int CS = ((C + 3) & ~3) + 4;
    const size_t lds = ((size_t)(20 + kTileCPB * 4) * CS + kTileCPB * 41) * sizeof(float);
    if ((int64_t)lds > 65536) return FACE_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(cp_density_bwd_kernel, dim3((unsigned)N), dim3(nthr), lds, (hipStream_t)stream, R, ld_R, env,
                       msg, ld_msg, msg_row, Y, ld_Y, row_ptr, M, C, gA, dR, ld_dR, dmsg, ld_dmsg, dY, ld_dY, denv);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_cp_radial_fwd(const float* h2, int32_t ld_h2, int32_t H, const float* w, const float* b,
                                  const float* env, const float* msg, int32_t ld_msg, const int32_t* msg_row,
                                  const float* Y, int32_t ld_Y, const int32_t* row_ptr, int64_t N, int64_t E,
                                  int32_t C, float* const* A_ranks, int64_t atom_stride, int64_t x_stride, float* R,
                                  int32_t ld_R, void* stream) {
    if (N < 0 || E < 0 || C <= 0 || H < 16 || H > 64 || H % 16 || ld_h2 < H || ld_msg < C || ld_Y < 20 ||
        (R && ld_R < 4 * C))
        return FACE_ERR_ARG;
    if (N == 0) return 0;
    RankOut A;
    if ((E > 0 && (!h2 || !w)) || !msg || !Y || !row_ptr || !rank_out(A_ranks, atom_stride, x_stride, 20, A))
        return FACE_ERR_ARG;
    if (C % 16 || ld_h2 % 4 || !aligned16(h2) || !aligned16(w) || A.sx * 19 + C >= ((int64_t)1 << 31) ||
        (int64_t)ld_R * 16 >= ((int64_t)1 << 31))
        return FACE_ERR_UNSUPPORTED;
    const int nblk = C / 16;
    const int nparts = (nblk + 4) / 5;
    const int ncb = (nblk + nparts - 1) / nparts;   // 16-channel blocks per part, <= 5
    const int rows = 4 * (ncb < 2 ? 2 : ncb) * 16;   // the kernel's NCB rows (NCB >= 2)
    const int64_t max_lds = device_max_lds();
    const size_t lds = (size_t)rows * crf_stride(H) * sizeof(float);
    if ((int64_t)lds > max_lds) return FACE_ERR_UNSUPPORTED;
    // edge shares: one group per CU at most, and at least 8 tiles per wave; a multiple of 8
    // groups, so that blocks b and b + 8 (one XCD) hold the parts of one group
    int64_t ngrp = (E + 16 * 8 * kCrfWaves - 1) / (16 * 8 * kCrfWaves);
    const int64_t n_cu = device_cu_count();
    if (ngrp > n_cu) ngrp = n_cu;
    ngrp = ((ngrp < 1 ? 1 : ngrp) + 7) / 8 * 8;
    const dim3 grid((unsigned)(ngrp * nparts)), block(kCrfWaves * kWave);
    const hipStream_t st = (hipStream_t)stream;
#define FACE_CRF(HB_, NCB_)                                                                                       \
    do {                                                                                                          \
        auto kern = cp_radial_fwd_kernel<HB_, NCB_>;                                                              \
        if (lds > 65536 &&                                                                                        \
            hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) \
            return FACE_ERR_UNSUPPORTED;                                                                          \
        hipLaunchKernelGGL(kern, grid, block, lds, st, h2, ld_h2, w, b, env, msg, ld_msg, msg_row, Y, ld_Y,         \
                           row_ptr, N, C, nparts, A, R, ld_R);                                                    \
    } while (0)
#define FACE_CRF_H(NCB_)                    \
    switch (H / 16) {                       \
        case 1: FACE_CRF(1, NCB_); break;   \
        case 2: FACE_CRF(2, NCB_); break;   \
        case 3: FACE_CRF(3, NCB_); break;   \
        default: FACE_CRF(4, NCB_); break;  \
    }
    switch (ncb) {
        case 1:
        case 2: FACE_CRF_H(2); break;
        case 3: FACE_CRF_H(3); break;
        case 4: FACE_CRF_H(4); break;
        default: FACE_CRF_H(5); break;
    }
#undef FACE_CRF_H
#undef FACE_CRF
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_cp_radial_bwd(const float* R, int32_t ld_R, const float* env, const float* msg, int32_t ld_msg,
                                  const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr,
                                  int64_t N, int32_t M, int32_t C, const float* const* gA_ranks, int64_t atom_stride,
                                  int64_t x_stride, const float* w_t, int32_t H, float* dh2, int32_t ld_dh2,
                                  float* dmsg, int32_t ld_dmsg, float* dY, int32_t ld_dY, float* denv,
                                  void* stream) {
    if (N < 0 || C <= 0 || ld_R < 4 * C || ld_msg < C || ld_Y < 20 || (!row_ptr && M < 0)) return FACE_ERR_ARG;
    if (H < 16 || H > 64 || H % 16 || !w_t || ((uintptr_t)w_t & 15) || !dh2 || ld_dh2 < H) return FACE_ERR_ARG;
    if ((dmsg && ld_dmsg < C) || (dY && ld_dY < 20)) return FACE_ERR_ARG;
    if (N == 0) return 0;
    RankIn gA;
    if (!R || !msg || !Y || !rank_in(gA_ranks, atom_stride, x_stride, 20, gA)) return FACE_ERR_ARG;
    const hipStream_t st = (hipStream_t)stream;
    const int n_cu = device_cu_count();
    const size_t lds_res = (size_t)H * 4 * C * sizeof(float);
    if ((int64_t)lds_res <= device_max_lds() && gA.sx * 19 + C < ((int64_t)1 << 31) &&
        mfma_layout_ok(R, ld_R, msg, ld_msg, Y, ld_Y, C, gA, nullptr, 0, dmsg, ld_dmsg, dY, ld_dY, kResStep)) {
        // all of W^T resident in LDS: one workgroup per CU, every wave on its own share of the edges
        constexpr int kNW = 8;
#define FACE_CPRES(HB_)                                                                                          \
    do {                                                                                                         \
        auto kern = cp_radial_bwd_res_kernel<HB_, kNW>;                                                          \
        if (lds_res > 65536 && hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                                   (int)lds_res) != hipSuccess)                                  \
            return FACE_ERR_UNSUPPORTED;                                                                         \
        hipLaunchKernelGGL(kern, dim3((unsigned)n_cu), dim3(kNW * kWave), lds_res, st, R, ld_R, env, msg, ld_msg, \
                           msg_row, Y, ld_Y, row_ptr, N, M, C, gA, dmsg, ld_dmsg, dY, ld_dY, denv, w_t, dh2, ld_dh2); \
    } while (0)
        switch (H / 16) {
            case 1: FACE_CPRES(1); break;
            case 2: FACE_CPRES(2); break;
            case 3: FACE_CPRES(3); break;
            default: FACE_CPRES(4); break;
        }
#undef FACE_CPRES
        FACE_LAUNCH_CHECK();
        return 0;
    }
    if (!mfma_layout_ok(R, ld_R, msg, ld_msg, Y, ld_Y, C, gA, nullptr, 0, dmsg, ld_dmsg, dY, ld_dY))
        return FACE_ERR_UNSUPPORTED;
    // persistent workgroups, one per CU: W slab + one gA row per wave + per-wave tile counts
    const size_t lds = ((size_t)H * kSlabRS + (size_t)kLdsWaves * 20 * cp_mfma_stride(C) + kLdsWaves) * sizeof(float);
    if ((int64_t)lds > device_max_lds()) return FACE_ERR_UNSUPPORTED;
    const int64_t waves = N < (int64_t)n_cu * kLdsWaves ? N : (int64_t)n_cu * kLdsWaves;
    const dim3 grid((unsigned)((waves + kLdsWaves - 1) / kLdsWaves)), block(kLdsWaves * kWave);
#define FACE_CPR(HB_)                                                                                            \
    do {                                                                                                         \
        auto kern = cp_radial_bwd_lds_kernel<HB_>;                                                               \
        if (lds > 65536 &&                                                                                       \
            hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) \
            return FACE_ERR_UNSUPPORTED;                                                                         \
        hipLaunchKernelGGL(kern, grid, block, lds, st, R, ld_R, env, msg, ld_msg, msg_row, Y, ld_Y, row_ptr, N, M, C, \
                           gA, dmsg, ld_dmsg, dY, ld_dY, denv, w_t, dh2, ld_dh2);                                \
    } while (0)
    switch (H / 16) {
        case 1: FACE_CPR(1); break;
        case 2: FACE_CPR(2); break;
        case 3: FACE_CPR(3); break;
        default: FACE_CPR(4); break;
    }
#undef FACE_CPR
    FACE_LAUNCH_CHECK();
    return 0;
}
