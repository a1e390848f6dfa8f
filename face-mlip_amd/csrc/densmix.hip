// Factor density fused with the per-rank channel mixing (gfx950, fp32 matrix cores):
//
//   A_l[i, x, c] = (beta_l A_l[i, x, c] + sum_{b,k} D[i, x, b, k] W_l[c, b K + k]) * s[z_i, l C + c]
//   D[i, x, b, k] = sum_{e in row i} phi[e, b] msg[m(e), k] Y[e, x]
//
// (face/kernels.py:22-54 for D, face/model.py:503-506 for mix[l] and :530-533 for the element
// scale) with D never written to memory: a workgroup of 16 waves owns a tile of kDmTA = 4 atoms
// (all 20 monomials: 80 rows ordered rank-major, then monomial, then atom) and walks the B K
// columns of D in chunks of (16 basis functions) x (16 channels). Per chunk,
//   phase 1: four waves per atom (5 monomials each) build the D^T[k][b] blocks on the matrix
//            cores (A = msg^T, B = Y_x phi, the edge tile's Y staged in the wave's LDS slot), one
//            v4f LDS store per lane and block;
//   phase 2: the (row block, c-block) tiles of the output, 7 row blocks (rank 0 | 1 | 2 | 2 | 3 |
//            3 | 3: blocks hold the rows of one rank) by C/16, dealt to the 16 waves, accumulate
//            W_l[c, (b, k)] D[row, (b, k)] (A = W_l from L2, the next basis function's block
//            loaded ahead; B = the D rows from LDS) in registers that live across all chunks.
// The backward runs the same tiles the other way round, per chunk:
//   phase 2: dD = (gA s) W_l into LDS (A = W_l^T, B = the scaled upstream rows), tiles (basis
//            function, row block) dealt to 14 waves;
//   phase 1: the factor-density backward of face/kernels.py:56-118 against that chunk, four waves
//            per atom splitting the monomials, per 16-edge tile
//              S[e, b] = sum_k msg[e, k] dD[x, b, k],  dmsg[e, k] += sum_{x,b} Y[e, x] phi[e, b] dD[x, b, k],
//              dphi[e, b] += sum_x S Y[e, x],       dY[e, x] += sum_b S phi[e, b]
//            with the four waves' dphi / dmsg partials summed in LDS (dmsg is complete per chunk;
//            dphi and dY are summed over the chunks in place by the lanes that own them).
// Every sum has a fixed order (no atomics). B = 16, the 20 monomials up to rank 3, K a multiple of
// 16 up to 64, C a multiple of 16 up to 256.
#include "common.h"

namespace face {

constexpr int kDmTA = 4;                  // atoms per workgroup
constexpr int kDmWaves = 16;              // 4 per atom in phase 1, 4 per SIMD
constexpr int kDmS = 260;                 // LDS row stride of a D chunk (256 columns + 4)
constexpr int kDmLdsRows = 88;            // the last row block reads rows 72 .. 87
constexpr int kDmYS = 21;                 // row stride of a wave's Y tile

// Row blocks of the 80-row tile: rank, first row, valid rows. Rows of (rank l, monomial x,
// atom a) are dm_base(l) + (x - x0(l)) kDmTA + a.
__host__ __device__ constexpr int dm_base(int l) { return l == 0 ? 0 : (l == 1 ? 4 : (l == 2 ? 16 : 40)); }
__host__ __device__ constexpr int dm_x0(int l) { return l == 0 ? 0 : (l == 1 ? 1 : (l == 2 ? 4 : 10)); }
__device__ __forceinline__ void dm_block(int rb, int& l, int& r0, int& nv) {
    l = rb == 0 ? 0 : (rb == 1 ? 1 : (rb < 4 ? 2 : 3));
    r0 = rb == 0 ? 0 : (rb == 1 ? 4 : (rb == 2 ? 16 : (rb == 3 ? 32 : (rb == 4 ? 40 : (rb == 5 ? 56 : 72)))));
    nv = rb == 0 ? 4 : (rb == 1 ? 12 : ((rb == 3 || rb == 6) ? 8 : 16));
}
__device__ __forceinline__ int dm_row(int x, int a) {
    const int l = rank_of(x);
    return dm_base(l) + (x - dm_x0(l)) * kDmTA + a;
}

struct DmRanks {
    float* p[4];          // output (or upstream-gradient) rank blocks
    int64_t sa, sx;       // atom and monomial strides
    const float* w[4];    // forward: W_l (C, ld_w); backward: W_l^T (B K, ld_w)
    int64_t ld_w;
};

// The wave's 16-edge tile of Y (16 x 20, zero past the row end) into its LDS slot.
__device__ __forceinline__ void dm_stage_y(float* ys, const float* __restrict__ Y, int ld_Y, int64_t e0, int ne,
                                           int lane) {
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int u = 0; u < 5; ++u) {
        const int v = u * kWave + lane, t = v / 20, x = v - t * 20;
        ys[t * kDmYS + x] = t < ne ? Y[(e0 + t) * ld_Y + x] : 0.f;
    }
    __builtin_amdgcn_wave_barrier();
}

// ------------------------------------------------------------------ forward
template <int KB, int TPW>
__global__ __launch_bounds__(kDmWaves * kWave) void density_mix_fwd_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int64_t N, int C, DmRanks R, const float* __restrict__ ys_tab, int ld_s, const int32_t* __restrict__ group,
    int beta_mask) {
    constexpr int K = 16 * KB;
    __shared__ float sD[kDmLdsRows * kDmS];
    __shared__ float sY[kDmWaves][16 * kDmYS];
    const int lane = threadIdx.x & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int64_t n0 = (int64_t)blockIdx.x * kDmTA;
    const int ntask = 7 * (C / 16);
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    // rows past the tile's 80 (read by the last row block, never stored) hold zeros
    for (int v = threadIdx.x; v < (kDmLdsRows - 80) * kDmS; v += kDmWaves * kWave) sD[80 * kDmS + v] = 0.f;
    // phase-1 role: atom a, monomials x1 .. x1 + 4
    const int a = wv >> 2, x1 = 5 * (wv & 3);
    const int64_t n = n0 + a;
    int64_t e_beg = 0, e_end = 0;
    if (n < N) {
        e_beg = row_ptr[n];
        e_end = row_ptr[n + 1];
    }
    float* ys = sY[wv];
    v4f acc[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) acc[i] = z4;
#pragma unroll 1
    for (int kc = 0; kc < KB; ++kc) {
        // ---- phase 1: D^T[k][b] blocks of (atom a, monomial x) for channels 16 kc .. 16 kc + 15
        v4f dt[5];
#pragma unroll
        for (int xx = 0; xx < 5; ++xx) dt[xx] = z4;
        for (int64_t e0 = e_beg; e0 < e_end; e0 += 16) {
            const int ne = (int)min((int64_t)16, e_end - e0);
            dm_stage_y(ys, Y, ld_Y, e0, ne, lane);
            float mv[4], ph[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 4 * q + r;
                const int64_t e = e0 + min(t, ne - 1);       // clamped: loads stay in the row
                const int64_t row = msg_row ? (int64_t)msg_row[e] : e;
                mv[r] = msg[row * ld_msg + 16 * kc + j];
                const float p = phi[e * ld_phi + j];
                ph[r] = t < ne ? p : 0.f;                    // zero past the row end
            }
#pragma unroll
            for (int xx = 0; xx < 5; ++xx)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    dt[xx] = mfma_16x16x4(mv[r], ys[(4 * q + r) * kDmYS + x1 + xx] * ph[r], dt[xx]);
        }
        // dt[xx]: D^T[k = 4q + r][b = j] in register r -> LDS row (x, a), column 16 b + k
#pragma unroll
        for (int xx = 0; xx < 5; ++xx) st4(sD + dm_row(x1 + xx, a) * kDmS + 16 * j + 4 * q, dt[xx]);
        __syncthreads();
        // ---- phase 2: task i = (row block, c-block): acc += W_l[c, (b, k)] D[row, (b, k)] over the
        // chunk; per task the 16 basis functions in order, the next one's W block loaded ahead
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int t = wv + kDmWaves * i;
            if (t >= ntask) break;
            int l, r0, nv;
            dm_block(t % 7, l, r0, nv);
            const float* wp = R.w[l] + (int64_t)(16 * (t / 7) + j) * R.ld_w + 16 * kc + 4 * q;
            const float* dp = sD + (r0 + j) * kDmS + 4 * q;
            v4f wn = ld4(wp);
#pragma unroll 4
            for (int b = 0; b < 16; ++b) {
                const v4f wc = wn;
                if (b + 1 < 16) wn = ld4(wp + (b + 1) * K);
                const v4f dv = *reinterpret_cast<const v4f*>(dp + 16 * b);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i] = mfma_16x16x4(wc[r], dv[r], acc[i]);
            }
        }
        __syncthreads();                                    // chunk consumed before it is overwritten
    }
    // ---- epilogue: acc[i] holds out[c = 16 cb + 4q + r][row r0 + j]
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int t = wv + kDmWaves * i;
        if (t >= ntask) break;
        int l, r0, nv;
        dm_block(t % 7, l, r0, nv);
        if (j >= nv) continue;
        const int c = 16 * (t / 7) + 4 * q;
        const int loc = r0 + j - dm_base(l);
        const int64_t na = n0 + loc % kDmTA;
        if (na >= N) continue;
        float* out = R.p[l] + (int64_t)(loc / kDmTA) * R.sx + na * R.sa + c;
        v4f v = acc[i];
        if ((beta_mask >> l) & 1) v += ld4(out);
        if (ys_tab) v *= ld4(ys_tab + (int64_t)group[na] * ld_s + l * C + c);
        st4(out, v);
    }
}

// ------------------------------------------------------------------ backward
template <int KB>
__global__ __launch_bounds__(kDmWaves * kWave) void density_mix_bwd_kernel(
    const float* __restrict__ phi, int ld_phi, const float* __restrict__ msg, int ld_msg,
    const int32_t* __restrict__ msg_row, const float* __restrict__ Y, int ld_Y, const int32_t* __restrict__ row_ptr,
    int64_t N, int C, DmRanks R, const float* __restrict__ xs, int ld_s, const int32_t* __restrict__ group,
    float* __restrict__ dphi, int ld_dphi, float* __restrict__ dmsg, int ld_dmsg, float* __restrict__ dY,
    int ld_dY) {
    constexpr int K = 16 * KB;
    __shared__ float sD[kDmLdsRows * kDmS];
    __shared__ float sY[kDmWaves][16 * kDmYS];
    __shared__ float sP[kDmWaves][512];               // per wave: dphi (16 x 16) | dmsg chunk (16 x 16)
    const int lane = threadIdx.x & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int64_t n0 = (int64_t)blockIdx.x * kDmTA;
    const int CB = C / 16;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    // phase-2 role: row block rb2 (waves with rb2 = 7 rest), basis functions b2, b2 + 2, ...
    const int rb2 = wv & 7, b2 = wv >> 3;
    int l2 = 0, r02 = 0, nv2 = 0;
    if (rb2 < 7) dm_block(rb2, l2, r02, nv2);
    const float* grow = nullptr;                       // this lane's upstream row (c = 16 cc + 4q + r)
    const float* srow = nullptr;
    if (rb2 < 7 && j < nv2) {
        const int loc = r02 + j - dm_base(l2);
        const int64_t na = n0 + loc % kDmTA;
        if (na < N) {
            grow = R.p[l2] + (int64_t)(loc / kDmTA) * R.sx + na * R.sa + 4 * q;
            if (xs) srow = xs + (int64_t)group[na] * ld_s + l2 * C + 4 * q;
        }
    }
    // phase-1 role: atom a, monomials x1 .. x1 + 4; the tile count of the busiest atom (uniform)
    const int a = wv >> 2, xp = wv & 3, x1 = 5 * xp;
    const int64_t n = n0 + a;
    int64_t e_beg = 0, e_end = 0;
    if (n < N) {
        e_beg = row_ptr[n];
        e_end = row_ptr[n + 1];
    }
    int tiles = 0;
#pragma unroll
    for (int aa = 0; aa < kDmTA; ++aa) {
        const int64_t m = n0 + aa;
        if (m < N) tiles = max(tiles, (int)((row_ptr[m + 1] - row_ptr[m] + 15) / 16));
    }
    float* ys = sY[wv];
#pragma unroll 1
    for (int kc = 0; kc < KB; ++kc) {
        // ---- phase 2: dD[row][(b, k)] = sum_c gA[row][c] s[c] W_l^T[(b K + k)][c], k in chunk kc
        if (rb2 < 7) {
#pragma unroll 1
            for (int b = b2; b < 16; b += 2) {
                const float* wt = R.w[l2] + (int64_t)(b * K + 16 * kc + j) * R.ld_w + 4 * q;
                v4f d = z4;
                v4f wn = ld4(wt), gn = grow ? ld4(grow) : z4;
                if (srow) gn *= ld4(srow);
                for (int cc = 0; cc < CB; ++cc) {
                    const v4f w4 = wn, g4 = gn;
                    if (cc + 1 < CB) {                       // next channel block loaded ahead
                        wn = ld4(wt + 16 * (cc + 1));
                        gn = grow ? ld4(grow + 16 * (cc + 1)) : z4;
                        if (srow) gn *= ld4(srow + 16 * (cc + 1));
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) d = mfma_16x16x4(w4[r], g4[r], d);
                }
                // d: dD[row r0 + j][k = 4q + r] of basis b; only the block's own rows are written
                if (j < nv2) st4(sD + (r02 + j) * kDmS + 16 * b + 4 * q, d);
            }
        }
        __syncthreads();
        // ---- phase 1: the atom's edge tiles against the dD chunk (same trip count on every wave)
#pragma unroll 1
        for (int t = 0; t < tiles; ++t) {
            const int64_t e0 = e_beg + 16 * t;
            const int ne = (int)max((int64_t)0, min((int64_t)16, e_end - e0));
            v4f dph = z4, dm = z4;
            if (ne > 0) {
                dm_stage_y(ys, Y, ld_Y, e0, ne, lane);
                const bool oki = j < ne;
                const int64_t ei = e0 + min(j, ne - 1);
                const int64_t rowi = msg_row ? (int64_t)msg_row[ei] : ei;
                const v4f mA = oki ? ld4(msg + rowi * ld_msg + 16 * kc + 4 * q) : z4;
                const v4f ph4 = oki ? ld4(phi + ei * ld_phi + 4 * q) : z4;
                float phT[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) phT[r] = phi[(e0 + min(4 * q + r, ne - 1)) * ld_phi + j];
                float dyk[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
                for (int xx = 0; xx < 5; ++xx) {
                    const int x = x1 + xx;
                    const float* gx = sD + dm_row(x, a) * kDmS;     // dD_x[b][k] at 16 b + k
                    const v4f gv = *reinterpret_cast<const v4f*>(gx + 16 * j + 4 * q);
                    v4f sv = z4;
#pragma unroll
                    for (int r = 0; r < 4; ++r) sv = mfma_16x16x4(mA[r], gv[r], sv);     // S[e = 4q + r][b = j]
                    const float yi = ys[j * kDmYS + x];
#pragma unroll
                    for (int r = 0; r < 4; ++r) dm = mfma_16x16x4(yi * ph4[r], gx[16 * (4 * q + r) + j], dm);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        dph[r] = fmaf(sv[r], ys[(4 * q + r) * kDmYS + x], dph[r]);
                        float v = sv[r] * phT[r];
                        v = row16_sum(v);
                        if (j == xx) dyk[r] = v;
                    }
                }
                // dY of this wave's monomials (lane j < 5 owns monomial x1 + j), summed over the chunks
                if (dY && j < 5) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int te = 4 * q + r;
                        if (te < ne) {
                            float* p = dY + (e0 + te) * ld_dY + x1 + j;
                            *p = kc == 0 ? dyk[r] : *p + dyk[r];
                        }
                    }
                }
            }
            // the four waves' dphi / dmsg partials of this tile, summed by wave (a, 0)
            float* mine = sP[wv];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                mine[(4 * q + r) * 16 + j] = dph[r];
                mine[256 + (4 * q + r) * 16 + j] = dm[r];
            }
            __syncthreads();
            if (xp == 0 && ne > 0) {
#pragma unroll
                for (int w = 1; w < 4; ++w) {
                    const float* o = sP[wv + w];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        dph[r] += o[(4 * q + r) * 16 + j];
                        dm[r] += o[256 + (4 * q + r) * 16 + j];
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int te = 4 * q + r;
                    if (te < ne) {
                        const int64_t e = e0 + te;
                        if (dmsg) dmsg[e * ld_dmsg + 16 * kc + j] = dm[r];
                        if (dphi) {
                            float* p = dphi + e * ld_dphi + j;
                            *p = kc == 0 ? dph[r] : *p + dph[r];
                        }
                    }
                }
            }
            __syncthreads();                                // partials read before the next tile writes
        }
        // (the last __syncthreads of the tile loop also orders this chunk's reads of sD before the
        // next chunk's phase 2; with no tiles, the one below does)
        __syncthreads();
    }
}

static bool dm_aligned(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace face

using namespace face;

extern "C" int face_density_mix_fwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg,
                                    const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr,
                                    int64_t N, int32_t B, int32_t K, int32_t C, const float* const* w_ranks,
                                    int64_t ld_w, float* const* A_ranks, int64_t atom_stride, int64_t x_stride,
                                    const float* y_scale, int32_t ld_scale, const int32_t* group, int32_t beta_mask,
                                    void* stream) {
    if (N < 0 || B != 16 || K < 16 || K > 64 || K % 16 || C < 16 || C > 256 || C % 16 || ld_phi < B || ld_msg < K ||
        ld_Y < 20 || ld_w < B * K || atom_stride < 1 || x_stride < 1)
        return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!phi || !msg || !Y || !row_ptr || !w_ranks || !A_ranks || (y_scale && (!group || ld_scale < 4 * C)))
        return FACE_ERR_ARG;
    DmRanks R{};
    for (int l = 0; l < 4; ++l) {
        R.p[l] = A_ranks[l];
        R.w[l] = w_ranks[l];
        if (!R.p[l] || !R.w[l]) return FACE_ERR_ARG;
        if (!dm_aligned(R.p[l]) || !dm_aligned(R.w[l])) return FACE_ERR_UNSUPPORTED;
    }
    if (atom_stride % 4 || x_stride % 4 || ld_w % 4 || (y_scale && (ld_scale % 4 || !dm_aligned(y_scale))))
        return FACE_ERR_UNSUPPORTED;
    R.sa = atom_stride, R.sx = x_stride, R.ld_w = ld_w;
    const dim3 grid((unsigned)((N + kDmTA - 1) / kDmTA)), block(kDmWaves * kWave);
    const hipStream_t st = (hipStream_t)stream;
    const int ntask = 7 * (C / 16);
    const int tpw = (ntask + kDmWaves - 1) / kDmWaves;                 // 1 .. 7
#define FACE_DMF(KB_, TPW_)                                                                                    \
    hipLaunchKernelGGL((density_mix_fwd_kernel<KB_, TPW_>), grid, block, 0, st, phi, ld_phi, msg, ld_msg, msg_row, \
                       Y, ld_Y, row_ptr, N, C, R, y_scale, ld_scale, group, beta_mask)
#define FACE_DMF_K(TPW_)                    \
    switch (K / 16) {                       \
        case 1: FACE_DMF(1, TPW_); break;   \
        case 2: FACE_DMF(2, TPW_); break;   \
        case 3: FACE_DMF(3, TPW_); break;   \
        default: FACE_DMF(4, TPW_); break;  \
    }
    if (tpw <= 1) {
        FACE_DMF_K(1)
    } else if (tpw <= 3) {
        FACE_DMF_K(3)
    } else if (tpw <= 5) {
        FACE_DMF_K(5)
    } else {
        FACE_DMF_K(7)
    }
#undef FACE_DMF_K
#undef FACE_DMF
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_density_mix_bwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg,
                                    const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr,
                                    int64_t N, int32_t B, int32_t K, int32_t C, const float* const* wt_ranks,
                                    int64_t ld_wt, const float* const* gA_ranks, int64_t atom_stride,
                                    int64_t x_stride, const float* x_scale, int32_t ld_scale, const int32_t* group,
                                    float* dphi, int32_t ld_dphi, float* dmsg, int32_t ld_dmsg, float* dY,
                                    int32_t ld_dY, void* stream) {
    if (N < 0 || B != 16 || K < 16 || K > 64 || K % 16 || C < 16 || C > 256 || C % 16 || ld_phi < B || ld_msg < K ||
        ld_Y < 20 || ld_wt < C || atom_stride < 1 || x_stride < 1 || (dphi && ld_dphi < B) ||
        (dmsg && ld_dmsg < K) || (dY && ld_dY < 20))
        return FACE_ERR_ARG;
    if (N == 0 || (!dphi && !dmsg && !dY)) return 0;
    if (!phi || !msg || !Y || !row_ptr || !wt_ranks || !gA_ranks || (x_scale && (!group || ld_scale < 4 * C)))
        return FACE_ERR_ARG;
    DmRanks R{};
    for (int l = 0; l < 4; ++l) {
        R.p[l] = const_cast<float*>(gA_ranks[l]);
        R.w[l] = wt_ranks[l];
        if (!R.p[l] || !R.w[l]) return FACE_ERR_ARG;
        if (!dm_aligned(R.p[l]) || !dm_aligned(R.w[l])) return FACE_ERR_UNSUPPORTED;
    }
    if (atom_stride % 4 || x_stride % 4 || ld_wt % 4 || ld_msg % 4 || ld_phi % 4 || !dm_aligned(msg) ||
        !dm_aligned(phi) || (x_scale && (ld_scale % 4 || !dm_aligned(x_scale))))
        return FACE_ERR_UNSUPPORTED;
    R.sa = atom_stride, R.sx = x_stride, R.ld_w = ld_wt;
    const dim3 grid((unsigned)((N + kDmTA - 1) / kDmTA)), block(kDmWaves * kWave);
    const hipStream_t st = (hipStream_t)stream;
#define FACE_DMB(KB_)                                                                                           \
    hipLaunchKernelGGL((density_mix_bwd_kernel<KB_>), grid, block, 0, st, phi, ld_phi, msg, ld_msg, msg_row, Y,  \
                       ld_Y, row_ptr, N, C, R, x_scale, ld_scale, group, dphi, ld_dphi, dmsg, ld_dmsg, dY, ld_dY)
    switch (K / 16) {
        case 1: FACE_DMB(1); break;
        case 2: FACE_DMB(2); break;
        case 3: FACE_DMB(3); break;
        default: FACE_DMB(4); break;
    }
#undef FACE_DMB
    FACE_LAUNCH_CHECK();
    return 0;
}
