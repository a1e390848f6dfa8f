// Row-block linear layers of the node features on the fp32 matrix cores (gfx950):
//
//   y[m, :] = (beta y[m, :] + (x[m, :] * xs[m, :]) W^T + bias) * ys[m, :]    (per problem: x, W, y, beta)
//
// for the tall activations of a pass, (k_l N, C) blocks against weights of at most a few
// hundred columns: mix, tmix and proj (face/model.py:498-533, :537-544) and their input
// gradients. xs / ys are per-atom scale rows picked by the atom's element (the elem_scale
// factor of face/model.py:530-533) and are optional, as are beta and bias. Up to four
// problems (the four ranks) share one launch.
//
// Work: a workgroup of NW waves (16 on large problems, 8 or 4 on small ones) owns a slice of
// NS = 16 NB output columns and 32 NW rows; the slice's weight block W[n0 : n0 + NS, 0 : K] sits in LDS (row stride
// K + 4) as the A operand of v_mfma_f32_16x16x4f32, the rows of x stream through registers as
// B operands (K index q of instruction r of chunk kc = input column 16 kc + 4q + r), one chunk
// of 16 columns ahead, and the wave keeps its 32 x NS outputs in registers over the whole K
// loop. D = W . x^T holds output column 4q + r of row j in register r of lane j + 16q, one
// float4 store of y[m][n .. n + 3] per lane and block.
//
// Side operands never wait on memory inside or after the K loop: the scale rows of every group
// (the ys columns of the slice, the xs columns of the problem) and the slice's bias are staged
// in LDS with the weight slice, and beta y is loaded into the accumulators before the K loop
// (its loads complete under the first x rows'). The epilogue therefore reads LDS only, then
// stores. (Epilogue loads from memory cost one full memory latency each: with 80 accumulator
// registers held, the compiler could not keep them in flight together.)
#include "common.h"

#include <algorithm>
#include <cstdlib>
#include <cstdio>
#include <map>
#include <mutex>
#include <vector>

namespace face {

constexpr int kGemmBB = 2;                 // 16-row blocks per wave
constexpr int kGemmMaxProbs = 8;                // problems per launch
constexpr int kGemmMaxGroups = 64;         // scale-table rows (elements) staged in LDS

struct GemmProb {
    const float* x;
    int64_t ld_x, m;
    const float* w;
    int64_t ld_w;
    float* y;
    int64_t ld_y;
    int n, k, s_off, tiles, slices;        // tiles of 32 NW rows, slices of NS columns
    float beta;
    const float* x2;                       // input columns k >= k1 (column k - k1), or null
    int64_t ld_x2;
    int k1, x_op;                          // x_op on columns < k1: 0 none, 1 silu, 2 * silu'(xz)
    const float* xz;
    int64_t ld_xz;
    const float* bias;
    const float* y0;                       // initial sum beta * y0 (columns < n_y0), null: y
    int64_t ld_y0;
    int n_y0;
    int64_t first_block;                   // first work item of this problem
    int64_t cost0;                         // summed cost of the items of the problems before it
    int cost;                              // cost of one of its items (~ K + fixed per-item work)
};

// silu and its derivative with the hardware exp2 and reciprocal (about 1 ulp each)
__device__ __forceinline__ float gemm_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.44269504088896341f * x));
}
__device__ __forceinline__ v4f gemm_silu(v4f x) {
    v4f o;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = x[r] * gemm_sigmoid(x[r]);
    return o;
}
__device__ __forceinline__ v4f gemm_dsilu(v4f g, v4f z) {       // g * d silu(z) / dz
    v4f o;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float sg = gemm_sigmoid(z[r]);
        o[r] = g[r] * (sg * (1.f + z[r] * (1.f - sg)));
    }
    return o;
}

struct GemmArgs {
    GemmProb p[kGemmMaxProbs];
    int64_t items;                         // (problem, slice, tile) work items over all problems
    int64_t total_cost;
    int n_probs, w_kn, NS;
    const float *xs, *ys;
    int any_bias;                          // some problem has a bias (side table present)
    int ld_s, n_groups;
    const int32_t* group;
    int64_t period;
    int side_off, kmax;                    // LDS offset (floats) of the side tables; largest K
    int xcd_order;                         // one-item launches: items in XCD-contiguous ranges
};

// LDS side tables of a launch, after the weight slice (floats): ys [n_groups][16 NB] (slice
// columns), xs [n_groups][kmax] (problem columns), bias [16 NB] -- each present only when its
// operand is.
struct GemmSide {
    float *ys, *xs, *bias;
    __device__ __forceinline__ GemmSide(float* base, const GemmArgs& A, int nsb) {
        ys = base;
        xs = ys + (A.ys ? A.n_groups * nsb : 0);
        bias = xs + (A.xs ? A.n_groups * A.kmax : 0);       // present when A.any_bias
    }
};

// Stage the side tables of (problem P, slice n0 .. n0 + ns) into LDS (callers synchronise);
// columns past ns are zero. The xs rows are restaged only with a new problem.
__device__ __forceinline__ void gemm_stage_side(const GemmArgs& A, const GemmProb& P, const GemmSide& S, int nsb, int n0,
                                                int ns, bool new_prob, int tid) {
    const int nthr = blockDim.x;
    if (A.ys) {
        for (int v = tid; v < A.n_groups * nsb; v += nthr) {
            const int g = v / nsb, c = v - g * nsb;
            S.ys[v] = c < ns ? A.ys[(int64_t)g * A.ld_s + P.s_off + n0 + c] : 0.f;
        }
    }
    if (A.xs && new_prob) {
        for (int v = tid; v < A.n_groups * P.k; v += nthr) {
            const int g = v / P.k, k = v - g * P.k;
            S.xs[g * A.kmax + k] = A.xs[(int64_t)g * A.ld_s + P.s_off + k];
        }
    }
    if (A.any_bias) {
        for (int c = tid; c < nsb; c += nthr) S.bias[c] = (c < ns && P.bias) ? P.bias[n0 + c] : 0.f;
    }
}

// XM: input mode -- 0 plain, 1 the per-group x scale (xs), 2 the per-problem transform x_op
template <int NB, int NW, bool PERSIST, int XM>
__global__ __launch_bounds__(NW * kWave) void rows_gemm_kernel(GemmArgs A) {
    constexpr bool XS = XM == 1, XO = XM == 2;
    extern __shared__ float sW[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int j = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    auto item_at = [&](int64_t target) -> int64_t {     // first item starting at or past target
        int p = 0;
#pragma unroll 1
        for (int k = 1; k < A.n_probs; ++k)
            if (target >= A.p[k].cost0) p = k;
        const int64_t i = A.p[p].first_block + (target - A.p[p].cost0 + A.p[p].cost - 1) / A.p[p].cost;
        return min(i, A.items);
    };
    const bool one = !PERSIST || A.items <= gridDim.x;
    const int64_t it_beg = one ? blockIdx.x : item_at(A.total_cost * (int64_t)blockIdx.x / gridDim.x);
    const int64_t it_end = one ? min(A.items, (int64_t)blockIdx.x + 1) : item_at(A.total_cost * ((int64_t)blockIdx.x + 1) / gridDim.x);
    int cur_pi = -1, cur_slice = -1;
    // Work items: (problem, column slice, row tile). Persistent runs walk 32-row wave tiles,
    // slice by slice: the workgroup stages a slice once, then its waves take the run's tiles of
    // that slice round robin (at most one tile of imbalance per wave); one item per workgroup is a
    // tile of 32 NW rows.
    auto locate = [&](int64_t it, int& pi, int& slice, int64_t& tile) {
        pi = 0;
#pragma unroll 1
        for (int k = 1; k < A.n_probs; ++k)
            if (it >= A.p[k].first_block) pi = k;
        const int64_t local = it - A.p[pi].first_block;
        slice = PERSIST ? (int)(local / A.p[pi].tiles) : (int)(local % A.p[pi].slices);
        tile = PERSIST ? local - (int64_t)slice * A.p[pi].tiles : local / A.p[pi].slices;
    };
    // stage the weight slice and the side tables of (pi, slice) unless they are staged
    auto stage = [&](int pi, int slice) __attribute__((always_inline)) {
        const GemmProb& P = A.p[pi];
        const int K = P.k, SK = K + 4;
        const int n0 = slice * A.NS;
        const int ns = min(A.NS, P.n - n0);                             // a multiple of 16
        const GemmSide side(sW + A.side_off, A, 16 * NB);
        if (pi != cur_pi || slice != cur_slice) {
            // stage W[n0 : n0 + ns, :] as rows of K (+ 4 pad); rows ns .. 16 NB - 1 are zero, so
            // the MFMA loop below runs all NB blocks without branches
            if (PERSIST) __syncthreads();                                // every wave is done with the old slice
            // the thread index through an empty asm: the staging addresses are rebuilt per staging
            // instead of being held (spilled) across the persistent loop
            int tid = threadIdx.x;
            asm volatile("" : "+v"(tid));
            // four loads per thread issued before their LDS stores (a loop that stores each
            // float4 before loading the next waits a memory latency per round)
            const float* __restrict__ wsrc = P.w;
            const int64_t ldw = P.ld_w;
            const int nthr = blockDim.x;
            if (!A.w_kn) {
                const int nk4 = K / 4, tot = 16 * NB * nk4;
                for (int v0 = tid; v0 < tot; v0 += 4 * nthr) {
                    v4f b[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int v = v0 + u * nthr, r = v / nk4, c4 = v - r * nk4;
                        b[u] = (v < tot && r < ns) ? ld4(wsrc + (int64_t)(n0 + r) * ldw + 4 * c4) : z4;
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int v = v0 + u * nthr, r = v / nk4, c4 = v - r * nk4;
                        if (v < tot) st4(sW + r * SK + 4 * c4, b[u]);
                    }
                }
            } else {                                                     // W given as (K, n)
                // item (k4, r): four coalesced reads down column n0 + r, one float4 into row r
                const int nr = 16 * NB, tot = nr * (K / 4);
                for (int v0 = tid; v0 < tot; v0 += 2 * nthr) {
                    v4f b[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int v = v0 + u * nthr, k4 = v / nr, r = v - k4 * nr;
                        b[u] = z4;
                        if (v < tot && r < ns) {
                            const float* col = wsrc + (int64_t)(4 * k4) * ldw + n0 + r;
#pragma unroll
                            for (int c = 0; c < 4; ++c) b[u][c] = col[c * ldw];
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int v = v0 + u * nthr, k4 = v / nr, r = v - k4 * nr;
                        if (v < tot) st4(sW + r * SK + 4 * k4, b[u]);
                    }
                }
            }
            gemm_stage_side(A, P, side, 16 * NB, n0, ns, pi != cur_pi, tid);
            __syncthreads();
            cur_pi = pi, cur_slice = slice;
        }
    };
    // rows m0 .. m0 + 31 of problem pi against the staged slice
    auto compute = [&](int pi, int slice, int64_t m0) __attribute__((always_inline)) {
        const GemmProb& P = A.p[pi];
        const int K = P.k, SK = K + 4;
        const int n0 = slice * A.NS;
        const int ns = min(A.NS, P.n - n0);
        const GemmSide side(sW + A.side_off, A, 16 * NB);
        if (m0 >= P.m) return;
        // rows as 32-bit element offsets from the problem's base pointers (the host checks that
        // every operand's rows fit), so that each row costs one register per operand
        bool ok[kGemmBB];
        int rcs[kGemmBB];
        int xo[kGemmBB], yo[kGemmBB];
        int xso[kGemmBB], yso[kGemmBB];                                  // LDS offsets of the row's scale rows
#pragma unroll
        for (int bb = 0; bb < kGemmBB; ++bb) {
            const int64_t row = m0 + 16 * bb + j;
            ok[bb] = row < P.m;
            rcs[bb] = ok[bb] ? (int)row : 0;
            xo[bb] = rcs[bb] * (int)P.ld_x + 4 * q;
            yo[bb] = rcs[bb] * (int)P.ld_y + 4 * q;
            const int g = A.group ? A.group[rcs[bb] % A.period] : 0;
            xso[bb] = g * A.kmax + 4 * q;
            yso[bb] = g * (16 * NB) + 4 * q;
        }
        // input column block kc of row bb: x for columns < k1, x2 beyond (the second range only in
        // the XM = 2 kernels; k1 is a multiple of 16)
        auto x_at = [&](int bb, int kc) -> const float* {
            const int c0 = 16 * kc;
            if (!XO) return P.x + (xo[bb] + c0);
            return c0 < P.k1 ? P.x + (xo[bb] + c0) : P.x2 + (rcs[bb] * (int)P.ld_x2 + (c0 - P.k1) + 4 * q);
        };
        auto load_x = [&](int kc, v4f (&xv)[kGemmBB], v4f (&zv)[kGemmBB]) {
#pragma unroll
            for (int bb = 0; bb < kGemmBB; ++bb) {
                xv[bb] = ok[bb] ? ld4(x_at(bb, kc)) : z4;
                if (XO && P.x_op == 2 && 16 * kc < P.k1)
                    zv[bb] = ok[bb] ? ld4(P.xz + (rcs[bb] * (int)P.ld_xz + 16 * kc + 4 * q)) : z4;
            }
        };
        // accumulators start at beta y (XM = 2: beta y0 over its first n_y0 columns), the loads
        // in flight with the first x rows, else zero
        v4f acc[NB][kGemmBB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int bb = 0; bb < kGemmBB; ++bb) {
                acc[nb][bb] = z4;
                if (P.beta != 0.f && ok[bb] && 16 * nb < ns) {
                    if (!XO) {
                        acc[nb][bb] = ld4(P.y + (yo[bb] + n0 + 16 * nb));
                    } else if (n0 + 16 * nb + 4 * q < P.n_y0) {
                        acc[nb][bb] = P.y0 ? ld4(P.y0 + (rcs[bb] * (int)P.ld_y0 + n0 + 16 * nb + 4 * q))
                                           : ld4(P.y + (yo[bb] + n0 + 16 * nb));
                    }
                    if (P.beta != 1.f) acc[nb][bb] *= P.beta;
                }
            }
        const int nkc = K / 16;
        v4f xn[kGemmBB], zn[kGemmBB];
        load_x(0, xn, zn);
#pragma unroll 1
        for (int kc = 0; kc < nkc; ++kc) {
            v4f xv[kGemmBB];
#pragma unroll
            for (int bb = 0; bb < kGemmBB; ++bb) {
                xv[bb] = xn[bb];
                if (XS) xv[bb] *= *reinterpret_cast<const v4f*>(side.xs + xso[bb] + 16 * kc);
                if (XO && 16 * kc < P.k1) {
                    if (P.x_op == 1) xv[bb] = gemm_silu(xv[bb]);
                    else if (P.x_op == 2) xv[bb] = gemm_dsilu(xv[bb], zn[bb]);
                }
            }
            if (kc + 1 < nkc) load_x(kc + 1, xn, zn);
            // weight blocks read one block ahead of their MFMAs (LDS latency under the MFMA chain)
            const float* wrow = sW + j * SK + 16 * kc + 4 * q;
            v4f wa = *reinterpret_cast<const v4f*>(wrow);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const v4f wn = nb + 1 < NB ? *reinterpret_cast<const v4f*>(wrow + 16 * (nb + 1) * SK) : wa;
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int bb = 0; bb < kGemmBB; ++bb) acc[nb][bb] = mfma_16x16x4(wa[r], xv[bb][r], acc[nb][bb]);
                wa = wn;
            }
            // issue order: reads of blocks 0 and 1, then per block its 4 kGemmBB MFMAs followed by
            // the read of block nb + 2, so every read has a block of MFMAs to hide under
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if (nb == 0) __builtin_amdgcn_sched_group_barrier(0x100, (NB > 1 ? 2 : 1) + (XS ? kGemmBB : 0), 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 4 * kGemmBB, 0);
                if (nb + 2 < NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
        // epilogue: bias and y scale from LDS, then the stores
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (16 * nb < ns) {
                const v4f bias = A.any_bias ? *reinterpret_cast<const v4f*>(side.bias + 16 * nb + 4 * q) : z4;
#pragma unroll
                for (int bb = 0; bb < kGemmBB; ++bb) {
                    v4f v = acc[nb][bb] + bias;
                    if (A.ys) v *= *reinterpret_cast<const v4f*>(side.ys + yso[bb] + 16 * nb);
                    if (ok[bb]) st4(P.y + (yo[bb] + n0 + 16 * nb), v);
                }
            }
        }
    };
    if (PERSIST) {
        int64_t it = it_beg;
        while (it < it_end) {                                            // uniform over the workgroup
            int pi, slice;
            int64_t t;
            locate(it, pi, slice, t);
            const GemmProb& P = A.p[pi];
            const int64_t seg_end = min(it_end, P.first_block + (int64_t)(slice + 1) * P.tiles);
            stage(pi, slice);
            for (int64_t w = it + wv; w < seg_end; w += NW)
                compute(pi, slice, (w - P.first_block - (int64_t)slice * P.tiles) * (16 * kGemmBB));
            it = seg_end;
        }
    } else {
        int pi, slice;
        int64_t t;
        // XCD-aware item order (xcd_order): workgroup b runs on XCD b % 8, so each XCD takes a
        // contiguous range of items and the column slices of a row tile share its L2 for the rows
        int64_t item = blockIdx.x;
        if (A.xcd_order) {
            const int64_t nbk = gridDim.x, bx = blockIdx.x, xcd = bx & 7, per = nbk >> 3, rem = nbk & 7;
            item = xcd * per + (xcd < rem ? xcd : rem) + (bx >> 3);
        }
        locate(item, pi, slice, t);
        stage(pi, slice);
        compute(pi, slice, (t * NW + wv) * (16 * kGemmBB));
    }
}

// ------------------------------------------------------------------ K-chunked row GEMM
// The whole-K weight slice of rows_gemm_kernel leaves narrow column slices once K grows (K = 1024:
// 32 columns), and every slice re-reads its x rows. Here the weight slice of NS = 16 NB columns
// (up to 256) is streamed through LDS in chunks of 32 k (row stride 36 floats: the 16 rows one
// instruction reads sit on distinct banks), double-buffered: the next chunk's loads are issued
// before the current chunk's products and written to the other buffer after them, one barrier
// per chunk. As in rows_gemm_kernel each of the 8 waves streams 32 x rows as B operands (two
// 16-column steps ahead) and keeps its 32 x NS outputs in registers over the whole K loop.
// Workgroups take the items (problem, 256-row tile, column slice), slice fastest, in an
// XCD-aware order (workgroup b runs on XCD b % 8, each XCD a contiguous range of items) so that
// the slices of a row tile read its rows from one L2. The epilogue (bias, beta y, y scale)
// loads all its operands before its stores.
constexpr int kKcWaves = 8, kKcK = 32, kKcS = 36;

template <int NB>
__global__ __launch_bounds__(kKcWaves * kWave) void rows_gemm_kc_kernel(GemmArgs A) {
    constexpr int NSB = 16 * NB;                              // columns of the slice buffer
    constexpr int WI = (NSB * (kKcK / 4) + kKcWaves * kWave - 1) / (kKcWaves * kWave);   // float4 items per thread
    __shared__ float sW[2][NSB * kKcS];
    extern __shared__ float sSide[];                          // side tables (GemmSide), dynamic
    const int tid = threadIdx.x, lane = tid & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    const int64_t nbk = gridDim.x, bx = blockIdx.x, xcd = bx & 7, kx = bx >> 3;
    const int64_t per = nbk >> 3, rem = nbk & 7;
    const int64_t it = xcd * per + (xcd < rem ? xcd : rem) + kx;
    int pi = 0;
#pragma unroll
    for (int k = 1; k < kGemmMaxProbs; ++k)
        if (k < A.n_probs && it >= A.p[k].first_block) pi = k;
    const GemmProb& P = A.p[pi];
    const int64_t local = it - P.first_block;
    const int64_t tile = local / P.slices;
    const int slice = (int)(local - tile * P.slices);
    const int n0 = slice * A.NS, K = P.k;
    const int ns = min(A.NS, P.n - n0);
    // weight chunk staging: item v = col * 8 + k4 (w as (n, k)) or k * (NSB / 4) + c4 (w as (k, n))
    auto load_w = [&](int k0, v4f (&bw)[WI]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < WI; ++u) {
            const int v = u * kKcWaves * kWave + tid;
            v4f t = z4;
            if (v < NSB * (kKcK / 4)) {
                if (!A.w_kn) {
                    const int col = v >> 3, k = k0 + 4 * (v & 7);
                    if (col < ns && k < K) t = ld4(P.w + (int64_t)(n0 + col) * P.ld_w + k);
                } else {
                    const int k = k0 + v / (NSB / 4), c4 = v % (NSB / 4);
                    if (k < K && 4 * c4 < ns) t = ld4(P.w + (int64_t)k * P.ld_w + n0 + 4 * c4);
                }
            }
            bw[u] = t;
        }
    };
    auto store_w = [&](int buf, const v4f (&bw)[WI]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < WI; ++u) {
            const int v = u * kKcWaves * kWave + tid;
            if (v < NSB * (kKcK / 4)) {
                if (!A.w_kn) {
                    st4(&sW[buf][(v >> 3) * kKcS + 4 * (v & 7)], bw[u]);
                } else {
                    const int kk = v / (NSB / 4), c4 = v % (NSB / 4);
#pragma unroll
                    for (int c = 0; c < 4; ++c) sW[buf][(4 * c4 + c) * kKcS + kk] = bw[u][c];
                }
            }
        }
    };
    const int64_t m0 = (tile * kKcWaves + wv) * (16 * kGemmBB);
    const GemmSide side(sSide, A, NSB);
    bool ok[kGemmBB];
    const float* xr[kGemmBB];
    const float* x2r[kGemmBB];
    float* yr[kGemmBB];
    int xso[kGemmBB], yso[kGemmBB];                            // LDS offsets of the row's scale rows
#pragma unroll
    for (int bb = 0; bb < kGemmBB; ++bb) {
        const int64_t row = m0 + 16 * bb + j;
        ok[bb] = row < P.m;
        const int64_t rc = ok[bb] ? row : 0;
        xr[bb] = P.x + rc * P.ld_x + 4 * q;
        x2r[bb] = P.x2 + rc * P.ld_x2 + 4 * q;
        yr[bb] = P.y + rc * P.ld_y + 4 * q;
        const int g = A.group ? A.group[rc % A.period] : 0;
        xso[bb] = g * A.kmax + 4 * q;
        yso[bb] = g * NSB + 4 * q;
    }
    const int nks = K / 16;                                    // 16-column steps of x
    // x rows of 16-column step ks (columns >= k1 from x2, k1 % 16 == 0) and, for x_op 2, the
    // matching pre-activation rows
    auto load_x = [&](int ks, v4f (&xv)[kGemmBB], v4f (&zv)[kGemmBB]) __attribute__((always_inline)) {
#pragma unroll
        for (int bb = 0; bb < kGemmBB; ++bb) {
            xv[bb] = (ok[bb] && ks < nks) ? ld4(16 * ks < P.k1 ? xr[bb] + 16 * ks : x2r[bb] + (16 * ks - P.k1)) : z4;
            if (P.x_op == 2 && 16 * ks < P.k1)
                zv[bb] = (ok[bb] && ks < nks) ? ld4(P.xz + (m0 + 16 * bb + j) * P.ld_xz + 16 * ks + 4 * q) : z4;
        }
    };
    {
        v4f bw[WI];
        load_w(0, bw);
        store_w(0, bw);
    }
    gemm_stage_side(A, P, side, NSB, n0, ns, true, tid);
    // accumulators start at beta y (loads in flight with the first x rows), else zero
    v4f acc[NB][kGemmBB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int bb = 0; bb < kGemmBB; ++bb) {
            acc[nb][bb] = z4;
            const int c = n0 + 16 * nb + 4 * q;
            if (P.beta != 0.f && ok[bb] && 16 * nb < ns && c < P.n_y0) {
                acc[nb][bb] = P.y0 ? ld4(P.y0 + (m0 + 16 * bb + j) * P.ld_y0 + c) : ld4(yr[bb] + n0 + 16 * nb);
                if (P.beta != 1.f) acc[nb][bb] *= P.beta;
            }
        }
    v4f x0[kGemmBB], x1[kGemmBB], z0[kGemmBB], z1[kGemmBB];
    load_x(0, x0, z0);
    load_x(1, x1, z1);
    __syncthreads();
    const int nchunk = (K + kKcK - 1) / kKcK;
#pragma unroll 1
    for (int c = 0; c < nchunk; ++c) {
        const int buf = c & 1;
        const bool more = c + 1 < nchunk;
        v4f bw[WI];
        if (more) load_w((c + 1) * kKcK, bw);
#pragma unroll
        for (int s2 = 0; s2 < kKcK / 16; ++s2) {
            const int ks = 2 * c + s2;
            if (ks >= nks) break;
            v4f xv[kGemmBB];
#pragma unroll
            for (int bb = 0; bb < kGemmBB; ++bb) {
                xv[bb] = x0[bb];
                if (A.xs) xv[bb] *= *reinterpret_cast<const v4f*>(side.xs + xso[bb] + 16 * ks);
                if (P.x_op == 1 && 16 * ks < P.k1) xv[bb] = gemm_silu(xv[bb]);
                if (P.x_op == 2 && 16 * ks < P.k1) xv[bb] = gemm_dsilu(xv[bb], z0[bb]);
                x0[bb] = x1[bb];
                z0[bb] = z1[bb];
            }
            load_x(ks + 2, x1, z1);                           // two 16-column steps ahead
            const float* wrow = sW[buf] + j * kKcS + 16 * s2 + 4 * q;
            v4f wa = *reinterpret_cast<const v4f*>(wrow);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const v4f wn = nb + 1 < NB ? *reinterpret_cast<const v4f*>(wrow + 16 * (nb + 1) * kKcS) : wa;
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int bb = 0; bb < kGemmBB; ++bb) acc[nb][bb] = mfma_16x16x4(wa[r], xv[bb][r], acc[nb][bb]);
                wa = wn;
            }
        }
        if (more) store_w(buf ^ 1, bw);
        __syncthreads();
    }
    // epilogue: bias and y scale from LDS, then the stores
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if (16 * nb < ns) {
            const v4f bias = A.any_bias ? *reinterpret_cast<const v4f*>(side.bias + 16 * nb + 4 * q) : z4;
#pragma unroll
            for (int bb = 0; bb < kGemmBB; ++bb) {
                v4f v = acc[nb][bb] + bias;
                if (A.ys) v *= *reinterpret_cast<const v4f*>(side.ys + yso[bb] + 16 * nb);
                if (ok[bb]) st4(yr[bb] + n0 + 16 * nb, v);
            }
        }
    }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Route of a launch: the K-chunked kernel for K >= 1024 with at least two 256-row tiles per CU
// (whole-K slices are then at most 32 columns wide, and every slice re-reads the x rows);
// measured on 2M-row problems: K = 1024, n = 256 9.18 against 10.0 ms (in the 100k-atom step's
// mix forward 9.7 against 11.8 ms); at K = 512 (64-column slices, n = 768) the whole-K kernel
// stays faster (12.9 against 13.9 ms), at K = 768 with (k, n) weights too (the 100k-atom proj
// backward 6.3 against 7.7 ms), and so it does for small row counts. FACE_ROWS_GEMM_KC=0 / 1 in
// the environment forces either kernel.
// Whole-K slices narrower than 64 columns (K >= ~600) re-read every x row once per 16-32 columns:
// the K-chunked kernel also serves those (the readout input layer, K = 10 C) once there are a
// few of its 256-row tiles per CU.
static bool use_kc_gemm(int K, int ns_max, int n_widest, int64_t rows) {
    const char* e = getenv("FACE_ROWS_GEMM_KC");
    if (e && (e[0] == '0' || e[0] == '1')) return e[0] == '1';
    const int64_t n_cu = device_cu_count();
    return K >= 1024 && n_widest > ns_max && (rows >= n_cu * 512 || (ns_max < 64 && rows >= n_cu * 32));
}

}  // namespace face

using namespace face;

// Validate problem s and fill p (everything but the tiling); 0 or a FACE_ERR_* status.
static int fill_prob(const face_lin_problem& s, int w_kn, bool scaled, const float* x_scale, const float* y_scale,
                     int ld_scale, GemmProb& p) {
    if (s.m < 0 || s.n < 16 || s.n % 16 || s.k < 16 || s.k % 16 || s.ld_y < s.n || s.ld_w < (w_kn ? s.n : s.k))
        return FACE_ERR_ARG;
    const int k1 = s.x2 ? s.k1 : s.k;
    if (k1 < 0 || k1 > s.k || k1 % 16 || s.ld_x < k1 || (s.x2 && s.ld_x2 < s.k - k1)) return FACE_ERR_ARG;
    if (s.x_op < 0 || s.x_op > 2 || (s.x_op == 2 && (!s.xz || s.ld_xz < k1)) || (s.x_op && x_scale)) return FACE_ERR_ARG;
    if (s.y0 && (s.n_y0 < 0 || s.n_y0 > s.n || s.n_y0 % 4 || s.ld_y0 < s.n_y0)) return FACE_ERR_ARG;
    if (scaled && (s.s_off < 0 || s.s_off % 4 || s.s_off + (x_scale ? s.k : 0) > ld_scale ||
                   s.s_off + (y_scale ? s.n : 0) > ld_scale))
        return FACE_ERR_ARG;
    if (s.m > 0 && (!s.x || !s.w || !s.y)) return FACE_ERR_ARG;
    // rows_gemm_kernel addresses rows by 32-bit element offsets from each operand's base
    const int64_t lim = (int64_t)1 << 31;
    if (s.m * s.ld_x >= lim || s.m * s.ld_y >= lim || (s.x2 && s.m * s.ld_x2 >= lim) ||
        (s.x_op == 2 && s.m * s.ld_xz >= lim) || (s.y0 && s.m * s.ld_y0 >= lim))
        return FACE_ERR_UNSUPPORTED;
    if (s.ld_x % 4 || s.ld_y % 4 || !al16(s.x) || !al16(s.y) || (!w_kn && (!al16(s.w) || s.ld_w % 4)) ||
        (s.x2 && (!al16(s.x2) || s.ld_x2 % 4)) || (s.x_op == 2 && (!al16(s.xz) || s.ld_xz % 4)) ||
        (s.bias && !al16(s.bias)) || (s.y0 && (!al16(s.y0) || s.ld_y0 % 4)))
        return FACE_ERR_UNSUPPORTED;
    p.x = s.x, p.ld_x = s.ld_x, p.m = s.m, p.w = s.w, p.ld_w = s.ld_w, p.y = s.y, p.ld_y = s.ld_y, p.n = s.n;
    p.k = s.k, p.s_off = s.s_off, p.beta = s.beta;
    p.x2 = s.x2 ? s.x2 : s.x, p.ld_x2 = s.x2 ? s.ld_x2 : s.ld_x, p.k1 = k1;
    p.x_op = s.x_op, p.xz = s.x_op == 2 ? s.xz : s.x, p.ld_xz = s.x_op == 2 ? s.ld_xz : s.ld_x;
    p.bias = s.bias;
    p.y0 = s.y0, p.ld_y0 = s.y0 ? s.ld_y0 : 0, p.n_y0 = s.y0 ? s.n_y0 : s.n;
    return 0;
}

// Everything a sliced launch needs but its shape (waves per workgroup, column slices).
struct RowsCtx {
    GemmArgs A;                                  // problems filled, tiling not yet
    const face_lin_problem* probs;
    int n_probs, K, n_widest, ns_max, max_lds, n_cu, n_groups;
    bool w_kn, x_scale, y_scale, any_bias, any_ext;
    hipStream_t st;
    // LDS floats of the side tables for a slice of ns columns (GemmSide)
    int side_floats(int ns) const {
        return (y_scale ? n_groups * ns : 0) + (x_scale ? n_groups * K : 0) + (any_bias ? ns : 0);
    }
};

// 16-wave workgroups (4 waves per SIMD hide the row loads) unless that leaves CUs idle; else 8
// (the staged weight slice serves twice the rows of 4 waves), except for several column slices
// of a (K, n) weight, measured better with 4.
static int default_nw(const RowsCtx& c, int NS) {
    auto wgs_for = [&](int nw) {
        int64_t t = 0;
        for (int i = 0; i < c.n_probs; ++i) t += (c.probs[i].m + 16 * kGemmBB * nw - 1) / (16 * kGemmBB * nw);
        return t;
    };
    bool kn_slices = false;
    for (int i = 0; i < c.n_probs; ++i)
        if (c.w_kn && c.probs[i].m > 0 && c.probs[i].n > NS) kn_slices = true;
    return wgs_for(16) >= c.n_cu ? 16 : (!kn_slices || wgs_for(8) >= c.n_cu ? 8 : 4);
}

// One launch of rows_gemm_kernel with NW waves per workgroup and the widest problem split into
// n_sl column slices (NS = its width rounded up to 16 columns); FACE_ERR_UNSUPPORTED, before
// anything is launched, if that shape does not fit.
static int launch_rows(const RowsCtx& c, int NW, int n_sl, int xcd_order = 0) {
    if (n_sl < 1 || (NW != 4 && NW != 8 && NW != 16)) return FACE_ERR_UNSUPPORTED;
    const int NS = ((c.n_widest + n_sl - 1) / n_sl + 15) / 16 * 16;
    if (NS > c.ns_max || NS > 160) return FACE_ERR_UNSUPPORTED;
    GemmArgs A = c.A;
    A.xcd_order = xcd_order;
    int max_n = 16;
    int64_t blocks = 0, total_cost = 0;
    for (int i = 0; i < c.n_probs; ++i) {
        const face_lin_problem& s = c.probs[i];
        GemmProb& p = A.p[i];
        p.tiles = (int)((s.m + 16 * kGemmBB * NW - 1) / (16 * kGemmBB * NW));
        p.slices = (s.n + NS - 1) / NS;
        p.first_block = blocks;
        p.cost0 = total_cost;
        p.cost = s.k + 64;
        blocks += (int64_t)p.tiles * p.slices;
        total_cost += (int64_t)p.tiles * p.slices * p.cost;
        if (s.n > max_n) max_n = s.n;
    }
    for (int i = c.n_probs; i < kGemmMaxProbs; ++i) A.p[i].first_block = A.p[i].cost0 = INT64_MAX;
    if (blocks == 0) return 0;
    A.NS = NS;
    A.items = blocks;
    A.total_cost = total_cost;
    const int nb = (max_n < NS ? max_n : NS) / 16;
    A.side_off = nb * 16 * (c.K + 4);
    const size_t lds = ((size_t)A.side_off + c.side_floats(nb * 16)) * sizeof(float);
    // persistent grid: as many workgroups as fit on the device at once, each on a contiguous run
    // of the work items
    int64_t wg_cu = (int64_t)c.max_lds / (int64_t)lds;
    if (wg_cu > 32 / NW) wg_cu = 32 / NW;
    if (wg_cu < 1) wg_cu = 1;
    // Persistent runs when the work outnumbers the resident workgroups and no weight slice has to
    // be staged again per row tile: single-slice problems, or (n, K) weights whose slices stage
    // from contiguous rows. Otherwise one work item per workgroup, tile by tile, so the slices of
    // a row tile share its rows in cache (measured better for multi-slice (K, n) weights of
    // large K and for launches that fit the device at once).
    bool multi_slice = false;
    for (int i = 0; i < c.n_probs; ++i)
        if (A.p[i].slices > 1 && A.p[i].tiles > 0) multi_slice = true;
    const bool persist = blocks > c.n_cu * wg_cu && (!c.w_kn || !multi_slice);
    if (persist) {
        // persistent runs count 32-row wave tiles as items (the cost split can then end a run
        // inside a workgroup tile; the run's waves share its tiles)
        blocks = total_cost = 0;
        for (int i = 0; i < c.n_probs; ++i) {
            GemmProb& p = A.p[i];
            p.tiles = (int)((c.probs[i].m + 16 * kGemmBB - 1) / (16 * kGemmBB));
            p.first_block = blocks;
            p.cost0 = total_cost;
            blocks += (int64_t)p.tiles * p.slices;
            total_cost += (int64_t)p.tiles * p.slices * p.cost;
        }
        A.items = blocks;
        A.total_cost = total_cost;
    }
    const int64_t grid = persist ? c.n_cu * wg_cu : blocks;
    const hipStream_t st = c.st;
#define FACE_GEMM_P(NB_, P_, X_)                                                                            \
    do {                                                                                                    \
        auto kern = NW == 16 ? rows_gemm_kernel<NB_, 16, P_, X_>                                            \
                             : (NW == 8 ? rows_gemm_kernel<NB_, 8, P_, X_> : rows_gemm_kernel<NB_, 4, P_, X_>); \
        if (lds > 65536 &&                                                                                  \
            hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != \
                hipSuccess)                                                                                 \
            return FACE_ERR_UNSUPPORTED;                                                                    \
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NW * kWave), lds, st, A);                      \
    } while (0)
    const int xm = c.x_scale ? 1 : (c.any_ext ? 2 : 0);
#define FACE_GEMM(NB_)                     \
    do {                                   \
        if (persist && xm == 1)            \
            FACE_GEMM_P(NB_, true, 1);     \
        else if (persist && xm == 2)       \
            FACE_GEMM_P(NB_, true, 2);     \
        else if (persist)                  \
            FACE_GEMM_P(NB_, true, 0);     \
        else if (xm == 1)                  \
            FACE_GEMM_P(NB_, false, 1);    \
        else if (xm == 2)                  \
            FACE_GEMM_P(NB_, false, 2);    \
        else                               \
            FACE_GEMM_P(NB_, false, 0);    \
    } while (0)
    switch (nb) {
        case 1: FACE_GEMM(1); break;
        case 2: FACE_GEMM(2); break;
        case 3: FACE_GEMM(3); break;
        case 4: FACE_GEMM(4); break;
        case 5: FACE_GEMM(5); break;
        case 6: FACE_GEMM(6); break;
        case 7: FACE_GEMM(7); break;
        case 8: FACE_GEMM(8); break;
        case 9: FACE_GEMM(9); break;
        default: FACE_GEMM(10); break;
    }
#undef FACE_GEMM
#undef FACE_GEMM_P
    FACE_LAUNCH_CHECK();
    return 0;
}

// Launch shapes picked per problem signature by timing. The shape that the rules above pick is
// near the best on most launches, but measured 20-30 % off on some small ones (e.g. 17,280 rows
// of 96 -> 512 columns with an input scale: 32 against 26 us; 26,880 rows of 512 -> 96: 48 against
// 33 us), and the best shape moves irregularly with the row count. So the first call of a
// signature (device, problem shapes, transposition, scales, kernel form) times every shape of
// 4, 8 or 16 waves and distinct slice widths (three launches each, then the three fastest and the
// rule's own five times more, also with an XCD-aware item order for one-item launches) and keeps
// the fastest unless it beats the rule's by less than 2 %.
// Every shape computes each output with the same instructions in the same order, so results are
// bitwise the same whatever the shape. Timing needs launches that can run again with the same
// result: only calls whose problems all have beta = 0 (or read beta y0 from another tensor), on a
// stream that is not being captured, are timed; others use a shape timed earlier for the same
// signature, else the rules. FACE_GEMM_TUNE=0 in the environment keeps the rules.
struct ShapePlan {
    int nw, n_sl, xcd;
};
static std::mutex g_plan_mu;
static std::map<std::vector<int64_t>, ShapePlan> g_plans;

static void pick_shape(const RowsCtx& c, ShapePlan& plan) {
    const int NW = plan.nw, n_sl = plan.n_sl;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    std::vector<int64_t> key = {dev, c.n_probs, c.w_kn, c.x_scale, c.y_scale, c.n_groups, c.any_ext, c.any_bias};
    for (int i = 0; i < c.n_probs; ++i) {
        key.push_back(c.probs[i].m);
        key.push_back(c.probs[i].n);
        key.push_back(c.probs[i].k);
    }
    {
        std::lock_guard<std::mutex> lk(g_plan_mu);
        auto it = g_plans.find(key);
        if (it != g_plans.end()) {
            plan = it->second;
            return;
        }
    }
    const char* env = getenv("FACE_GEMM_TUNE");
    if (env && env[0] == '0') return;
    for (int i = 0; i < c.n_probs; ++i) {
        const face_lin_problem& s = c.probs[i];
        if (s.beta != 0.f && (!s.y0 || s.y0 == s.y)) return;          // accumulating: not re-runnable
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(c.st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return;
    std::vector<ShapePlan> cand = {{NW, n_sl, 0}};
    for (int nw : {16, 8, 4})
        for (int ns = 16; ns <= c.ns_max && ns <= 160; ns += 16) {
            const int k = (c.n_widest + ns - 1) / ns;
            if (k > 32) continue;
            bool seen = false;
            for (const ShapePlan& p : cand) seen = seen || (p.nw == nw && p.n_sl == k);
            if (!seen) cand.push_back({nw, k, 0});
        }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        if (e0) (void)hipEventDestroy(e0);
        return;
    }
    auto time_it = [&](const ShapePlan& p, int reps) -> float {   // us per launch, < 0 if it does not run
        if (launch_rows(c, p.nw, p.n_sl, p.xcd) != 0) return -1.f;
        if (hipEventRecord(e0, c.st) != hipSuccess) return -1.f;
        for (int r = 0; r < reps; ++r)
            if (launch_rows(c, p.nw, p.n_sl, p.xcd) != 0) return -1.f;
        float ms = 0.f;
        if (hipEventRecord(e1, c.st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
            hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
            return -1.f;
        return 1000.f * ms / reps;
    };
    std::vector<std::pair<float, int>> t1;
    for (int i = 0; i < (int)cand.size(); ++i) {
        const float t = time_it(cand[i], 3);
        if (t >= 0.f) t1.push_back({t, i});
    }
    ShapePlan best = cand[0];
    if (!t1.empty()) {
        std::sort(t1.begin(), t1.end());
        const float t_rule = time_it(cand[0], 5);
        float t_best = t_rule;
        // the three fastest and the rule's shape again, each also with the XCD-aware item order
        for (int r = 0; r < 3 && r < (int)t1.size(); ++r) {
            if (t1[r].second == 0) continue;
            const float t = time_it(cand[t1[r].second], 5);
            if (t >= 0.f && (t_best < 0.f || t < t_best)) t_best = t, best = cand[t1[r].second];
        }
        for (int r = -1; r < 3 && r < (int)t1.size(); ++r) {
            if (r >= 0 && t1[r].second == 0) continue;
            ShapePlan p = r < 0 ? cand[0] : cand[t1[r].second];
            p.xcd = 1;
            const float t = time_it(p, 5);
            if (t >= 0.f && (t_best < 0.f || t < t_best)) t_best = t, best = p;
        }
        if (t_rule >= 0.f && !(t_best < 0.98f * t_rule)) best = cand[0];
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    plan = best;
    std::lock_guard<std::mutex> lk(g_plan_mu);
    g_plans[key] = best;
}

extern "C" int face_rows_linear(const face_lin_problem* probs, int32_t n_probs, int32_t w_kn, const float* x_scale,
                                const float* y_scale, int32_t ld_scale, int32_t n_groups, const int32_t* group,
                                int64_t period, void* stream) {
    if (!probs || n_probs < 1 || n_probs > kGemmMaxProbs) return FACE_ERR_ARG;
    int K = 16;
    bool any_bias = false, any_op = false, any_ext = false;
    for (int i = 0; i < n_probs; ++i) {
        if (probs[i].k < 16 || probs[i].k % 16) return FACE_ERR_ARG;
        if (probs[i].k > K) K = probs[i].k;
        if (probs[i].bias) any_bias = true;
        if (probs[i].x_op) any_op = true;
        if (probs[i].x_op || probs[i].x2 || probs[i].y0) any_ext = true;     // the XM = 2 kernels
    }
    const bool scaled = x_scale || y_scale;
    if (scaled && (!group || period < 1 || ld_scale < 1 || n_groups < 1 || n_groups > kGemmMaxGroups))
        return FACE_ERR_ARG;
    if (!scaled) n_groups = 1;
    if ((x_scale && !al16(x_scale)) || (y_scale && !al16(y_scale)) || (scaled && ld_scale % 4))
        return FACE_ERR_UNSUPPORTED;
    GemmArgs A{};
    A.n_probs = n_probs, A.w_kn = w_kn ? 1 : 0, A.any_bias = any_bias ? 1 : 0, A.xs = x_scale, A.ys = y_scale;
    A.ld_s = ld_scale, A.n_groups = n_groups, A.group = group, A.period = period, A.kmax = K;
    for (int i = 0; i < n_probs; ++i) {
        const int st = fill_prob(probs[i], A.w_kn, scaled, x_scale, y_scale, ld_scale, A.p[i]);
        if (st) return st;
    }
    // LDS floats of the side tables for a slice of ns columns (GemmSide)
    auto side_floats = [&](int ns) {
        return (y_scale ? n_groups * ns : 0) + (x_scale ? n_groups * K : 0) + (any_bias ? ns : 0);
    };
    // column slice: the weight slice (NS x (K + 4) floats) and the side tables must fit in LDS, at
    // most 160 columns, and the widest problem splits into slices of equal width (multiples of 16)
    const int max_lds = device_max_lds();
    int ns_max = 160;
    while (ns_max >= 16 && 4 * ((int64_t)ns_max * (K + 4) + side_floats(ns_max)) > max_lds) ns_max -= 16;
    int n_widest = 16;
    for (int i = 0; i < n_probs; ++i)
        if (probs[i].n > n_widest) n_widest = probs[i].n;
    int n_sl = ns_max >= 16 ? (n_widest + ns_max - 1) / ns_max : 1;
    // small problems: narrower slices until there are two workgroups per CU (each slice re-reads
    // its rows, from L2)
    {
        int64_t wg4 = 0;
        for (int i = 0; i < n_probs; ++i) wg4 += (probs[i].m + 16 * kGemmBB * 4 - 1) / (16 * kGemmBB * 4);
        const int n_cu = device_cu_count();
        while (ns_max >= 16 && wg4 * n_sl < 2 * n_cu && (n_widest + n_sl) / (n_sl + 1) >= 16) ++n_sl;
    }
    const int NS = ((n_widest + n_sl - 1) / n_sl + 15) / 16 * 16;
    int64_t rows_total = 0;
    for (int i = 0; i < n_probs; ++i) rows_total += probs[i].m > 0 ? probs[i].m : 0;
    if (use_kc_gemm(K, ns_max, n_widest, rows_total)) {
        // K-chunked weight slices of up to 256 columns (rows_gemm_kc_kernel; 192 with an input
        // transform, whose pre-activation rows take registers too)
        const int ns_cap = any_op ? 192 : 256;
        const int nsl = (n_widest + ns_cap - 1) / ns_cap;
        const int NSk = ((n_widest + nsl - 1) / nsl + 15) / 16 * 16;
        int64_t blocks = 0;
        for (int i = 0; i < n_probs; ++i) {
            const face_lin_problem& s = probs[i];
            if (!al16(s.w) || s.ld_w % 4) return FACE_ERR_UNSUPPORTED;
            GemmProb& p = A.p[i];
            p.tiles = (int)((s.m + 16 * kGemmBB * kKcWaves - 1) / (16 * kGemmBB * kKcWaves));
            p.slices = (s.n + NSk - 1) / NSk;
            p.first_block = blocks;
            blocks += (int64_t)p.tiles * p.slices;
        }
        for (int i = n_probs; i < kGemmMaxProbs; ++i) A.p[i].first_block = INT64_MAX;
        if (blocks == 0) return 0;
        A.NS = NSk;
        A.items = blocks;
        A.side_off = 0;
        const hipStream_t stk = (hipStream_t)stream;
        const int nbk = NSk <= 64 ? 4 : (NSk <= 128 ? 8 : (NSk <= 192 ? 12 : 16));
        const size_t side_lds = 4 * (size_t)side_floats(16 * nbk);
        const size_t static_lds = 2 * (size_t)(16 * nbk) * kKcS * sizeof(float);
        if ((int64_t)(side_lds + static_lds) > max_lds) return FACE_ERR_UNSUPPORTED;
#define FACE_GEMM_KC(NB_)                                                                                          \
    do {                                                                                                           \
        if (side_lds + static_lds > 65536 &&                                                                       \
            hipFuncSetAttribute((const void*)rows_gemm_kc_kernel<NB_>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                (int)side_lds) != hipSuccess)                                                      \
            return FACE_ERR_UNSUPPORTED;                                                                           \
        hipLaunchKernelGGL(rows_gemm_kc_kernel<NB_>, dim3((unsigned)blocks), dim3(kKcWaves * kWave), side_lds, stk, \
                           A);                                                                                     \
    } while (0)
        switch (nbk) {
            case 4: FACE_GEMM_KC(4); break;
            case 8: FACE_GEMM_KC(8); break;
            case 12: FACE_GEMM_KC(12); break;
            default: FACE_GEMM_KC(16); break;
        }
#undef FACE_GEMM_KC
        FACE_LAUNCH_CHECK();
        return 0;
    }
    if (ns_max < 16) return FACE_ERR_UNSUPPORTED;
    RowsCtx c;
    c.A = A, c.probs = probs, c.n_probs = n_probs, c.K = K, c.n_widest = n_widest, c.ns_max = ns_max;
    c.max_lds = max_lds, c.n_cu = device_cu_count(), c.w_kn = w_kn != 0, c.x_scale = x_scale != nullptr;
    c.y_scale = y_scale != nullptr, c.any_bias = any_bias, c.any_ext = any_ext, c.n_groups = n_groups;
    c.st = (hipStream_t)stream;
    if (x_scale && any_ext) return FACE_ERR_UNSUPPORTED;                 // x scale with split / op / y0
    // FACE_GEMM_SHAPE="nw,n_sl,xcd" forces one launch shape (no timing, nothing cached), for tests
    // that compare every shape's results; FACE_ERR_UNSUPPORTED if that shape does not fit
    if (const char* fs = getenv("FACE_GEMM_SHAPE")) {
        int nw = 0, ns = 0, xcd = 0;
        if (sscanf(fs, "%d,%d,%d", &nw, &ns, &xcd) == 3) return launch_rows(c, nw, ns, xcd ? 1 : 0);
    }
    ShapePlan plan{default_nw(c, NS), n_sl, 0};
    pick_shape(c, plan);
    return launch_rows(c, plan.nw, plan.n_sl, plan.xcd);
}
