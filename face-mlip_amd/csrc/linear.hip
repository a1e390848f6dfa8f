// Per-edge linear layers on the fp32 matrix cores (gfx950), for layers whose input is a
// per-edge feature row of K <= 64 values and whose output is a per-edge row of F values:
//
//   forward   Y[e] = X[e] W^T + b + T[idx[e]]                            (E, F)
//   backward  dX[e] = dY[e] W                                            (E, K)
//             dT[n] = sum of dY[e] over the edges e with idx[e] = n      (N, F), idx = col
//
// Users: the CP columns of the last radial layer, R = h2 W_cp^T + b_cp (face/model.py:469,
// :496-497; no table), and the pass message gather(msg(h)) + dir_mix(d) (face/model.py:488-493:
// X = d, T = msg(h), idx = col). The backward's table reduction walks each atom's reverse
// edges (rev) the way the gather backward does, so no atomics are needed and the sums are
// bitwise reproducible; the same pass applies W to each visited edge.
#include "common.h"

namespace face {

// ------------------------------------------------------------------ forward
// The (F, K) weight block sits whole in LDS (160 KB at F = 640, K = 64) as the A operand of
// v_mfma_f32_16x16x4f32; each wave loads the X rows of 16 BB edges once as B operands (K index
// q of instruction r of chunk kb = input feature 16 kb + 4q + r) and walks all output blocks, so
// the output streams out at the write rate: D = W . X^T holds output feature 4q + r of edge j
// in register r of lane j + 16q, one float4 store of Y[e][f .. f + 3] per lane and block.
// LDS image: lin_off / lin_layout (common.h).
constexpr int kLinWaves = 16;

template <int KB, int BB, int FB, bool HAS_B, bool HAS_T>
__global__ __launch_bounds__(kLinWaves * kWave) void edge_linear_fwd_kernel(
    const float* __restrict__ X, int ld_X, int64_t E, const float* __restrict__ w, const float* __restrict__ b,
    int F, int f_chunk, int S, int rot, const float* __restrict__ T, int ld_T, const int32_t* __restrict__ idx,
    float* __restrict__ Y, int ld_Y) {
    constexpr int K = 16 * KB, NCH = K / 4;
    extern __shared__ float sW[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int f_beg = blockIdx.y * f_chunk;
    const int nf = min(f_chunk, F - f_beg);                           // a multiple of 16
    const bool rt = rot != 0;
    for (int v0 = 0; v0 < nf * NCH; v0 += 4 * (int)blockDim.x) {
        v4f buf[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int v = v0 + u * (int)blockDim.x + tid;
            if (v < nf * NCH) buf[u] = ld4(w + (int64_t)(f_beg + v / NCH) * K + 4 * (v % NCH));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int v = v0 + u * (int)blockDim.x + tid;
            if (v < nf * NCH) st4(sW + lin_off(v / NCH, v % NCH, S, NCH, rt), buf[u]);
        }
    }
    __syncthreads();
    const int j = lane & 15, q = lane >> 4;
    const int wv_id = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int64_t ntile = (E + 16 * BB - 1) / (16 * BB);
    const int64_t stride = (int64_t)gridDim.x * kLinWaves;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    int64_t t = (int64_t)blockIdx.x * kLinWaves + wv_id;
    if (t >= ntile) return;
    // X rows (B operands) and table rows of a tile's 16 BB edges; rows past E repeat edge E - 1
    // (never stored). The next tile's rows are loaded while the current one computes, and moved
    // in before its output blocks start, so that no load is outstanding inside the block loop:
    // a wait there would also wait for the Y stores issued after it.
    v4f xn[BB][KB];
    int64_t trn[BB];
    auto load_tile = [&](int64_t tt) __attribute__((always_inline)) {
#pragma unroll
        for (int bb = 0; bb < BB; ++bb) {
            const int64_t e = tt * 16 * BB + 16 * bb + j;
            const int64_t ec = e < E ? e : E - 1;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) xn[bb][kb] = ld4(X + ec * ld_X + 16 * kb + 4 * q);
            trn[bb] = HAS_T ? (idx ? (int64_t)idx[ec] : ec) : 0;
        }
    };
    load_tile(t);
    for (; t < ntile; t += stride) {
        const int64_t e0 = t * 16 * BB;
        v4f xv[BB][KB];
        int64_t trow[BB];
#pragma unroll
        for (int bb = 0; bb < BB; ++bb) {
            trow[bb] = trn[bb];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) xv[bb][kb] = xn[bb][kb];
        }
        if (t + stride < ntile) load_tile(t + stride);
#pragma unroll 1
        for (int fb0 = 0; fb0 < nf; fb0 += 16 * FB) {
            // epilogue operands, issued ahead of the products: the bias through scalar loads
            // (16 features of a block are wave-uniform; lane (j, q) takes 4q .. 4q + 3), the
            // table rows as vector loads
            v4f bias[FB], tv[FB][BB];
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) {
                const int fc = min(fb0 + 16 * fb, nf - 16);
                bias[fb] = z4;
                if (HAS_B) {
                    const float* bp = b + f_beg + fc;
                    float bs[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u)      // wave-uniform values: scalar loads
                        bs[u] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(bp[u])));
#pragma unroll
                    for (int r = 0; r < 4; ++r) bias[fb][r] = q == 0 ? bs[r] : (q == 1 ? bs[4 + r] : (q == 2 ? bs[8 + r] : bs[12 + r]));
                }
#pragma unroll
                for (int bb = 0; bb < BB; ++bb)
                    tv[fb][bb] = HAS_T ? ld4(T + trow[bb] * ld_T + f_beg + fc + 4 * q) : z4;
            }
            v4f acc[FB][BB];
#pragma unroll
            for (int fb = 0; fb < FB; ++fb)
#pragma unroll
                for (int bb = 0; bb < BB; ++bb) acc[fb][bb] = z4;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                v4f wa[FB];
#pragma unroll
                for (int fb = 0; fb < FB; ++fb)
                    wa[fb] = fb0 + 16 * fb < nf
                                 ? lds4_at(sW, lin_off(fb0 + 16 * fb + j, 4 * kb + q, S, NCH, rt))
                                 : z4;
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int fb = 0; fb < FB; ++fb)
#pragma unroll
                        for (int bb = 0; bb < BB; ++bb) acc[fb][bb] = mfma_16x16x4(wa[fb][r], xv[bb][kb][r], acc[fb][bb]);
            }
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) {
                if (fb0 + 16 * fb < nf) {
                    const int f = f_beg + fb0 + 16 * fb + 4 * q;
#pragma unroll
                    for (int bb = 0; bb < BB; ++bb) {
                        const int64_t e = e0 + 16 * bb + j;
                        if (e < E) st4(Y + e * ld_Y + f, acc[fb][bb] + bias[fb] + tv[fb][bb]);
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------ backward
// One wave per atom n (persistent waves): the edges with idx = n are rev[e] for the edges e of
// row n. Per tile of 16 such edges the wave loads their dY rows as B operands (K index q of
// instruction r of chunk fc = output feature 16 fc + 4q + r), adds them into per-lane partial
// sums of dT[n], and multiplies them by W^T (A operand from an LDS image W^T[k][f], row stride
// F + 4) into dX: D = W^T . dY^T holds input feature 4q + r of edge j in register r of lane
// j + 16q. The 16 edge lanes of the partial sums are reduced once per atom.
constexpr int kLinBwdWaves = 8;

template <int KB, int FCB>
__global__ __launch_bounds__(kLinBwdWaves * kWave) void edge_linear_bwd_kernel(
    const float* __restrict__ dY, int ld_dY, const float* __restrict__ w, int F, const int32_t* __restrict__ row_ptr,
    const int32_t* __restrict__ rev, int64_t N, float* __restrict__ dX, int ld_dX, float* __restrict__ dT,
    int ld_dT) {
    constexpr int K = 16 * KB;
    extern __shared__ float sWT[];
    const int SW = F + 4;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    if (dX) {
        for (int v0 = 0; v0 < K * F; v0 += 4 * (int)blockDim.x) {
            float buf[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int v = v0 + u * (int)blockDim.x + tid;             // v = c * K + k: coalesced reads of w
                if (v < K * F) buf[u] = w[v];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int v = v0 + u * (int)blockDim.x + tid;
                if (v < K * F) sWT[(v % K) * SW + v / K] = buf[u];
            }
        }
        __syncthreads();
    }
    const int j = lane & 15, q = lane >> 4;
    const int nfc = F / 16;
    const int wv_id = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int64_t stride = (int64_t)gridDim.x * kLinBwdWaves;
    const v4f z4 = {0.f, 0.f, 0.f, 0.f};
    for (int64_t n = (int64_t)blockIdx.x * kLinBwdWaves + wv_id; n < N; n += stride) {
        const int64_t a = row_ptr[n], bnd = row_ptr[n + 1];
        v4f sums[FCB];
#pragma unroll
        for (int fc = 0; fc < FCB; ++fc) sums[fc] = z4;
        // the reverse-edge index of the next tile is loaded before this tile's stores: on gfx9 a
        // wait for a load also waits for every store issued before it
        int64_t ep_next = a + j < bnd ? (int64_t)rev[a + j] : 0;
        for (int64_t t0 = a; t0 < bnd; t0 += 16) {
            const int64_t er = t0 + j;
            const bool ok = er < bnd;
            const int64_t ep = ep_next;
            ep_next = t0 + 16 + j < bnd ? (int64_t)rev[t0 + 16 + j] : 0;
            v4f acc[KB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc[kb] = z4;
#pragma unroll
            for (int fc = 0; fc < FCB; ++fc) {
                if (fc < nfc) {
                    const v4f g = ok ? ld4(dY + ep * ld_dY + 16 * fc + 4 * q) : z4;
                    sums[fc] += g;
                    if (dX) {
#pragma unroll
                        for (int kb = 0; kb < KB; ++kb) {
                            const v4f wa = lds4_at(sWT, (16 * kb + j) * SW + 16 * fc + 4 * q);
#pragma unroll
                            for (int r = 0; r < 4; ++r) acc[kb] = mfma_16x16x4(wa[r], g[r], acc[kb]);
                        }
                    }
                }
            }
            if (dX && ok) {
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) st4(dX + ep * ld_dX + 16 * kb + 4 * q, acc[kb]);
            }
        }
        if (dT) {
#pragma unroll
            for (int fc = 0; fc < FCB; ++fc) {
                if (fc < nfc) {
                    v4f s = sums[fc];
#pragma unroll
                    for (int o = 1; o < 16; o <<= 1) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) s[r] += __shfl_xor(s[r], o, kWave);
                    }
                    if (j == 0) st4(dT + n * ld_dT + 16 * fc + 4 * q, s);
                }
            }
        }
    }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace face

using namespace face;

extern "C" int face_edge_linear_fwd(const float* x, int32_t ld_x, int64_t E, int32_t K, const float* w, const float* b,
                                    int32_t F, const float* tab, int32_t ld_tab, const int32_t* idx, float* y,
                                    int32_t ld_y, void* stream) {
    if (E < 0 || K < 16 || K > 64 || K % 16 || F < 16 || F % 16 || ld_x < K || ld_y < F || (tab && ld_tab < F))
        return FACE_ERR_ARG;
    if (E == 0) return 0;
    if (!x || !w || !y) return FACE_ERR_ARG;
    if (ld_x % 4 || ld_y % 4 || (tab && ld_tab % 4) || !aligned16(x) || !aligned16(w) || !aligned16(y) ||
        (b && !aligned16(b)) || (tab && !aligned16(tab)))
        return FACE_ERR_UNSUPPORTED;
    const int max_lds = device_max_lds();
    int S = 0, rot = 0, f_chunk = 0;
    if (!lin_layout(F, K, max_lds, S, rot, f_chunk)) return FACE_ERR_UNSUPPORTED;
    const size_t lds = (size_t)f_chunk * S * sizeof(float);
    // 32 edges per tile (BB = 2) for the plain head; the gathered-table form keeps 16 (BB = 1): its
    // table rows (FB x BB float4 per lane) on top of the 32-edge operands spill at 16 waves
    const int BB = tab ? 1 : 2;
    constexpr int FB = 2;
    const int64_t ntile = (E + 16 * BB - 1) / (16 * BB);
    int64_t wgs = device_cu_count();                  // persistent: one 16-wave workgroup per CU
    const int64_t need = (ntile + kLinWaves - 1) / kLinWaves;
    if (need < wgs) wgs = need;
    const dim3 grid((unsigned)wgs, (unsigned)((F + f_chunk - 1) / f_chunk)), block(kLinWaves * kWave);
    const hipStream_t st = (hipStream_t)stream;
#define FACE_LINF(KB_)                                                                                        \
    do {                                                                                                      \
        auto kern = b ? (tab ? edge_linear_fwd_kernel<KB_, 1, FB, true, true>                                 \
                             : edge_linear_fwd_kernel<KB_, 2, FB, true, false>)                               \
                      : (tab ? edge_linear_fwd_kernel<KB_, 1, FB, false, true>                                \
                             : edge_linear_fwd_kernel<KB_, 2, FB, false, false>);                             \
        if (lds > 65536 &&                                                                                    \
            hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=    \
                hipSuccess)                                                                                   \
            return FACE_ERR_UNSUPPORTED;                                                                      \
        hipLaunchKernelGGL(kern, grid, block, lds, st, x, ld_x, E, w, b, F, f_chunk, S, rot, tab, ld_tab, idx, \
                           y, ld_y);                                                                          \
    } while (0)
    switch (K / 16) {
        case 1: FACE_LINF(1); break;
        case 2: FACE_LINF(2); break;
        case 3: FACE_LINF(3); break;
        default: FACE_LINF(4); break;
    }
#undef FACE_LINF
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_edge_linear_bwd(const float* dy, int32_t ld_dy, int32_t F, const float* w, int32_t K,
                                    const int32_t* row_ptr, const int32_t* rev, int64_t N, float* dx, int32_t ld_dx,
                                    float* dtab, int32_t ld_dtab, void* stream) {
    if (N < 0 || K < 16 || K > 64 || K % 16 || F < 16 || F > 256 || F % 16 || ld_dy < F ||
        (dx && ld_dx < K) || (dtab && ld_dtab < F))
        return FACE_ERR_ARG;
    if (N == 0 || (!dx && !dtab)) return 0;
    if (!dy || !row_ptr || !rev || (dx && !w)) return FACE_ERR_ARG;
    if (ld_dy % 4 || (dx && ld_dx % 4) || (dtab && ld_dtab % 4) || !aligned16(dy) || (dx && !aligned16(dx)) ||
        (dtab && !aligned16(dtab)))
        return FACE_ERR_UNSUPPORTED;
    const size_t lds = dx ? (size_t)K * (F + 4) * sizeof(float) : 0;
    if ((int64_t)lds > device_max_lds()) return FACE_ERR_UNSUPPORTED;
    int64_t wgs = (int64_t)device_cu_count() * 2;
    const int64_t need = (N + kLinBwdWaves - 1) / kLinBwdWaves;
    if (need < wgs) wgs = need;
    const dim3 grid((unsigned)wgs), block(kLinBwdWaves * kWave);
    const hipStream_t st = (hipStream_t)stream;
    const int nfc = F / 16;
    const int fcb = nfc <= 2 ? nfc : (nfc <= 4 ? 4 : (nfc <= 8 ? 8 : (nfc <= 10 ? 10 : 16)));
#define FACE_LINB(KB_, FCB_)                                                                                   \
    do {                                                                                                       \
        auto kern = edge_linear_bwd_kernel<KB_, FCB_>;                                                         \
        if (lds > 65536 &&                                                                                     \
            hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=     \
                hipSuccess)                                                                                    \
            return FACE_ERR_UNSUPPORTED;                                                                       \
        hipLaunchKernelGGL(kern, grid, block, lds, st, dy, ld_dy, w, F, row_ptr, rev, N, dx, ld_dx, dtab, ld_dtab); \
    } while (0)
#define FACE_LINB_K(FCB_)                 \
    switch (K / 16) {                     \
        case 1: FACE_LINB(1, FCB_); break; \
        case 2: FACE_LINB(2, FCB_); break; \
        case 3: FACE_LINB(3, FCB_); break; \
        default: FACE_LINB(4, FCB_); break; \
    }
    switch (fcb) {
        case 1: FACE_LINB_K(1); break;
        case 2: FACE_LINB_K(2); break;
        case 4: FACE_LINB_K(4); break;
        case 8: FACE_LINB_K(8); break;
        case 10: FACE_LINB_K(10); break;
        default: FACE_LINB_K(16); break;
    }
#undef FACE_LINB_K
#undef FACE_LINB
    FACE_LAUNCH_CHECK();
    return 0;
}
