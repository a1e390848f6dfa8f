// Edge front-end (geometry, Bessel basis, envelope, monomials), row gathers and the
// atomic-free scatters that replace autograd's index_add (gfx950).
//
// Forward follows face/model.py:670-677 and :28-40, face/cartesian.py:34-46. The backward
// scatters use the reverse-edge map of a symmetric pair list: the edges whose neighbour is
// atom k are exactly the reverses of row k, so every scatter becomes a row reduction.
#include "common.h"

namespace face {

__device__ __forceinline__ void monomials20(float x, float y, float z, float* Y) {
    Y[0] = 1.f;
    Y[1] = x; Y[2] = y; Y[3] = z;
    Y[4] = x * x; Y[5] = y * y; Y[6] = z * z; Y[7] = x * y; Y[8] = x * z; Y[9] = y * z;
    Y[10] = x * x * x; Y[11] = y * y * y; Y[12] = z * z * z; Y[13] = x * x * y; Y[14] = x * x * z;
    Y[15] = x * y * y; Y[16] = y * y * z; Y[17] = x * z * z; Y[18] = y * z * z; Y[19] = x * y * z;
}

struct EdgeGeom {
    float v[3], r, u[3], x;
    bool valid;
};

__device__ __forceinline__ EdgeGeom edge_geom(const float* __restrict__ pos, const int32_t* __restrict__ recv,
                                              const int32_t* __restrict__ col, const float* __restrict__ shift,
                                              const uint8_t* __restrict__ mask, int64_t e, float rc) {
    EdgeGeom g;
    const int64_t i = recv[e], j = col[e];
#pragma unroll
    for (int a = 0; a < 3; ++a) g.v[a] = (pos[j * 3 + a] - pos[i * 3 + a]) + shift[e * 3 + a];
    g.valid = mask ? mask[e] != 0 : true;
    const float r2 = g.v[0] * g.v[0] + g.v[1] * g.v[1] + g.v[2] * g.v[2];
    g.r = sqrtf(g.valid ? r2 : 1.f);
#pragma unroll
    for (int a = 0; a < 3; ++a) g.u[a] = g.v[a] / g.r;
    g.x = g.r / rc;
    return g;
}

// envelope 1 - 28 x^6 + 48 x^7 - 21 x^8 (p = 6), zero at and beyond x = 1 and on masked edges
__device__ __forceinline__ float envelope(const EdgeGeom& g) {
    if (!g.valid || !(g.x < 1.f)) return 0.f;
    const float x2 = g.x * g.x, x6 = x2 * x2 * x2;
    return 1.f - 28.f * x6 + 48.f * x6 * g.x - 21.f * x6 * x2;
}
__device__ __forceinline__ float envelope_dr(const EdgeGeom& g, float rc) {
    if (!g.valid || !(g.x < 1.f)) return 0.f;
    const float x = g.x, x2 = x * x, x5 = x2 * x2 * x;
    return (-168.f * x5 + 336.f * x5 * x - 168.f * x5 * x2) / rc;
}

__global__ __launch_bounds__(256) void edge_geom_fwd_kernel(const float* __restrict__ pos,
                                                            const int32_t* __restrict__ recv,
                                                            const int32_t* __restrict__ col,
                                                            const float* __restrict__ shift,
                                                            const uint8_t* __restrict__ mask, int64_t E,
                                                            const float* __restrict__ freq, int nb, float rc,
                                                            float bes_scale, float* __restrict__ Y,
                                                            float* __restrict__ rb, float* __restrict__ env,
                                                            float* __restrict__ rout) {
    const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (e >= E) return;
    const EdgeGeom g = edge_geom(pos, recv, col, shift, mask, e, rc);
    float y[20];
    monomials20(g.u[0], g.u[1], g.u[2], y);
#pragma unroll
    for (int x = 0; x < 20; ++x) Y[e * 20 + x] = y[x];
    const float ev = envelope(g);
    if (env) env[e] = ev;
    if (rout) rout[e] = g.r;
    if (rb) {
        for (int n = 0; n < nb; ++n) rb[e * nb + n] = sinf(freq[n] * g.r) / g.r * bes_scale * ev;
    }
}

// dL/dvec of one edge from the upstream gradients of its outputs (Y, rb, env, r).
__device__ __forceinline__ void edge_dvec(const EdgeGeom& g, int64_t e, const float* __restrict__ freq, int nb, float rc,
                                          float bes_scale, const float* __restrict__ gY,
                                          const float* __restrict__ grb, const float* __restrict__ genv,
                                          const float* __restrict__ gr, float* out) {
    // d/du of the monomials contracted with gY
    float gu[3] = {0.f, 0.f, 0.f};
    if (gY) {
        const float* q = gY + e * 20;
        const float x = g.u[0], y = g.u[1], z = g.u[2];
        gu[0] = q[1] + 2.f * x * q[4] + y * q[7] + z * q[8] + 3.f * x * x * q[10] + 2.f * x * y * q[13] +
                2.f * x * z * q[14] + y * y * q[15] + z * z * q[17] + y * z * q[19];
        gu[1] = q[2] + 2.f * y * q[5] + x * q[7] + z * q[9] + 3.f * y * y * q[11] + x * x * q[13] +
                2.f * x * y * q[15] + 2.f * y * z * q[16] + z * z * q[18] + x * z * q[19];
        gu[2] = q[3] + 2.f * z * q[6] + x * q[8] + y * q[9] + 3.f * z * z * q[12] + x * x * q[14] +
                y * y * q[16] + 2.f * x * z * q[17] + 2.f * y * z * q[18] + x * y * q[19];
    }
    if (g.valid) {
        const float ev = envelope(g);
        float genv_t = genv ? genv[e] : 0.f;
        float g_r = gr ? gr[e] : 0.f;
        if (grb) {
            const float inv_r = 1.f / g.r;
            for (int n = 0; n < nb; ++n) {
                const float fr = freq[n] * g.r;
                const float s = sinf(fr), c = cosf(fr);
                const float bes = s * inv_r * bes_scale;
                const float dbes = bes_scale * (freq[n] * c * inv_r - s * inv_r * inv_r);
                const float q = grb[e * nb + n];
                genv_t = fmaf(q, bes, genv_t);
                g_r = fmaf(q * ev, dbes, g_r);
            }
        }
        g_r = fmaf(genv_t, envelope_dr(g, rc), g_r);
        const float gdotu = gu[0] * g.u[0] + gu[1] * g.u[1] + gu[2] * g.u[2];
#pragma unroll
        for (int a = 0; a < 3; ++a) out[a] = (gu[a] - gdotu * g.u[a]) / g.r + g_r * g.u[a];
    } else {
#pragma unroll
        for (int a = 0; a < 3; ++a) out[a] = gu[a];   // r := 1 is a constant on masked slots
    }
}

// Up to kEdgeGradSlots gradient buffers per edge input (Y, rb, envelope, r), null where absent:
// one per reader of the input in the forward (each reader gets its own view of the same tensor), so
// that their gradients are summed here, in a fixed order, instead of by separate addition launches.
constexpr int kEdgeGradSlots = 4;
struct EdgeGrads {
    const float* y[kEdgeGradSlots];
    const float* rb[kEdgeGradSlots];
    const float* env[kEdgeGradSlots];
    const float* r[kEdgeGradSlots];
};
__device__ __forceinline__ float slot_sum(const float* const (&p)[kEdgeGradSlots], int64_t i) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kEdgeGradSlots; ++k)
        if (p[k]) s += p[k][i];
    return s;
}
__device__ __forceinline__ bool any_slot(const float* const (&p)[kEdgeGradSlots]) {
    bool a = false;
#pragma unroll
    for (int k = 0; k < kEdgeGradSlots; ++k) a = a || p[k] != nullptr;
    return a;
}

// dL/dvec of one edge from its input gradients already summed over the readers' slots: q (20) the
// monomial gradients (has_y), qb (nb <= 16) the radial-basis gradients (has_rb), genv_t and g_r
// the envelope and distance gradients.
__device__ __forceinline__ void edge_dvec_sums(const EdgeGeom& g, const float* __restrict__ freq, int nb, float rc,
                                               float bes_scale, bool has_y, const float (&q)[20], bool has_rb,
                                               const float (&qb)[16], float genv_t, float g_r, float* out) {
    float gu[3] = {0.f, 0.f, 0.f};
    if (has_y) {
        const float x = g.u[0], y = g.u[1], z = g.u[2];
        gu[0] = q[1] + 2.f * x * q[4] + y * q[7] + z * q[8] + 3.f * x * x * q[10] + 2.f * x * y * q[13] +
                2.f * x * z * q[14] + y * y * q[15] + z * z * q[17] + y * z * q[19];
        gu[1] = q[2] + 2.f * y * q[5] + x * q[7] + z * q[9] + 3.f * y * y * q[11] + x * x * q[13] +
                2.f * x * y * q[15] + 2.f * y * z * q[16] + z * z * q[18] + x * z * q[19];
        gu[2] = q[3] + 2.f * z * q[6] + x * q[8] + y * q[9] + 3.f * z * z * q[12] + x * x * q[14] +
                y * y * q[16] + 2.f * x * z * q[17] + 2.f * y * z * q[18] + x * y * q[19];
    }
    if (g.valid) {
        const float ev = envelope(g);
        if (has_rb) {
            const float inv_r = 1.f / g.r;
#pragma unroll
            for (int n = 0; n < 16; ++n) {
                if (n < nb) {
                    const float fr = freq[n] * g.r;
                    const float sn = sinf(fr), c = cosf(fr);
                    const float bes = sn * inv_r * bes_scale;
                    const float dbes = bes_scale * (freq[n] * c * inv_r - sn * inv_r * inv_r);
                    genv_t = fmaf(qb[n], bes, genv_t);
                    g_r = fmaf(qb[n] * ev, dbes, g_r);
                }
            }
        }
        g_r = fmaf(genv_t, envelope_dr(g, rc), g_r);
        const float gdotu = gu[0] * g.u[0] + gu[1] * g.u[1] + gu[2] * g.u[2];
#pragma unroll
        for (int a = 0; a < 3; ++a) out[a] = (gu[a] - gdotu * g.u[a]) / g.r + g_r * g.u[a];
    } else {
#pragma unroll
        for (int a = 0; a < 3; ++a) out[a] = gu[a];   // r := 1 is a constant on masked slots
    }
}

__global__ __launch_bounds__(256) void edge_geom_bwd_kernel(
    const float* __restrict__ pos, const int32_t* __restrict__ recv, const int32_t* __restrict__ col,
    const float* __restrict__ shift, const uint8_t* __restrict__ mask, int64_t E, const float* __restrict__ freq,
    int nb, float rc, float bes_scale, const float* __restrict__ gY, const float* __restrict__ grb,
    const float* __restrict__ genv, const float* __restrict__ gr, float* __restrict__ gvec) {
    const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (e >= E) return;
    const EdgeGeom g = edge_geom(pos, recv, col, shift, mask, e, rc);
    float out[3];
    edge_dvec(g, e, freq, nb, rc, bes_scale, gY, grb, genv, gr, out);
#pragma unroll
    for (int a = 0; a < 3; ++a) gvec[e * 3 + a] = out[a];
}

// Edge backward with the own-row half of the force scatter folded in (CSR lists, no mask). One
// lane per edge computes dL/dvec_e as edge_geom_bwd_kernel does and writes it, as one 16-byte row
// (x, y, z, 0), to the slot of the edge's REVERSE, gvec_rev[rev e], so that row k of gvec_rev holds
// the dL/dvec of the edges whose neighbour is k, contiguous for the scatter that follows.
// Each wave takes a window of 64 consecutive edges, and every global load of the window is issued
// before the first use: the lane's own Y gradient rows (float4 pieces), the window's radial-basis
// gradient rows read as consecutive 4-byte pieces (256 bytes per instruction), summed over the
// slots in that layout and handed to each edge's lane through LDS (rows padded to nb + 1 floats
// against bank conflicts), then the geometry. Measured at the 24,000-atom liquid against a lane
// reading every row itself, each slot under its own branch: 151 -> 119 us; staging the Y rows
// through LDS as well: 131 us; basis rows read by their own lane (4-byte loads at a 32-byte
// stride): 138 us. The reverse-slot writes are scattered 16-byte rows: written in edge order
// instead (a timing probe only) the kernel takes 106 us; non-temporal stores: 139 us.
// The row's own sum is reduced inside the wave: rows are contiguous edge ranges, so a segmented
// scan over the window (segments = receiver atoms) leaves, at the last edge of each row inside the
// window, the sum of the row's edges in that window; it is written to wsum at that edge's index
// (the other wsum rows are never written or read). Every sum has a fixed order: no atomics.
__global__ __launch_bounds__(256) void edge_geom_bwd_seg_kernel(
    const float* __restrict__ pos, const int32_t* __restrict__ recv, const int32_t* __restrict__ col,
    const float* __restrict__ shift, const int32_t* __restrict__ rev, int64_t E, const float* __restrict__ freq,
    int nb, float rc, float bes_scale, EdgeGrads G, v4f* __restrict__ gvec_rev, v4f* __restrict__ wsum) {
    __shared__ float sB[4][17 * kWave];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int64_t e0 = ((int64_t)blockIdx.x * 4 + w) * kWave;   // the wave's window
    if (e0 >= E) return;                                // whole wave past the end (no workgroup barrier)
    const int nwin = E - e0 < kWave ? (int)(E - e0) : kWave;
    const int64_t e = e0 + lane;
    const bool valid = lane < nwin;
    const bool has_y = any_slot(G.y), has_rb = any_slot(G.rb);
    // every global load of the window issued first: the staged rows, then the lane's own operands
    v4f ay[5];
    float ab[16];
#pragma unroll
    for (int c = 0; c < 5; ++c) ay[c] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 16; ++c) ab[c] = 0.f;
    if (has_y && valid) {
#pragma unroll
        for (int s = 0; s < kEdgeGradSlots; ++s) {
            if (G.y[s]) {
                const v4f* src = reinterpret_cast<const v4f*>(G.y[s] + e * 20);
                v4f t[5];
#pragma unroll
                for (int c = 0; c < 5; ++c) t[c] = src[c];
#pragma unroll
                for (int c = 0; c < 5; ++c) ay[c] += t[c];
            }
        }
    }
    if (has_rb) {
#pragma unroll
        for (int s = 0; s < kEdgeGradSlots; ++s) {
            if (G.rb[s]) {
                const float* src = G.rb[s] + e0 * nb;
                float t[16];
#pragma unroll
                for (int c = 0; c < 16; ++c) {
                    const int f = c * kWave + lane;
                    t[c] = c < nb && f < nwin * nb ? src[f] : 0.f;
                }
#pragma unroll
                for (int c = 0; c < 16; ++c) ab[c] += t[c];
            }
        }
    }
    float genv_t = 0.f, g_r = 0.f;
    EdgeGeom g;
    int key = -1;
    int64_t r_e = 0;
    if (valid) {
        genv_t = slot_sum(G.env, e);
        g_r = slot_sum(G.r, e);
        g = edge_geom(pos, recv, col, shift, nullptr, e, rc);
        key = recv[e];
        r_e = rev[e];
    }
    if (has_rb) {
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            if (c < nb) {                                // piece f = edge f / nb, basis f % nb
                const int f = c * kWave + lane, ed = f / nb;
                sB[w][ed * (nb + 1) + (f - ed * nb)] = ab[c];
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    float q[20], qb[16];
#pragma unroll
    for (int k = 0; k < 20; ++k) q[k] = 0.f;
#pragma unroll
    for (int n = 0; n < 16; ++n) qb[n] = 0.f;
    if (has_y) {
#pragma unroll
        for (int c = 0; c < 5; ++c) {
#pragma unroll
            for (int r = 0; r < 4; ++r) q[4 * c + r] = ay[c][r];
        }
    }
    if (has_rb) {
#pragma unroll
        for (int n = 0; n < 16; ++n)
            if (n < nb) qb[n] = sB[w][lane * (nb + 1) + n];
    }
    float out[3] = {0.f, 0.f, 0.f};
    if (valid) {
        edge_dvec_sums(g, freq, nb, rc, bes_scale, has_y, q, has_rb, qb, genv_t, g_r, out);
        gvec_rev[r_e] = v4f{out[0], out[1], out[2], 0.f};
    }
    // segmented inclusive scan: keys are non-decreasing along the wave, so equal keys d lanes
    // apart bound a run of one row
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const float p0 = __shfl_up(out[0], d, kWave), p1 = __shfl_up(out[1], d, kWave), p2 = __shfl_up(out[2], d, kWave);
        const int kp = __shfl_up(key, d, kWave);
        if (lane >= d && kp == key) {
            out[0] += p0;
            out[1] += p1;
            out[2] += p2;
        }
    }
    const int kn = __shfl_down(key, 1, kWave);
    if (valid && (lane == kWave - 1 || kn != key)) wsum[e] = v4f{out[0], out[1], out[2], 0.f};
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ X, int ld_X,
                                                          const int32_t* __restrict__ idx, int64_t E, int F,
                                                          float* __restrict__ out, int ld_out) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= E * F) return;
    const int64_t e = t / F;
    const int f = (int)(t - e * F);
    out[e * ld_out + f] = X[(int64_t)idx[e] * ld_X + f];
}

// dX[k, f] = sum_{e in row k} g[rev[e], f]; thread = (k, f), row walked in order, eight gathers
// issued per round.
__global__ __launch_bounds__(256) void gather_rows_bwd_kernel(const float* __restrict__ g, int ld_g,
                                                              const int32_t* __restrict__ row_ptr,
                                                              const int32_t* __restrict__ rev, int64_t N, int F,
                                                              float* __restrict__ dX, int ld_dX) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= N * F) return;
    const int64_t k = t / F;
    const int f = (int)(t - k * F);
    const int64_t e1 = row_ptr[k + 1];
    float s = 0.f;
    int64_t e = row_ptr[k];
    for (; e + 8 <= e1; e += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = g[(int64_t)rev[e + u] * ld_g + f];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; e < e1; ++e) s += g[(int64_t)rev[e] * ld_g + f];
    dX[k * ld_dX + f] = s;
}

__global__ __launch_bounds__(256) void segment_sum_kernel(const float* __restrict__ g, int ld_g,
                                                          const int32_t* __restrict__ row_ptr, int64_t N, int F,
                                                          float* __restrict__ out, int ld_out) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= N * F) return;
    const int64_t k = t / F;
    const int f = (int)(t - k * F);
    float s = 0.f;
    for (int64_t e = row_ptr[k]; e < row_ptr[k + 1]; ++e) s += g[e * ld_g + f];
    out[k * ld_out + f] = s;
}

// grad[k] = sign * sum_{e in row k} (g[rev e] - g[e]). G lanes per atom (a power of two <= 64,
// ~half the mean row length): lane l takes edges l, l + G, ... of the row two at a time, so
// the row's own g and rev entries are read coalesced and every lane has two reverse-edge
// gathers in flight; the G partial sums are then reduced by butterfly shuffles.
template <int G>
__global__ __launch_bounds__(256) void force_scatter_kernel(const float* __restrict__ gvec,
                                                            const int32_t* __restrict__ row_ptr,
                                                            const int32_t* __restrict__ rev, int64_t N, float sign,
                                                            float* __restrict__ grad) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int l = threadIdx.x & (G - 1);
    const int64_t k = t / G;
    const bool live = k < N;                            // whole groups of G lanes share k
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
    const int64_t e0 = live ? row_ptr[k] : 0, e1 = live ? row_ptr[k + 1] : 0;
    for (int64_t e = e0 + l; e < e1; e += 2 * G) {
        const int64_t f = e + G;
        const bool two = f < e1;
        const int64_t r = rev[e], rf = two ? (int64_t)rev[f] : r;
        const float a0 = gvec[r * 3 + 0], a1 = gvec[r * 3 + 1], a2 = gvec[r * 3 + 2];
        const float b0 = gvec[e * 3 + 0], b1 = gvec[e * 3 + 1], b2 = gvec[e * 3 + 2];
        const float c0 = gvec[rf * 3 + 0], c1 = gvec[rf * 3 + 1], c2 = gvec[rf * 3 + 2];
        const int64_t fe = two ? f : e;
        const float d0 = gvec[fe * 3 + 0], d1 = gvec[fe * 3 + 1], d2 = gvec[fe * 3 + 2];
        s0 += a0 - b0;
        s1 += a1 - b1;
        s2 += a2 - b2;
        if (two) {
            s0 += c0 - d0;
            s1 += c1 - d1;
            s2 += c2 - d2;
        }
    }
    s0 = group_sum(s0, G);
    s1 = group_sum(s1, G);
    s2 = group_sum(s2, G);
    if (live && l == 0) {
        grad[k * 3 + 0] = sign * s0;
        grad[k * 3 + 1] = sign * s1;
        grad[k * 3 + 2] = sign * s2;
    }
}

// grad[k] = sign * sum_{e in row k} (gvec_rev[e] - own_e), own_e = wsum[e] at the last edge of the
// row in each 64-edge window (e % 64 == 63 or e == end of row) and 0 elsewhere: the force scatter
// as one contiguous pass over each row (gvec_rev and wsum from edge_geom_bwd_seg_kernel, 16-byte
// rows). G lanes per atom read the row's entries coalesced; partial sums reduced by butterfly
// shuffles.
template <int G>
__global__ __launch_bounds__(256) void force_scatter_rows_kernel(const v4f* __restrict__ gvec_rev,
                                                                 const v4f* __restrict__ wsum,
                                                                 const int32_t* __restrict__ row_ptr, int64_t N,
                                                                 float sign, float* __restrict__ grad) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int l = threadIdx.x & (G - 1);
    const int64_t k = t / G;
    const bool live = k < N;                            // whole groups of G lanes share k
    const int64_t e0 = live ? row_ptr[k] : 0, e1 = live ? row_ptr[k + 1] : 0;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
    for (int64_t e = e0 + l; e < e1; e += G) {
        const v4f a = gvec_rev[e];
        s0 += a[0];
        s1 += a[1];
        s2 += a[2];
        if ((e & (kWave - 1)) == kWave - 1 || e == e1 - 1) {
            const v4f b = wsum[e];
            s0 -= b[0];
            s1 -= b[1];
            s2 -= b[2];
        }
    }
    s0 = group_sum(s0, G);
    s1 = group_sum(s1, G);
    s2 = group_sum(s2, G);
    if (live && l == 0) {
        grad[k * 3 + 0] = sign * s0;
        grad[k * 3 + 1] = sign * s1;
        grad[k * 3 + 2] = sign * s2;
    }
}

// ---------------------------------------------------------------- directional edge features
// Node tables: V element (component a, atom n, channel k) at V[a*v_sq + n*v_sn + k] (3 rows),
// M likewise (6 rows, sym storage).
// d[e] = [u.V_j | Y2w.M_j | u.V_i | Y2w.M_i] (4 x Kd), u = Y[1:4], Y2w = Y[4:10] * (1,1,1,2,2,2),
// j = col[e], i = recv[e]   (face/model.py:474-493).
struct DirTables {
    const float* V;
    const float* M;
    int64_t v_sn, v_sq, m_sn, m_sq;
    __device__ __forceinline__ float at(int q, int64_t n, int k) const {
        return q < 3 ? V[q * v_sq + n * v_sn + k] : M[(q - 3) * m_sq + n * m_sn + k];
    }
};

__device__ __forceinline__ void dir_weights(const float* __restrict__ y, float* w) {
    w[0] = y[1]; w[1] = y[2]; w[2] = y[3];
    w[3] = y[4]; w[4] = y[5]; w[5] = y[6];
    w[6] = y[7] * 2.f; w[7] = y[8] * 2.f; w[8] = y[9] * 2.f;
}

__global__ __launch_bounds__(256) void dir_feats_fwd_kernel(DirTables T, int Kd, const int32_t* __restrict__ recv,
                                                            const int32_t* __restrict__ col,
                                                            const float* __restrict__ Y, int64_t E,
                                                            float* __restrict__ d) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= E * Kd) return;
    const int64_t e = t / Kd;
    const int k = (int)(t - e * Kd);
    float w[9];
    dir_weights(Y + e * 20, w);
    const int64_t j = col[e], i = recv[e];
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        a0 = fmaf(w[q], T.at(q, j, k), a0);
        a2 = fmaf(w[q], T.at(q, i, k), a2);
    }
#pragma unroll
    for (int q = 3; q < 9; ++q) {
        a1 = fmaf(w[q], T.at(q, j, k), a1);
        a3 = fmaf(w[q], T.at(q, i, k), a3);
    }
    float* de = d + e * 4 * Kd + k;
    de[0] = a0;
    de[Kd] = a1;
    de[2 * Kd] = a2;
    de[3 * Kd] = a3;
}

// Row form of the dL/dY kernel below for Kd == 16: one wave per receiver atom, lane (j, q) on
// channel kd = j of the row's edges e0 + 4s + q; the receiver's 9 table rows at channel j are
// loaded once per atom, so an edge gathers only its neighbour's. (The same row form of the
// forward measured slower than its per-edge kernel: 186 against 170 us at 24,000 atoms.)
constexpr int kDirWaves = 4;

// dL/dY of the directional features, row form (Kd == 16): the 9 products per (edge, channel)
// summed over the 16 channel lanes of a group with DPP row sums; lane j of the group then writes
// monomial j of the edge's gY row (and lanes j < 4 monomials 16 .. 19, all zero).
__global__ __launch_bounds__(kDirWaves * kWave) void dir_feats_bwd_row_kernel(DirTables T, const int32_t* __restrict__ col,
                                                                            const int32_t* __restrict__ row_ptr,
                                                                            const float* __restrict__ gd, int64_t N,
                                                                            float* __restrict__ gY) {
    constexpr int Kd = 16;
    const int lane = threadIdx.x & (kWave - 1), j = lane & 15, q = lane >> 4;
    const int64_t i = (int64_t)blockIdx.x * kDirWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (i >= N) return;
    const int64_t e0 = row_ptr[i], e1 = row_ptr[i + 1];
    if (e1 <= e0) return;
    float Ti[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) Ti[k] = T.at(k, i, j);
    const int64_t ns = (e1 - e0 + 3) / 4;
    for (int64_t st = 0; st < ns; ++st) {                 // uniform: every lane takes part in the row sums
        const int64_t e = e0 + 4 * st + q;
        const int64_t ec = e < e1 ? e : e1 - 1;
        const int64_t c = col[ec];
        float Tj[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) Tj[k] = T.at(k, c, j);
        const float* g = gd + ec * 4 * Kd + j;
        const float g0 = g[0], g1 = g[Kd], g2 = g[2 * Kd], g3 = g[3 * Kd];
        float acc[9];
#pragma unroll
        for (int k = 0; k < 3; ++k) acc[k] = row16_sum(g0 * Tj[k] + g2 * Ti[k]);
#pragma unroll
        for (int k = 3; k < 9; ++k) acc[k] = row16_sum(g1 * Tj[k] + g3 * Ti[k]);
        if (e < e1) {
            // monomial x = j: 0 for x = 0 and x >= 10, acc[x - 1] for x = 1..6, 2 acc[x - 1] for 7..9
            float v = 0.f;
#pragma unroll
            for (int k = 0; k < 9; ++k)
                if (j == k + 1) v = k < 6 ? acc[k] : 2.f * acc[k];
            float* o = gY + e * 20;
            o[j] = v;
            if (j < 4) o[16 + j] = 0.f;
        }
    }
}

// dL/dY for the directional features (monomials 1..9; 0 and 10..19 are written as 0).
// Thread = (edge, channel slot); the KP lanes of an edge (KP = Kd rounded up to a power of two,
// <= 64) sum their partial products with butterfly shuffles.
__global__ __launch_bounds__(256) void dir_feats_bwd_edge_kernel(DirTables T, int Kd, int KP,
                                                                 const int32_t* __restrict__ recv,
                                                                 const int32_t* __restrict__ col,
                                                                 const float* __restrict__ gd, int64_t E,
                                                                 float* __restrict__ gY) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;   // grid covers E*KP rounded up to 256
    const int64_t e = t / KP;
    const int k = (int)(t - e * KP);
    const bool ok = e < E && k < Kd;
    float acc[9];
#pragma unroll
    for (int q = 0; q < 9; ++q) acc[q] = 0.f;
    if (ok) {
        const int64_t j = col[e], i = recv[e];
        const float* g = gd + e * 4 * Kd + k;
        const float g0 = g[0], g1 = g[Kd], g2 = g[2 * Kd], g3 = g[3 * Kd];
#pragma unroll
        for (int q = 0; q < 3; ++q) acc[q] = g0 * T.at(q, j, k) + g2 * T.at(q, i, k);
#pragma unroll
        for (int q = 3; q < 9; ++q) acc[q] = g1 * T.at(q, j, k) + g3 * T.at(q, i, k);
    }
#pragma unroll
    for (int q = 0; q < 9; ++q) acc[q] = group_sum(acc[q], KP);
    if (e < E && k == 0) {
        float* o = gY + e * 20;
        o[0] = 0.f;
#pragma unroll
        for (int q = 0; q < 6; ++q) o[1 + q] = acc[q];
#pragma unroll
        for (int q = 6; q < 9; ++q) o[1 + q] = 2.f * acc[q];
#pragma unroll
        for (int x = 10; x < 20; ++x) o[x] = 0.f;
    }
}

// dL/dT[q, n, k] = sum_{e in row n} ( gd[rev e, s(q) Kd + k] w_q(rev e) + gd[e, (2 + s(q)) Kd + k] w_q(e) ),
// s(q) = 0 for the V rows, 1 for the M rows: the neighbour half through the reverse map, the
// receiver half from the row itself. Thread = (atom n, channel k). gV / gM share V / M's layout.
__global__ __launch_bounds__(256) void dir_feats_bwd_node_kernel(int Kd, int64_t v_sn, int64_t v_sq, int64_t m_sn,
                                                                 int64_t m_sq, const int32_t* __restrict__ row_ptr,
                                                                 const int32_t* __restrict__ rev,
                                                                 const float* __restrict__ Y,
                                                                 const float* __restrict__ gd, int64_t N,
                                                                 float* __restrict__ gV, float* __restrict__ gM) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= N * Kd) return;
    const int64_t n = t / Kd;
    const int k = (int)(t - n * Kd);
    float acc[9];
#pragma unroll
    for (int q = 0; q < 9; ++q) acc[q] = 0.f;
    for (int64_t e = row_ptr[n]; e < row_ptr[n + 1]; ++e) {
        const int64_t r = rev[e];
        float wr[9], we[9];
        dir_weights(Y + r * 20, wr);
        dir_weights(Y + e * 20, we);
        const float gr0 = gd[r * 4 * Kd + k], gr1 = gd[r * 4 * Kd + Kd + k];
        const float ge2 = gd[e * 4 * Kd + 2 * Kd + k], ge3 = gd[e * 4 * Kd + 3 * Kd + k];
#pragma unroll
        for (int q = 0; q < 3; ++q) acc[q] += gr0 * wr[q] + ge2 * we[q];
#pragma unroll
        for (int q = 3; q < 9; ++q) acc[q] += gr1 * wr[q] + ge3 * we[q];
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) gV[q * v_sq + n * v_sn + k] = acc[q];
#pragma unroll
    for (int q = 3; q < 9; ++q) gM[(q - 3) * m_sq + n * m_sn + k] = acc[q];
}

// Per-row scalar sums with one workgroup per row (few, long rows: energies per structure).
__global__ __launch_bounds__(256) void row_sum_kernel(const float* __restrict__ g, int ld_g,
                                                      const int32_t* __restrict__ row_ptr,
                                                      float* __restrict__ out, int ld_out) {
    __shared__ float part[256];
    const int64_t k = blockIdx.x;
    const int tid = threadIdx.x;
    float s = 0.f;
    for (int64_t e = row_ptr[k] + tid; e < row_ptr[k + 1]; e += 256) s += g[e * ld_g];
    part[tid] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) part[tid] += part[tid + o];
        __syncthreads();
    }
    if (tid == 0) out[k * ld_out] = part[0];
}

// ------------------------------------------------------------------ atom energies
// e_at[a] = e0[a] + scale (e_1[a] + ...) added pass by pass, and E[s] = the sum of e_at over the
// atoms of structure s (contiguous, [struct_ptr[s], struct_ptr[s+1])) (face/model.py:680-690), in
// two launches: the per-atom energies over a fixed device-wide grid (the pass energies are often
// columns of wider rows, one cache line per atom and pass), then one workgroup of 1024 threads per
// structure summing the contiguous e_at in a fixed order. One workgroup doing both read every
// strided pass energy through a single CU: 63 us at 24,000 atoms, 231 us at 100,000.
constexpr int kMaxEnergyTerms = 8;
constexpr int kEnergyThreads = 1024, kEnergyUnroll = 16;
constexpr int kEnergyRowThreads = 256, kEnergyRowBlocks = 512;
struct EnergyTerms {
    const float* e[kMaxEnergyTerms];
    int64_t ld[kMaxEnergyTerms];
    int n;
};

// e_at over atoms [0, struct_ptr[nstr]), grid-stride
__global__ __launch_bounds__(kEnergyRowThreads) void atom_energy_rows_kernel(const float* __restrict__ e0,
                                                                             const float* __restrict__ scale,
                                                                             EnergyTerms T,
                                                                             const int32_t* __restrict__ struct_ptr,
                                                                             int64_t nstr, float* __restrict__ e_at) {
    const int64_t N = struct_ptr[nstr];
    const float sc = *scale;
    for (int64_t a = (int64_t)blockIdx.x * kEnergyRowThreads + threadIdx.x; a < N;
         a += (int64_t)gridDim.x * kEnergyRowThreads) {
        float x[kMaxEnergyTerms];
#pragma unroll
        for (int p = 0; p < kMaxEnergyTerms; ++p) x[p] = p < T.n ? T.e[p][a * T.ld[p]] : 0.f;
        float v = e0[a];
#pragma unroll
        for (int p = 0; p < kMaxEnergyTerms; ++p)
            if (p < T.n) v += sc * x[p];
        e_at[a] = v;
    }
}

// E[k] = sum of e_at over structure k: thread t adds atoms beg + t, beg + t + 1024, ... in order,
// then the waves and the workgroup in a fixed order
__global__ __launch_bounds__(kEnergyThreads) void atom_energy_sum_kernel(const float* __restrict__ e_at,
                                                                         const int32_t* __restrict__ struct_ptr,
                                                                         float* __restrict__ E) {
    __shared__ float part[kEnergyThreads / kWave];
    const int64_t k = blockIdx.x, beg = struct_ptr[k], end = struct_ptr[k + 1];
    const int tid = threadIdx.x;
    float s = 0.f;
    for (int64_t a0 = beg + tid; a0 < end; a0 += kEnergyThreads * kEnergyUnroll) {
        float v[kEnergyUnroll];
#pragma unroll
        for (int u = 0; u < kEnergyUnroll; ++u) {
            const int64_t a = a0 + u * kEnergyThreads;
            v[u] = a < end ? e_at[a] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kEnergyUnroll; ++u)
            if (a0 + u * kEnergyThreads < end) s += v[u];
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, kWave);
    if ((tid & (kWave - 1)) == 0) part[tid / kWave] = s;
    __syncthreads();
    if (tid == 0) {
        float t = 0.f;
        for (int w = 0; w < kEnergyThreads / kWave; ++w) t += part[w];
        E[k] = t;
    }
}

// ge[a] = scale (gE[s] + g_at[a]) for the atoms a of structure s (either term may be absent)
__global__ __launch_bounds__(kEnergyThreads) void atom_energy_bwd_kernel(const float* __restrict__ gE,
                                                                         const float* __restrict__ g_at,
                                                                         const float* __restrict__ scale,
                                                                         const int32_t* __restrict__ struct_ptr,
                                                                         float* __restrict__ ge) {
    const int64_t k = blockIdx.x, beg = struct_ptr[k], end = struct_ptr[k + 1];
    const float sc = *scale, gs = gE ? gE[k] : 0.f;
    for (int64_t a0 = beg + threadIdx.x; a0 < end; a0 += kEnergyThreads * kEnergyUnroll) {
        float x[kEnergyUnroll];
#pragma unroll
        for (int u = 0; u < kEnergyUnroll; ++u) {
            const int64_t a = a0 + u * kEnergyThreads;
            x[u] = (g_at && a < end) ? g_at[a] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kEnergyUnroll; ++u) {
            const int64_t a = a0 + u * kEnergyThreads;
            if (a < end) ge[a] = sc * (gs + x[u]);
        }
    }
}

static unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace face

using namespace face;

extern "C" int face_edge_geom_fwd(const float* pos, const int32_t* recv, const int32_t* col, const float* shift,
                                  const uint8_t* mask, int64_t E, const float* freq, int32_t n_basis, float rc,
                                  float bes_scale, float* Y, float* rb, float* env, float* r, void* stream) {
    if (E < 0 || n_basis < 0 || !(rc > 0.f) || (rb && (!freq || n_basis == 0))) return FACE_ERR_ARG;
    if (E == 0) return 0;
    if (!pos || !recv || !col || !shift || !Y) return FACE_ERR_ARG;
    hipLaunchKernelGGL(edge_geom_fwd_kernel, dim3(blocks_for(E)), dim3(256), 0, (hipStream_t)stream, pos, recv, col,
                       shift, mask, E, freq, n_basis, rc, bes_scale, Y, rb, env, r);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_edge_geom_bwd(const float* pos, const int32_t* recv, const int32_t* col, const float* shift,
                                  const uint8_t* mask, int64_t E, const float* freq, int32_t n_basis, float rc,
                                  float bes_scale, const float* gY, const float* grb, const float* genv,
                                  const float* gr, float* gvec, void* stream) {
    if (E < 0 || n_basis < 0 || !(rc > 0.f) || (grb && (!freq || n_basis == 0))) return FACE_ERR_ARG;
    if (E == 0) return 0;
    if (!pos || !recv || !col || !shift || !gvec) return FACE_ERR_ARG;
    hipLaunchKernelGGL(edge_geom_bwd_kernel, dim3(blocks_for(E)), dim3(256), 0, (hipStream_t)stream, pos, recv, col,
                       shift, mask, E, freq, n_basis, rc, bes_scale, gY, grb, genv, gr, gvec);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_edge_geom_bwd_seg(const float* pos, const int32_t* recv, const int32_t* col, const float* shift,
                                      const int32_t* rev, int64_t E, const float* freq, int32_t n_basis, float rc,
                                      float bes_scale, const float* const* gY, const float* const* grb,
                                      const float* const* genv, const float* const* gr, float* gvec_rev, float* wsum,
                                      void* stream) {
    if (E < 0 || n_basis < 0 || !(rc > 0.f)) return FACE_ERR_ARG;
    EdgeGrads G{};
    for (int k = 0; k < kEdgeGradSlots; ++k) {
        G.y[k] = gY ? gY[k] : nullptr;
        G.rb[k] = grb ? grb[k] : nullptr;
        G.env[k] = genv ? genv[k] : nullptr;
        G.r[k] = gr ? gr[k] : nullptr;
        if (G.rb[k] && (!freq || n_basis == 0 || n_basis > 16)) return FACE_ERR_ARG;
        if (G.y[k] && ((uintptr_t)G.y[k] & 15)) return FACE_ERR_UNSUPPORTED;     // 16-byte pieces of Y rows
    }
    if (E == 0) return 0;
    if (!pos || !recv || !col || !shift || !rev || !gvec_rev || !wsum) return FACE_ERR_ARG;
    if (((uintptr_t)gvec_rev & 15) || ((uintptr_t)wsum & 15)) return FACE_ERR_UNSUPPORTED;
    const unsigned grid = (unsigned)((E + 4 * kWave - 1) / (4 * kWave));
    hipLaunchKernelGGL(edge_geom_bwd_seg_kernel, dim3(grid), dim3(4 * kWave), 0, (hipStream_t)stream, pos, recv, col,
                       shift, rev, E, freq, n_basis, rc, bes_scale, G, reinterpret_cast<v4f*>(gvec_rev),
                       reinterpret_cast<v4f*>(wsum));
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_force_scatter_rows(const float* gvec_rev, const float* wsum, const int32_t* row_ptr, int64_t N,
                                       int32_t mean_row, float sign, float* grad, void* stream) {
    if (N < 0) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!gvec_rev || !wsum || !row_ptr || !grad) return FACE_ERR_ARG;
    if (((uintptr_t)gvec_rev & 15) || ((uintptr_t)wsum & 15)) return FACE_ERR_UNSUPPORTED;
    const hipStream_t st = (hipStream_t)stream;
    const v4f* gv = reinterpret_cast<const v4f*>(gvec_rev);
    const v4f* ws = reinterpret_cast<const v4f*>(wsum);
    // lanes per row ~ a third of the mean row length: two or three edges per lane
    if (mean_row <= 24) {
        hipLaunchKernelGGL(force_scatter_rows_kernel<8>, dim3(blocks_for(N * 8)), dim3(256), 0, st, gv, ws, row_ptr,
                           N, sign, grad);
    } else {
        hipLaunchKernelGGL(force_scatter_rows_kernel<16>, dim3(blocks_for(N * 16)), dim3(256), 0, st, gv, ws,
                           row_ptr, N, sign, grad);
    }
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_gather_rows(const float* X, int32_t ld_X, const int32_t* idx, int64_t E, int32_t F, float* out,
                                int32_t ld_out, void* stream) {
    if (E < 0 || F < 0 || ld_X < F || ld_out < F) return FACE_ERR_ARG;
    if (E == 0 || F == 0) return 0;
    if (!X || !idx || !out) return FACE_ERR_ARG;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_for(E * F)), dim3(256), 0, (hipStream_t)stream, X, ld_X, idx,
                       E, F, out, ld_out);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_gather_rows_bwd(const float* g, int32_t ld_g, const int32_t* row_ptr, const int32_t* rev,
                                    int64_t N, int32_t F, float* dX, int32_t ld_dX, void* stream) {
    if (N < 0 || F < 0 || ld_g < F || ld_dX < F) return FACE_ERR_ARG;
    if (N == 0 || F == 0) return 0;
    if (!g || !row_ptr || !rev || !dX) return FACE_ERR_ARG;
    hipLaunchKernelGGL(gather_rows_bwd_kernel, dim3(blocks_for(N * F)), dim3(256), 0, (hipStream_t)stream, g, ld_g,
                       row_ptr, rev, N, F, dX, ld_dX);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_segment_sum(const float* g, int32_t ld_g, const int32_t* row_ptr, int64_t N, int32_t F,
                                float* out, int32_t ld_out, void* stream) {
    if (N < 0 || F < 0 || ld_g < F || ld_out < F) return FACE_ERR_ARG;
    if (N == 0 || F == 0) return 0;
    if (!g || !row_ptr || !out) return FACE_ERR_ARG;
    if (F == 1)
        hipLaunchKernelGGL(row_sum_kernel, dim3((unsigned)N), dim3(256), 0, (hipStream_t)stream, g, ld_g, row_ptr, out,
                           ld_out);
    else
        hipLaunchKernelGGL(segment_sum_kernel, dim3(blocks_for(N * F)), dim3(256), 0, (hipStream_t)stream, g, ld_g,
                           row_ptr, N, F, out, ld_out);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_atom_energy_fwd(const float* e0, const float* scale, const float* const* e, const int64_t* ld_e,
                                    int32_t n_e, const int32_t* struct_ptr, int64_t nstr, float* e_at, float* E,
                                    void* stream) {
    if (nstr < 0 || n_e < 0 || n_e > kMaxEnergyTerms || (n_e > 0 && (!e || !ld_e))) return FACE_ERR_ARG;
    if (nstr == 0) return 0;
    if (!e0 || !scale || !struct_ptr || !e_at || !E) return FACE_ERR_ARG;
    EnergyTerms T{};
    T.n = n_e;
    for (int p = 0; p < n_e; ++p) {
        if (!e[p] || ld_e[p] < 1) return FACE_ERR_ARG;
        T.e[p] = e[p];
        T.ld[p] = ld_e[p];
    }
    hipLaunchKernelGGL(atom_energy_rows_kernel, dim3(kEnergyRowBlocks), dim3(kEnergyRowThreads), 0,
                       (hipStream_t)stream, e0, scale, T, struct_ptr, nstr, e_at);
    FACE_LAUNCH_CHECK();
    hipLaunchKernelGGL(atom_energy_sum_kernel, dim3((unsigned)nstr), dim3(kEnergyThreads), 0, (hipStream_t)stream,
                       e_at, struct_ptr, E);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_atom_energy_bwd(const float* gE, const float* g_at, const float* scale, const int32_t* struct_ptr,
                                    int64_t nstr, float* ge, void* stream) {
    if (nstr < 0) return FACE_ERR_ARG;
    if (nstr == 0) return 0;
    if (!scale || !struct_ptr || !ge) return FACE_ERR_ARG;
    hipLaunchKernelGGL(atom_energy_bwd_kernel, dim3((unsigned)nstr), dim3(kEnergyThreads), 0, (hipStream_t)stream, gE,
                       g_at, scale, struct_ptr, ge);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_force_scatter(const float* gvec, const int32_t* row_ptr, const int32_t* rev, int64_t N,
                                  float sign, float* grad, void* stream) {
    if (N < 0) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!gvec || !row_ptr || !rev || !grad) return FACE_ERR_ARG;
    constexpr int G = 16;                               // rows of ~10-70 pairs: one or two sweeps
    hipLaunchKernelGGL(force_scatter_kernel<G>, dim3(blocks_for(N * G)), dim3(256), 0, (hipStream_t)stream, gvec,
                       row_ptr, rev, N, sign, grad);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_dir_feats_fwd(const float* V, int64_t v_sn, int64_t v_sq, const float* M, int64_t m_sn,
                                  int64_t m_sq, int32_t Kd, const int32_t* recv, const int32_t* col, const float* Y,
                                  int64_t E, float* d, void* stream) {
    if (E < 0 || Kd <= 0) return FACE_ERR_ARG;
    if (E == 0) return 0;
    if (!V || !M || !recv || !col || !Y || !d) return FACE_ERR_ARG;
    DirTables T{V, M, v_sn, v_sq, m_sn, m_sq};
    hipLaunchKernelGGL(dir_feats_fwd_kernel, dim3(blocks_for(E * Kd)), dim3(256), 0, (hipStream_t)stream, T, Kd, recv,
                       col, Y, E, d);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_dir_feats_bwd(const float* V, int64_t v_sn, int64_t v_sq, const float* M, int64_t m_sn,
                                  int64_t m_sq, int32_t Kd, const int32_t* row_ptr, const int32_t* recv,
                                  const int32_t* col, const int32_t* rev, const float* Y, const float* gd, int64_t N,
                                  int64_t E, float* gV, float* gM, float* gY, void* stream) {
    if (E < 0 || N < 0 || Kd <= 0 || Kd > 64) return FACE_ERR_ARG;
    if (!V || !M || !row_ptr || !recv || !col || !rev || !Y || !gd || (!gV != !gM)) return FACE_ERR_ARG;
    DirTables T{V, M, v_sn, v_sq, m_sn, m_sq};
    hipStream_t st = (hipStream_t)stream;
    if (gY && E > 0 && Kd == 16 && N > 0) {
        hipLaunchKernelGGL(dir_feats_bwd_row_kernel, dim3((unsigned)((N + kDirWaves - 1) / kDirWaves)),
                           dim3(kDirWaves * kWave), 0, st, T, col, row_ptr, gd, N, gY);
    } else if (gY && E > 0) {
        int KP = 1;
        while (KP < Kd) KP <<= 1;
        hipLaunchKernelGGL(dir_feats_bwd_edge_kernel, dim3(blocks_for(E * KP)), dim3(256), 0, st, T, Kd, KP, recv, col,
                           gd, E, gY);
    }
    if (gV && N > 0)
        hipLaunchKernelGGL(dir_feats_bwd_node_kernel, dim3(blocks_for(N * Kd)), dim3(256), 0, st, Kd, v_sn, v_sq,
                           m_sn, m_sq, row_ptr, rev, Y, gd, N, gV, gM);
    FACE_LAUNCH_CHECK();
    return 0;
}
