// GPU pair-list build with the semantics of ASE neighbor_list("ijS") as used by
// face/neighbors.py:12-15 and face/datasets.py:51 (gfx950).
//
// The accept test is evaluated in fp64 with a fixed operation order (no FMA contraction,
// correctly rounded sqrt):
//   shift_c = (S0*cell[0][c] + S1*cell[1][c]) + S2*cell[2][c]
//   d_c     = (pos[j][c] - pos[i][c]) + shift_c
//   keep    iff sqrt((d0*d0 + d1*d1) + d2*d2) < rc, and not (i == j and S == 0)
// Rows come out sorted by (j, S lexicographic).
//
// Two candidate generators share that test:
//   small structures: each atom scans all atoms of its structure and every image that can
//                     lie within rc (molecule batches, small cells);
//   cell list:        one fully periodic structure binned in fractional coordinates; each atom
//                     scans the (2s+1)^3 neighbouring bins with their periodic images.
#include "common.h"

namespace face {

struct NbrGrid {
    int nb[3];   // bins per axis
    int s[3];    // bins searched on each side
};

__device__ __forceinline__ bool pair_within(const double* __restrict__ pos, int64_t i, int64_t j,
                                            const double* __restrict__ cell, int s0, int s1, int s2, double rc,
                                            double* shv) {
    double d[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const double sh = __dadd_rn(__dadd_rn(__dmul_rn((double)s0, cell[c]), __dmul_rn((double)s1, cell[3 + c])),
                                    __dmul_rn((double)s2, cell[6 + c]));
        shv[c] = sh;
        d[c] = __dadd_rn(__dsub_rn(pos[j * 3 + c], pos[i * 3 + c]), sh);
    }
    const double r2 = __dadd_rn(__dadd_rn(__dmul_rn(d[0], d[0]), __dmul_rn(d[1], d[1])), __dmul_rn(d[2], d[2]));
    return __dsqrt_rn(r2) < rc;
}

__device__ __forceinline__ double frac_coord(const double* __restrict__ pos, int64_t i, const double* __restrict__ inv,
                                             int c) {
    return __dadd_rn(__dadd_rn(__dmul_rn(pos[i * 3 + 0], inv[c]), __dmul_rn(pos[i * 3 + 1], inv[3 + c])),
                     __dmul_rn(pos[i * 3 + 2], inv[6 + c]));
}

__device__ __forceinline__ int64_t pair_key(int64_t j, int s0, int s1, int s2) {
    return (j << 30) | ((int64_t)(s0 + 512) << 20) | ((int64_t)(s1 + 512) << 10) | (int64_t)(s2 + 512);
}

// Emits one accepted pair: either counts it or writes it into the row (sorted insertion
// for the cell-list generator, whose candidate order is not canonical).
struct RowWriter {
    int64_t base;
    int cap;
    int n;
    int64_t* key;
    int32_t* col;
    int32_t* S;
    float* shift;
    int32_t* overflow;
};

__device__ __forceinline__ void emit_sorted(RowWriter& w, int64_t j, int s0, int s1, int s2) {
    if (w.key) {
        if (w.n >= w.cap || s0 < -512 || s0 > 511 || s1 < -512 || s1 > 511 || s2 < -512 || s2 > 511) {
            atomicAdd(w.overflow, 1);
        } else {
            const int64_t k = pair_key(j, s0, s1, s2);
            int p = w.n;
            while (p > 0 && w.key[w.base + p - 1] > k) {
                w.key[w.base + p] = w.key[w.base + p - 1];
                --p;
            }
            w.key[w.base + p] = k;
        }
    }
    ++w.n;
}

__device__ __forceinline__ void emit_direct(RowWriter& w, int64_t j, int s0, int s1, int s2, const double* shv) {
    if (w.col) {
        if (w.n >= w.cap) {
            atomicAdd(w.overflow, 1);
        } else {
            const int64_t e = w.base + w.n;
            w.col[e] = (int32_t)j;
            w.S[e * 3 + 0] = s0;
            w.S[e * 3 + 1] = s1;
            w.S[e * 3 + 2] = s2;
#pragma unroll
            for (int c = 0; c < 3; ++c) w.shift[e * 3 + c] = (float)shv[c];
        }
    }
    ++w.n;
}

// ----------------------------------------------------------------------- small structures
__global__ __launch_bounds__(256) void nbr_small_kernel(const double* __restrict__ pos, int64_t N,
                                                        const int32_t* __restrict__ atom_struct,
                                                        const int32_t* __restrict__ struct_ptr,
                                                        const double* __restrict__ cell_all,
                                                        const double* __restrict__ inv_all,
                                                        const int32_t* __restrict__ pbc_all, double rc,
                                                        int32_t* __restrict__ counts,
                                                        const int32_t* __restrict__ row_ptr, int32_t* col,
                                                        int32_t* S, float* shift, int32_t* overflow) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int s = atom_struct[i];
    const int64_t a0 = struct_ptr[s], a1 = struct_ptr[s + 1];
    const double* cell = cell_all + 9 * (int64_t)s;
    const double* inv = inv_all + 9 * (int64_t)s;
    const int32_t* pbc = pbc_all + 3 * (int64_t)s;
    const bool any = pbc[0] || pbc[1] || pbc[2];
    double fi[3] = {0, 0, 0}, w[3] = {0, 0, 0};
    if (any) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            fi[c] = frac_coord(pos, i, inv, c);
            const double l = sqrt(inv[c] * inv[c] + inv[3 + c] * inv[3 + c] + inv[6 + c] * inv[6 + c]);
            w[c] = rc * l;   // rc / face distance
        }
    }
    RowWriter wr{row_ptr ? (int64_t)row_ptr[i] : 0, row_ptr ? row_ptr[i + 1] - row_ptr[i] : 0, 0, nullptr, col, S,
                 shift, overflow};
    for (int64_t j = a0; j < a1; ++j) {
        int lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            if (!pbc[c]) continue;
            const double df = frac_coord(pos, j, inv, c) - fi[c];
            lo[c] = (int)floor(-df - w[c]) - 1;
            hi[c] = (int)ceil(-df + w[c]) + 1;
        }
        for (int s0 = lo[0]; s0 <= hi[0]; ++s0)
            for (int s1 = lo[1]; s1 <= hi[1]; ++s1)
                for (int s2 = lo[2]; s2 <= hi[2]; ++s2) {
                    if (i == j && s0 == 0 && s1 == 0 && s2 == 0) continue;
                    double shv[3];
                    if (pair_within(pos, i, j, cell, s0, s1, s2, rc, shv)) emit_direct(wr, j, s0, s1, s2, shv);
                }
    }
    if (counts) counts[i] = wr.n;
}

// ----------------------------------------------------------------------- cell list
__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t < n) p[t] = v;
}

__global__ __launch_bounds__(256) void nbr_bin_kernel(const double* __restrict__ pos, int64_t N,
                                                      const double* __restrict__ inv, NbrGrid grid,
                                                      int32_t* __restrict__ bin_of, int32_t* __restrict__ wrap,
                                                      int32_t* __restrict__ bin_count) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= N) return;
    int b[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const double f = frac_coord(pos, i, inv, c);
        const double w = floor(f);
        int bc = (int)((f - w) * grid.nb[c]);
        bc = bc < 0 ? 0 : (bc >= grid.nb[c] ? grid.nb[c] - 1 : bc);
        b[c] = bc;
        wrap[i * 3 + c] = (int32_t)w;
    }
    const int bin = b[0] + grid.nb[0] * (b[1] + grid.nb[1] * b[2]);
    bin_of[i] = bin;
    atomicAdd(&bin_count[bin], 1);
}

// Exclusive scan of n counts into out[0..n] by one workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(const int32_t* __restrict__ in, int64_t n,
                                                              int32_t* __restrict__ out) {
    __shared__ int32_t part[1024];
    const int tid = threadIdx.x;
    const int64_t chunk = (n + 1023) / 1024;
    const int64_t b = tid * chunk, e = min(n, b + chunk);
    int32_t s = 0;
    for (int64_t q = b; q < e; ++q) s += in[q];
    part[tid] = s;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const int32_t v = tid >= o ? part[tid - o] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int32_t run = tid ? part[tid - 1] : 0;
    for (int64_t q = b; q < e; ++q) {
        out[q] = run;
        run += in[q];
    }
    if (tid == 1023) out[n] = part[1023];
}

__global__ __launch_bounds__(256) void nbr_scatter_kernel(int64_t N, const int32_t* __restrict__ bin_of,
                                                          const int32_t* __restrict__ bin_start,
                                                          int32_t* __restrict__ bin_fill,
                                                          int32_t* __restrict__ bin_atoms) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int bin = bin_of[i];
    const int slot = atomicAdd(&bin_fill[bin], 1);
    bin_atoms[bin_start[bin] + slot] = (int32_t)i;
}

__global__ __launch_bounds__(256) void nbr_cell_kernel(const double* __restrict__ pos, int64_t N,
                                                       const double* __restrict__ cell, NbrGrid grid, double rc,
                                                       const int32_t* __restrict__ bin_of,
                                                       const int32_t* __restrict__ wrap,
                                                       const int32_t* __restrict__ bin_start,
                                                       const int32_t* __restrict__ bin_atoms,
                                                       int32_t* __restrict__ counts,
                                                       const int32_t* __restrict__ row_ptr, int64_t* key,
                                                       int32_t* col, int32_t* S, float* shift, int32_t* overflow) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int bin = bin_of[i];
    const int bi[3] = {bin % grid.nb[0], (bin / grid.nb[0]) % grid.nb[1], bin / (grid.nb[0] * grid.nb[1])};
    const int wi[3] = {wrap[i * 3 + 0], wrap[i * 3 + 1], wrap[i * 3 + 2]};
    RowWriter wr{row_ptr ? (int64_t)row_ptr[i] : 0, row_ptr ? row_ptr[i + 1] - row_ptr[i] : 0, 0, key, nullptr,
                 nullptr, nullptr, overflow};
    for (int d2 = -grid.s[2]; d2 <= grid.s[2]; ++d2)
        for (int d1 = -grid.s[1]; d1 <= grid.s[1]; ++d1)
            for (int d0 = -grid.s[0]; d0 <= grid.s[0]; ++d0) {
                const int n[3] = {bi[0] + d0, bi[1] + d1, bi[2] + d2};
                int img[3], m[3];
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    img[c] = (n[c] >= 0 ? n[c] : n[c] - grid.nb[c] + 1) / grid.nb[c];   // floor division
                    m[c] = n[c] - img[c] * grid.nb[c];
                }
                const int nbin = m[0] + grid.nb[0] * (m[1] + grid.nb[1] * m[2]);
                for (int q = bin_start[nbin]; q < bin_start[nbin + 1]; ++q) {
                    const int64_t j = bin_atoms[q];
                    const int s0 = img[0] + wi[0] - wrap[j * 3 + 0];
                    const int s1 = img[1] + wi[1] - wrap[j * 3 + 1];
                    const int s2 = img[2] + wi[2] - wrap[j * 3 + 2];
                    if (i == j && s0 == 0 && s1 == 0 && s2 == 0) continue;
                    double shv[3];
                    if (pair_within(pos, i, j, cell, s0, s1, s2, rc, shv)) emit_sorted(wr, j, s0, s1, s2);
                }
            }
    if (counts) counts[i] = wr.n;
    if (key && wr.n <= wr.cap) {   // decode the sorted keys of this row
        for (int p = 0; p < wr.n; ++p) {
            const int64_t e = wr.base + p;
            const int64_t k = key[e];
            const int s0 = (int)((k >> 20) & 1023) - 512, s1 = (int)((k >> 10) & 1023) - 512,
                      s2 = (int)(k & 1023) - 512;
            col[e] = (int32_t)(k >> 30);
            S[e * 3 + 0] = s0;
            S[e * 3 + 1] = s1;
            S[e * 3 + 2] = s2;
#pragma unroll
            for (int c = 0; c < 3; ++c)
                shift[e * 3 + c] = (float)__dadd_rn(
                    __dadd_rn(__dmul_rn((double)s0, cell[c]), __dmul_rn((double)s1, cell[3 + c])),
                    __dmul_rn((double)s2, cell[6 + c]));
        }
    }
}

// ----------------------------------------------------------------------- reverse map, padded view
__device__ __forceinline__ int cmp_edge(int32_t ca, const int32_t* Sa, int32_t cb, int sb0, int sb1, int sb2) {
    if (ca != cb) return ca < cb ? -1 : 1;
    if (Sa[0] != sb0) return Sa[0] < sb0 ? -1 : 1;
    if (Sa[1] != sb1) return Sa[1] < sb1 ? -1 : 1;
    if (Sa[2] != sb2) return Sa[2] < sb2 ? -1 : 1;
    return 0;
}

__global__ __launch_bounds__(256) void nbr_rev_kernel(const int32_t* __restrict__ row_ptr,
                                                      const int32_t* __restrict__ col, const int32_t* __restrict__ S,
                                                      int64_t N, int32_t* __restrict__ rev,
                                                      int32_t* __restrict__ missing) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= N) return;
    for (int64_t e = row_ptr[i]; e < row_ptr[i + 1]; ++e) {
        const int64_t j = col[e];
        const int t0 = -S[e * 3], t1 = -S[e * 3 + 1], t2 = -S[e * 3 + 2];
        int64_t lo = row_ptr[j], hi = row_ptr[j + 1];   // rows are sorted by (col, S)
        int64_t found = -1;
        while (lo < hi) {
            const int64_t mid = (lo + hi) >> 1;
            const int c = cmp_edge(col[mid], S + mid * 3, (int32_t)i, t0, t1, t2);
            if (c == 0) {
                found = mid;
                break;
            }
            if (c < 0) lo = mid + 1;
            else hi = mid;
        }
        if (found < 0) {
            atomicAdd(missing, 1);
            found = e;
        }
        rev[e] = (int32_t)found;
    }
}

__global__ __launch_bounds__(256) void nbr_rev_shift_kernel(const int32_t* __restrict__ row_ptr,
                                                            const int32_t* __restrict__ col,
                                                            const float* __restrict__ shift, int64_t N,
                                                            int32_t* __restrict__ rev, int32_t* __restrict__ missing) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= N) return;
    for (int64_t e = row_ptr[i]; e < row_ptr[i + 1]; ++e) {
        const int64_t j = col[e];
        const float t0 = -shift[e * 3], t1 = -shift[e * 3 + 1], t2 = -shift[e * 3 + 2];
        int64_t found = -1;
        for (int64_t q = row_ptr[j]; q < row_ptr[j + 1]; ++q) {
            if (col[q] == (int32_t)i && shift[q * 3] == t0 && shift[q * 3 + 1] == t1 && shift[q * 3 + 2] == t2) {
                found = q;
                break;
            }
        }
        if (found < 0) {
            atomicAdd(missing, 1);
            found = e;
        }
        rev[e] = (int32_t)found;
    }
}

__global__ __launch_bounds__(256) void nbr_padded_kernel(const int32_t* __restrict__ row_ptr,
                                                         const int32_t* __restrict__ col,
                                                         const float* __restrict__ shift,
                                                         const int32_t* __restrict__ atom_struct,
                                                         const int32_t* __restrict__ struct_ptr, int64_t N, int M,
                                                         int64_t* __restrict__ nbr, float* __restrict__ shift_pad,
                                                         uint8_t* __restrict__ mask) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= N * M) return;
    const int64_t i = t / M;
    const int m = (int)(t - i * M);
    const int64_t e = row_ptr[i] + m;
    const bool ok = e < row_ptr[i + 1];
    nbr[t] = ok ? (int64_t)col[e] : (int64_t)struct_ptr[atom_struct[i]];
#pragma unroll
    for (int c = 0; c < 3; ++c) shift_pad[t * 3 + c] = ok ? shift[e * 3 + c] : 0.f;
    mask[t] = ok ? 1 : 0;
}

static unsigned nblk(int64_t n) { return (unsigned)((n + 255) / 256); }

static bool grid_from(const int32_t* nb, NbrGrid& g) {
    for (int c = 0; c < 3; ++c) {
        g.nb[c] = nb[c];
        g.s[c] = nb[3 + c];
        if (g.nb[c] <= 0 || g.s[c] < 0 || g.s[c] > 64) return false;
    }
    return true;
}

}  // namespace face

using namespace face;

extern "C" int face_nbr_bin(const double* pos, int64_t N, const double* inv_cell, const int32_t* nb, int32_t* bin_of,
                            int32_t* wrap, int32_t* bin_count, int32_t* bin_start, int32_t* bin_fill,
                            int32_t* bin_atoms, void* stream) {
    NbrGrid g;
    if (N < 0 || !nb || !grid_from(nb, g)) return FACE_ERR_ARG;
    const int64_t nbins = (int64_t)g.nb[0] * g.nb[1] * g.nb[2];
    if (nbins > (1 << 26)) return FACE_ERR_CAPACITY;
    if (!pos || !inv_cell || !bin_of || !wrap || !bin_count || !bin_start || !bin_fill || !bin_atoms)
        return FACE_ERR_ARG;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(fill_i32_kernel, dim3(nblk(nbins)), dim3(256), 0, st, bin_count, nbins, 0);
    hipLaunchKernelGGL(fill_i32_kernel, dim3(nblk(nbins)), dim3(256), 0, st, bin_fill, nbins, 0);
    if (N > 0)
        hipLaunchKernelGGL(nbr_bin_kernel, dim3(nblk(N)), dim3(256), 0, st, pos, N, inv_cell, g, bin_of, wrap,
                           bin_count);
    hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, st, bin_count, nbins, bin_start);
    if (N > 0)
        hipLaunchKernelGGL(nbr_scatter_kernel, dim3(nblk(N)), dim3(256), 0, st, N, bin_of, bin_start, bin_fill,
                           bin_atoms);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_nbr_count(const double* pos, int64_t N, const int32_t* atom_struct, const int32_t* struct_ptr,
                              const double* cell, const double* inv_cell, const int32_t* pbc, double rc,
                              const int32_t* nb, const int32_t* bin_of, const int32_t* wrap, const int32_t* bin_start,
                              const int32_t* bin_atoms, int32_t* counts, void* stream) {
    if (N < 0 || !(rc > 0.0) || !counts) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!pos || !cell) return FACE_ERR_ARG;
    hipStream_t st = (hipStream_t)stream;
    if (bin_atoms) {
        NbrGrid g;
        if (!nb || !grid_from(nb, g) || !bin_of || !wrap || !bin_start) return FACE_ERR_ARG;
        hipLaunchKernelGGL(nbr_cell_kernel, dim3(nblk(N)), dim3(256), 0, st, pos, N, cell, g, rc, bin_of, wrap,
                           bin_start, bin_atoms, counts, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
    } else {
        if (!atom_struct || !struct_ptr || !inv_cell || !pbc) return FACE_ERR_ARG;
        hipLaunchKernelGGL(nbr_small_kernel, dim3(nblk(N)), dim3(256), 0, st, pos, N, atom_struct, struct_ptr, cell,
                           inv_cell, pbc, rc, counts, nullptr, nullptr, nullptr, nullptr, nullptr);
    }
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_nbr_fill(const double* pos, int64_t N, const int32_t* atom_struct, const int32_t* struct_ptr,
                             const double* cell, const double* inv_cell, const int32_t* pbc, double rc,
                             const int32_t* nb, const int32_t* bin_of, const int32_t* wrap, const int32_t* bin_start,
                             const int32_t* bin_atoms, const int32_t* row_ptr, int64_t* key, int32_t* col, int32_t* S,
                             float* shift, int32_t* overflow, void* stream) {
    if (N < 0 || !(rc > 0.0)) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!pos || !cell || !row_ptr || !col || !S || !shift || !overflow) return FACE_ERR_ARG;
    hipStream_t st = (hipStream_t)stream;
    if (bin_atoms) {
        NbrGrid g;
        if (!nb || !grid_from(nb, g) || !bin_of || !wrap || !bin_start || !key) return FACE_ERR_ARG;
        hipLaunchKernelGGL(nbr_cell_kernel, dim3(nblk(N)), dim3(256), 0, st, pos, N, cell, g, rc, bin_of, wrap,
                           bin_start, bin_atoms, nullptr, row_ptr, key, col, S, shift, overflow);
    } else {
        if (!atom_struct || !struct_ptr || !inv_cell || !pbc) return FACE_ERR_ARG;
        hipLaunchKernelGGL(nbr_small_kernel, dim3(nblk(N)), dim3(256), 0, st, pos, N, atom_struct, struct_ptr, cell,
                           inv_cell, pbc, rc, nullptr, row_ptr, col, S, shift, overflow);
    }
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_nbr_rev(const int32_t* row_ptr, const int32_t* col, const int32_t* S, int64_t N, int32_t* rev,
                            int32_t* missing, void* stream) {
    if (N < 0) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!row_ptr || !col || !S || !rev || !missing) return FACE_ERR_ARG;
    hipLaunchKernelGGL(nbr_rev_kernel, dim3(nblk(N)), dim3(256), 0, (hipStream_t)stream, row_ptr, col, S, N, rev,
                       missing);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_nbr_rev_shift(const int32_t* row_ptr, const int32_t* col, const float* shift, int64_t N,
                                  int32_t* rev, int32_t* missing, void* stream) {
    if (N < 0) return FACE_ERR_ARG;
    if (N == 0) return 0;
    if (!row_ptr || !col || !shift || !rev || !missing) return FACE_ERR_ARG;
    hipLaunchKernelGGL(nbr_rev_shift_kernel, dim3(nblk(N)), dim3(256), 0, (hipStream_t)stream, row_ptr, col, shift,
                       N, rev, missing);
    FACE_LAUNCH_CHECK();
    return 0;
}

extern "C" int face_nbr_padded(const int32_t* row_ptr, const int32_t* col, const float* shift,
                               const int32_t* atom_struct, const int32_t* struct_ptr, int64_t N, int32_t M,
                               int64_t* nbr, float* shift_pad, uint8_t* mask, void* stream) {
    if (N < 0 || M < 0) return FACE_ERR_ARG;
    if (N == 0 || M == 0) return 0;
    if (!row_ptr || !col || !shift || !atom_struct || !struct_ptr || !nbr || !shift_pad || !mask) return FACE_ERR_ARG;
    hipLaunchKernelGGL(nbr_padded_kernel, dim3(nblk(N * (int64_t)M)), dim3(256), 0, (hipStream_t)stream, row_ptr, col,
                       shift, atom_struct, struct_ptr, N, M, nbr, shift_pad, mask);
    FACE_LAUNCH_CHECK();
    return 0;
}
