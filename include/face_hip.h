/* C-ABI of the MI355X-native FACE hot path (libface_hip.so, gfx950).
 *
 * Conventions
 *   - Every pointer is a device pointer unless the comment says "host".
 *   - Every entry point enqueues work on `stream` (a hipStream_t; NULL = the null stream),
 *     never synchronises, never allocates: outputs and workspaces are passed in.
 *   - Return value: 0 on success, a positive hipError_t from the launch, or a negative
 *     FACE_ERR_* code for an argument the kernels cannot serve. face_hip_error_string()
 *     names either kind.
 *   - Floating point data are fp32, row-major; `ld_*` arguments are row strides in elements.
 *   - Edge lists are grouped by receiver atom i. `row_ptr` (N+1, int32) gives row i as edges
 *     [row_ptr[i], row_ptr[i+1]); row_ptr == NULL means the reference's padded-dense layout
 *     (N, M): row i is edges [i*M, (i+1)*M), masked slots included (their radial weight is 0).
 *
 * Reference interfaces replaced (albert-hzbn/face-mlip):
 *   face/kernels.py:135-172      FactorDensity / factor_density   -> face_density_fwd / _bwd
 *   face/kernels.py:135-172 + face/model.py:503-506  factor density + mix[l]
 *                                                                  -> face_density_mix_fwd / _bwd
 *   face/model.py:496-502        CP pooling bmm                   -> face_cp_density_fwd / _bwd
 *   face/node_kernel.py:164-209  NodeAlgebra / node_algebra       -> face_node_fwd / _bwd
 *   face/model.py:244-249,332    node algebra + readout LayerNorm -> face_node_ln_fwd / _bwd
 *   face/model.py:286-296        gated equivariant outputs V*gv, Ms*gm -> face_eq_gate_fwd / _bwd
 *   face/model.py:140,332        readout nn.LayerNorm             -> face_layer_norm_fwd / _bwd
 *   face/neighbors.py:7-37       padded_graph (ASE neighbor_list) -> face_nbr_* (count, fill, rev, padded)
 *   face/model.py:670-677        edge geometry + Bessel basis     -> face_edge_geom_fwd / _bwd
 *   face/model.py:465-469        radial MLP (rad_in, pair, radial) -> face_radial_fwd / _bwd
 *   face/model.py:407-418,466-467 RadialSpline (compile_radial)   -> face_radial_spline_fwd / _bwd
 *                                                                    (+ face_radial_spline_order)
 *   face/model.py:469,488-493    CP radial columns; gather(msg(h)) + dir_mix(d)
 *                                                                  -> face_edge_linear_fwd / _bwd
 *   face/model.py:498-533,537-544 mix / tmix / proj (+ elem_scale)   -> face_rows_linear
 *   face/model.py:474-493        directional edge features        -> face_dir_feats_fwd / _bwd
 *   face/model.py:514-533        transport sums + transport map   -> face_transport_fwd / _bwd
 *   face/model.py:680-690        atom energies + per-structure sum -> face_atom_energy_fwd / _bwd
 *   face/model.py:670,464,692-694 index_select gathers and their index_add backward
 *                                                                  -> face_gather_rows, face_gather_rows_bwd,
 *                                                                     face_force_scatter
 */
#ifndef FACE_HIP_H
#define FACE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FACE_ERR_ARG (-1)         /* invalid shape, stride or null pointer */
#define FACE_ERR_UNSUPPORTED (-2) /* shape outside the instantiated kernel variants */
#define FACE_ERR_CAPACITY (-3)    /* a row or bin exceeds the kernel's capacity */
#define FACE_ERR_SCRATCH (-4)     /* input exceeds the fixed scratch of an allocation-free entry point */

const char* face_hip_error_string(int code);
/* ABI version of this header (bumped on any signature change). */
int face_hip_abi_version(void);

/* ---------------------------------------------------------------- rank-block outputs
 * Density outputs and their upstream gradients are addressed per monomial rank l (x ranges
 * 0 | 1-3 | 4-9 | 10-19): element (atom i, monomial x, column c) lives at
 *     ranks[l(x)] + i * atom_stride + (x - x0(l)) * x_stride + c
 * ranks: host array of 4 device pointers (only ranks 0 and 1 are read when NX == 4).
 * The reference layout (N, NX, W) is ranks[l] = base + x0(l) * W, atom_stride = NX * W,
 * x_stride = W; a (k_l, N, W) tensor per rank is ranks[l] = D_l, atom_stride = W, x_stride = N * W.
 *
 * ---------------------------------------------------------------- factor density
 * D[i, x, b*K + k] = sum_{e in row i} phi[e, b] * msg[m(e), k] * Y[e, x],  x < NX
 * where m(e) = msg_row ? msg_row[e] : e (msg_row gathers rows of a node table directly).
 * phi (E, ld_phi >= B), msg (*, ld_msg >= K), Y (E, ld_Y >= NX), D: rank blocks of width B*K.
 * NX is 20 (monomials up to rank 3, face/cartesian.py:11-17) or 4 (1, u: the transport sums
 * of face/model.py:515-522, which are this contraction with msg = gathered transport tables).
 * Replaces FactorDensity.forward / dens_fwd (face/kernels.py:137-149, :22-54).            */
int face_density_fwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg, const int32_t* msg_row,
                     const float* Y, int32_t ld_Y, int32_t NX, const int32_t* row_ptr, int64_t N, int32_t M,
                     int32_t B, int32_t K, float* const* D_ranks, int64_t atom_stride, int64_t x_stride,
                     void* stream);

/* Backward of face_density_fwd for upstream G = dL/dD (rank blocks of width B*K):
 *   dphi[e,b] = sum_{x,k} G[i,x,b,k] Y[e,x] msg[m(e),k]
 *   dmsg[e,k] = sum_{x,b} G[i,x,b,k] Y[e,x] phi[e,b]     (per EDGE, also when msg_row != NULL)
 *   dY[e,x]   = sum_{b,k} G[i,x,b,k] phi[e,b] msg[m(e),k]
 * Any of dphi / dmsg / dY may be NULL (not computed). max_row = longest row (M when padded).
 * Replaces FactorDensity.backward / dens_bwd (face/kernels.py:151-167, :56-118).           */
int face_density_bwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg, const int32_t* msg_row,
                     const float* Y, int32_t ld_Y, int32_t NX, const int32_t* row_ptr, int64_t N, int32_t M,
                     int32_t max_row, int32_t B, int32_t K, const float* const* G_ranks, int64_t atom_stride,
                     int64_t x_stride, float* dphi, int32_t ld_dphi, float* dmsg, int32_t ld_dmsg, float* dY,
                     int32_t ld_dY, void* stream);

/* ---------------------------------------------------------------- factor density fused with mix
 * The factor density above (B = 16, NX = 20, CSR rows) followed by the per-rank channel mixing
 * and element scale, with D kept on chip (LDS, one chunk of 16 basis functions x 16 channels at a
 * time) instead of written:
 *   A_l[i, x, c] = (beta_l A_l[i, x, c] + sum_{b,k} D[i, x, b, k] W_l[c, b K + k]) * ys[group[i], l C + c]
 * w_ranks: 4 device pointers to W_l (C, ld_w >= B K) row-major (face/model.py:445 mix[l].weight);
 * A_ranks: 4 output rank blocks (k_l, N, C)-addressed by atom_stride / x_stride (multiples of 4,
 * 16-byte aligned); beta_l = bit l of beta_mask (the block already holds the transport mix of
 * face/model.py:530-533); y_scale (n_el, ld_scale >= 4C) the elem_scale / avg_nb table, group (N)
 * int32 element index, or NULL (no scale). K a multiple of 16 up to 64, C a multiple of 16 up to
 * 256. Replaces FactorDensity.forward (face/kernels.py:137-149) + mix (face/model.py:503-506). */
int face_density_mix_fwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg, const int32_t* msg_row,
                         const float* Y, int32_t ld_Y, const int32_t* row_ptr, int64_t N, int32_t B, int32_t K,
                         int32_t C, const float* const* w_ranks, int64_t ld_w, float* const* A_ranks,
                         int64_t atom_stride, int64_t x_stride, const float* y_scale, int32_t ld_scale,
                         const int32_t* group, int32_t beta_mask, void* stream);
/* Its backward for gA (rank blocks): dD = (gA * x_scale) W_l recomputed on chip per chunk, then
 * dphi (E, ld_dphi), dmsg (E, ld_dmsg) per edge and dY (E, ld_dY) as face_density_bwd (any may be
 * NULL). wt_ranks: W_l^T (B K, ld_wt >= C) row-major. Replaces FactorDensity.backward
 * (face/kernels.py:151-167) + the mix backward. */
int face_density_mix_bwd(const float* phi, int32_t ld_phi, const float* msg, int32_t ld_msg, const int32_t* msg_row,
                         const float* Y, int32_t ld_Y, const int32_t* row_ptr, int64_t N, int32_t B, int32_t K,
                         int32_t C, const float* const* wt_ranks, int64_t ld_wt, const float* const* gA_ranks,
                         int64_t atom_stride, int64_t x_stride, const float* x_scale, int32_t ld_scale,
                         const int32_t* group, float* dphi, int32_t ld_dphi, float* dmsg, int32_t ld_dmsg, float* dY,
                         int32_t ld_dY, void* stream);

/* ---------------------------------------------------------------- CP density
 * A[i, x, c] = sum_{e in row i} env[e] * R[e, l(x), c] * msg[m(e), c] * Y[e, x],  l(x) = rank of x
 * R (E, ld_R >= 4C) laid out [rank][channel] (the radial output BEFORE the cutoff envelope),
 * env (E) the envelope (NULL = 1), msg (*, ld_msg >= C), Y (E, ld_Y >= 20), A: rank blocks of
 * width C. The rank-diagonal blocks of the reference's (N,20,4,C) bmm with the envelope
 * multiply of face/model.py:469 folded in (face/model.py:496-502).                          */
int face_cp_density_fwd(const float* R, int32_t ld_R, const float* env, const float* msg, int32_t ld_msg,
                        const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr, int64_t N,
                        int32_t M, int32_t C, float* const* A_ranks, int64_t atom_stride, int64_t x_stride,
                        void* stream);

/* Backward for gA = dL/dA (rank blocks): dR (E, ld_dR), dmsg (E, ld_dmsg) per edge, dY (E, ld_dY),
 * denv (E). Any output may be NULL. Served on the matrix cores when C is a multiple of 32
 * (C <= 800) and every row / rank block is 16-byte aligned; otherwise C <= 256. */
int face_cp_density_bwd(const float* R, int32_t ld_R, const float* env, const float* msg, int32_t ld_msg,
                        const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr, int64_t N,
                        int32_t M, int32_t max_row, int32_t C, const float* const* gA_ranks, int64_t atom_stride,
                        int64_t x_stride, float* dR, int32_t ld_dR, float* dmsg, int32_t ld_dmsg, float* dY,
                        int32_t ld_dY, float* denv, void* stream);

/* CP pooling forward fused with the CP columns of the last radial layer (face/model.py:469-472,
 * 496-502): R = h2 W^T + b (W (4C, H) row-major, b (4C) or NULL) computed on the matrix cores, written
 * to R (E, ld_R >= 4C; NULL = not written) for the backward, and pooled into A as
 * face_cp_density_fwd from the same registers (R is not read back). E = row_ptr[N] (the number of
 * edges; sizes the launch); row_ptr is required (CSR rows). Served when C is a multiple of 16,
 * H in {16, 32, 48, 64}, h2 and W are 16-byte aligned with ld_h2 % 4 == 0 and the part of W one
 * workgroup holds fits LDS; FACE_ERR_UNSUPPORTED otherwise (then R = h2 W^T + b by
 * face_edge_linear_fwd and face_cp_density_fwd give the same result). A equals
 * face_cp_density_fwd's within fp32 rounding (another summation order); R is bitwise
 * face_edge_linear_fwd's. */
int face_cp_radial_fwd(const float* h2, int32_t ld_h2, int32_t H, const float* w, const float* b, const float* env,
                       const float* msg, int32_t ld_msg, const int32_t* msg_row, const float* Y, int32_t ld_Y,
                       const int32_t* row_ptr, int64_t N, int64_t E, int32_t C, float* const* A_ranks,
                       int64_t atom_stride, int64_t x_stride, float* R, int32_t ld_R, void* stream);

/* CP pooling backward fused with the CP columns of the last radial layer (face/model.py:469-472):
 * with R = h2 W^T + b (W (4C, H)), returns dh2 (E, ld_dh2) = dR W instead of dR, computed on the
 * matrix cores inside the pooling kernel. w_t = W^T (H, 4C) row-major, 16-byte aligned;
 * H in {16, 32, 48, 64}; C a multiple of 32 and the layout conditions of the matrix-core
 * path above. Other arguments as face_cp_density_bwd (dmsg, dY, denv may be NULL). */
int face_cp_radial_bwd(const float* R, int32_t ld_R, const float* env, const float* msg, int32_t ld_msg,
                       const int32_t* msg_row, const float* Y, int32_t ld_Y, const int32_t* row_ptr, int64_t N,
                       int32_t M, int32_t C, const float* const* gA_ranks, int64_t atom_stride, int64_t x_stride,
                       const float* w_t, int32_t H, float* dh2, int32_t ld_dh2, float* dmsg, int32_t ld_dmsg,
                       float* dY, int32_t ld_dY, float* denv, void* stream);

/* ---------------------------------------------------------------- node algebra
 * Per (atom n, channel c) invariants of symmetric Cartesian tensors
 *   inputs  P1,Q1,S1 (3 comps), P2,Q2,S2 (6, order xx,yy,zz,xy,xz,yz), P3,Q3 (10, face/cartesian.py:14-15)
 *   inv[0..7] = P1.Q1, P2:Q2, P3:Q3, P1.Q2.S1, tr(P2 Q2 S2), (P3:Q2).S1, (P3:Q3):S2, P3[Q1,S1,Q1]
 *   V  = a0 P1 + a1 Q2 S1 + a2 P3:Q2 + a3 P2 Q1
 *   Mf = b0 P2 + b1 P1 (x) Q1 + b2 P2 Q2 + b3 P3.S1                      (only when eq != 0)
 * ins: host array of 8 device pointers (P1,Q1,S1,P2,Q2,S2,P3,Q3); in_strides: host array of
 * 8 x 3 int64 element strides (atom, channel, component). a, b: (4, C) contiguous device arrays.
 * inv: strides (atom, channel, family); V: (atom, channel, component).
 * Mf: mf_mode 0 -> full 3x3 (component a*3+d); 1 -> symmetrised 0.5(Mf+Mf^T) in 6-component storage.
 * Replaces NodeAlgebra.forward / node_fwd (face/node_kernel.py:168-184, :18-64).          */
int face_node_fwd(const float* const* ins, const int64_t* in_strides, const float* a, const float* b, float* inv,
                  const int64_t* inv_strides, float* V, const int64_t* V_strides, float* Mf,
                  const int64_t* Mf_strides, int32_t mf_mode, int64_t N, int32_t C, int32_t eq, void* stream);

/* Backward: gI (8 families), gV (3), gM (mf_mode as above) with host stride arrays; any of them
 * may be NULL (= zero). outs: host array of 8 device pointers dP1..dQ3 (symmetric storage) with
 * out_strides (8 x 3). da, db: (N, C, 4) per-(atom, channel) partials, or NULL when not needed
 * (forces only). Replaces NodeAlgebra.backward / node_bwd (face/node_kernel.py:186-204, :66-151). */
int face_node_bwd(const float* const* ins, const int64_t* in_strides, const float* a, const float* b,
                  const float* gI, const int64_t* gI_strides, const float* gV, const int64_t* gV_strides,
                  const float* gM, const int64_t* gM_strides, int32_t mf_mode, float* const* outs,
                  const int64_t* out_strides, float* da, float* db, int64_t N, int32_t C, int32_t eq, void* stream);
/* Node algebra fused with the readout LayerNorm (face/model.py:244-249, :140, :332): the row
 * x = [P0 | inv_1 .. inv_8] (9C, family-major) of every atom is formed in registers and written
 * normalised: y[n, k C + c] = (x - mean) rstd ln_w[kC + c] + ln_b[kC + c] (row stride ld_y), with
 * stats[2n] = mean, stats[2n + 1] = rstd = 1 / sqrt(biased var + eps); P0 (N, C) row stride p0_sn;
 * V / Mf as face_node_fwd. C <= 256. The row x itself is not written. */
int face_node_ln_fwd(const float* const* ins, const int64_t* in_strides, const float* p0, int64_t p0_sn,
                     const float* a, const float* b, const float* ln_w, const float* ln_b, float eps, float* y,
                     int64_t ld_y, float* stats, float* V, const int64_t* V_strides, float* Mf,
                     const int64_t* Mf_strides, int32_t mf_mode, int64_t N, int32_t C, int32_t eq, void* stream);
/* Backward of face_node_ln_fwd for gy = dL/dy (row stride ld_gy) and gV, gM (may be NULL): the row
 * recomputed from the inputs, dx = rstd (g - mean(g) - xh mean(g xh)), g = gy ln_w; dx's first C
 * entries go to dp0 (row stride dp0_sn), the others through the node-algebra backward into outs
 * (as face_node_bwd, with da / db). No LayerNorm weight gradients. */
int face_node_ln_bwd(const float* const* ins, const int64_t* in_strides, const float* p0, int64_t p0_sn,
                     const float* a, const float* b, const float* ln_w, const float* gy, int64_t ld_gy,
                     const float* stats, const float* gV, const int64_t* gV_strides, const float* gM,
                     const int64_t* gM_strides, int32_t mf_mode, float* const* outs, const int64_t* out_strides,
                     float* dp0, int64_t dp0_sn, float* da, float* db, int64_t N, int32_t C, int32_t eq,
                     void* stream);


/* Gated equivariant outputs of a pass: Vo = V * gv, Mo = Ms * gm per (atom, channel), with
 * gvm = [gv | gm] (N, 2C) the gate row; V (3, N, C), Ms (6, N, C), Vo, Mo likewise, all
 * contiguous (C % 4 == 0 and 16-byte aligned, else FACE_ERR_UNSUPPORTED).
 * Replaces `V * gv[..., None], Ms * gm[..., None]` of face/model.py:286-287 and :295-296. */
int face_eq_gate_fwd(const float* V, const float* Ms, const float* gvm, int64_t N, int32_t C, float* Vo, float* Mo,
                     void* stream);

/* Backward of face_eq_gate_fwd for upstream gVo (3, N, C), gMo (6, N, C): dV = gVo * gv,
 * dMs = gMo * gm, dgvm = [sum_a gVo[a] V[a] | sum_k gMo[k] Ms[k]] (N, 2C). */
int face_eq_gate_bwd(const float* V, const float* Ms, const float* gvm, const float* gVo, const float* gMo, int64_t N,
                     int32_t C, float* dV, float* dMs, float* dgvm, void* stream);

/* LayerNorm of the readout's invariant row (face/model.py:140, :332): y = (x - mean) * rstd * w + b
 * over rows of F features, biased variance, rstd = 1 / sqrt(var + eps); mean, rstd (N) are
 * written for the backward. x, y (N, F) contiguous, F % 4 == 0, F <= 2048, 16-byte aligned
 * (else FACE_ERR_UNSUPPORTED). */
int face_layer_norm_fwd(const float* x, int64_t N, int32_t F, const float* w, const float* b, float eps, float* y,
                        float* mean, float* rstd, void* stream);

/* Input gradient of face_layer_norm_fwd: dx = rstd (g - mean(g) - xh mean(g xh)), g = dy w,
 * xh = (x - mean) rstd. No weight gradients. */
int face_layer_norm_bwd(const float* x, const float* dy, int64_t N, int32_t F, const float* w, const float* mean,
                        const float* rstd, float* dx, void* stream);

/* ---------------------------------------------------------------- neighbour build
 * Pair set of ASE neighbor_list("ijS", atoms, rc) as used by face/neighbors.py:12-15 and
 * face/datasets.py:51: all (i, j, S) with |pos[j] - pos[i] + S.cell| < rc in fp64,
 * S integer (0 on non-periodic axes), (i, i, 0) excluded; rows sorted by j then S.
 *
 * Batch description (device): pos (N,3) fp64; atom_struct (N) int32 structure of each atom;
 * struct_ptr (nstr+1) int32 atom ranges; cell (nstr,9) fp64 rows = lattice vectors;
 * inv_cell (nstr,9) fp64 = inverse of cell (zeros for non-periodic structures);
 * pbc (nstr,3) int32.
 *
 * Small-structure path (bin_atoms == NULL): every atom tests every atom of its structure and
 * every image that can lie within rc. Cell-list path (one fully periodic structure, nstr == 1,
 * cell / inv_cell then point at its 9 values): nb is a HOST int32[6] = bins per axis (3) then
 * bins searched on each side (3), each bin at least rc wide along its reciprocal axis unless
 * the search width compensates; bin_of (N), wrap (N,3) = floor(fractional coordinate),
 * bin_start (nbins+1) and bin_atoms (N) come from face_nbr_bin (bin_count, bin_fill: nbins
 * int32 workspaces).                                                                        */
int face_nbr_bin(const double* pos, int64_t N, const double* inv_cell, const int32_t* nb, int32_t* bin_of,
                 int32_t* wrap, int32_t* bin_count, int32_t* bin_start, int32_t* bin_fill, int32_t* bin_atoms,
                 void* stream);
/* counts[i] = number of pairs of atom i. */
int face_nbr_count(const double* pos, int64_t N, const int32_t* atom_struct, const int32_t* struct_ptr,
                   const double* cell, const double* inv_cell, const int32_t* pbc, double rc, const int32_t* nb,
                   const int32_t* bin_of, const int32_t* wrap, const int32_t* bin_start, const int32_t* bin_atoms,
                   int32_t* counts, void* stream);
/* Writes row i of the CSR list: col (E) int32 global neighbour index, S (E,3) int32,
 * shift (E,3) fp32 = fp32(S . cell) computed in fp64; row_ptr (N+1) int32 from a scan of counts.
 * key (E) int64 is workspace. Returns FACE_ERR_CAPACITY via *overflow (device int32) if a row
 * found more pairs than counted (cannot happen for unchanged inputs).                    */
int face_nbr_fill(const double* pos, int64_t N, const int32_t* atom_struct, const int32_t* struct_ptr,
                  const double* cell, const double* inv_cell, const int32_t* pbc, double rc, const int32_t* nb,
                  const int32_t* bin_of, const int32_t* wrap, const int32_t* bin_start, const int32_t* bin_atoms,
                  const int32_t* row_ptr, int64_t* key, int32_t* col, int32_t* S, float* shift, int32_t* overflow,
                  void* stream);
/* rev[e] = index of the reverse edge (j, i, -S) of e = (i, j, S); missing[0] counts edges
 * without one (a non-symmetric list). */
int face_nbr_rev(const int32_t* row_ptr, const int32_t* col, const int32_t* S, int64_t N, int32_t* rev,
                 int32_t* missing, void* stream);
/* Reverse map for an edge list given by fp32 shift vectors (e.g. a padded graph converted
 * to CSR): the reverse of (i, j, shift) is (j, i, -shift) with bitwise-equal components. */
int face_nbr_rev_shift(const int32_t* row_ptr, const int32_t* col, const float* shift, int64_t N, int32_t* rev,
                       int32_t* missing, void* stream);
/* Padded view of face/neighbors.py:27-33: nbr (N,M) int64 (padding -> first atom of the
 * atom's structure), shift_pad (N,M,3) fp32 (padding 0), mask (N,M) uint8. */
int face_nbr_padded(const int32_t* row_ptr, const int32_t* col, const float* shift, const int32_t* atom_struct,
                    const int32_t* struct_ptr, int64_t N, int32_t M, int64_t* nbr, float* shift_pad, uint8_t* mask,
                    void* stream);

/* ---------------------------------------------------------------- edge geometry
 * Per edge e = (i -> col[e], shift[e]) (recv[e] = i): vec = pos[col] - pos[i] + shift,
 * r = |vec| (r := 1 where mask[e] == 0), u = vec / r, Y = monomials(u) (20),
 * bes_n = sin(freq[n] r) / r * bes_scale (freq[n] = (n+1) pi / rc, bes_scale = sqrt(2/rc) as the
 * caller computes them), env = (1 - 28x^6 + 48x^7 - 21x^8)[x<1] * mask, x = r/rc, rb = bes * env. face/model.py:670-677, :28-40, face/cartesian.py:34-46.
 * mask may be NULL (all edges valid). Outputs: Y (E,20), rb (E,nb), env (E), r (E) (may be NULL). */
int face_edge_geom_fwd(const float* pos, const int32_t* recv, const int32_t* col, const float* shift,
                       const uint8_t* mask, int64_t E, const float* freq, int32_t n_basis, float rc, float bes_scale,
                       float* Y, float* rb, float* env, float* r, void* stream);
/* dL/dvec (E,3) from gY (E,20), grb (E,nb), genv (E), gr (E) (any may be NULL = 0). */
int face_edge_geom_bwd(const float* pos, const int32_t* recv, const int32_t* col, const float* shift,
                       const uint8_t* mask, int64_t E, const float* freq, int32_t n_basis, float rc, float bes_scale,
                       const float* gY, const float* grb, const float* genv, const float* gr, float* gvec,
                       void* stream);

/* ---------------------------------------------------------------- radial MLP
 * Hidden layers and the phi columns of the radial MLP of a factorised pass
 * (face/model.py:465-469, rb = bessel * envelope as at face/model.py:676):
 *   u1 = rb W_in^T + b_in + pair_tab[pair[e]],  hid = silu(u1)          (E, H)
 *   u2 = hid W1^T + b1,                         h2  = silu(u2)          (E, H)
 *   phi = (h2 W_phi^T + b_phi) * env[e]                                 (E, B)
 * rb (E, ld_rb >= n_basis), n_basis <= 16; pair (E) int32 element-pair row of pair_tab
 * (n_pair, H); W_in (H, n_basis), W1 (H, H), W_phi (B, H) row-major effective weights
 * (any 1/sqrt(fan_in) factor applied); H in {16, 32, 48, 64}, B <= 64. env may be NULL (= 1).
 * h2 (E, ld_h2) is optional (NULL: not written; 16-byte aligned rows otherwise) -- the CP
 * columns of the last radial layer are a GEMM on it.                                       */
int face_radial_fwd(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair, const float* env,
                    int64_t E, const float* w_in, const float* b_in, const float* pair_tab, int32_t n_pair,
                    int32_t H, const float* w1, const float* b1, const float* w_phi, const float* b_phi, int32_t B,
                    float* h2, int32_t ld_h2, float* phi, int32_t ld_phi, void* stream);
/* Backward for gh2 = dL/dh2 (may be NULL = 0; 16-byte aligned rows) and gphi = dL/dphi
 * (plus gphi2, same layout, when phi has a second reader; may be NULL):
 * grb (E, ld_grb) = dL/drb, genv (E) = dL/denv through phi (either may be NULL). The
 * weights receive no gradient (forces only). */
int face_radial_bwd(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair, const float* env,
                    int64_t E, const float* w_in, const float* b_in, const float* pair_tab, int32_t n_pair,
                    int32_t H, const float* w1, const float* b1, const float* w_phi, const float* b_phi, int32_t B,
                    const float* gh2, int32_t ld_gh2, const float* gphi, const float* gphi2, int32_t ld_gphi,
                    float* grb, int32_t ld_grb, float* genv, void* stream);
/* The radial MLPs of n_sets (<= 4) passes over the same edges in one launch (the passes'
 * radial functions are independent of each other, face/model.py:465-469 per pass): weights is a
 * host array of 7 n_sets device pointers (w_in, b_in, pair_tab, w1, b1, w_phi, b_phi of set k at
 * 7k .. 7k + 6), h2 / phi host arrays of n_sets outputs (h2 may be NULL, or hold NULL entries);
 * each set as face_radial_fwd. */
int face_radial_fwd_sets(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair, const float* env,
                         int64_t E, int32_t n_sets, const float* const* weights, int32_t n_pair, int32_t H, int32_t B,
                         float* const* h2, int32_t ld_h2, float* const* phi, int32_t ld_phi, void* stream);
/* Backward of face_radial_fwd_sets: host arrays of n_sets gh2 / gphi / gphi2 / grb / genv (the
 * arrays other than gphi may be NULL; entries may be NULL), each set as face_radial_bwd. */
int face_radial_bwd_sets(const float* rb, int32_t ld_rb, int32_t n_basis, const int32_t* pair, const float* env,
                         int64_t E, int32_t n_sets, const float* const* weights, int32_t n_pair, int32_t H, int32_t B,
                         const float* const* gh2, int32_t ld_gh2, const float* const* gphi, const float* const* gphi2,
                         int32_t ld_gphi, float* const* grb, int32_t ld_grb, float* const* genv, void* stream);

/* ---------------------------------------------------------------- compiled radial (splines)
 * RadialSpline.forward (face/model.py:407-418), the table lookup that FACE.compile_radial
 * (face/model.py:644-655) puts in place of the radial MLP: T, dT (P, G, F) row-major hold the
 * values and exact r-derivatives of the radial functions of each element pair on the grid
 * r_g = g * dr; for edge e, x = clamp(r[e] / dr, 0, G - 1), i = min(floor x, G - 2), t = x - i,
 *   S[e, f] = h00 T[p][i][f] + h10 dr dT[p][i][f] + h01 T[p][i+1][f] + h11 dr dT[p][i+1][f]
 * (cubic Hermite basis), p = pair[e] (clamped into [0, P)). Columns f < nb: phi[e][f] =
 * S[e,f] * env[e] (face/model.py:467; env may be NULL: factor 1); columns f >= nb (the CP
 * radials, enveloped inside the pooling kernels): R[e][f - nb] = S[e,f]. G >= 2, dr > 0,
 * 0 <= nb <= F; phi is unused when nb = 0, R when nb = F. order (E, may be NULL): the
 * permutation of the edges in which to visit them (face_radial_spline_order), no effect on the
 * results. */
int face_radial_spline_fwd(const float* r, const int32_t* pair, int64_t E, const float* T, const float* dT, int32_t P,
                           int32_t G, int32_t F, float dr, const float* env, int32_t nb, const int32_t* order,
                           float* phi, int32_t ld_phi, float* R, int32_t ld_R, void* stream);
/* Its backward for upstream gphi (E, ld_gphi >= nb) and gR (E, ld_gR >= F - nb) (either may be
 * NULL = 0): gr[e] = sum_f g[e,f] dphi_or_R[e,f]/dr (0 where r / dr lies outside [0, G - 1], as
 * through the clamp), genv[e] = sum_{f < nb} gphi[e,f] S[e,f] (genv may be NULL). */
int face_radial_spline_bwd(const float* r, const int32_t* pair, int64_t E, const float* T, const float* dT, int32_t P,
                           int32_t G, int32_t F, float dr, const float* env, int32_t nb, const int32_t* order,
                           const float* gphi, int32_t ld_gphi, const float* gR, int32_t ld_gR, float* gr, float* genv,
                           void* stream);
/* No counterpart in the reference (its index_select gathers in edge order): the edges sorted by
 * table cell (pair, grid interval) into order (E), a permutation, so that the spline kernels
 * read each table row from L2 for the whole run of edges that needs it -- worth it when the
 * tables (8 P G F bytes) are far larger than L2. work: P * G int32 of scratch. */
int face_radial_spline_order(const float* r, const int32_t* pair, int64_t E, int32_t P, int32_t G, float dr,
                             int32_t* work, int32_t* order, void* stream);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP-graph capture, tight serving loops, harnesses that forbid hipMalloc): face_radial_spline_order
 * without the `work` argument. Its P * G sort counters live in a fixed device array of the library,
 * FACE_SPLINE_ORDER_SCRATCH int32 (4 MiB) per GPU, held until the process ends; P * G above that
 * returns FACE_ERR_SCRATCH before any launch. The entry point allocates nothing (no hipMalloc /
 * hipFree); the counters are cleared by a kernel at the start of every call. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (e.g. on two streams) race. */
#define FACE_SPLINE_ORDER_SCRATCH (1 << 20)
int face_radial_spline_order_noalloc(const float* r, const int32_t* pair, int64_t E, int32_t P, int32_t G, float dr,
                                     int32_t* order, void* stream);

/* ---------------------------------------------------------------- row-block linear layers
 * One problem: x (m, ld_x >= k) rows, w (n, k) row-major with row stride ld_w (w_kn = 0) or
 * (k, n) with row stride ld_w (w_kn = 1), y (m, ld_y >= n); n and k multiples of 16.
 * Optional per problem (NULL / 0 = absent):
 *   x2, ld_x2, k1   input columns k >= k1 are read from x2 (column k - k1): x = [x | x2], the
 *                   concatenation of two activations without a copy (k1 a multiple of 16; k1 = k
 *                   when x2 is NULL);
 *   x_op, xz, ld_xz transform of the input columns k < k1 as they load: 0 none, 1 silu(x),
 *                   2 x * silu'(xz) (xz (m, ld_xz) the pre-activation, for backward chains);
 *   bias            (n) added to every row;
 *   y0, ld_y0, n_y0 initial value of the sum: beta * y0[r, c] for columns c < n_y0 (a multiple
 *                   of 4), 0 beyond; y0 NULL: beta * y[r, :] (y0 may be another tensor, e.g. a
 *                   residual). */
typedef struct {
    const float* x;
    int64_t ld_x, m;
    const float* w;
    int64_t ld_w;
    float* y;
    int64_t ld_y;
    int32_t n, k, s_off;
    float beta;
    const float* x2;
    int64_t ld_x2;
    int32_t k1, x_op;
    const float* xz;
    int64_t ld_xz;
    const float* bias;
    const float* y0;
    int64_t ld_y0;
    int32_t n_y0, pad_;
} face_lin_problem;
/* For each problem (1..8 of them, host array):
 *   y[r, :] = (beta y0[r, :] + (op(x)[r, :] * xs[r, :]) w^T + bias) * ys[r, :]
 * with xs[r, k] = x_scale[group[r % period] * ld_scale + s_off + k] and ys likewise over the
 * n output columns, group values in [0, n_groups) (n_groups <= 64: the scale tables' rows, staged
 * in LDS); x_scale, y_scale may be NULL (beta = 0: y0 / y is not read). The linear layers of the
 * node features: mix / tmix / proj (face/model.py:498-533, :537-544) with the elem_scale factor,
 * the readout MLP (face/model.py:331-339: [inv | h] W0^T + b0, then SiLU-on-load layers, the
 * residual as y0) and their input gradients (w_kn = 1). x, x2, xz, y, y0, bias and the scale
 * tables 16-byte aligned, every ld and s_off a multiple of 4; FACE_ERR_UNSUPPORTED when an operand
 * spans 2^31 elements or more (m * ld of x, x2, xz, y or y0: rows are addressed by 32-bit offsets). */
int face_rows_linear(const face_lin_problem* probs, int32_t n_probs, int32_t w_kn, const float* x_scale,
                     const float* y_scale, int32_t ld_scale, int32_t n_groups, const int32_t* group, int64_t period,
                     void* stream);

/* ---------------------------------------------------------------- per-edge linear layers
 * Forward: y (E, ld_y) = x (E, ld_x) w^T + b + tab[idx[e]], w (F, K) row-major, b (F) and tab
 * (N, ld_tab) optional (NULL), idx NULL = row e of tab. K in {16, 32, 48, 64}, F a multiple
 * of 16; x, w, b, tab, y 16-byte aligned and ld_* multiples of 4 (else FACE_ERR_UNSUPPORTED).
 * Replaces the last nn.Linear of the radial MLP for the CP columns (face/model.py:469 with the
 * split at :496-497; tab NULL) and gather(msg(h)) + dir_mix(d) (face/model.py:488-493: x = d,
 * w = dir_mix weight, b = its bias, tab = msg(h), idx = col). */
int face_edge_linear_fwd(const float* x, int32_t ld_x, int64_t E, int32_t K, const float* w, const float* b,
                         int32_t F, const float* tab, int32_t ld_tab, const int32_t* idx, float* y, int32_t ld_y,
                         void* stream);
/* Backward of face_edge_linear_fwd with idx = col of a CSR graph with reverse-edge map rev:
 * dx (E, ld_dx) = dy w and dtab (N, ld_dtab) row n = sum of dy[e] over the edges with col = n
 * (rev[e] for e in row n); either output may be NULL. F <= 256. The reduction has a fixed
 * order (no atomics). */
int face_edge_linear_bwd(const float* dy, int32_t ld_dy, int32_t F, const float* w, int32_t K,
                         const int32_t* row_ptr, const int32_t* rev, int64_t N, float* dx, int32_t ld_dx, float* dtab,
                         int32_t ld_dtab, void* stream);

/* ---------------------------------------------------------------- directional edge features
 * Node tables of Kd channels: V element (component a, atom n, channel k) at
 * V[a*v_sq + n*v_sn + k] (3 components), M likewise (6 components, sym storage).
 * d (E, 4*Kd) = [u.V_j | u^T M_j u | u.V_i | u^T M_i u] with u = Y[e,1:4], u^T M u =
 * sum_q Y[e,4+q] * (1,1,1,2,2,2)_q * M_q, j = col[e], i = recv[e]
 * (face/model.py:474-493, the per-edge d fed to dir_mix).                                  */
int face_dir_feats_fwd(const float* V, int64_t v_sn, int64_t v_sq, const float* M, int64_t m_sn, int64_t m_sq,
                       int32_t Kd, const int32_t* recv, const int32_t* col, const float* Y, int64_t E, float* d,
                       void* stream);
/* Backward for gd = dL/dd (E, 4*Kd): gV, gM (same layouts as V, M; both or neither) through the
 * reverse-edge map (no atomics), gY (E, 20) (monomials 0 and 10..19 written as zero; may be NULL).
 * Kd <= 64. */
int face_dir_feats_bwd(const float* V, int64_t v_sn, int64_t v_sq, const float* M, int64_t m_sn, int64_t m_sq,
                       int32_t Kd, const int32_t* row_ptr, const int32_t* recv, const int32_t* col, const int32_t* rev,
                       const float* Y, const float* gd, int64_t N, int64_t E, float* gV, float* gM, float* gY,
                       void* stream);

/* ---------------------------------------------------------------- transport moments
 * D[i, b, kd, :] = scale * sum_{e in row i} phi[e, b] * F(u_e, V_j[kd], M_j[kd]),
 * F = [V (3) | M u (3) | M (6) | sym(u (x) V) (6)], j = col[e], u = Y[e, 1:4]: the transport sums of
 * face/model.py:514-528 ([1,u] (x) phi (x) [V|M] mapped by its (36,18) transport map), written as
 * D1 (3, N, B*2*Kd) = [V | M u] and D2 (6, N, B*2*Kd) = [M | sym(u V)], channel b*2Kd + t*Kd + kd.
 * Tables V, M as for the directional features (the transport half of the channels).
 * B * Kd <= 1024.                                                                            */
int face_transport_fwd(const float* phi, int32_t ld_phi, int32_t B, const float* V, int64_t v_sn, int64_t v_sq,
                       const float* M, int64_t m_sn, int64_t m_sq, int32_t Kd, const float* Y, int32_t ld_Y,
                       const int32_t* col, const int32_t* row_ptr, int64_t N, float scale, float* D1, float* D2,
                       void* stream);
/* Backward for gD1, gD2 (layouts of D1, D2): dphi (E, ld_dphi) (may be NULL), dT_edge (E, 9, Kd)
 * per-edge table gradient (workspace), gV / gM (table gradients through the reverse map; both or
 * neither, written in V / M's layout), gY: du is ADDED to gY[e, 1..3] (gY must hold the other
 * contributions, e.g. face_dir_feats_bwd's output; may be NULL). B <= 32, Kd <= 64.          */
int face_transport_bwd(const float* phi, int32_t ld_phi, int32_t B, const float* V, int64_t v_sn, int64_t v_sq,
                       const float* M, int64_t m_sn, int64_t m_sq, int32_t Kd, const float* Y, int32_t ld_Y,
                       const int32_t* col, const int32_t* row_ptr, const int32_t* rev, int64_t N, int32_t max_row,
                       float scale, const float* gD1, const float* gD2, float* dphi, int32_t ld_dphi, float* dT_edge,
                       float* gV, float* gM, float* gY, void* stream);

/* ---------------------------------------------------------------- gathers and scatters
 * out[e, :] = X[idx[e], :] for F features (X row stride ld_X, out row stride ld_out). */
int face_gather_rows(const float* X, int32_t ld_X, const int32_t* idx, int64_t E, int32_t F, float* out,
                     int32_t ld_out, void* stream);
/* Backward of a gather along col of a symmetric edge list, without atomics:
 * dX[k, :] = sum_{e in row k} g[rev[e], :]  (the edges with col == k are the reverses of row k). */
int face_gather_rows_bwd(const float* g, int32_t ld_g, const int32_t* row_ptr, const int32_t* rev, int64_t N,
                         int32_t F, float* dX, int32_t ld_dX, void* stream);
/* Row sums: out[k, :] = sum_{e in row k} g[e, :]. */
int face_segment_sum(const float* g, int32_t ld_g, const int32_t* row_ptr, int64_t N, int32_t F, float* out,
                     int32_t ld_out, void* stream);
/* Atom energies and their per-structure sums (replaces e_at = E0[z] + sum_p scale * e_p and the
 * index_add over batch, face/model.py:680-690): e_at[a] = e0[a] + scale[0] * e_p[a * ld_e[p]],
 * added pass by pass over the n_e (<= 8) passes (host arrays e, ld_e of device pointers / strides),
 * and E[s] = sum of e_at over the atoms [struct_ptr[s], struct_ptr[s+1]) of structure s (atoms of
 * a structure contiguous; fixed summation order). scale is a device scalar.                */
int face_atom_energy_fwd(const float* e0, const float* scale, const float* const* e, const int64_t* ld_e,
                         int32_t n_e, const int32_t* struct_ptr, int64_t nstr, float* e_at, float* E, void* stream);
/* Backward: ge[a] = scale[0] * (gE[s] + g_at[a]) for the atoms a of structure s, the gradient of
 * every pass's e_p; gE (nstr) or g_at (N) may be NULL (zero).                               */
int face_atom_energy_bwd(const float* gE, const float* g_at, const float* scale, const int32_t* struct_ptr,
                         int64_t nstr, float* ge, void* stream);
/* dE/dpos from dE/dvec (vec_e = pos[col e] - pos[i] + shift): grad[k] = sum_{e in row k} (gvec[rev e] - gvec[e]).
 * Writes grad (N,3) (forces are its negative: sign = -1 writes -grad). */
int face_force_scatter(const float* gvec, const int32_t* row_ptr, const int32_t* rev, int64_t N, float sign,
                       float* grad, void* stream);
/* The same force scatter without reverse-edge gathers, in two passes over a CSR list (no mask):
 * face_edge_geom_bwd_seg computes dL/dvec of every edge as face_edge_geom_bwd does and writes it
 * to the slot of the edge's reverse, gvec_rev[rev e], as a 16-byte row (x, y, z, 0) of an (E,4)
 * buffer; its own-row sums are reduced per window of 64 consecutive edges (e / 64) and written to
 * wsum (E,4) at the last edge of the row in the window (wsum's other rows are left unwritten).
 * Both buffers 16-byte aligned; Y gradient buffers too. face_force_scatter_rows then writes
 * grad[k] = sign * sum_{e in row k} (gvec_rev[e] - [e is the row's last edge in its window] wsum[e]),
 * reading each row contiguously. mean_row (~E/N) picks the lanes per row. Fixed summation
 * order, no atomics. Replaces the index_add backward of pos[nbr] - pos[i] (face/model.py:670;
 * forces = -grad at :692-694). gY, grb, genv, gr each point to 4 gradient buffers of that input
 * (entries may be null; a null array means none), summed in slot order: one per reader of the
 * input in the forward, so no separate accumulation of the readers' gradients is needed. */
int face_edge_geom_bwd_seg(const float* pos, const int32_t* recv, const int32_t* col, const float* shift,
                           const int32_t* rev, int64_t E, const float* freq, int32_t n_basis, float rc, float bes_scale,
                           const float* const* gY, const float* const* grb, const float* const* genv,
                           const float* const* gr, float* gvec_rev, float* wsum, void* stream);
int face_force_scatter_rows(const float* gvec_rev, const float* wsum, const int32_t* row_ptr, int64_t N,
                            int32_t mean_row, float sign, float* grad, void* stream);

#ifdef __cplusplus
}
#endif
#endif
