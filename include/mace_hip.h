/*
 * mace_hip.h — C ABI of libmace_hip.so, the MI355X (gfx950) backend of mace_hip_kernels.
 *
 * The reference (Yike-Ye/mace-mps-kernels) JIT-compiles one generated Metal library per layer with
 * torch.mps.compile_shader and calls its kernels as lib.<kernel>(tensors..., n, threads=...).  This library is the
 * HIP replacement of that boundary: per-layer HIP source (generated in Python with the layer's coupling
 * coefficients as literals) is compiled by hipRTC into a gfx950 code object, loaded as a module, and its kernels are
 * launched on the caller's HIP stream.  Plain pointers and sizes only; no torch types.
 *
 * Conventions
 *   - Every function returns 0 on success or a nonzero hipError_t / hiprtcResult code; mh_last_error() then holds a
 *     message (per calling thread).
 *   - All device pointers are caller-owned (torch allocations); the library never allocates or frees tensor memory
 *     and never synchronises the stream.  Inputs must be contiguous fp32 / int32 in the layouts below.
 *   - A module is bound to the device that was current when it was loaded; launching it with another device current
 *     is an error.  Module handles are immutable after mh_module_bind, so concurrent launches are safe.
 *
 * Layouts (e3nn "mul_ir"), MUL channels, NINS instructions:
 *   x   [N, X_DIM]       node features, block b at x_off[b] + u*(2l_b+1) + m
 *   Y   [E, Y_DIM]       edge spherical harmonics
 *   W   [E, NINS*MUL]    per-edge weights, instruction k / channel u at k*MUL + u
 *   out [N, OUT_DIM]     instruction k output block at o_off[k] + u*(2l_k+1) + m;  out[n] = Σ_{e: recv(e)=n} TP(...)
 *   X   [N, C, N_ELL]    symmetric-contraction input;  T [n_elem, R, C] polynomial table;  elem [N] int32
 */
#ifndef MACE_HIP_H
#define MACE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mh_module mh_module;

/* kernel slots a module can bind (mh_module_bind) */
enum mh_kernel_kind {
    MH_CONV_FWD = 0,     /* receiver rows over the receiver CSR                                   */
    MH_CONV_BWD = 1,     /* fused d/dx, d/dW, d/dY: sender rows over the sender CSR               */
    MH_CONV_BWD_WY = 2,  /* d/dW, d/dY only: chunks of consecutive edges, no CSR                  */
    MH_SC_FWD = 3,       /* node rows                                                             */
    MH_SC_BWD = 4,       /* node rows                                                             */
    MH_CONV_BWD_R = 5,   /* d/dW, d/dY and per-edge dX messages: receiver rows over the receiver CSR */
    MH_CONV_GXSUM = 6,   /* dX = sum of an edge-row array over the sender CSR: sender rows        */
    MH_SC_FWD_G = 7,     /* groups of consecutive nodes of an element-sorted order                */
    MH_SC_BWD_G = 8,     /* groups of consecutive nodes of an element-sorted order                */
    MH_CONV_BWD_RC = 9,  /* MH_CONV_BWD_R with the weights factored as W0 * cutoff per edge       */
    MH_CONV_FWD_C = 10,  /* MH_CONV_FWD skipping edges whose cutoff is 0                          */
    MH_SH_FWD = 11,      /* edge spherical harmonics: one edge per thread                         */
    MH_SH_BWD = 12,      /* their gradient with respect to the edge vectors                       */
    MH_LIN_FWD = 13,     /* node-wise equivariant linear (optionally modulated by scalar attrs)    */
    MH_LIN_BWD = 14,     /* its input gradient (the same map with transposed weights)              */
    MH_MLP_FWD = 15,     /* radial MLP: per-edge weights from the edge features, 64 edges a block  */
    MH_MLP_BWD = 16,     /* its input gradient (hidden layers recomputed)                          */
    MH_EMB_FWD = 17,     /* radial embedding: Bessel basis x polynomial cutoff of the edge lengths */
    MH_EMB_BWD = 18,     /* its gradient with respect to the lengths                               */
    MH_PERM_FWD = 19,    /* per-node permutation irreps layout -> [mul, sum (2l+1)]                */
    MH_PERM_BWD = 20,    /* its inverse                                                            */
    MH_GEOM_FWD = 21,    /* edge vectors and lengths from positions, edge list and shifts          */
    MH_GEOM_BWD = 22,    /* their gradient: per-atom CSR sums (one wave per atom)                  */
    MH_SC_FWD_I = 23,    /* MH_SC_FWD reading x in e3nn's irreps layout                            */
    MH_SC_BWD_I = 24,    /* MH_SC_BWD reading x and writing its gradient in the irreps layout      */
    MH_SC_FWD_GI = 25,   /* MH_SC_FWD_G in the irreps layout                                       */
    MH_SC_BWD_GI = 26,   /* MH_SC_BWD_G in the irreps layout                                       */
    MH_READOUT_FWD = 27, /* readout head: per-node energy from the node features, 16 nodes a block  */
    MH_READOUT_BWD = 28, /* its input gradient                                                     */
    MH_SC_JVP = 29,      /* symmetric contraction: directional derivative of the output, node rows */
    MH_SC_BWD2 = 30,     /* directional derivative of the x-gradient (a Hessian-vector product)     */
    MH_SC_JVP_I = 31,    /* MH_SC_JVP in the irreps layout                                          */
    MH_SC_BWD2_I = 32,   /* MH_SC_BWD2 in the irreps layout                                         */
    MH_CSR_FILL = 33,    /* graph build: zero the per-node counters (grid y = the two index rows)   */
    MH_CSR_COUNT = 34,   /* int32 copy of the indices (clamped, flagged) and per-node edge counts   */
    MH_CSR_SCAN = 35,    /* rowptr = exclusive scan of the counts (one workgroup per index row)     */
    MH_CSR_SCATTER = 36, /* each edge into its node's segment (any order)                           */
    MH_CSR_RANK = 37,    /* each segment's edges in increasing edge order                           */
    MH_SH_JVP = 38,      /* edge spherical harmonics: derivative along a direction of the vectors   */
    MH_SH_BWD2 = 39,     /* derivative of their vector gradient along that direction                */
    MH_EMB_JVP = 40,     /* radial embedding: derivative along a direction of the lengths           */
    MH_EMB_BWD2 = 41,    /* derivative of its length gradient along that direction                  */
    MH_GEOM_JVP = 42,    /* edge geometry, behind a double backward: per-edge second-order terms     */
    MH_READOUT_JVP = 43, /* SiLU readout head: derivative of the energy along a direction of x       */
    MH_READOUT_BWD2 = 44,/* derivative of its input gradient along that direction                   */
    MH_CSR_SORT = 45,    /* graph build: sort each segment longer than the counting kernel handles  */
    MH_MLP_HID = 46,     /* radial MLP's hidden layers only: last hidden activations h [E, HL]      */
    MH_MLP_HIDB = 47,    /* their backward from the fused convolution's partial dL/d(c h)           */
    MH_CONV_FWD_M = 48,  /* convolution forward with the MLP's output layer fused (grid_y: tiles)  */
    MH_CONV_BWD_M = 49,  /* its backward: dX messages, gY and dL/d(c h) partials (grid_y: tiles)   */
    MH_CONV_GYSUM = 50,  /* gY = sum of the fused backward's per-channel-tile partials             */
    MH_SC_FWD_S = 51,    /* symmetric contraction, coefficient rows staged in LDS (grid_y: blocks)  */
    MH_SC_BWD_S = 52,    /* its x-gradient                                                          */
    MH_SC_FWD_SI = 53,   /* MH_SC_FWD_S in the irreps layout                                        */
    MH_SC_BWD_SI = 54,   /* MH_SC_BWD_S in the irreps layout                                        */
    MH_NL_SETUP = 55,    /* neighbour list: per-structure bounding box, images, bin grid            */
    MH_NL_ZERO = 56,     /* zero an int32 array                                                     */
    MH_NL_BINS = 57,     /* each atom's bin, per-bin counts                                         */
    MH_NL_SCAN = 58,     /* bin offsets (one workgroup)                                             */
    MH_NL_PLACE = 59,    /* atoms into their bins                                                   */
    MH_NL_COUNT = 60,    /* edges per sender (one wave per sender)                                  */
    MH_NL_OFFSETS = 61,  /* edges per structure, each sender's segment start (one workgroup)        */
    MH_NL_FILL = 62,     /* edges of each sender, ordered, and its padding (one wave per sender)    */
    MH_SPECIES_ORDER = 63, /* element index, stable element order and contraction slots (one workgroup) */
    MH_MLP_JVP = 64,     /* radial MLP: derivative of its output along a direction of the features  */
    MH_MLP_BWD2 = 65,    /* derivative of its feature gradient along that direction                 */
    MH_GEOM_SEGSUM = 66, /* per-structure sums of 3x3 rows (the stress displacement's gather backward) */
    MH_NL_BASES = 67,    /* neighbour list: each structure's first edge slot (one workgroup)        */
    MH_EDGE_COUNT = 68,  /* edge compaction: kept edges per workgroup of 4096                       */
    MH_EDGE_PLACE = 69,  /* edge compaction: the row list                                           */
    MH_GEOM_SEGSUM1 = 70, /* per-structure sums of one column (MACE's energy sums)                  */
    MH_EDGE_PAIR = 71,   /* shared radial-MLP rows of an edge and its reverse                         */
    MH_CONV_FWD_CR = 72, /* conv fwd, W0 * cutoff with W0 rows through a row map (cacheable loads)     */
    MH_MLP_H3 = 73,      /* radial MLP: last hidden activations of the listed rows, h3 [slot][HL]       */
    MH_MLP_OUT = 74,     /* its output layer, weight-stationary: persistent waves over 16-edge tiles    */
    MH_EDGE_FWD = 75,    /* edge geometry, spherical harmonics and radial embedding in one pass          */
    MH_EDGE_BWD = 76,    /* the harmonics' and the embedding's backward in one pass                      */
    MH_MLP_BWD_P = 77,   /* radial MLP backward over shared rows, an edge's and its partner's gW0 summed   */
    MH_LIN_BWD_SUM = 78, /* node linear backward over the sum of three gradients of its output               */
    MH_NUM_KINDS = 79
};

/* flags of mh_conv_bwd */
#define MH_WANT_GX 1
#define MH_WANT_GWY 2
/* flag of mh_conv_bwd_recv (factored weights only): cutoff[e] == -0.0 exactly marks an edge outside the cutoff
 * envelope's support, where the envelope's derivative is zero */
#define MH_CUT_MASKED 4
/* with MH_CUT_MASKED: the masked edges' gW rows are left unwritten (not zeroed) */
#define MH_CUT_NOZERO 8

/* Message of the last failing call on this thread ("" if none).  No reference counterpart (Metal errors surface
 * from torch there). */
const char* mh_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int mh_version(void);

/* Launch log of the process, for profiling and tests that check which kernels ran: while enabled, every successful
 * launch, from any thread (autograd runs backward passes on threads of its own), appends the symbol bound to the
 * launched slot.  mh_launch_log(1) enables it, mh_launch_log(0)
 * disables and clears it; both return the previous state.  mh_launch_log_take copies the names, each followed by
 * ';', oldest first, into buf (NUL-terminated) and clears the log when it fitted; it returns the log's length (call
 * with buf NULL to size the buffer).  No reference counterpart (Metal kernels are named in the reference's own
 * source). */
int mh_launch_log(int enable);
size_t mh_launch_log_take(char* buf, size_t len);

/* Path of the HIP runtime library this .so is bound to (must be the one torch loaded). */
const char* mh_hip_runtime_path(void);

/* hipRTC-compile `source` with space-separated `options` into a code object (malloc'ed, release with
 * mh_free_code).  Needs no GPU.  Replaces the compile half of torch.mps.compile_shader (reference conv.py:280,
 * symmetric.py:165). */
int mh_compile(const char* source, const char* options, void** code, size_t* code_size);
void mh_free_code(void* code);

/* Load a code object on the current device.  Replaces the load half of torch.mps.compile_shader. */
int mh_module_load(const void* code, size_t code_size, mh_module** out);
int mh_module_unload(mh_module* m);

/* Attach kernel `name` of the module to slot `kind` with its launch shape: `block_threads` threads per workgroup,
 * each workgroup covering `rows_per_block` rows of the launch (receivers, senders, nodes or edges).  Replaces the
 * threads=/group_size= launch arguments of the reference (conv.py:247, 264, 269; symmetric.py:140, 154). */
int mh_module_bind(mh_module* m, int kind, const char* name, int block_threads, int rows_per_block);
/* As mh_module_bind, with a second grid dimension of grid_y workgroups (1..65535); mh_module_bind uses 1. */
int mh_module_bind_grid(mh_module* m, int kind, const char* name, int block_threads, int rows_per_block,
                        int grid_y);

/* Fused convolution forward: out[n] = Σ_{p in rowptr[n]..rowptr[n+1]} TP(x[senders[e]], Y[e], W[e]), e = eids[p].
 * rowptr/eids: receiver-sorted CSR.  Replaces lib.conv_fwd (reference conv.py:109-141, launched at conv.py:247). */
int mh_conv_fwd(mh_module* m, const float* x, const float* Y, const float* W, const int32_t* rowptr,
                const int32_t* eids, const int32_t* senders, float* out, int32_t N, void* stream);

/* mh_conv_fwd for weights W0[e] * cutoff[e] (W passed as the unscaled W0 [E, NW], cutoff [E]; the kernel scales
 * each edge's weights in registers, so the product is never stored): an edge with cutoff[e] == 0 contributes exactly
 * zero and is skipped (the padding of fixed-size graphs, and neighbour-list entries beyond the cutoff radius).  Same
 * result as mh_conv_fwd on W0 * cutoff up to the sign of zero sums.  No reference counterpart. */
int mh_conv_fwd_cut(mh_module* m, const float* x, const float* Y, const float* W, const int32_t* rowptr,
                    const int32_t* eids, const int32_t* senders, const float* cutoff, float* out, int32_t N,
                    void* stream);
/* mh_conv_fwd_cut with edge e's W0 row read at row wrow[e] of W (wrow [E] int32 on the device; NULL: row e), so
 * that edges with equal radial-MLP rows can share one (mh_edge_pairs).  With a row map it launches MH_CONV_FWD_CR
 * (the same kernel with cacheable W0 loads: a shared row is read twice), without one MH_CONV_FWD_C.  No reference
 * counterpart. */
int mh_conv_fwd_cut_rows(mh_module* m, const float* x, const float* Y, const float* W, const int32_t* rowptr,
                         const int32_t* eids, const int32_t* senders, const float* cutoff, const int32_t* wrow,
                         float* out, int32_t N, void* stream);

/* d/dx only, over the sender-sorted CSR: gx[s] = Σ_{e: sender(e)=s} ∂TP/∂x · g[receivers[e]].
 * Replaces lib.conv_bwd_x (reference conv.py:144-176, launched at conv.py:264).  Runs the MH_CONV_BWD kernel with
 * flags = MH_WANT_GX. */
int mh_conv_bwd_x(mh_module* m, const float* g, const float* Y, const float* W, const int32_t* rowptr_s,
                  const int32_t* eids_s, const int32_t* receivers, float* gx, int32_t N, void* stream);

/* d/dW and d/dY per edge: gW[e, k*MUL+u] = ∂TP/∂W · g[recv(e)],  gY[e, j] = Σ_u W·∂TP/∂Y · g[recv(e)].
 * Replaces lib.conv_bwd_wy (reference conv.py:179-222, launched at conv.py:269). */
int mh_conv_bwd_wy(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                   const int32_t* senders, const int32_t* receivers, float* gW, float* gY, int32_t E, void* stream);

/* Fused backward over the sender-sorted CSR: one pass computes any of gx (flags & MH_WANT_GX) and gW, gY
 * (flags & MH_WANT_GWY), reading W once and gathering the g row of every edge's receiver.  Outputs not wanted may
 * be NULL.  mace_hip_kernels uses it when only gx is wanted; it replaces the pair lib.conv_bwd_x +
 * lib.conv_bwd_wy (reference conv.py:252-270). */
int mh_conv_bwd(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                const int32_t* rowptr_s, const int32_t* eids_s, const int32_t* receivers, float* gx, float* gW,
                float* gY, int32_t N, int32_t flags, void* stream);

/* Backward in receiver order, the path mace_hip_kernels uses whenever gW and gY are wanted (flags must hold
 * MH_WANT_GWY).  Kernel MH_CONV_BWD_R walks the receiver CSR (rowptr_r, eids_r, senders: the forward's), keeps
 * g[r] in registers for the whole row and writes gW[e] and gY[e].  With MH_WANT_GX it also writes each edge's dX
 * message work[e, :] = Σ_k W·∂TP/∂x · g[r] ([E, X_DIM] floats of caller-owned scratch), and kernel MH_CONV_GXSUM
 * then sums them over the sender CSR (rowptr_s, eids_s) in CSR order: gx[s] = Σ_{p} work[eids_s[p], :].  No
 * atomics; the result is deterministic.  Together the two kernels replace lib.conv_bwd_wy + lib.conv_bwd_x
 * (reference conv.py:144-222, launched at conv.py:259-270).  Without MH_WANT_GX, rowptr_s, eids_s, gx and work
 * may be NULL.
 * Factored weights: with `cutoff` non-NULL ([E] floats) the weights are W = W0 * cutoff[e] (MACE multiplies the
 * radial MLP output by the cutoff envelope before the convolution) and `W` must point to W0.  Then `gW` receives
 * ∂/∂W0 = ∂/∂W * cutoff[e] and `g_cutoff` ([E]) receives ∂/∂cutoff[e] = Σ_{k,u} ∂/∂W[e,k,u] * W0[e,k,u], so the caller
 * need not differentiate the product itself (kernel MH_CONV_BWD_RC; no reference counterpart).
 * With MH_CUT_MASKED in `flags` (factored weights only) an edge whose cutoff is -0.0 exactly is taken to lie outside
 * the envelope's support (mace_hip_kernels' radial embedding writes -0.0 there, where the envelope's derivative is
 * zero): its gW, gY and g_cutoff rows are written as zeros without reading W0 or x, and it has no dX message.  Only
 * g_cutoff differs from the unmasked call (it is the exact partial derivative there), and only where whatever
 * produced the cutoff multiplies it by a zero derivative.  MH_CUT_NOZERO as well: the masked edges' gW rows are
 * not written at all (for a caller whose consumer of gW skips them, as mh_mlp_bwd_rows does). */
int mh_conv_bwd_recv(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                     const int32_t* rowptr_r, const int32_t* eids_r, const int32_t* senders,
                     const int32_t* rowptr_s, const int32_t* eids_s, float* work, float* gx, float* gW, float* gY,
                     const float* cutoff, float* g_cutoff, int32_t N, int32_t flags, void* stream);
/* mh_conv_bwd_recv with factored weights whose W0 rows are read at wrow[e] (as mh_conv_fwd_cut_rows; NULL: row e).
 * gW stays per edge: row e receives ∂/∂W0 of edge e.  No reference counterpart. */
int mh_conv_bwd_recv_rows(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                          const int32_t* rowptr_r, const int32_t* eids_r, const int32_t* senders,
                          const int32_t* rowptr_s, const int32_t* eids_s, float* work, float* gx, float* gW, float* gY,
                          const float* cutoff, float* g_cutoff, const int32_t* wrow, int32_t N, int32_t flags,
                          void* stream);

/* Symmetric contraction forward: out[b, off + c*M + m] = Σ_terms T[elem[b], r0+m, c] Π X[b, c, idx].
 * Replaces lib.sc_fwd (reference symmetric.py:82-105, launched at symmetric.py:140). */
int mh_sc_fwd(mh_module* m, const float* X, const int32_t* elem, const float* T, float* out, int32_t N,
              void* stream);

/* Symmetric contraction backward: GX[b, c, i] = Σ_terms (Σ_m T·G) ∂(Π X)/∂X_i.
 * Replaces lib.sc_bwd (reference symmetric.py:106-131, launched at symmetric.py:154). */
int mh_sc_bwd(mh_module* m, const float* X, const int32_t* elem, const float* T, const float* G, float* GX,
              int32_t N, void* stream);

/* The symmetric contraction over groups of nodes: `order` [N] is a permutation of the nodes, sorted by element for
 * speed (any permutation gives the same results).  Each workgroup takes rows_per_block consecutive entries of `order`; when they
 * share an element every coefficient row loaded serves all of them.  Same results as mh_sc_fwd / mh_sc_bwd (the
 * per-node arithmetic is identical).  Both replace the reference's lib.sc_fwd / lib.sc_bwd (symmetric.py:82-131,
 * launched at symmetric.py:140, 154) with a grouping the reference does not have; bind MH_SC_FWD_G / MH_SC_BWD_G
 * with rows_per_block = the GROUP the kernels were generated for. */
int mh_sc_fwd_sorted(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     float* out, int32_t N, void* stream);
int mh_sc_bwd_sorted(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     const float* G, float* GX, int32_t N, void* stream);

/* The symmetric contraction on x in e3nn's irreps layout X [N, sum_k C d_k] (block k of dimension d_k = 2l+1 holds
 * channel c's components at C o_k + c d_k + m, o_k the sum of the earlier d) instead of [N, C, n_ell]: the tensor
 * MACE passes through reshape_irreps, read and differentiated in place, so that permutation never runs; GX comes
 * back in the same layout.  order NULL: one node per workgroup (kernels MH_SC_FWD_I / MH_SC_BWD_I, rows_per_block
 * 1); else as mh_sc_fwd_sorted / mh_sc_bwd_sorted (MH_SC_FWD_GI / MH_SC_BWD_GI).  Same results as the [N, C, n_ell]
 * entry points on the permuted input.  No reference counterpart: the reference reshapes first (MACE's
 * reshape_irreps) and launches lib.sc_fwd / lib.sc_bwd on the result (symmetric.py:140, 154). */
int mh_sc_fwd_irreps(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     float* out, int32_t N, void* stream);
int mh_sc_bwd_irreps(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     const float* G, float* GX, int32_t N, void* stream);

/* The symmetric contraction with the element's coefficient table streamed through LDS: each workgroup takes
 * rows_per_block consecutive entries of `slots` [nslots] (node ids, -1 for an empty slot; every group of
 * rows_per_block entries holds nodes of one element and starts with a node, or is empty from its first entry on,
 * which ends the workgroup at once) and one 64-channel block (grid_y).  TS is the table in the staged layout
 * (rows in the kernel's walk order, chunk by chunk, symmetric.pack_staged), copied to LDS once per workgroup, so
 * every coefficient read from L2 serves all nodes of the group.  layout 0: X, GX as [N, C, n_ell] (MH_SC_FWD_S /
 * MH_SC_BWD_S); 1: e3nn's irreps layout as in mh_sc_fwd_irreps (MH_SC_FWD_SI / MH_SC_BWD_SI).  nslots must be a
 * multiple of rows_per_block.  Same results as mh_sc_fwd / mh_sc_bwd up to fp32 rounding of the same per-node
 * sums.  Replace the reference's lib.sc_fwd / lib.sc_bwd (symmetric.py:82-131, launched at symmetric.py:140, 154)
 * with the per-element tables in LDS, as its kernels intend (symmetric.py:91, 98, 101). */
int mh_sc_fwd_staged(mh_module* m, const float* X, const int32_t* slots, int32_t nslots, const int32_t* elem,
                     const float* TS, float* out, int32_t N, int32_t layout, void* stream);
int mh_sc_bwd_staged(mh_module* m, const float* X, const int32_t* slots, int32_t nslots, const int32_t* elem,
                     const float* TS, const float* G, float* GX, int32_t N, int32_t layout, void* stream);

/* Second derivatives of the symmetric contraction, behind a double backward.  With P(X) the contraction of
 * mh_sc_fwd and V a direction in the layout of X:
 *   mh_sc_jvp:  out = d/de P(X + eV) at e = 0 (the forward-mode derivative; [N, out_dim] like mh_sc_fwd), which is
 *               the gradient of <V, dL/dX> with respect to G;
 *   mh_sc_bwd2: GX = d/de (dP/dX(X + eV))^T G at e = 0 (a Hessian-vector product of <G, P>), the gradient of
 *               <V, dL/dX> with respect to X.
 * layout 0: X, V, GX as [N, C, n_ell] (kernels MH_SC_JVP / MH_SC_BWD2); 1: e3nn's irreps layout as in
 * mh_sc_fwd_irreps (MH_SC_JVP_I / MH_SC_BWD2_I).  One node per workgroup (rows_per_block 1).  No reference
 * counterpart: the reference raises on a double backward (symmetric.py:147-149). */
int mh_sc_jvp(mh_module* m, const float* X, const float* V, const int32_t* elem, const float* T, float* out,
              int32_t N, int32_t layout, void* stream);
int mh_sc_bwd2(mh_module* m, const float* X, const float* V, const int32_t* elem, const float* T, const float* G,
               float* GX, int32_t N, int32_t layout, void* stream);

/* Both CSRs of an edge list in one call: edge_index [2, E] int64 (row 0 senders, row 1 receivers, contiguous) over
 * n nodes.  Writes keys [2, E] int32 (the indices, clamped into [0, n)), rowptr [2, n + 1] int32 and eids [2, E] int32:
 * row r lists the edges grouped by index r, node k's edges at eids[r, rowptr[r, k] .. rowptr[r, k + 1]) in
 * increasing edge order (what a stable sort by the index gives).  *bad is set to 1 when an index was outside [0, n)
 * and 0 otherwise.  work: 4 (n + 1) + 2 E int32 of caller-owned scratch.  Device work only (no host
 * synchronisation, no memset), so it can be captured in a HIP graph; results do not depend on the order in which
 * atomics land.  Bind MH_CSR_FILL / _COUNT / _SCATTER / _RANK with 256 threads and rows_per_block 256, MH_CSR_SCAN
 * with 1024 threads and rows_per_block 1, MH_CSR_SORT with 256 threads and rows_per_block 1 (one workgroup per node),
 * all with grid y = 2 (mh_module_bind_grid).  Replaces the reference's
 * csr_by (conv.py:229-235: a stable argsort per CSR and per layer, then a count). */
int mh_graph_build(mh_module* m, const int64_t* edge_index, int64_t E, int32_t n, int32_t* keys, int32_t* rowptr,
                   int32_t* eids, int32_t* work, int32_t* bad, void* stream);

/* mh_graph_build for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation): the same arguments but `work`, with the same results, calling no hipMalloc / hipFree.  The
 * scratch is a device array the library owns, MH_GRAPH_SCRATCH_INTS int32 (16 MiB) per GPU, held until the process
 * ends; a call whose 4 (n + 1) + 2 E exceeds it returns an error without launching anything.  Every call on a GPU
 * uses that GPU's one array (the kernels clear what must start at zero), so calls that overlap on one GPU (two
 * streams, two threads) race and must be ordered by the caller.  The array used is that of the stream's device, which
 * must be the module's (else an error).  No counterpart in the reference; it is for the callers that cannot
 * allocate. */
#define MH_GRAPH_SCRATCH_INTS (4 << 20)
int mh_graph_build_noalloc(mh_module* m, const int64_t* edge_index, int64_t E, int32_t n, int32_t* keys,
                           int32_t* rowptr, int32_t* eids, int32_t* bad, void* stream);

/* Neighbour list of a batch of B structures (atoms ptr[b] .. ptr[b + 1] of pos [N, 3] float64, cell [B, 3, 3]
 * float64 with the lattice vectors as rows, pbc [B, 3] int32): every (sender i, receiver j, unit shift o) with
 * |pos[j] + o cell - pos[i]| < r_max (float64, no fused multiply-add), o over the translations
 * max(ceil(r_max / h_k), floor(r_max / h_k + s_k)) deep along each periodic direction (h_k the spacing of lattice
 * planes k, s_k the span of the structure's fractional coordinates along k, so atoms outside the cell keep every
 * edge; at most 64 deep), without (i, i, 0); ordered by sender,
 * then receiver, then o (lexicographic).  e_pad > 0: structure b's edges fill [b e_pad, (b + 1) e_pad) (e_total =
 * B e_pad), each sender's real edges followed by its share of padding edges (self-loops with unit shift (0, 0, kz),
 * kz = ceil((r_max + 1) / |c_2|), spread round-robin over the structure's atoms); a structure with more edges fills
 * its e_pad slots with e_pad of them.  e_pad == 0: the edges back to back, e_total their number.  Outputs: edge_index [2, e_total]
 * int64 (row 0 senders, row 1 receivers), unit_shifts and shifts (= unit_shifts cell) [e_total, 3] as float64
 * (out_f64) or float32, n_edges [B] int32 = each structure's real edge count (above e_pad when it overflowed; -1
 * when it needs padding and cannot have any: no atoms, or c_2 = 0, its slots then holding zero-length self-loops;
 * -1 also when the image search was cut at 64 translations, atoms spread over more than 64 cells).
 * edge_index NULL: only n_edges (size the exact layout with it, then call again).  work: caller-owned device scratch
 * of mh_neighbour_list_work_size(B, N, e_total) bytes.  Device work only (no host synchronisation, no memset), so a
 * padded build can be captured in a HIP graph; deterministic.  Bind MH_NL_SETUP with 256 threads and rows_per_block
 * 1, MH_NL_ZERO / _BINS / _PLACE with 256 and 256, MH_NL_SCAN / _OFFSETS / _BASES with 1024 and 1 (MH_NL_OFFSETS
 * runs one workgroup per structure), MH_NL_COUNT / _FILL with 256 and 4 (a wave per sender).  No reference
 * counterpart: the reference takes MACE's host-built graphs and recommends fixed-size padded ones for long runs
 * (README.md:77-78); this builds them on the GPU. */
size_t mh_neighbour_list_work_size(int32_t B, int32_t N, int64_t e_total);
int mh_neighbour_list(mh_module* m, const double* pos, const double* cell, const int32_t* pbc, const int64_t* ptr,
                      int32_t B, int32_t N, double r_max, int64_t e_pad, int64_t e_total, int64_t* edge_index,
                      void* unit_shifts, void* shifts, int32_t out_f64, int32_t* n_edges, void* work, void* stream);

/* The species order of N nodes from one-hot attributes attrs [N, ne] float32 (ne <= MH_SPECIES_MAX_ELEM): elem [N]
 * int32 = the first maximum of each row (torch.argmax; reference symmetric.py:169), order [N] int32 = the nodes
 * stably sorted by elem, slots [nslots] int32 = that order with each element's run padded with -1 to a multiple of
 * `group`, then -1 (nslots >= ceil(N / group) group + ne group: the symmetric contraction's staged kernels walk
 * `group` slots of one element per workgroup).  One workgroup (bind MH_SPECIES_ORDER with 1024 threads, rows_per_block
 * 1); deterministic, no host synchronisation.  No reference counterpart (the reference takes argmax per call and has
 * no grouped kernels). */
#define MH_SPECIES_MAX_ELEM 128
int mh_species_order(mh_module* m, const float* attrs, int32_t N, int32_t ne, int32_t* elem, int32_t* order,
                     int32_t* slots, int32_t nslots, int32_t group, void* stream);

/* Edge spherical harmonics Y[e, :] = Y_{0..l_max}(vec[e] / |vec[e]|) (vec [E, 3], Y [E, (l_max+1)^2]; e3nn's real
 * basis, y polar axis) and their backward gvec[e] = dL/dvec[e] from gY.  The kernels are generated per (l_max,
 * normalisation).  No reference counterpart: the reference leaves the model's edge spherical harmonics on e3nn's
 * o3.SphericalHarmonics(normalize=True), which these replace in the model's forward (edge vectors -> edge attrs). */
int mh_sh_fwd(mh_module* m, const float* vec, float* Y, int64_t E, void* stream);
int mh_sh_bwd(mh_module* m, const float* vec, const float* gY, float* gvec, int64_t E, void* stream);

/* Second derivatives of the edge spherical harmonics, behind a double backward (dvec [E, 3] a direction):
 * mh_sh_jvp writes dY = (dY/dvec) dvec [E, (l_max+1)^2], the gradient of <dvec, dL/dvec> with respect to gY;
 * mh_sh_bwd2 writes the derivative of mh_sh_bwd's gvec along dvec for the given gY (a Hessian-vector product of
 * <gY, Y>), the gradient of <dvec, dL/dvec> with respect to vec.  The first-order statements run on dual numbers.
 * Bind MH_SH_JVP / MH_SH_BWD2 with 256 threads and 256 edges per block.  No reference counterpart (the reference
 * leaves the harmonics on e3nn and raises on a double backward). */
int mh_sh_jvp(mh_module* m, const float* vec, const float* dvec, float* dY, int64_t E, void* stream);
int mh_sh_bwd2(mh_module* m, const float* vec, const float* dvec, const float* gY, float* gvec, int64_t E,
               void* stream);

/* The same for the radial embedding (dlen [E] a direction of the lengths): mh_emb_jvp writes the derivatives of the
 * features [E, n] and of the cutoff [E] along dlen; mh_emb_bwd2 the derivative of mh_emb_bwd's glen along dlen for
 * the given gfeats and gcutoff (gcutoff may be NULL).  Bind MH_EMB_JVP / MH_EMB_BWD2 like MH_EMB_*. */
int mh_emb_jvp(mh_module* m, const float* len, const float* dlen, float* dfeats, float* dcutoff, int64_t E,
               void* stream);
int mh_emb_bwd2(mh_module* m, const float* len, const float* dlen, const float* gfeats, const float* gcutoff,
                float* glen, int64_t E, void* stream);

/* Second derivatives of the edge geometry, behind a double backward.  With d_e = ggpos[recv[e]] - ggpos[send[e]]
 * + ggshifts[e] (either may be NULL: zero) and u = vec / |vec|: dgvec = d, dglen = u.d, and h = glen (d - u (u.d)) /
 * |vec| (0 at |vec| = 0; glen NULL: 0), which mh_geom_bwd (h as gvec, glen NULL) sums onto the atoms and shifts.
 * Bind MH_GEOM_JVP with 256 threads and 256 edges per block.  No reference counterpart (MACE's
 * get_edge_vectors_and_lengths runs on PyTorch, and the reference raises on a double backward). */
int mh_geom_jvp(mh_module* m, const float* vec, const float* len, const float* ggpos, const float* ggshifts,
                const int32_t* send, const int32_t* recv, const float* glen, float* dgvec, float* dglen, float* h,
                int64_t E, void* stream);

/* Per-structure sums of 3x3 rows, out[b] = sum of g[row] over the rows of segment b: perm[seg[b]] ..
 * perm[seg[b + 1] - 1] (perm [M] int32), or rows seg[b] .. seg[b + 1] - 1 with perm NULL (seg [B + 1] int64, g [M, 9],
 * out [B, 9]).  The backward of MACE's per-structure gathers in get_symmetric_displacement (the symmetric strain by
 * atom, the strained cell by edge: segments from the batch's ptr and the sender CSR).  One workgroup per structure
 * (bind MH_GEOM_SEGSUM with 256 threads and rows_per_block 1); fixed summation order.  No reference counterpart. */
int mh_geom_segsum(mh_module* m, const float* g, const int32_t* perm, const int64_t* seg, float* out, int32_t B,
                   void* stream);
/* The same for one column, out[b] = sum of g[seg[b]] .. g[seg[b + 1] - 1] (g [M], seg [B + 1] int64, out [B]):
 * MACE's per-structure energy sums (scatter_sum of the node energies by the sorted batch vector), deterministic
 * where an atomic index_add is not.  Bind MH_GEOM_SEGSUM1 with 256 threads and rows_per_block 1.  No reference
 * counterpart. */
int mh_geom_segsum1(mh_module* m, const float* g, const int64_t* seg, float* out, int32_t B, void* stream);

/* Second derivatives of a SiLU readout head, behind a double backward (v [N, Din] a direction of x): mh_readout_jvp
 * writes de = (de/dx) v [N]; mh_readout_bwd2 the derivative of mh_readout_bwd's gx along v for the given g [N]
 * (zeros outside the scalar block).  One thread per node; bind MH_READOUT_JVP / MH_READOUT_BWD2 with 256 threads
 * and 256 nodes per block.  No reference counterpart (the readouts stay on PyTorch there). */
int mh_readout_jvp(mh_module* m, const float* x, const float* v, float* de, int64_t N, void* stream);
int mh_readout_bwd2(mh_module* m, const float* x, const float* v, const float* g, float* gx, int64_t N, void* stream);

/* Node-wise equivariant linear out[n] = L(x[n], attrs[n]) for N nodes (x [N, Din], out [N, Dout], fp32, the e3nn
 * irreps layout [.., u * (2l+1) + m] per block).  Without attrs (attrs NULL) it is e3nn's o3.Linear:
 *   out[n, o, w, m] = sum_{i: irrep_i = irrep_o} sum_u x[n, i, u, m] W_io[u, w];
 * with V scalar attrs it is the tensor product x (x) attrs over 0e attrs (MACE's skip_tp, FullyConnectedTensorProduct
 * with node_attrs):
 *   out[n, o, w, m] = sum_i sum_{u, v} x[n, i, u, m] attrs[n, v] W_io[u, v, w],
 * terms whose attrs are zero over a whole tile of nodes skipped.  W holds the module's weights (path normalisation folded in) in the layout of the module's kernel
 * family: for the bf16 family (attribute-free maps with >= 1024 outputs) each fp32 value split exactly into three
 * bf16 parts (uint16 bit patterns) in streaming order — per output block, column group of up to 64 channels, input
 * block and chunk of 32 input channels, a [part][channel / 8][column][8] slice; for the fp32 family the float32
 * blocks W_io[u, v, w] one after another.  The block layout, family and offsets are compiled into the module (attrs
 * must not be NULL for a module with attributes).  order (NULL: identity) is an optional permutation of the N nodes
 * in which the kernels walk them — the results do not depend on it; sorting the nodes by species (the one-hot
 * attrs' argmax) lets a workgroup skip every attribute term but one.  Outputs are scaled by alpha (1 for the plain
 * map; MACE divides the interaction linear's output by avg_num_neighbors).  mh_lin_bwd computes gx from g [N, Dout] the
 * same way with the transposed weights Wt_oi[w, v, u].  No reference counterpart: the reference leaves the model's
 * linears and skip_tp on e3nn (o3.Linear / o3.FullyConnectedTensorProduct in the interaction and product blocks). */
int mh_lin_fwd(mh_module* m, const float* x, const float* attrs, const void* W, float* out, const int32_t* order,
               float alpha, int32_t N, void* stream);
int mh_lin_bwd(mh_module* m, const float* g, const float* attrs, const void* Wt, float* gx, const int32_t* order,
               float alpha, int32_t N, void* stream);
/* mh_lin_fwd with a residual: out = alpha * L(x) + res, res [N, Dout] (NULL: none), the addition done in the store
 * (rounded as a separate multiply and add, so the result equals mh_lin_fwd's output plus res computed apart).  For
 * callers that add a tensor of the output's shape to the map's output (MACE's product block:
 * linear(node_feats) + sc), which then needs no addition kernel of its own.  No reference counterpart. */
int mh_lin_fwd_res(mh_module* m, const float* x, const float* attrs, const void* W, float* out, const int32_t* order,
                   float alpha, const float* res, int32_t N, void* stream);
/* mh_lin_bwd over the sum of three gradients of the output, gx = alpha L^T ((g + g2) + g3), the sum formed as the
 * kernel loads them (g, g2, g3 [N, Dout], none NULL), for an output read by three consumers that each give it a
 * gradient (MACE's product output: the readout and the next interaction block's skip_tp and linear_up).  The module
 * binds MH_LIN_BWD_SUM to the kernel `linear.source_sum` generates (fp32 family, as MH_LIN_BWD's grid).  No
 * reference counterpart. */
int mh_lin_bwd_sum(mh_module* m, const float* g, const float* g2, const float* g3, const float* attrs, const void* Wt,
                   float* gx, const int32_t* order, float alpha, int32_t N, void* stream);

/* Readout head e[n] = R(x[n]) for N nodes (x [N, D], e [N], fp32): MACE's LinearReadoutBlock (e = x_s . w) or
 * NonLinearReadoutBlock (e = w2 . (c silu(x_s W1))), x_s the scalar (0e) block of the node features; the weights,
 * the activation constant and the block offset are compiled into the module.  mh_readout_bwd gives gx = dL/dx
 * (the whole row, zeros outside the scalar block) from g = dL/de.  No reference counterpart: the reference leaves
 * MACE's readout heads on e3nn. */
int mh_readout_fwd(mh_module* m, const float* x, float* e, int64_t N, void* stream);
int mh_readout_bwd(mh_module* m, const float* x, const float* g, float* gx, int64_t N, void* stream);

/* Radial MLP W0[e] = MLP(ef[e]) for E edges (ef [E, n_basis], W0 [E, n_out], fp32): bias-free layers h <- c_i *
 * silu(h A_i) and a linear output layer, MACE's conv_tp_weights (an e3nn FullyConnectedNet).  Wh holds the hidden
 * layers' fp32 weights in the module's LDS layout; Wl the output layer [n_hidden_last, n_out] split exactly into
 * three bf16 parts (bit patterns), cut into chunks of 32 columns (the last zero-padded): for mh_mlp_fwd
 * [chunk][part][hidden / 8][column][8] with the hidden index in the kernel's MFMA operand order, for mh_mlp_bwd
 * [chunk][part][column / 8][hidden][8] (HipRadialMLP packs both).  The layer widths are compiled into the module.
 * mh_mlp_bwd gives gef = dL/def from gW0 = dL/dW0.  No reference counterpart: the reference leaves the radial MLP
 * on e3nn (FullyConnectedNet in MACE's interaction blocks). */
int mh_mlp_fwd(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, float* W0, int64_t E,
               void* stream);
int mh_mlp_bwd(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, const float* gW0, float* gef,
               int64_t E, void* stream);
/* The same over a row list: slot i < count[0] computes edge rows[i] (W0 row, or gef row from the gW0 row); the
 * edges of the slots from count[0] to E - 1 are not computed: mh_mlp_fwd_rows leaves their W0 rows unwritten and
 * mh_mlp_bwd_rows writes zero gef rows for them without reading their gW0 rows.  rows [E] int32 is a permutation
 * of 0 .. E - 1 and count [1] int32 lives on the device (both from mh_edge_compact: the edges inside the cutoff's
 * support first), so no host synchronisation is needed; rows and count both NULL is mh_mlp_fwd / mh_mlp_bwd.  No
 * reference counterpart. */
int mh_mlp_fwd_rows(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, float* W0, int64_t E,
                    const int32_t* rows, const int32_t* count, void* stream);
/* mh_mlp_fwd_rows with the output layer weight-stationary (what the patched model runs): MH_MLP_H3 writes the last
 * hidden activations of slot i < count[0] to h3 [E, HL] (fp32, slot order, features in the output layer's K order;
 * caller-owned scratch), then MH_MLP_OUT
 * runs a persistent grid of 4-wave workgroups; every wave keeps one block of 64 output columns of the bf16x3-split
 * output layer in registers (Wo, packed [ncb][4][HL / 32][3][64 lanes][8] bf16), the four waves of a workgroup take
 * four consecutive blocks and share each 16-slot tile of their XCD's share through LDS, storing W0 row rows[i] (rows
 * and count NULL: every slot, row = slot).  WhT: the hidden layers' transposed weights of mh_mlp_fwd.  ncb: the
 * number of 64-column blocks the module was generated for (the grid is sized so that every workgroup keeps one group
 * of four blocks).  Bind MH_MLP_H3 with 256 threads and 64 slots per block, MH_MLP_OUT with 256 threads.  Same
 * results as mh_mlp_fwd_rows to fp32 rounding; no atomics.  No reference counterpart. */
int mh_mlp_fwd_ws(mh_module* m, const float* ef, const float* WhT, const uint16_t* Wo, float* h3, float* W0,
                  int64_t E, const int32_t* rows, const int32_t* count, int32_t ncb, void* stream);
int mh_mlp_bwd_rows(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, const float* gW0, float* gef,
                    int64_t E, const int32_t* rows, const int32_t* count, void* stream);
/* mh_mlp_bwd_rows over the rows mh_edge_pairs shares between an edge and its exact reverse: slot i < count[0]
 * (edge e = rows[i], a row the forward computed) projects gW0[e] + gW0[partner[e]] when partner[e] >= 0 (the one
 * edge that reads e's W0 row, from mh_edge_pairs with vec), else gW0[e]; gef[e] receives the row's gradient and
 * every edge of the slots from count[0] on (the partners and the edges outside the support) a zero row.  The sum of
 * the two edges' gef rows is what mh_mlp_bwd_rows gives them (to fp32 rounding), which is all that reaches the
 * positions when the features are the same function of both edges' lengths and the two vectors are exact
 * negations; the per-edge split is not kept.  rows, count and partner are required.  Bind MH_MLP_BWD_P as
 * MH_MLP_BWD.  No reference counterpart. */
int mh_mlp_bwd_pairs(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, const float* gW0,
                     float* gef, int64_t E, const int32_t* rows, const int32_t* count, const int32_t* partner,
                     void* stream);

/* The edge rows of a cutoff column (cutoff [E] fp32): rows [E] int32 = the edges whose cutoff is not -0.0 exactly
 * (inside the cutoff envelope's support, as mace_hip_kernels' radial embedding marks it), in increasing order, then
 * the others; count [1] int32 = how many are inside.  work: device scratch of mh_edge_compact_work_size(E) bytes.
 * Module of conv.graph_source(); bind MH_EDGE_COUNT and MH_EDGE_PLACE with 1024 threads and 4096 edges per block.
 * Deterministic (no atomics), device work only.  No reference counterpart (the reference has no edge masks). */
size_t mh_edge_compact_work_size(int64_t E);
int mh_edge_compact(mh_module* m, const float* cutoff, int64_t E, int32_t* rows, int32_t* count, void* work,
                    void* stream);

/* Radial-MLP rows shared between an edge and its reverse.  ef [E, nf] fp32 are the MLP's input rows, cutoff [E] as
 * for mh_edge_compact, the receiver CSR (rowptr_r, eids_r) and sender CSR (rowptr_s, eids_s) of the graph and the
 * int32 senders / receivers of every edge (mh_graph_build).  For an edge e = s -> r inside the support with r < s,
 * the first edge r -> s into s (in CSR order) that is inside the support and whose ef row equals e's bit for bit
 * gives e's W0 row: wrow[e] = that edge (equal inputs give bitwise-equal MLP rows); every other edge has
 * wrow[e] = e.  rows [E] int32 lists the edges that need a row of their own (inside the support and not mapped to
 * a partner) in increasing order, then the others; count [1] = how many need one (mh_mlp_fwd_rows takes rows and
 * count as they are).  srows / scount receive, from the same pass, what mh_edge_compact gives for the cutoff (the
 * edges inside the support first: mh_mlp_bwd_rows's list).  work: mh_edge_pairs_work_size(E) bytes of device
 * scratch.  Module of conv.graph_source(); bind MH_EDGE_PAIR with 256 threads and 4 nodes per block, MH_EDGE_COUNT
 * and MH_EDGE_PLACE as for mh_edge_compact.  Deterministic, no atomics in global memory, device work only.
 * vec [E, 3] fp32 (the edge vectors) and partner [E] int32, both NULL or both given: with them a partner must also be
 * e's exact reverse (vec of the partner == -vec[e], component by component), every edge's row is read by at most
 * one other edge, and partner[e2] = the edge that reads e2's row (-1: none), the map mh_mlp_bwd_pairs takes; a node
 * with more than 2048 incoming edges then shares none of its rows.  No reference counterpart. */
size_t mh_edge_pairs_work_size(int64_t E);
int mh_edge_pairs(mh_module* m, const float* ef, int32_t nf, const float* cutoff, const int32_t* rowptr_r,
                  const int32_t* eids_r, const int32_t* rowptr_s, const int32_t* eids_s, const int32_t* senders,
                  const int32_t* receivers, int32_t N, int64_t E, const float* vec, int32_t* wrow, int32_t* partner,
                  int32_t* rows, int32_t* count, int32_t* srows, int32_t* scount, void* work, void* stream);

/* Second derivatives of the radial MLP, behind a double backward (ev [E, n_basis] a direction of the features):
 * mh_mlp_jvp writes dW0 = (dW0/def) ev [E, n_out], the gradient of <ev, dL/def> with respect to gW0; mh_mlp_bwd2
 * writes the derivative of mh_mlp_bwd's gef along ev for the given gW0 (the Hessian-vector product
 * sum_k gW0_k d^2 W0_k / def^2 ev), the gradient of <ev, dL/def> with respect to ef.  The first-order kernels run on
 * dual numbers (each hidden layer carries a tangent; the output layer is the same bf16 three-part product); the
 * weights are packed as for mh_mlp_fwd (mh_mlp_jvp) and mh_mlp_bwd (mh_mlp_bwd2).  Bind MH_MLP_JVP with 256 threads
 * and 64 edges per block, MH_MLP_BWD2 with 256 and 64.  No reference counterpart (the reference leaves the MLP on
 * e3nn and raises on a double backward). */
int mh_mlp_jvp(mh_module* m, const float* ef, const float* ev, const float* Wh, const uint16_t* Wl, float* dW0,
               int64_t E, void* stream);
int mh_mlp_bwd2(mh_module* m, const float* ef, const float* ev, const float* Wh, const uint16_t* Wl, const float* gW0,
                float* gev, int64_t E, void* stream);

/* The convolution with the radial MLP's output layer inside it (no reference counterpart: the reference streams the
 * materialised weights, W [E, NINS*MUL], through lib.conv_fwd and writes their gradient in lib.conv_bwd_wy,
 * conv.py:127, 203-209).  MACE's tp_weights = MLP(ef) * cutoff with the MLP's last layer A [HL, NINS*MUL] linear, so
 * W[e] = cutoff[e] * h[e] A with h [E, HL] the last hidden activations: the kernels read c*h and form W on the matrix
 * cores per edge tile, at fp32 accuracy (exact three-way bf16 splits of c*h and A, six partial products).
 *   mh_mlp_hid:       hc = cutoff * h from the MLP's hidden layers (module of radial.source, Wh the forward's hidden
 *                     weights), as the convolutions' MFMA operand: [E][HL / 32][3 bf16 parts][4][8] uint16, K position
 *                     8 q + t of step s holding feature 32 s + 16 (t / 4) + 4 q + t % 4;
 *   mh_conv_fwd_mlp:  out as mh_conv_fwd_cut on W = hc A (edges with cutoff == 0 skipped); Wf = A packed per channel
 *                     tile with its rows in hc's K order (conv_mlp.FusedSpec.pack_fwd).  Bind MH_CONV_FWD_M with rows_per_block = the
 *                     receivers per workgroup and grid_y = channel tiles x instruction groups: the grid is grid_y
 *                     times ceil(N / rows_per_block) workgroups;
 *   mh_conv_bwd_mlp:  from g [N, OUT_DIM]: gY [E, Y_DIM], gx (flags & MH_WANT_GX: dX messages in work [E, X_DIM],
 *                     summed over the sender CSR) and the per-channel-tile partials of dL/d(cutoff * h),
 *                     gh_parts [NCT, E, HL] (gY_parts [NCT, E, Y_DIM rounded up to 4] is scratch); Wb = A packed for
 *                     the transposed product (conv_mlp.pack_bwd).  eids_r / receivers / senders: the receiver CSR's
 *                     edge order and the int32 edge endpoints.  Bind MH_CONV_BWD_M with rows_per_block = waves per
 *                     workgroup and grid_y = NCT (the channel tiles), MH_CONV_GYSUM with 256 threads and 256 edges per
 *                     block, MH_CONV_GXSUM as for mh_conv_bwd_recv;
 *   mh_mlp_hid_bwd:   gcut[e] = sum_j P[e, j] h[e, j] and gef = dL/def through the hidden layers with dL/dh = cutoff P,
 *                     P the sum of the nparts slices of gparts [nparts, E, HL] (Wh the backward's hidden weights).
 * All sums run in a fixed order: results are bitwise repeatable. */
int mh_mlp_hid(mh_module* m, const float* ef, const float* Wh, const float* cutoff, uint16_t* hc, int64_t E,
               void* stream);
int mh_mlp_hid_bwd(mh_module* m, const float* ef, const float* Wh, const float* gparts, int32_t nparts,
                   const float* cutoff, float* gef, float* gcut, int64_t E, void* stream);
int mh_conv_fwd_mlp(mh_module* m, const float* x, const float* Y, const uint16_t* h, const float* cutoff,
                    const int32_t* rowptr, const int32_t* eids, const int32_t* senders, const uint16_t* Wf, float* out,
                    int32_t N, void* stream);
int mh_conv_bwd_mlp(mh_module* m, const float* x, const float* g, const float* Y, const uint16_t* h,
                    const float* cutoff, const int32_t* eids_r, const int32_t* receivers, const int32_t* senders,
                    const int32_t* rowptr_s, const int32_t* eids_s, const uint16_t* Wf, const uint16_t* Wb,
                    float* work, float* gx, float* gY_parts, float* gh_parts, float* gY, int32_t E, int32_t N,
                    int32_t flags, void* stream);

/* Radial embedding of E edge lengths (len [E]): cutoff[e] = polynomial envelope of len[e] / r_max (0 beyond r_max)
 * and feats[e, n] = sqrt(2 / r_max) sin(w_n len[e]) / len[e] * cutoff[e] (feats [E, n_basis]); r_max, the envelope
 * power and the w_n are compiled into the module.  mh_emb_bwd gives glen from gfeats and gcutoff (gcutoff may be
 * NULL: no gradient reaches the cutoff).  No reference counterpart: the reference leaves MACE's
 * RadialEmbeddingBlock (BesselBasis x PolynomialCutoff) on PyTorch. */
int mh_emb_fwd(mh_module* m, const float* len, float* feats, float* cutoff, int64_t E, void* stream);
int mh_emb_bwd(mh_module* m, const float* len, const float* gfeats, const float* gcutoff, float* glen, int64_t E,
               void* stream);
/* The edge geometry, the spherical harmonics and the radial embedding of the same edges in one pass (a module
 * generated by edgefeat.source(SHSpec, EmbSpec); bind MH_EDGE_FWD and MH_EDGE_BWD with 256 threads and 256 edges per
 * block).  mh_edge_fwd writes what mh_geom_fwd, then mh_sh_fwd on its vectors and mh_emb_fwd on its lengths would:
 * vec [E, 3], len [E], Y [E, DIM], feats [E, n], cutoff [E].  mh_edge_bwd writes what mh_sh_bwd and mh_emb_bwd would:
 * gvec [E, 3] = (dY/dv)^T gY and glen [E] = dL/dlen from gfeats [E, n] and gcutoff [E] (gcutoff NULL: none).  No
 * reference counterpart (these modules stay on e3nn / MACE there). */
int mh_edge_fwd(mh_module* m, const float* pos, const int32_t* send, const int32_t* recv, const float* shifts,
                float* vec, float* len, float* Y, float* feats, float* cutoff, int64_t E, void* stream);
int mh_edge_bwd(mh_module* m, const float* vec, const float* len, const float* gY, const float* gfeats,
                const float* gcutoff, float* gvec, float* glen, int64_t E, void* stream);
/* mh_edge_bwd for outputs that two consumers read: gY2 [E, DIM], gfeats2 [E, n] and gcutoff2 [E] (each may be NULL)
 * are a second consumer's gradients of the same outputs, added to the first's per element (gY + gY2, ...) before
 * use, so that no separate sum of the two runs (the results are those of mh_edge_bwd on the sums).  No reference
 * counterpart. */
int mh_edge_bwd2(mh_module* m, const float* vec, const float* len, const float* gY, const float* gfeats,
                 const float* gcutoff, const float* gY2, const float* gfeats2, const float* gcutoff2, float* gvec,
                 float* glen, int64_t E, void* stream);

/* Per-node permutation of N rows from e3nn's irreps layout (block l at off_l, index off_l + u (2l+1) + m) to
 * [mul, sum_l (2l+1)] (index u D + o_l + m), the block table compiled into the module; mh_perm_bwd applies the inverse
 * (gx from gy).  No reference counterpart: the reference leaves MACE's reshape_irreps on PyTorch. */
int mh_perm_fwd(mh_module* m, const float* x, float* y, int32_t N, void* stream);
int mh_perm_bwd(mh_module* m, const float* gy, float* gx, int32_t N, void* stream);

/* Edge geometry: vec[e] = pos[recv[e]] - pos[send[e]] + shifts[e] and len[e] = |vec[e]| for E edges (pos [N, 3],
 * shifts/vec [E, 3], len [E]).  mh_geom_bwd: gpos[n] = sum_{recv[e] = n} gv[e] - sum_{send[e] = n} gv[e] with
 * gv[e] = gvec[e] + glen[e] vec[e] / len[e] (0 where len is 0), over the receiver and sender CSRs of the edge list
 * (rowptr [N + 1], eids [E]); gshifts (may be NULL) receives gv; gvec or glen NULL count as zero.  No reference
 * counterpart: the reference leaves MACE's get_edge_vectors_and_lengths on PyTorch. */
int mh_geom_fwd(mh_module* m, const float* pos, const int32_t* send, const int32_t* recv, const float* shifts,
                float* vec, float* len, int64_t E, void* stream);
int mh_geom_bwd(mh_module* m, const float* vec, const float* len, const float* gvec, const float* glen,
                const int32_t* rowptr_r, const int32_t* eids_r, const int32_t* rowptr_s, const int32_t* eids_s,
                float* gpos, float* gshifts, int32_t N, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MACE_HIP_H */
