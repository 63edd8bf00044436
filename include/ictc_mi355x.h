/* C ABI of the MI355X (gfx950) ICTC-O3 equivariant-operator library.
 *
 * libictc_mi355x.so exports these entry points.  Every pointer is a device
 * pointer (HBM) unless stated otherwise; every size is int64_t; `stream` is a
 * hipStream_t passed as void* (nullptr = the null stream).  Calls only enqueue
 * work on `stream` (no host synchronisation, no allocation) and return 0 on
 * success or a negative code; ictc_last_error() then describes the failure
 * (thread-local, valid until the next failing call on the same thread).
 *
 * Layouts (FP32, row-major, "component-major, channel-minor" = the reference's
 * packed ir_mul layout, operators.py:283-308):
 *   features [rows, C*(LI+1)^2]  degree l, component m at ((l*l+m)*C + c)
 *   harmonics [E, (LE+1)^2]      degree l, component m at (l*l+m)
 *   gates    [E, P*C]            path p (natural-parity order) at (p*C + c)
 *   weight   [P, C] or NULL      fixed per-path coefficients (NULL = all ones)
 *   output   [rows, C*NO]        degree-major, path slot, then [2l+1, C]
 * Paths are the natural-parity triangle set of (LI, LE, LO) in the order of
 * operators.py:206-207; supported degrees are 0..3 and channels 1..256.
 */
#ifndef ICTC_MI355X_H
#define ICTC_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ICTC_OK = 0,
  ICTC_ERR_ARGUMENT = -1,    /* invalid shape / degree / channel count / null pointer */
  ICTC_ERR_UNSUPPORTED = -2, /* configuration outside the compiled coverage */
  ICTC_ERR_RUNTIME = -3      /* HIP launch / runtime failure */
};

/* Library version (major*10000 + minor*100 + patch). */
int ictc_version(void);

/* Description of the last failure on the calling thread. */
const char* ictc_last_error(void);

/* Number of paths and output components (units of C) of a natural-parity TP;
 * returns a negative code for unsupported degrees.  Host-only. */
int ictc_tp_shape(int input_lmax, int edge_lmax, int output_lmax, int* num_paths, int* out_components);

/* ---- Per-edge tensor product -------------------------------------------
 * Replaces the generated_forward launch of _Edge.forward
 * (ictc_o3/operators.py:106-127 -> backends/k100/generated_cartesian_message.py:376-383):
 *   out[e] = sum_p gate[e,p] * w[p] * CG_p(features[e], harmonics[e])         */
int ictc_tp_fwd(int input_lmax, int edge_lmax, int output_lmax, int channels,
                const float* features, const float* harmonics, const float* gates,
                const float* weight, int64_t edges, float* out, void* stream);

/* First adjoint of ictc_tp_fwd; replaces generated_adjoint of _Edge.backward
 * (operators.py:129-158 -> generated_cartesian_message.py:386-407).  Any of
 * dfeatures [E, C*(LI+1)^2], dharmonics [E,(LE+1)^2], dgates [E,P*C] may be
 * NULL to skip that role (required_gradients pruning,
 * autograd/adjoint_requirements.py:13-27).  Outputs are overwritten.
 * dharmonics with more than 64 channels needs a workspace of
 * ictc_tp_workspace_bytes(edge_lmax, channels, edges) bytes (the channel
 * groups' partial sums, added in group order; NULL/0 when not needed).       */
int64_t ictc_tp_workspace_bytes(int edge_lmax, int channels, int64_t edges);
int ictc_tp_bwd(int input_lmax, int edge_lmax, int output_lmax, int channels,
                const float* features, const float* harmonics, const float* gates,
                const float* weight, const float* grad, int64_t edges,
                float* dfeatures, float* dharmonics, float* dgates, void* workspace,
                int64_t workspace_bytes, void* stream);

/* Mixed second derivative of ictc_tp_bwd: the derivative of the first
 * adjoint (features, harmonics, gates; grad) -> (dfeatures, dharmonics,
 * dgates) along tangents tfeatures / tharmonics / tgates of its three outputs
 * (NULL = zero tangent).  Replaces generated_second
 * (backends/k100/generated_message_second.py:178,330-368, edge mode) and the
 * _EdgeAdjoint.backward composition (operators.py:72-103):
 *   dgrad      = fwd(tf, h, g) + fwd(f, th, g) + fwd(f, h, tg)   [E, C*NO]
 *   dfeatures  = dx(th, g, grad) + dx(h, tg, grad)               [E, C*(LI+1)^2]
 *   dharmonics = dy(tf, g, grad) + dy(f, tg, grad)               [E, (LE+1)^2]
 *   dgates     = dg(tf, h, grad) + dg(f, th, grad)               [E, P*C]
 * NULL outputs are skipped; non-NULL outputs are fully overwritten.
 * workspace as in ictc_tp_bwd.                                               */
int ictc_tp_second(int input_lmax, int edge_lmax, int output_lmax, int channels,
                   const float* features, const float* harmonics, const float* gates,
                   const float* weight, const float* grad, const float* tfeatures,
                   const float* tharmonics, const float* tgates, int64_t edges,
                   float* dgrad, float* dfeatures, float* dharmonics, float* dgates, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* ---- Receiver / source sorted CSR ---------------------------------------
 * Replaces topology() (backends/k100/generated_csr_forward.py:22-31: bincount,
 * cumsum, stable argsort).  keys [E] int64 node ids; builds
 *   ptr   [nodes + 2] int32: edges of node n are order[ptr[n] .. ptr[n+1]);
 *         ptr[nodes] .. ptr[nodes+1] holds edges whose key is out of range;
 *   order [E] int32, a stable sort of edge ids by key.
 * workspace must hold ictc_csr_workspace_bytes(edges, nodes) bytes.  order
 * NULL: the caller guarantees keys already in non-decreasing order with every
 * key in [0, nodes) (a receiver-sorted edge list, e.g. the neighbour list's);
 * only ptr is built, the order is the identity (pass NULL as dst_order), and
 * workspace may be NULL.                                                       */
int64_t ictc_csr_workspace_bytes(int64_t edges, int64_t nodes);
int ictc_csr_build(const int64_t* keys, int64_t edges, int64_t nodes, int32_t* ptr,
                   int32_t* order, void* workspace, int64_t workspace_bytes, void* stream);

/* ---- Spatial row order --------------------------------------------------
 * No counterpart in the reference (its kernels visit rows in index order).
 * order [N] int32 = the rows sorted (stably) by the 30-bit Morton key of the
 * grid cell floor(pos / spacing), pos [N,3] FP32; used as the row order (dst_rows / src_rows) of the
 * graph-message calls.  workspace: ictc_morton_workspace_bytes(N) bytes.      */
int64_t ictc_morton_workspace_bytes(int64_t rows);
int ictc_morton_order(const float* pos, int64_t rows, float spacing, int32_t* order, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* Row order of the receiver-owned passes (no counterpart in the reference):
 * out [N] int32 = rows (a spatial order, e.g. ictc_morton_order's) when the
 * mean distance between consecutively numbered atoms, pos [N,3] FP32, exceeds
 * twice the mean distance between consecutive entries of rows, else the
 * identity 0 .. N-1.  A lattice or domain-ordered numbering keeps index order
 * (it streams receiver-sorted gate rows sequentially); a scattered one gets
 * the spatial order.  Decided on the device (no host copy), deterministically;
 * either order gives the same message results bit for bit.  workspace:
 * ictc_receiver_rows_workspace_bytes(N) bytes.                               */
int64_t ictc_receiver_rows_workspace_bytes(int64_t rows);
int ictc_receiver_rows(const float* pos, int64_t rows, const int32_t* order, int32_t* out, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* ---- Graph message (gather -> TP -> gate -> mask -> receiver sum) --------
 * Replaces PackedGraphMessage.forward's native launches
 * (operators.py:382-409 -> ops/rematerialized_message.py:166-205 ->
 * generated_csr_forward.py:187-192 / generated_cartesian_message.py:376-383):
 *   out[n] = sum_{e: dst[e]=n} mask[e] * TP(features[src[e]], harmonics[e], gates[e])
 * features [nodes, C*(LI+1)^2]; out [nodes, C*NO] is fully overwritten.
 * dst_ptr/dst_order: ictc_csr_build over dst (dst_order NULL = edges already
 * sorted by dst with no out-of-range ids).  mask may be NULL.  dst_rows
 * [nodes] int32 (NULL = 0..nodes-1) is the order in which output rows are
 * visited: a permutation of 0..nodes-1, e.g. spatial (ictc_morton_order), so
 * that the neighbour rows gathered by concurrent waves share the L2.  It
 * changes no result bit.  Entries outside [0, nodes) are skipped.  (When the
 * edge arrays are stored receiver-sorted, index order also streams the gate
 * rows sequentially and is the better choice.)  Deterministic: one owner per
 * output row, no floating-point atomics.  gate_rows [edges] int32 (NULL =
 * edge e reads gate row e) maps each edge to the row of `gates` it reads:
 * the rows shared by an edge and its reverse (ictc_edge_pairs).               */
int ictc_msg_fwd(int input_lmax, int edge_lmax, int output_lmax, int channels,
                 const float* features, const float* harmonics, const float* gates,
                 const float* weight, const float* mask, const int64_t* src,
                 int64_t nodes, int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                 const int32_t* dst_rows, float* out, const int32_t* gate_rows, void* stream);

/* First adjoint of ictc_msg_fwd; replaces _first
 * (ops/rematerialized_message.py:25-83 -> generated_adjoint /
 * generated_csr_adjoint.py:199-293 source_adjoint).  dfeatures uses the
 * source-sorted CSR (src_ptr/src_order from ictc_csr_build over src);
 * dharmonics and dgates use the receiver-sorted CSR, visiting receivers in
 * dst_rows order; dfeatures visits sources in src_rows order (both as
 * dst_rows of ictc_msg_fwd; NULL = index order).  NULL outputs are skipped;
 * non-NULL outputs are fully overwritten.  dharmonics with more than 64
 * channels needs ictc_tp_workspace_bytes(edge_lmax, channels, edges) bytes of
 * workspace.                                                                  */
int ictc_msg_bwd(int input_lmax, int edge_lmax, int output_lmax, int channels,
                 const float* features, const float* harmonics, const float* gates,
                 const float* weight, const float* mask, const int64_t* src, const int64_t* dst,
                 int64_t nodes, int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                 const int32_t* src_ptr, const int32_t* src_order, const int32_t* dst_rows,
                 const int32_t* src_rows, const float* grad,
                 float* dfeatures, float* dharmonics, float* dgates, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* ictc_msg_bwd with dgates (required) as an input-output: the gate gradient
 * is added to the [E, P*C] rows dgates holds (each element read and written
 * by one lane: dgates <- dgates + gradient), every other output as in
 * ictc_msg_bwd.  No counterpart in the reference, whose autograd adds the
 * gate gradients of the first-order and mixed second-order passes with a
 * separate tensor add; for training callers that hold the mixed second
 * derivative's gate gradient when the first-order adjoint runs, so that the
 * sum is formed in the adjoint's own store.                                  */
int ictc_msg_bwd_accumulate(int input_lmax, int edge_lmax, int output_lmax, int channels,
                            const float* features, const float* harmonics, const float* gates,
                            const float* weight, const float* mask, const int64_t* src, const int64_t* dst,
                            int64_t nodes, int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                            const int32_t* src_ptr, const int32_t* src_order, const int32_t* dst_rows,
                            const int32_t* src_rows, const float* grad,
                            float* dfeatures, float* dharmonics, float* dgates, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* ictc_msg_bwd for a caller that holds gtangent [E, P*C] = d gates / d r
 * (ictc_radial_gates_tangent_fwd) and wants the edge-length gradient rather
 * than the gate gradient: dr [E] (required) = sum over paths and channels of
 * dgates * gtangent, formed in registers, so dgates is never written.
 * dfeatures / dharmonics (NULL = skipped) are those of ictc_msg_bwd up to FP32
 * rounding (the same products, which the two kernels may contract into FMAs
 * differently).
 * More than 64 channels need ictc_msg_bwd_tangent_workspace_bytes bytes of
 * workspace.  gates and gtangent rows are read through gate_rows as in
 * ictc_msg_fwd (dr stays per edge).  Same reference boundary as ictc_msg_bwd (_first,
 * ops/rematerialized_message.py:25-83) composed with the radial adjoint the
 * reference's force autograd runs through `fc` (layers.py:826-835).          */
int64_t ictc_msg_bwd_tangent_workspace_bytes(int edge_lmax, int channels, int64_t edges);
int ictc_msg_bwd_tangent(int input_lmax, int edge_lmax, int output_lmax, int channels,
                         const float* features, const float* harmonics, const float* gates,
                         const float* weight, const float* mask, const int64_t* src, const int64_t* dst,
                         int64_t nodes, int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                         const int32_t* src_ptr, const int32_t* src_order, const int32_t* dst_rows,
                         const int32_t* src_rows, const float* grad, const float* gtangent,
                         float* dfeatures, float* dharmonics, float* dr, void* workspace,
                         int64_t workspace_bytes, const int32_t* gate_rows, void* stream);

/* ---- Fused radial-gate message (energy + forces) ---------------------------
 * Replaces the reference's streamed gate message for frozen-weight force
 * inference (ictc_o3/ops/streamed_gate_message.py:51-57, _StreamedGate
 * :87-223): the gates [E, P*C] = h3 . W4^T are formed per edge tile inside the
 * message kernels from the radial MLP's last hidden activation h3 [E, 64]
 * (ictc_radial_mlp_tangent_fwd) and never materialised; h3 and t3 rows are
 * read through gate_rows as in ictc_msg_fwd (NULL = row e).  W4 [P*C, 64] is the
 * last Linear of `fc` (layers.py:826-835), folded with the TP path weight
 * [P, C] (may be NULL = ones) and split once into the MFMA operand layout
 * (ictc_fused_weight_split, ictc_fused_weight_bytes bytes, 16-byte aligned).
 * Compiled degree triples: ictc_fused_supported (input <= 2, edge = output
 * = 2; channels a multiple of 64 up to 256); others return
 * ICTC_ERR_UNSUPPORTED.  ictc_msg_fused_fwd writes out [N, NO*C] exactly as
 * ictc_msg_fwd with gates = h3 . W4^T.  ictc_msg_fused_bwd_tangent is
 * ictc_msg_bwd_tangent with gtangent = t3 . W4^T (t3 = d h3 / dr): dr [E]
 * (required), dharmonics [E, NY] and dfeatures (NULL = skipped; with
 * dfeatures NULL the receiver-owned pass runs and the source CSR is unused).  */
int ictc_fused_supported(int input_lmax, int edge_lmax, int output_lmax, int channels);
int64_t ictc_fused_weight_bytes(int paths, int channels);
int ictc_fused_weight_split(const float* W4, const float* tp_weight, int paths, int channels, void* out,
                            int64_t out_bytes, void* stream);
int ictc_msg_fused_fwd(int input_lmax, int edge_lmax, int output_lmax, int channels, const float* features,
                       const float* harmonics, const float* h3, const void* w4split, const float* mask,
                       const int64_t* src, int64_t nodes, int64_t edges, const int32_t* dst_ptr,
                       const int32_t* dst_order, const int32_t* dst_rows, float* out,
                       const int32_t* gate_rows, void* stream);
int ictc_msg_fused_bwd_tangent(int input_lmax, int edge_lmax, int output_lmax, int channels, const float* features,
                               const float* harmonics, const float* h3, const float* t3, const void* w4split,
                               const float* mask, const int64_t* src, const int64_t* dst, int64_t nodes,
                               int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                               const int32_t* src_ptr, const int32_t* src_order, const int32_t* dst_rows,
                               const int32_t* src_rows, const float* grad, float* dfeatures, float* dharmonics,
                               float* dr, const int32_t* gate_rows, void* stream);

/* ---- Species form of the degree-0-input radial message ----------------------
 * No direct counterpart in the reference: it evaluates the first layer's
 * message like every other (streamed_gate_message.py:87-223 over the gates
 * of layers.py:826-835, scatter-sum of the TP, layers.py:1042-1368).  In the
 * first layer the features are a function of the species alone
 * (x[s] = xtab[species[s]], xtab [S, C] = linear_up of the embedding table),
 * so for the paths (0, l, l) the message factorises through the hidden
 * space of the radial MLP:
 *   out[d, lm, c] = sum_{sp,k} Wf_l[c, (sp,k)] H[d, lm, (sp,k)],
 *   H[d, lm, (sp,k)] = sum_{e -> d, species[src e] = sp} m_e Y_lm(e) h3_e[k],
 *   Wf_l[c, (sp,k)] = coef_l xtab[sp, c] w[l, c] W4[l C + c, k],
 * with coef_l the path's CG constant and w the TP path weight [P, C]
 * (NULL = ones).  ictc_species_message_fwd writes out [N, (L+1)^2 * C]
 * exactly as ictc_msg_fused_fwd with input degree 0 and features
 * xtab[species]; ictc_species_message_bwd writes dharmonics [E, NY] and
 * dr [E] exactly as ictc_msg_fused_bwd_tangent without dfeatures (the
 * features do not depend on positions).  Edges whose source or its species
 * is out of range contribute nothing; edges whose receiver is out of range
 * get zero gradients.  edge_lmax == output_lmax <= 2, 1 <= S <= 4, any
 * channel count up to 256.  Workspace: ictc_species_message_workspace_bytes
 * (H or Z: N * NY * S * 64 floats, plus the two [P, C, S*64] projection operands); the
 * caller allocates it, the entry points do not.                              */
int64_t ictc_species_message_workspace_bytes(int edge_lmax, int species, int channels, int64_t nodes);
int ictc_species_message_fwd(int edge_lmax, int output_lmax, int channels, int species, const float* xtab,
                             const int64_t* node_species, const float* harmonics, const float* h3, const float* W4,
                             const float* tp_weight, const float* mask, const int64_t* src, int64_t nodes,
                             int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                             const int32_t* dst_rows, const int32_t* gate_rows, float* out, void* workspace,
                             int64_t workspace_bytes, void* stream);
int ictc_species_message_bwd(int edge_lmax, int output_lmax, int channels, int species, const float* xtab,
                             const int64_t* node_species, const float* harmonics, const float* h3, const float* t3,
                             const float* W4, const float* tp_weight, const float* mask, const int64_t* src,
                             int64_t nodes, int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                             const int32_t* dst_rows, const int32_t* gate_rows, const float* grad,
                             float* dharmonics, float* dr, void* workspace, int64_t workspace_bytes, void* stream);

/* ---- Edge pairs for shared radial gates ------------------------------------
 * No direct counterpart in the reference, which evaluates the radial MLP
 * `fc` on every directed edge (layers.py:826-835); the gates depend on the
 * edge length only, and an edge (s -> d, shift S) and its reverse
 * (d -> s, shift -S) have bitwise-equal lengths, so they can share one gate
 * row.  For each edge the reverse is looked up in the receiver CSR of its
 * source (dst_ptr/dst_order of ictc_csr_build over dst); shifts [E, 3] (NULL
 * = all zero) are compared exactly.  Writes gate_rows [E] (the row edge e
 * reads, in 0..count-1), reps [E] (reps[j] = the edge whose gates fill row j,
 * the first count entries) and count [1] int32 on the device.  An edge with
 * src < dst (src == dst: shift zero or lexicographically positive) owns a
 * row; any other edge reads the row of its reverse (the first in CSR order)
 * or, without one, owns a row; owners are numbered in edge order
 * (deterministic).  Workspace: ictc_edge_pairs_workspace_bytes(E)
 * bytes (-1 = 2^30 edges or more).                                         */
int64_t ictc_edge_pairs_workspace_bytes(int64_t edges);
int ictc_edge_pairs(const int64_t* src, const int64_t* dst, const float* shifts, int64_t nodes, int64_t edges,
                    const int32_t* dst_ptr, const int32_t* dst_order, int32_t* gate_rows, int32_t* reps,
                    int32_t* count, void* workspace, int64_t workspace_bytes, void* stream);

/* ictc_edge_pairs plus the source-sorted CSR from the same reverse lookup (it
 * replaces the stable sort of ictc_csr_build over src for a symmetric list).
 * When every edge has a reverse and the map edge -> reverse is one-to-one,
 * the edges leaving node n are the reverses of the edges entering it, so the
 * source CSR's ptr equals dst_ptr; src_order [E] int32 then receives those
 * edges in edge order per node (exactly ictc_csr_build's stable order over
 * src) and src_ok [1] int32 = 1.  Otherwise src_ok = 0 and src_order holds no
 * meaning (build the source CSR with ictc_csr_build).  The same workspace.   */
int ictc_edge_pairs_src_csr(const int64_t* src, const int64_t* dst, const float* shifts, int64_t nodes, int64_t edges,
                            const int32_t* dst_ptr, const int32_t* dst_order, int32_t* gate_rows, int32_t* reps,
                            int32_t* count, int32_t* src_order, int32_t* src_ok, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* Mixed second derivative of ictc_msg_bwd along tangents of its outputs
 * (tfeatures [nodes, C*(LI+1)^2], tharmonics [E, NY], tgates [E, P*C]; NULL =
 * zero tangent); replaces generated_second (graph mode,
 * generated_message_second.py:78-204,232-310) behind
 * rematerialized_message._Adjoint.backward (ops/rematerialized_message.py:146-163)
 * and the formula of ops/fused_message.py:677-729 (_second_raw):
 *   dgrad[n]   = sum_{e->n} mask (fwd(tf[src], h, g) + fwd(f[src], th, g) + fwd(f[src], h, tg))
 *   dfeatures[s] = sum_{e: src=s} mask (dx(th, g, grad[dst]) + dx(h, tg, grad[dst]))
 *   dharmonics[e] = mask (dy(tf[src], g, grad[dst]) + dy(f[src], tg, grad[dst]))
 *   dgates[e]  = mask (dg(tf[src], h, grad[dst]) + dg(f[src], th, grad[dst]))
 * CSR arguments, row orders and output conventions as in ictc_msg_bwd
 * (dgrad, dharmonics, dgates: receiver CSR; dfeatures: source CSR; workspace
 * for dharmonics beyond 64 channels).                                         */
int ictc_msg_second(int input_lmax, int edge_lmax, int output_lmax, int channels,
                    const float* features, const float* harmonics, const float* gates,
                    const float* weight, const float* mask, const int64_t* src, const int64_t* dst,
                    int64_t nodes, int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order,
                    const int32_t* src_ptr, const int32_t* src_order, const int32_t* dst_rows,
                    const int32_t* src_rows, const float* grad, const float* tfeatures,
                    const float* tharmonics, const float* tgates, float* dgrad, float* dfeatures,
                    float* dharmonics, float* dgates, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* ---- Direction harmonics --------------------------------------------------
 * Replaces direction_harmonics (operators.py:471-490 ->
 * ops/generated_direction_harmonics.py:152-170, backends/k100/
 * hip_direction_harmonics.py:35-63): directions [E,3] -> Y [E,(lmax+1)^2]
 * packed by degree, Y_l = s_l t_l(n) G_l B_l (ictd_irreps.py:1153-1208).      */
int ictc_sh_fwd(const float* directions, int64_t edges, int lmax, float* out, void* stream);
/* ddirections [E,3] = J^T grad (overwritten). */
int ictc_sh_bwd(const float* directions, const float* grad, int64_t edges, int lmax,
                float* ddirections, void* stream);

/* Second-order pieces of the harmonic map, used by force-loss training (the
 * mixed derivatives of hip_direction_harmonics.py's adjoint,
 * ops/generated_direction_harmonics.py:112-149):
 *   ictc_sh_jvp: out [E,(lmax+1)^2] = J(n) h            (h [E,3])
 *   ictc_sh_hvp: out [E,3] = Hess_n(sum_k grad_k Y_k) h  (grad [E,(lmax+1)^2]) */
int ictc_sh_jvp(const float* directions, const float* tangent, int64_t edges, int lmax, float* out,
                void* stream);
int ictc_sh_hvp(const float* directions, const float* grad, const float* tangent, int64_t edges, int lmax,
                float* out, void* stream);

/* ---- Radial path elementwise maps -----------------------------------------
 * ictc_silu replaces the normalized-SiLU kernels (operators.py:631-636 ->
 * backends/k100/hip_activation.py:11-36): n elements, scale s,
 *   mode 0: out = s x sig(x)   1: out = grad s silu'(x)   2: out = grad tangent s silu''(x)
 * ictc_radial replaces mace_radial_embedding (mace_ictc/models/radial_basis.py:
 * 42-92, Bessel x polynomial cutoff of order poly_p, no sqrt(num_basis) norm):
 *   order 0: out [E,K] = b_k(r);  1: out [E] = sum_k grad[e,k] b_k'(r);
 *   order 2: out [E] = tangent[e] sum_k grad[e,k] b_k''(r);  3: out [E,K] = b_k'(r) tangent[e] */
int ictc_silu(int mode, const float* x, const float* grad, const float* tangent, float scale, int64_t n,
              float* out, void* stream);
int ictc_radial(int order, const float* r, const float* grad, const float* tangent, int64_t edges, int num_basis,
                float cutoff, int poly_p, float* out, void* stream);

/* ---- Packed channel linears (MFMA) ------------------------------------------
 * Replaces the per-degree channel maps of EquivariantChannelLinearSO3
 * (ictd_irreps.py:207-227), the product o3.Linear (products.py:817) and
 * PathPreservingLinearSO3 (layers.py:317-355, common.py:368-374), and their
 * input adjoints, on the packed layout: for each degree l <= lmax and
 * component m, out[n, out_offsets[l] + (p*(2l+1) + m)*Cout + c] =
 *   scales[l] * sum_{q, c'} W_l[p*Cout + c, q*Cin + c'] in[n, in_offsets[l] + (q*(2l+1) + m)*Cin + c'],
 * p < out_paths[l], q < in_paths[l]; W_l = weights[l] (device pointer),
 * row-major [out_paths*Cout, in_paths*Cin].  Channel counts multiples of 16,
 * strides and offsets in floats (multiples of 4), 16-byte aligned operands.
 * Host arrays: in_paths, in_offsets, out_paths, out_offsets, weights, scales
 * (lmax + 1 entries each).  FP32 MFMA, FP32 accumulate.                       */
int ictc_packed_linear(int lmax, int channels_in, int channels_out, const float* in, int64_t in_stride,
                       const int* in_paths, const int64_t* in_offsets, float* out, int64_t out_stride,
                       const int* out_paths, const int64_t* out_offsets, const float* const* weights,
                       const float* scales, int64_t nodes, void* stream);

/* ---- Gate projection --------------------------------------------------------
 * Replaces the last Linear of the radial MLP `fc` as the gate projection
 * (layers.py:826-835; streamed_gate_message.py:51-57 `_gate_projection`):
 * out [E, gates] = hidden [E, 64] . weight^T, weight [gates, 64] row-major
 * (nn.Linear layout), gates a positive multiple of 16, operands 16-byte
 * aligned.  bf16 MFMA with a three-way operand split (FP32-level accuracy,
 * FP32 range).                                                                 */
int ictc_gate_gemm_fwd(const float* hidden, int64_t edges, int hidden_width, const float* weight, int gates,
                       float* out, void* stream);

/* Adjoint of ictc_gate_gemm_fwd with respect to the hidden layer (replaces
 * the library GEMM `grad @ weight` in the gate projection's backward,
 * streamed_gate_message.py:51-57 / the autograd of layers.py:826-835):
 * dhidden [E, 64] = grad [E, gates] . weight, gates a positive multiple of 64
 * up to 768, operands 16-byte aligned; same split-bf16 arithmetic.  The
 * per-slice partial sums are added in a fixed order (deterministic).          */
int ictc_gate_gemm_bwd(const float* grad, int64_t edges, int gates, const float* weight, int hidden_width,
                       float* dhidden, void* stream);
/* ictc_gate_gemm_bwd over a column block of a wider gradient: grad rows have
 * pitch grad_pitch (>= gates, a multiple of 4), weight holds the block's
 * `gates` rows; accumulate != 0 adds to dhidden.  Wider projections (more than
 * 768 gates, e.g. 17 paths x 128 channels) run as blocks of at most 768
 * columns accumulated in column order (deterministic).                        */
int ictc_gate_gemm_bwd_strided(const float* grad, int64_t grad_pitch, int64_t edges, int gates, const float* weight,
                               int hidden_width, float* dhidden, int accumulate, void* stream);

/* Channel-linear GEMM: c [m, n] = a [m, k] . b [n, k]^T (accumulate != 0: c +=),
 * row-major with row pitches lda, ldb, ldc, FP32 MFMA products and sums.
 * Replaces the library GEMMs torch runs for the channel linears' forward and
 * input adjoint in the training path and for the readouts: the per-degree and
 * per-path maps (layers.py:317-355, ictd_irreps.py:207-227 linear_up), the
 * element-conditioned self connection (layers.py:21-87) and the readouts
 * (heads.py:12-27; pure_cartesian_ictd_layers.py:89-115).                      */
int ictc_gemm_nt(const float* a, int64_t m, int64_t k, int64_t lda, const float* b, int64_t n, int64_t ldb, float* c,
                 int64_t ldc, int accumulate, void* stream);
/* Per-graph energy: out [graphs] (FP64) = sum of values [n] over atoms with
 * batch [n] == graph, a fixed-order reduction (deterministic, no atomics);
 * replaces the per-graph scatter of hp/runtime.py:86-113.  batch_sorted != 0
 * promises an ascending batch (each graph's atoms contiguous, as the
 * reference's collate builds it): each graph then binary-searches its range,
 * O(n + graphs); batch_sorted == 0 accepts any order at O(graphs * n).        */
int ictc_graph_sum(const float* values, const int64_t* batch, int64_t n, int64_t graphs, int batch_sorted,
                   double* out, void* stream);

/* Element-conditioned self connection (ElementConditionedLinearSO3,
 * layers.py:21-87, applied at layers.py:1042-1100 as the model's sc =
 * self_connection[species](h)): out[n] = M_s x[n] with s = species[n], M_s =
 * W[s] ([S, C, C], output by input) or, transpose != 0, W[s]^T (the input
 * adjoint).  The nodes come in species order: perm [nodes] int32 node ids
 * sorted by species (stable), offsets [S + 2] int32 with species s at sorted
 * rows offsets[s] .. offsets[s + 1] and group S (rows offsets[S] .. nodes)
 * the nodes whose species is outside [0, S), which get zero rows.  Each
 * 64-row tile of one species stages its weights once; FP32 MFMA.  C = 64 or
 * 128; x row pitch ldx (a multiple of 4, 16-byte aligned), out pitch ldo.     */
int ictc_species_linear(const float* x, int64_t ldx, int64_t nodes, int channels, const float* W, int species_count,
                        const int32_t* perm, const int32_t* offsets, int transpose, float* out, int64_t ldo,
                        void* stream);
/* Weight gradient of ictc_species_linear: out[s] = sum over the nodes n of
 * species s of a[n] b[n]^T ([S, C, C]; the autograd weight gradient of the
 * same layer, layers.py:21-87).  Same perm / offsets; sorted rows are cut
 * into tiles of rows_per_tile (a multiple of 32) within one species, whose
 * partial products go to the workspace
 * (ictc_species_outer_workspace_bytes) and are added per species in tile
 * order (deterministic; zeros for a species with no nodes).                  */
int64_t ictc_species_outer_workspace_bytes(int64_t nodes, int channels, int species_count, int rows_per_tile);
int ictc_species_outer(const float* a, int64_t lda, const float* b, int64_t ldb, int64_t nodes, int channels,
                       int species_count, const int32_t* perm, const int32_t* offsets, int rows_per_tile, float* out,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* Weight gradient of a per-edge linear (replaces the library GEMM dW = dy^T x
 * that autograd runs for every Linear of the radial MLP fc in the force-loss
 * training step, mace_ictc/models/mace/layers.py:826-835 via
 * radial_checkpoint.py:133-164): out [m, n] = a^T b with a [k, m] (row pitch
 * lda) and b [k, n] (row pitch ldb), split-bf16 MFMA (each operand as three
 * bf16 parts, six products kept: FP32-level accuracy).  The k rows are split into
 * chunks whose partial products go to the workspace
 * (ictc_gemm_tn_workspace_bytes(k, m, n) bytes) and are added in a fixed
 * order (deterministic).  k = 0 writes zeros.                                  */
int64_t ictc_gemm_tn_workspace_bytes(int64_t k, int64_t m, int64_t n);
int ictc_gemm_tn(const float* a, int64_t k, int64_t m, int64_t lda, const float* b, int64_t n, int64_t ldb,
                 float* out, void* workspace, int64_t workspace_bytes, void* stream);
/* ictc_gemm_tn over grouped rows and blocked columns, for the weight
 * gradient of one degree of a packed channel linear (the per-degree
 * dW_l = dout_l^T x_l of EquivariantChannelLinearSO3 / the path-preserving
 * linear, ictd_irreps.py:207-227, in the force-loss training step): the k =
 * groups * rows_per_group rows are (group g, member i) pairs and an operand's
 * element (row (g, i), column c) is at
 *   p[g * ldg + i * ldr + (c / cg) * ldc + c % cg]
 * (for a packed [N, paths, 2l+1, C] block: g the node, i the component, c =
 * (path, channel), ldr = C, cg = C, ldc = (2l+1) C).  Same arithmetic and
 * workspace (ictc_gemm_tn_workspace_bytes(groups * rows_per_group, m, n)) as
 * ictc_gemm_tn; k below 2^31.                                                 */
int ictc_gemm_tn_grouped(const float* a, int64_t a_ldg, int64_t a_ldr, int a_cg, int64_t a_ldc, const float* b,
                         int64_t b_ldg, int64_t b_ldr, int b_cg, int64_t b_ldc, int64_t groups, int rows_per_group,
                         int64_t m, int64_t n, float* out, void* workspace, int64_t workspace_bytes, void* stream);

/* ---- Periodic radius graph ---------------------------------------------------
 * Replaces the host neighbour search the reference delegates to ASE / matscipy
 * / torch_cluster (examples/predict.py:62, utils/graph_utils.py:217-297):
 * all directed pairs with 1e-20 < |vec|^2 < cutoff^2, vec = pos[dst] - pos[src]
 * + shift @ cell (backbone.py:940-944), periodic self-images included, edges
 * receiver-sorted in a fixed order.  cell: host [3][3] (rows = lattice
 * vectors); ncell: host [3] cells per direction, each >= 3 with cell width >=
 * cutoff.  Two calls: _count writes the edge count to edges (device int64[1]),
 * then the caller allocates src/dst [E] int64 and shifts [E,3] float and calls
 * _fill with the same workspace (ictc_neighbors_workspace_bytes bytes).      */
int64_t ictc_neighbors_workspace_bytes(int64_t atoms, const int* ncell);
int ictc_neighbors_count(const float* pos, int64_t atoms, const double* cell, double cutoff, const int* ncell,
                         void* workspace, int64_t workspace_bytes, int64_t* edges, void* stream);
int ictc_neighbors_fill(const float* pos, int64_t atoms, const double* cell, double cutoff, const int* ncell,
                        const void* workspace, int64_t workspace_bytes, int64_t* src, int64_t* dst, float* shifts,
                        void* stream);
/* _fill into arrays of `capacity` edges: the walk writes the first `capacity`
 * edges (those at list positions below it) and skips the rest, so it can be
 * launched before the edge count reaches the host, into arrays sized by an
 * estimate; when the count exceeds the capacity, call _fill again into arrays
 * of the exact size.  ictc_neighbors_fill is this with no limit.             */
int ictc_neighbors_fill_capacity(const float* pos, int64_t atoms, const double* cell, double cutoff,
                                 const int* ncell, const void* workspace, int64_t workspace_bytes, int64_t* src,
                                 int64_t* dst, float* shifts, int64_t capacity, void* stream);

/* ---- Edge geometry ---------------------------------------------------------
 * Replaces the edge-vector block of the model forward
 * (mace_ictc/models/pure_cartesian_ictd_layers.py:1288-1297, backbone.py:944):
 * vec = pos[dst] - pos[src] + shift (shift [E,3] may be NULL), r = |vec|,
 * n = vec / max(r, 1e-8), mask = [r <= cutoff] (mask may be NULL).  pos [N,3].
 * The adjoint takes dr [E] and dn [E,3] (either may be NULL = zero) and writes
 * dpos [N,3] = sum over incoming edges - sum over outgoing edges of d vec, as
 * a gather over the receiver- and source-sorted CSRs (ictc_csr_build over dst
 * and over src; dst_order NULL = edges already receiver-sorted), in CSR order: deterministic, no atomics.  dshift [E,3] (may
 * be NULL) receives d vec per edge.  Every src/dst id must lie in [0, N).     */
int ictc_edge_geometry_fwd(const float* pos, const float* shift, const int64_t* src, const int64_t* dst,
                           int64_t nodes, int64_t edges, float cutoff, float* r, float* n, float* mask,
                           void* stream);
/* Edge geometry and direction harmonics in one pass, for the first-order
 * (energy + forces) route: the edge-vector block above (r, n, mask) and
 * Y [E,(lmax+1)^2] = ictc_sh_fwd(n) (the harmonics of the model forward,
 * pure_cartesian_ictd_layers.py:1298), lmax 0..3, each value exactly as the
 * two separate calls compute it (bitwise).  n [E,3] is kept for the adjoint.  The
 * adjoint ictc_edge_harmonics_bwd takes dr [E] and dY (either may be NULL =
 * zero), plus dr2 / dY2 of a second consumer of r and Y (NULL = none; added
 * to dr / dY first, as autograd would sum them), and writes dvec [E,3] per edge (ictc_sh_bwd's dn folded with dr as
 * ictc_edge_geometry_bwd does); ictc_edge_vector_bwd then gathers dvec into
 * dpos, in the same order, so dpos is that of ictc_sh_bwd followed by
 * ictc_edge_geometry_bwd to FP32 rounding.  Y, dY and dY2 are 16-byte aligned. */
int ictc_edge_harmonics_fwd(const float* pos, const float* shift, const int64_t* src, const int64_t* dst,
                            int64_t nodes, int64_t edges, float cutoff, int lmax, float* r, float* n, float* mask,
                            float* Y, void* stream);
int ictc_edge_harmonics_bwd(const float* r, const float* n, const float* dr, const float* dY, const float* dr2,
                            const float* dY2, int64_t edges, int lmax, float* dvec, void* stream);

/* Unit vectors of edge vectors that are themselves autograd inputs (the
 * second-order route of pure_cartesian_ictd_layers.py:1288-1297, where the
 * reference composes norm and division): order 0: v [E, 3] -> out0 = r [E],
 * out1 = n [E, 3] (n = v / max(r, 1e-8)); order 1: the adjoint out0 = gv
 * [E, 3] from r, n and the cotangents gr [E], gn [E, 3] (either nullable);
 * order 2: that adjoint's derivative for a cotangent h [E, 3] on gv:
 * out0 = d v, out1 = d gr, out2 = d gn (each nullable).                      */
int ictc_edge_unit(int order, const float* v, const float* r, const float* n, const float* gr, const float* gn,
                   const float* h, int64_t edges, float* out0, float* out1, float* out2, void* stream);
/* Cartesian image shifts of the edges, replacing `edge_shifts @ cell[batch[src]]`
 * (backbone.py:940-944, the shift term of vec): out [E,3] = shifts [E,3] (lattice
 * coordinates) times the 3x3 cell (rows = lattice vectors) of the edge's graph,
 * cell [cells,3,3]; with cells == 1 every edge uses cell 0 (batch/src may be NULL),
 * else graph batch[src[e]] (batch [nodes], src [E]).  Each component is
 * (s0 c0j + s1 c1j) + s2 c2j, every operation rounded on its own, so an edge and
 * its reverse (shift -S) get exactly negated shifts (the premise of
 * ictc_edge_pairs' shared rows).  An edge whose source or graph id is out of
 * range gets NaN.                                                             */
int ictc_shift_vectors(const float* shifts, int64_t edges, const float* cell, int64_t cells, const int64_t* batch,
                       const int64_t* src, int64_t nodes, float* out, void* stream);
int ictc_edge_geometry_bwd(const float* r, const float* n, const float* dr, const float* dn, int64_t nodes,
                           int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order, const int32_t* src_ptr,
                           const int32_t* src_order, float* dshift, float* dpos, void* stream);

/* Adjoint of the edge-vector gather alone (the training path differentiates
 * vec = pos[dst] - pos[src] + shift twice, backbone.py:944 under
 * create_graph): dpos [N,3] = sum over incoming edges - sum over outgoing
 * edges of dvec [E,3], the same CSR-order gather as ictc_edge_geometry_bwd
 * (deterministic, no atomics; it replaces the index_put scatter-adds of the
 * gathers' autograd).                                                          */
int ictc_edge_vector_bwd(const float* dvec, int64_t nodes, int64_t edges, const int32_t* dst_ptr,
                         const int32_t* dst_order, const int32_t* src_ptr, const int32_t* src_order, float* dpos,
                         void* stream);

/* ---- Fused radial MLP (hidden layers) ---------------------------------------
 * Replaces the hidden part of the interaction's radial MLP `fc`
 * (mace_ictc/models/mace/layers.py:826-835, radial_basis.py:42-92) and its
 * first adjoint: r [E] -> R = radial basis (num_basis 8, cutoff polynomial of
 * order poly_p >= 2) -> a1 = s silu(R W1^T) -> a2 = s silu(a1 W2^T) ->
 * a3 = s silu(a2 W3^T), written to a3 [E,64].  W1 [64,8], W2/W3 [64,64]
 * row-major (nn.Linear layout).  The adjoint recomputes the forward, takes
 * da3 [E,64] and writes dr [E]; dz1..dz3 (pre-activation gradients) and a1, a2
 * [E,64] may be NULL and are only needed for weight gradients.  MFMA FP32.  */
int ictc_radial_mlp_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, float silu_scale, float* a3, void* stream);
/* Fused radial gates: ictc_radial_mlp_fwd followed by the gate projection
 * (ictc_gate_gemm_fwd with weight W4 [gates, 64]) without writing the hidden
 * activation: out [E, gates] = a3 . W4^T; gates a positive multiple of 16,
 * out 16-byte aligned.  workspace (ictc_radial_gates_workspace_bytes(gates),
 * 16-byte aligned) receives W4 split into bf16 parts in MFMA operand order.
 * Replaces the whole of `fc` (layers.py:826-835) as the reference's radial
 * path computes it before streamed_gate_message.py:51-57.                    */
int64_t ictc_radial_gates_workspace_bytes(int gates);
int ictc_radial_gates_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                          const float* W1, const float* W2, const float* W3, const float* W4, int gates,
                          float silu_scale, float* out, void* workspace, int64_t workspace_bytes, void* stream);
/* ictc_radial_gates_fwd that also writes tangent [E, gates] = d out / d r
 * (forward mode through the MLP, same split-bf16 arithmetic).  For
 * energy-and-forces callers that need no weight gradient: the force term of
 * the gates is then sum over gates of dout * tangent per edge, which
 * ictc_msg_bwd_tangent forms inside the message adjoint, so neither the gate
 * gradient [E, gates] nor the MLP adjoint is materialised.  No single
 * reference counterpart: it replaces the autograd pass through `fc`
 * (layers.py:826-835) that the reference's force computation runs.          */
int ictc_radial_gates_tangent_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                                  const float* W1, const float* W2, const float* W3, const float* W4, int gates,
                                  float silu_scale, float* out, float* tangent, void* workspace,
                                  int64_t workspace_bytes, void* stream);
/* ictc_radial_gates_tangent_fwd without a workspace argument and without any
 * allocation: the split W4 goes to a static device array of
 * ICTC_NOALLOC_MAX_GATES * 384 bytes (1.5 MiB) that each GPU holds until the
 * process ends.  No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc); gates above ICTC_NOALLOC_MAX_GATES fail with
 * ICTC_ERR_ARGUMENT.  All calls on one GPU share the array: calls that
 * overlap in time on one GPU (different streams or threads) race.            */
#define ICTC_NOALLOC_MAX_GATES 4096
int ictc_radial_gates_tangent_fwd_noalloc(const float* r, int64_t edges, int num_basis, int hidden, float cutoff,
                                          int poly_p, const float* W1, const float* W2, const float* W3,
                                          const float* W4, int gates, float silu_scale, float* out, float* tangent,
                                          void* stream);
/* ictc_radial_mlp_fwd that also writes t3 [E, 64] = d a3 / dr (forward mode
 * through the MLP): the hidden state and tangent the fused radial-gate
 * message projects (the `fc` of layers.py:826-835 without its last Linear).  */
int ictc_radial_mlp_tangent_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                                const float* W1, const float* W2, const float* W3, float silu_scale, float* a3,
                                float* t3, void* stream);
int ictc_radial_mlp_bwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, float silu_scale, const float* da3,
                        float* dr, float* dz1, float* dz2, float* dz3, float* a1, float* a2, void* stream);
/* Derivative of ictc_radial_mlp_bwd's dr for a cotangent rho [E] on it: what
 * torch's double backward through `fc` (layers.py:826-835, without its last
 * Linear) computes in a force-loss training step.  With dr = da3 . t3
 * (t3 = d a3 / dr), writes dr_out [E] = d (rho dr) / dr, dda3 [E, 64] =
 * rho t3 (nullable), and, when the six row arrays are given (all or none),
 * the rows whose products are the weight gradients over 2E rows:
 * d W3 = z3rows^T a2rows, d W2 = z2rows^T a1rows, d W1 = z1rows^T brows
 * (z/a rows [2E, 64] 16-byte aligned, brows [2E, 8] 8-byte aligned).  v
 * [E, 64] (nullable) is a cotangent of a3 itself: dr_out and the rows then
 * also carry ictc_radial_mlp_bwd's adjoint for da3 = v (the sum of both
 * derivatives in one pass).  dr_out null: only dda3 is written.            */
int ictc_radial_mlp_bwd2(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                         const float* W1, const float* W2, const float* W3, float silu_scale, const float* da3,
                         const float* rho, const float* v, float* dr_out, float* dda3, float* z3rows,
                         float* a2rows, float* z2rows, float* a1rows, float* z1rows, float* brows, void* stream);

/* ---- Symmetric contraction (bridge-U, correlation 1..3) -------------------
 * Replaces the SC circuits of ICTDBridgeUSymmetricContractionSO3.forward
 * (ictc_o3/ops/symmetric_contraction.py:98-147 -> factorized_contraction.py:
 * 197-266 -> backends/k100/hip_circuit.py:28-115 run / :223 mixed / :248 reduce):
 *   out[n, L, m, c] = sum_nu sum_p W(L,nu)[s_n, p, c] U(L,nu)[m, i1..inu, p] x[n,i1,c]..x[n,inu,c]
 * with U the MACE coupling folded into the ICTC basis.  x [N, C*(lmax+1)^2]
 * and out [N, C*sum_{L<=target}(2L+1)] use the packed component-major layout;
 * species [N] int64 (out-of-range species give zero rows); weights is a host
 * array of 12 device pointers, entry L*3 + (nu-1) -> W(L,nu) [S, P, C]
 * (reference layout, _mace_symmetric_contraction.py:152-155), NULL where P=0.
 * Compiled for (lmax, target_lmax) with lmax <= 2, target <= lmax, and
 * lmax 3 with target 0..2; channels 1..4096.                                  */
int ictc_sc_shape(int lmax, int target_lmax, int correlation, int* paths /* [12] */, int* num_weights);
/* Measurement helper with no reference counterpart: the number of (monomial x
 * weight-combination) terms the forward evaluates per (node, channel), summed
 * over output components; algorithmic forward FLOPs = 2 * terms * N * C.
 * Returns the count (>= 0) or a negative error code.                          */
int ictc_sc_terms(int lmax, int target_lmax, int correlation);
int ictc_sc_fwd(int lmax, int target_lmax, int correlation, int channels, const float* x, const int64_t* species,
                int num_species, const float* const* weights, int64_t nodes, float* out, void* stream);
/* dx = d(grad . out)/dx (overwritten). */
int ictc_sc_bwd_x(int lmax, int target_lmax, int correlation, int channels, const float* x,
                  const int64_t* species, int num_species, const float* const* weights, int64_t nodes,
                  const float* grad, float* dx, void* stream);
/* dW(L,nu)[s] = sum over nodes of species s (deterministic chunked reduction over
 * the species-sorted CSR from ictc_csr_build(species, nodes, num_species)).
 * workspace: ictc_sc_workspace_bytes(...) bytes.  dweights: 12 device pointers. */
int64_t ictc_sc_workspace_bytes(int lmax, int target_lmax, int correlation, int channels, int64_t nodes,
                                int num_species);
int ictc_sc_bwd_w(int lmax, int target_lmax, int correlation, int channels, const float* x, int num_species,
                  int64_t nodes, const float* grad, const int32_t* species_ptr, const int32_t* species_order,
                  float* const* dweights, void* workspace, int64_t workspace_bytes, void* stream);
/* Mixed second derivatives (force-loss training, hip_circuit.py:223):
 *   jvp: out = J_x(out) h;  hvp: dx = Hess_x(grad . out) h;
 *   bwd_w_jvp: dW = d/dW (grad . J_x(out) h).                                   */
int ictc_sc_jvp(int lmax, int target_lmax, int correlation, int channels, const float* x, const int64_t* species,
                int num_species, const float* const* weights, int64_t nodes, const float* tangent, float* out,
                void* stream);
int ictc_sc_hvp(int lmax, int target_lmax, int correlation, int channels, const float* x, const int64_t* species,
                int num_species, const float* const* weights, int64_t nodes, const float* grad,
                const float* tangent, float* dx, void* stream);
int ictc_sc_bwd_w_jvp(int lmax, int target_lmax, int correlation, int channels, const float* x, int num_species,
                      int64_t nodes, const float* grad, const float* tangent, const int32_t* species_ptr,
                      const int32_t* species_order, float* const* dweights, void* workspace,
                      int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ICTC_MI355X_H */
