/*
 * holo_mi355x.h -- C ABI of the MI355X (gfx950) path-ordered attention forward.
 *
 * The reference (SiddhiMali/HolonomyAwareAttention) exposes this path as a
 * PyTorch module and one Triton operator; it has no native ABI. The entry
 * points below replace, one for one, the pieces of that path:
 *
 *   holo_geom_scan_fwd  replaces PathOrderedGeometricMHA._geometry after the
 *                       projections (link rotations, prefix products,
 *                       holonomy: core/attention_fast_chunked.py:73-96) and
 *                       the query/key/value transports (:108-110);
 *   holo_attn_fwd       replaces HoloAttnFn.apply / run_fwd_kernel /
 *                       fwd_kernel (kernel/attention_kernel.py:40-134,166-172):
 *                       causal online-softmax attention on the transported
 *                       queries/keys/values and the back-rotation
 *                       out_i = P_i o_i (core/attention_fast_chunked.py:119-171);
 *   holo_attn_masked_fwd replaces the reference's exact path for every other
 *                       call (any mask, inert mode: kernel/attention_fast.py:
 *                       129-166, reached from kernel/attention_kernel.py:211-213);
 *   holo_quat_to_dense  expands the stored rotations to the reference's dense
 *                       geometry tensors {"C": P, "H": Hol}
 *                       (core/attention_fast_chunked.py:175-177);
 *   holo_attn_bwd       replaces HoloAttnFn.backward (kernel/attention_kernel.py:
 *                       174-187, which recomputes the reference forward under
 *                       autograd): gradients of the attention output with
 *                       respect to q, k, v and the link generator outputs;
 *   holo_attn_masked_train_fwd, holo_attn_masked_bwd
 *                       the exact path's forward with its log-sum-exp and its
 *                       backward (torch autograd through kernel/attention_fast.py:
 *                       78-166 in the reference);
 *   holo_attn_masked_dropout_fwd, holo_attn_masked_dropout_bwd,
 *   holo_dropout_keep_mask
 *                       the same pair with attention dropout (the nn.Dropout on
 *                       the softmax weights, kernel/attention_fast.py:160), and
 *                       the keep mask it draws.
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller; no entry point
 *     allocates device memory. Work that needs scratch takes a caller
 *     workspace whose size comes from the matching *_workspace_size query.
 *   - `stream` is a hipStream_t (0 = the null stream). Calls are asynchronous,
 *     never synchronise the host and keep no state between calls.
 *   - Return value 0 is success; otherwise one of holo_status, with a message
 *     available from holo_last_error() (thread-local).
 *   - Rotation model: head dimension d holds nb = floor(d/3) SO(3) blocks on
 *     dims 3b..3b+2; the remaining d - 3nb dims are not rotated. A block's
 *     three link parameters (a0, a1, a2) are the skew entries A[0][1], A[0][2],
 *     A[1][2] (row-major upper triangle, core/utils.py:20-26).
 *   - Rotations are stored as quaternions (w, x, y, z), fp32, one per block:
 *     P (B, H, T, nb, 4). The rotation matrix of q is the homogeneous map
 *     R(q) = (1/|q|^2) * [...]; exp(A) for a block is the quaternion
 *     (cos(th/2), sin(th/2)/th * (-a2, a1, -a0)), th = |a|.
 */
#ifndef HOLO_MI355X_H
#define HOLO_MI355X_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define HOLO_API __attribute__((visibility("default")))
#else
#define HOLO_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef enum holo_status {
  HOLO_OK = 0,
  HOLO_ERR_INVALID_ARG = 1,   /* null pointer, bad stride or dtype          */
  HOLO_ERR_BAD_SHAPE = 2,     /* inconsistent sizes (ValueError upstream)   */
  HOLO_ERR_UNSUPPORTED = 3,   /* outside the kernel path (NotImplementedError) */
  HOLO_ERR_WORKSPACE = 4,     /* workspace missing or too small             */
  HOLO_ERR_LAUNCH = 5         /* HIP reported an error at launch            */
} holo_status;

typedef enum holo_dtype {
  HOLO_F32 = 0,
  HOLO_BF16 = 1,
  /* fp16: only as the operand type of the transported qh / kh / vh_t between
     holo_geom_scan_fwd and holo_attn_fwd on the bf16 path (11-bit
     significands at the bf16 matrix-core rate; finite range +-65504)       */
  HOLO_F16 = 2
} holo_dtype;

/* Bits of a chained workspace's status word (holo_workspace_status).       */
typedef enum holo_ws_status {
  /* a chained carry wait ran out of polls (impossible in a conforming
     launch); the affected outputs were written as NaN                      */
  HOLO_WS_TIMEOUT = 1,
  /* holo_geom_scan_fwd: a transported value exceeded the finite range of
     op_dtype (fp16); it was stored as +-inf                                 */
  HOLO_WS_OVERFLOW = 2
} holo_ws_status;

/* Storage of the prefix rotations P (one quaternion per block and token). */
typedef enum holo_quat_format {
  /* (w, x, y, z) fp32, 16 bytes                                             */
  HOLO_QUAT_F32 = 0,
  /* round(32767 * q / |q|) as int16, 8 bytes: the rotation of a quaternion
     does not depend on its norm, so the stored integers are used as they are;
     quantisation moves a rotated vector by about 6e-5 of its length        */
  HOLO_QUAT_SNORM16 = 1
} holo_quat_format;

typedef enum holo_gen_mode {
  /* a_t = edge_scale * (gq_t + gk_{(t+1) mod T})  (core/attention_fast_chunked.py:80-84) */
  HOLO_GEN_ADDITIVE = 0,
  /* a_t = edge_scale * g_t, g supplied by the caller in `gq`, e.g. the
     interaction edge-MLP output (core/attention_fast_chunked.py:73-79)       */
  HOLO_GEN_DIRECT = 1
} holo_gen_mode;

/* Attention mode (PathOrderedGeometricMHA(mode=...), core/attention.py:31-40). */
typedef enum holo_mode {
  /* arc transport: key j reaches query i along the ring arc j -> i, through
     the closing edge (the holonomy) when i < j                              */
  HOLO_MODE_CAUSAL = 0,
  /* endpoint transport P_i^T P_j (the holonomy never enters)                */
  HOLO_MODE_INERT = 1
} holo_mode;

/* Message for the last failing call on this thread ("" if none). */
HOLO_API const char* holo_last_error(void);

/* ABI version: (major << 16) | minor. */
HOLO_API int holo_abi_version(void);

/* Padded head dimension used by the kh / vh_t layouts (d rounded up to 32). */
HOLO_API int holo_padded_head_dim(int d);

/* Padded sequence length used by the kh / vh_t layouts (T rounded up to 64). */
HOLO_API int64_t holo_padded_seq_len(int64_t T);

/*
 * holo_qkvg_proj_fwd: the layer's input projections in one hand-written
 * gfx950 GEMM (bf16 operands, fp32 accumulation), replacing the q/k/v
 * projection and the additive link generator
 * (core/attention_fast_chunked.py:69-71 and :80-84):
 *   qkv[r][n] = sum_c x[r][c] w_qkv[n][c]                        bf16, n < n_qkv
 *   g[r][n]   = sum_c x[r][c] w_gq[n][c] + x[r'][c] w_gk[n][c]   fp32, n < n_gen
 * for token rows r = b*T + t, r' = b*T + (t+1) mod T: g is the generator sum
 * before edge_scale, the input of holo_geom_scan_fwd in HOLO_GEN_DIRECT mode
 * (a_t = edge_scale * g_t), so gq and gk are never stored. x is (M, K) with
 * row stride x_row_stride (M = B*T); weights are row-major (n, K), the
 * nn.Linear layout. K a multiple of 64; n_qkv, n_gen multiples of 4 (n_gen
 * may be 0: then w_gq, w_gk and g are unused); pointers 16-byte aligned, row
 * strides whole 16-byte multiples.
 */
HOLO_API int holo_qkvg_proj_fwd(int64_t M, int64_t T, int K, int n_qkv, int n_gen,
                       const void* x, int64_t x_row_stride,
                       const void* w_qkv, const void* w_gq, const void* w_gk,
                       void* qkv, int64_t qkv_row_stride, float* g, int64_t g_row_stride, void* stream);

/*
 * holo_edge_hidden_fwd: the interaction generator's first edge-MLP layer on
 * the same hand-written GEMM, replacing the pair [x_t ; x_{t+1}], its Linear
 * and the GELU (core/attention_fast_chunked.py:56-59 and :73-76), with the
 * q/k/v projection (:69) in the same launch:
 *   qkv[r][n] = sum_c x[r][c] w_qkv[n][c]                                 bf16, n < n_qkv
 *   hid[r][n] = GELU(bf16(sum_c x[r][c] w1[n][c] + x[r'][c] w1[n][K + c] + b1[n]))   bf16, n < n_hid
 * for token rows r = b*T + t, r' = b*T + (t+1) mod T (the reference's roll),
 * GELU the exact erf form (nn.GELU()). w1 is edge_mlp[0].weight, (n_hid, 2K)
 * with row stride w1_row_stride >= 2K; b1 its bias (n_hid). n_qkv may be 0
 * (w_qkv and qkv unused). K a multiple of 64, n_qkv and n_hid multiples of
 * 4, pointers 16-byte aligned, row strides whole 16-byte multiples.
 */
HOLO_API int holo_edge_hidden_fwd(int64_t M, int64_t T, int K, int n_qkv, int n_hid,
                         const void* x, int64_t x_row_stride, const void* w_qkv,
                         const void* w1, int64_t w1_row_stride, const void* b1,
                         void* qkv, int64_t qkv_row_stride, void* hid, int64_t hid_row_stride, void* stream);

/*
 * holo_gemm_f32out_fwd: c (M, N) fp32 = a (M, K) bf16 w^T, w (N, K)
 * contiguous bf16 (the nn.Linear layout): the edge MLP's last layer
 * (core/attention_fast_chunked.py:59 and :76) with its sums kept in fp32, the
 * gq operand of holo_geom_scan_fwd (its bias goes in as gk with row stride
 * 0). K a multiple of 64, N a multiple of 4, pointers 16-byte aligned, a's
 * row stride a whole 16-byte multiple, c's a multiple of 4.
 */
HOLO_API int holo_gemm_f32out_fwd(int64_t M, int K, int N, const void* a, int64_t a_row_stride,
                         const void* w, float* c, int64_t c_row_stride, void* stream);

/* Workspace bytes for holo_geom_scan_fwd. */
HOLO_API size_t holo_geom_scan_workspace_size(int B, int64_t T, int H, int d);

/*
 * Status word of the last call that used a chained workspace (a
 * holo_geom_scan_fwd or holo_attn_bwd workspace; its first 256 bytes hold the
 * ticket counter and this word): copies the 32-bit word, a set of
 * holo_ws_status bits (0 = clean), into *status, which may be device memory
 * or pinned host memory, with an asynchronous copy on `stream` (the caller
 * synchronises before reading a host copy). Diagnostics, not the hot path.
 */
HOLO_API int holo_workspace_status(const void* workspace, size_t workspace_bytes, unsigned* status, void* stream);

/*
 * Link rotations, chunked prefix-product scan and key/value transport.
 *
 * Inputs (token-major as the projections produce them):
 *   gq, gk : dtype `gen_dtype` (fp32, or bf16 with bf16 k/v), element (b, t, h, j)
 *            at ptr[(b*T + t)*row_stride + h*head_stride + j], j < 3*nb.
 *            In HOLO_GEN_DIRECT mode gk must be NULL. Link parameters are
 *            accumulated and composed in fp32 whatever their storage type.
 *            A gk row stride of 0 reads the same row for every token: with
 *            HOLO_GEN_ADDITIVE that gives a_t = edge_scale * (gq_t + c) for a
 *            per-head constant c (e.g. the interaction edge MLP's output bias,
 *            with gq its unbiased output).
 *   q, k, v: dtype `io_dtype` (HOLO_F32 or HOLO_BF16),
 *            element (b, t, h, c) at ptr[(b*T + t)*row_stride + h*head_stride + c], c < d.
 *   mode   : HOLO_MODE_CAUSAL transports u^ = P^T u (the written formulas);
 *            HOLO_MODE_INERT transports u' = P u instead (the endpoint
 *            transport of inert mode, kernel/attention_fast.py:142-144), for
 *            holo_attn_masked_fwd in that mode.
 * Outputs, in `op_dtype` (HOLO_F32 with fp32 inputs; HOLO_BF16 or HOLO_F16
 * with bf16 inputs: the operand type of the attention call that reads them;
 * an fp16 value beyond +-65504 is stored as inf and sets HOLO_WS_OVERFLOW):
 *   qh   (B, H, Tp, Dp)        qh[t] = P_t^T q_t   (Tp = padded T, Dp = padded d)
 *   kh   (B, H, Tp, Dp)        kh[t] = P_t^T k_t
 *   vh_t (B, H, Tp/64, Dp, 64) key tiles of 64 stored transposed:
 *                               vh_t[b][h][t/64][c][t%64] = (P_t^T v_t)[c]
 *        Padding (t >= T or c >= d) is written as zero.
 *   P    (B, H, T, nb, 4)      quaternions of the prefix products in `p_format`
 *                               (fp32 or int16, holo_quat_format)
 *                               P_0 = I, P_{t+1} = G_t P_t   (:89-94)
 *   hol  (B, H, nb, 4)         fp32 holonomy G_close P_{T-1} (:95), or NULL.
 * The scan composes within chunks of 64 links and re-anchors each chunk on the
 * product of all earlier chunks, which each chunk's workgroup publishes for
 * the next one in `workspace` (a chained scan): the inputs are read once. The
 * workspace is cleared by the call itself (a fill kernel on `stream`); two
 * calls that share one workspace must not run concurrently. Its status word
 * (holo_workspace_status) reports a carry time-out or an fp16 overflow.
 */
HOLO_API int holo_geom_scan_fwd(int B, int64_t T, int H, int d,
                       int gen_mode, float edge_scale, int io_dtype, int op_dtype, int gen_dtype,
                       int p_format, int mode,
                       const void* gq, int64_t gq_row_stride, int64_t gq_head_stride,
                       const void* gk, int64_t gk_row_stride, int64_t gk_head_stride,
                       const void* q, int64_t q_row_stride, int64_t q_head_stride,
                       const void* k, int64_t k_row_stride, int64_t k_head_stride,
                       const void* v, int64_t v_row_stride, int64_t v_head_stride,
                       void* qh, void* kh, void* vh_t, float* P, float* hol,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * holo_geom_scan_fwd_static: holo_geom_scan_fwd (same arguments, same
 * results) with its chained scan state in a static device array of
 * HOLO_SCAN_STATIC_SCRATCH_BYTES per device instead of a caller workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation); it calls no allocating routine. Inputs whose state
 * (holo_geom_scan_workspace_size) exceeds the array are rejected with
 * HOLO_ERR_UNSUPPORTED. Every call on a device shares that device's array:
 * calls that overlap in time on one device race (the state is cleared at the
 * start of each call, on `stream`). The array's address is resolved on the
 * first call on each device, with that device current.
 */
#define HOLO_SCAN_STATIC_SCRATCH_BYTES ((size_t)32 << 20)
HOLO_API int holo_geom_scan_fwd_static(int B, int64_t T, int H, int d,
                       int gen_mode, float edge_scale, int io_dtype, int op_dtype, int gen_dtype,
                       int p_format, int mode,
                       const void* gq, int64_t gq_row_stride, int64_t gq_head_stride,
                       const void* gk, int64_t gk_row_stride, int64_t gk_head_stride,
                       const void* q, int64_t q_row_stride, int64_t q_head_stride,
                       const void* k, int64_t k_row_stride, int64_t k_head_stride,
                       const void* v, int64_t v_row_stride, int64_t v_head_stride,
                       void* qh, void* kh, void* vh_t, float* P, float* hol, void* stream);

/*
 * Causal path-ordered attention on transported queries/keys/values.
 *   qh, kh, vh_t, P : as written by holo_geom_scan_fwd (same B, T, H, d,
 *                     op_dtype, p_format)
 *   o    : output in `out_dtype`, element (b, t, h, c) at
 *          o[(b*T + t)*o_row_stride + h*o_head_stride + c]
 *          o_i = P_i * sum_{j<=i} softmax_j(scale * qh_i . kh_j) * vh_j
 *   lse  : optional (null to skip), (B, H, Tp) fp32: per query, log2 of the
 *          softmax normaliser in units of scale*log2(e) times the score (what
 *          holo_attn_bwd recomputes the probabilities from)
 * op_dtype is the type of qh, kh, vh_t and of the softmax weights on the
 * matrix core: HOLO_BF16 or HOLO_F16 (16-bit MFMA with fp32 accumulation and
 * softmax) or HOLO_F32 (fp32 MFMA throughout). out_dtype: HOLO_F32, or
 * HOLO_BF16 with 16-bit operands.
 */
HOLO_API int holo_attn_fwd(int B, int64_t T, int H, int d, int op_dtype, int out_dtype, int p_format, float scale,
                  const void* qh, const void* kh, const void* vh_t, const void* P,
                  void* o, int64_t o_row_stride, int64_t o_head_stride,
                  float* lse, void* stream);

/* Workspace bytes of holo_attn_masked_fwd (has_mask: a mask will be passed). */
HOLO_API size_t holo_attn_masked_workspace_size(int B, int64_t T, int H, int d, int dtype, int mode,
                                                int has_mask);

/*
 * Path-ordered attention for any mask and either mode: the reference's exact
 * path (kernel/attention_fast.py:129-166), which its kernel module runs for
 * every call that is not causal + exactly tril(T) (kernel/attention_kernel.py:
 * 203-213), e.g. no mask, the ring mask (core/utils.py:59-75) or inert mode.
 *   mode HOLO_MODE_CAUSAL: qh, kh, vh_t from holo_geom_scan_fwd in that mode,
 *     hol required:
 *       s_ij = scale * qh_i . (Hol kh_j if i < j else kh_j)
 *       o_i  = P_i (sum_{j<=i} a_ij vh_j + Hol sum_{j>i} a_ij vh_j)
 *   mode HOLO_MODE_INERT: qh, kh, vh_t from the scan in inert mode (u' = P u),
 *     hol unused:
 *       s_ij = scale * qh_i . kh_j,   o_i = P_i^T sum_j a_ij vh_j
 *   a_ij = softmax_j over the allowed keys; mask (T, T), element (i, j) at
 *   mask[i * mask_row_stride + j], nonzero = allowed, NULL = every pair
 *   allowed. Disallowed scores are -inf, so a row that allows no key is NaN
 *   (as torch.softmax gives). Workspace: holo_attn_masked_workspace_size
 *   bytes (the wrap queries Hol^T qh and the mask as bits), filled by the call.
 */
HOLO_API int holo_attn_masked_fwd(int B, int64_t T, int H, int d, int dtype, int p_format, int mode, float scale,
                         const void* qh, const void* kh, const void* vh_t, const void* P, const float* hol,
                         const uint8_t* mask, int64_t mask_row_stride,
                         void* o, int64_t o_row_stride, int64_t o_head_stride,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * holo_attn_masked_train_fwd: holo_attn_masked_fwd for training (the forward
 * whose gradient holo_attn_masked_bwd computes; in the reference, torch
 * autograd records kernel/attention_fast.py:78-166): P in fp32 quaternions
 * (HOLO_QUAT_F32), and lse (B, H, Tp) fp32 receives each row's log2-domain
 * log-sum-exp of the scaled scores over both branches (-inf for a row that
 * allows no key). Same workspace as holo_attn_masked_fwd.
 */
HOLO_API int holo_attn_masked_train_fwd(int B, int64_t T, int H, int d, int dtype, int mode, float scale,
                         const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                         const uint8_t* mask, int64_t mask_row_stride,
                         void* o, int64_t o_row_stride, int64_t o_head_stride, float* lse,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of holo_attn_bwd. */
HOLO_API size_t holo_attn_bwd_workspace_size(int B, int64_t T, int H, int d, int dtype);

/*
 * holo_attn_bwd: given dout = dL/do for the output o of holo_attn_fwd, writes
 *   dq, dk, dv  (dtype of q: element (b, t, h, c) at ptr[(b*T + t)*row_stride + h*head_stride + c])
 *   dgq, dgk    (fp32, layout of gq / gk): gradients of the generator outputs;
 *               additive: a_t = edge_scale (gq_t + gk_{t+1 mod T}); direct: a_t =
 *               edge_scale g_t (dgk, gk unused).
 * Saved forward state: gq, gk (fp32) as given to holo_geom_scan_fwd; qh, kh,
 * vh_t and P (p_format HOLO_QUAT_F32) as it wrote them; o and lse as
 * holo_attn_fwd wrote them (lse (B, H, Tp) fp32: pass a non-null lse to the
 * forward). All gradients are accumulated in fp32; the attention products
 * use the forward's dtype on the matrix cores. Calls sharing a workspace must
 * not overlap in time.
 */
HOLO_API int holo_attn_bwd(int B, int64_t T, int H, int d, int gen_mode, float edge_scale,
                  int io_dtype, int gen_dtype, float scale,
                  const void* gq, int64_t gq_row_stride, int64_t gq_head_stride,
                  const void* gk, int64_t gk_row_stride, int64_t gk_head_stride,
                  const void* qh, const void* kh, const void* vh_t, const float* P, const float* lse,
                  const void* o, int64_t o_row_stride, int64_t o_head_stride,
                  const void* dout, int64_t dout_row_stride, int64_t dout_head_stride,
                  void* dq, int64_t dq_row_stride, int64_t dq_head_stride,
                  void* dk, int64_t dk_row_stride, int64_t dk_head_stride,
                  void* dv, int64_t dv_row_stride, int64_t dv_head_stride,
                  float* dgq, int64_t dgq_row_stride, int64_t dgq_head_stride,
                  float* dgk, int64_t dgk_row_stride, int64_t dgk_head_stride,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of holo_attn_masked_bwd (mode and has_mask as the call's). */
HOLO_API size_t holo_attn_masked_bwd_workspace_size(int B, int64_t T, int H, int d, int dtype, int mode,
                                                    int has_mask);

/*
 * holo_attn_masked_bwd: the gradient of the exact path (any mask, either
 * mode), as torch autograd takes it through kernel/attention_fast.py:78-166
 * in the reference. Arguments as holo_attn_bwd's, plus the call's mode, the
 * holonomy hol (causal mode) and the mask; qh, kh, vh_t, P, hol from
 * holo_geom_scan_fwd in that mode, o and lse from holo_attn_masked_train_fwd.
 * In causal mode the holonomy Hol = G_{T-1} P_{T-1} carries the wrap branch,
 * so the closing edge (a_{T-1} = edge_scale (gq_{T-1} + gk_0)) gets a
 * gradient; in inert mode it does not. A row that allows no key has a NaN
 * output; its NaN reaches the link gradients of that token and every
 * earlier one, and contributes nothing to dq, dk, dv. Calls sharing a
 * workspace must not overlap in time.
 */
HOLO_API int holo_attn_masked_bwd(int B, int64_t T, int H, int d, int gen_mode, float edge_scale,
                  int io_dtype, int gen_dtype, int mode, float scale,
                  const void* gq, int64_t gq_row_stride, int64_t gq_head_stride,
                  const void* gk, int64_t gk_row_stride, int64_t gk_head_stride,
                  const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                  const float* lse, const uint8_t* mask, int64_t mask_row_stride,
                  const void* o, int64_t o_row_stride, int64_t o_head_stride,
                  const void* dout, int64_t dout_row_stride, int64_t dout_head_stride,
                  void* dq, int64_t dq_row_stride, int64_t dq_head_stride,
                  void* dk, int64_t dk_row_stride, int64_t dk_head_stride,
                  void* dv, int64_t dv_row_stride, int64_t dv_head_stride,
                  float* dgq, int64_t dgq_row_stride, int64_t dgq_head_stride,
                  float* dgk, int64_t dgk_row_stride, int64_t dgk_head_stride,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * Attention dropout of the exact path (kernel/attention_fast.py:160, an
 * nn.Dropout(p) on the softmax weights, active in training; core/attention.py:
 * 190). Pair (i, j) of head bh = b*H + h is kept when word j % 4 of
 * Philox4x32-10 (Salmon et al., SC 2011) at counter (i, j / 4, bh, offset)
 * under key (seed mod 2^32, seed / 2^32) is >= round(p * 2^32); kept weights
 * are multiplied by 1 / (1 - p). The mask is a function of (seed, offset)
 * and is never stored: the forward and the backward regenerate it, so a
 * backward must be given the forward's p, seed and offset. 0 <= p < 1.
 *
 * holo_attn_masked_dropout_fwd: holo_attn_masked_train_fwd with dropout: o_i
 * takes a_ij * keep_ij / (1 - p) in place of a_ij; lse is the softmax's, as
 * without dropout.
 */
HOLO_API int holo_attn_masked_dropout_fwd(int B, int64_t T, int H, int d, int dtype, int mode, float scale,
                         float dropout_p, uint64_t seed, uint32_t offset,
                         const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                         const uint8_t* mask, int64_t mask_row_stride,
                         void* o, int64_t o_row_stride, int64_t o_head_stride, float* lse,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * holo_attn_masked_dropout_bwd: holo_attn_masked_bwd for the output of
 * holo_attn_masked_dropout_fwd (same dropout_p, seed and offset); the
 * workspace is holo_attn_masked_bwd_workspace_size's.
 */
HOLO_API int holo_attn_masked_dropout_bwd(int B, int64_t T, int H, int d, int gen_mode, float edge_scale,
                  int io_dtype, int gen_dtype, int mode, float scale,
                  float dropout_p, uint64_t seed, uint32_t offset,
                  const void* gq, int64_t gq_row_stride, int64_t gq_head_stride,
                  const void* gk, int64_t gk_row_stride, int64_t gk_head_stride,
                  const void* qh, const void* kh, const void* vh_t, const float* P, const float* hol,
                  const float* lse, const uint8_t* mask, int64_t mask_row_stride,
                  const void* o, int64_t o_row_stride, int64_t o_head_stride,
                  const void* dout, int64_t dout_row_stride, int64_t dout_head_stride,
                  void* dq, int64_t dq_row_stride, int64_t dq_head_stride,
                  void* dk, int64_t dk_row_stride, int64_t dk_head_stride,
                  void* dv, int64_t dv_row_stride, int64_t dv_head_stride,
                  float* dgq, int64_t dgq_row_stride, int64_t dgq_head_stride,
                  float* dgk, int64_t dgk_row_stride, int64_t dgk_head_stride,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * holo_dropout_keep_mask: writes keep (B, H, T, T) uint8, element (b, h, i, j)
 * at keep[((b*H + h)*T + i)*T + j]: 1 where the calls above with the same
 * dropout_p, seed and offset keep pair (i, j), else 0 (for inspection and
 * tests).
 */
HOLO_API int holo_dropout_keep_mask(int B, int64_t T, int H, float dropout_p, uint64_t seed, uint32_t offset,
                                    uint8_t* keep, void* stream);

/*
 * Incremental decode (no counterpart in the reference, which only runs whole
 * sequences; row t of its forward, core/attention_fast_chunked.py:63-173, is
 * what these two calls produce for a new token t after tokens 0..t-1).
 *
 * Cache layouts (io dtype): kh_cache (B, H, capacity, Dp) and vh_cache
 * (B, H, capacity/64, Dp, 64), i.e. the scan's kh / vh_t layouts with
 * `capacity` (a multiple of 64) in place of Tp; rows 0..t-1 hold the
 * transported keys and values of the earlier tokens (e.g. copied from a scan
 * of the prefix). P (B, H, nb, 4) fp32 holds P_{t-1} on entry (identity for
 * t = 0) and P_t on return.
 *
 * holo_decode_geom_fwd: composes the link of edge t-1 -> t into P
 *   (additive: gq of token t-1 plus gk of token t; direct: g of edge t-1;
 *   neither is read when t = 0), writes qh = P_t^T q_t (B, H, Dp) and appends
 *   kh_t = P_t^T k_t, vh_t = P_t^T v_t as row t of the caches. Inputs are one
 *   token per (b, h): element (b, h, c) at ptr[b*batch_stride + h*head_stride + c].
 */
HOLO_API int holo_decode_geom_fwd(int B, int H, int d, int64_t t, int64_t capacity,
                         int gen_mode, float edge_scale, int io_dtype, int gen_dtype,
                         const void* gq, int64_t gq_batch_stride, int64_t gq_head_stride,
                         const void* gk, int64_t gk_batch_stride, int64_t gk_head_stride,
                         const void* q, int64_t q_batch_stride, int64_t q_head_stride,
                         const void* k, int64_t k_batch_stride, int64_t k_head_stride,
                         const void* v, int64_t v_batch_stride, int64_t v_head_stride,
                         float* P, void* qh, void* kh_cache, void* vh_cache, void* stream);

/* Workspace bytes for holo_decode_attn_fwd at position t. */
HOLO_API size_t holo_decode_attn_workspace_size(int B, int H, int d, int64_t t);

/*
 * holo_decode_attn_fwd: o_t = P_t sum_{j<=t} softmax_j(scale * qh . kh_j) vh_j
 *   over cache rows 0..t, written at o[b*o_batch_stride + h*o_head_stride + c].
 *   Split over 256-key segments with a merge; every cached key and value is
 *   read once.
 */
HOLO_API int holo_decode_attn_fwd(int B, int H, int d, int64_t t, int64_t capacity, int dtype, float scale,
                         const void* qh, const void* kh_cache, const void* vh_cache, const float* P,
                         void* o, int64_t o_batch_stride, int64_t o_head_stride,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Residual add fused with LayerNorm (the decoder stack's norms; no counterpart
 * in the reference's path ABI: it replaces the torch add and nn.LayerNorm of
 * the pre-LN block, experiments/session_cherry.py:292-294):
 *   h = x + delta  (rounded to dtype),  y = (h - mean) / sqrt(var + eps) * weight + bias
 * over the last dimension d of n rows (biased variance, fp32 statistics of the
 * rounded h). Rows at ptr[r * row_stride]; weight and bias have dtype `dtype`.
 * d a multiple of 16 bytes of dtype and at most 1024 such chunks (bf16: 8192,
 * fp32: 4096); row strides 16-byte multiples, pointers 16-byte aligned.
 */
HOLO_API int holo_add_layernorm_fwd(int64_t n, int d, int dtype, float eps,
                           const void* x, int64_t x_row_stride, const void* delta, int64_t delta_row_stride,
                           const void* weight, const void* bias,
                           void* h, int64_t h_row_stride, void* y, int64_t y_row_stride, void* stream);

/*
 * Expand fp32 quaternions (n, nb, 4) to dense fp32 rotation matrices (n, d, d):
 * block b on dims 3b..3b+2, identity on the leftover dims.
 */
HOLO_API int holo_quat_to_dense(int64_t n, int d, const float* quat, float* dense, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HOLO_MI355X_H */
