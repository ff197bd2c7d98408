// Kernel argument blocks and launchers shared by the C ABI and the kernels.
#pragma once

#include "holo_common.h"

namespace holo {

struct ScanArgs {
  int B, H, d, nb, nbx, Dp, gen_mode;
  int64_t T, Tp, nch;
  float edge_scale;
  const void* gq; int64_t gq_rs, gq_hs;
  const void* gk; int64_t gk_rs, gk_hs;
  const void* q; int64_t q_rs, q_hs;
  const void* k; int64_t k_rs, k_hs;
  const void* v; int64_t v_rs, v_hs;
  void* qh; void* kh; void* vh_t; float* P; float* hol;
  int p_format;    // 0: fp32 quaternions, 1: int16 (round(32767 q/|q|))
  int wide;        // 16-byte row path of the scan (d in {48, 72, 96}, aligned rows)
  int inert;       // transport u' = P u (inert mode) instead of u^ = P^T u
  float* incl;     // chained-scan state: chunk products (B, H, nch, nb, 4), then inclusive prefixes (same shape)
  unsigned* ticket;  // [0]: chunk ticket counter, [1]: status word (kStatusTimeout, kStatusOverflow)
};
size_t scan_state_bytes(int B, int64_t T, int H, int d);
constexpr int kScanGroup = 8;    // chunks per carry-chain hop of the scan when the chain lags

struct AttnArgs {
  int B, H, d, nb, Dp;
  int64_t T, Tp, nch;
  float scale_log2;                       // scale * log2(e)
  const void* qh; const void* kh; const void* vh_t; const void* P;
  void* o; int64_t o_rs, o_hs;
  int p_format;    // 0: fp32 quaternions, 1: int16 (round(32767 q/|q|))
  float* lse;      // optional (B, H, Tp): log2 of each query's softmax normaliser, in the
                   // log2 units of scale_log2 (max + log2(sum)); what the backward recomputes P from
};

// Attention for any mask and either mode (the exact path): mode 0 causal, with
// the wrap branch (key j > query i) through the holonomy; mode 1 inert.
struct MaskedArgs {
  int B, H, d, nb, Dp, mode;
  int64_t T, Tp;
  float scale_log2;
  const void* qh;
  const void* kh; const void* vh_t; const void* P; const float* hol;
  const uint64_t* mask_bits;             // (Tp, Tp/64): bit e of word w = allowed(i, 64 w + e); null = all
  const uint8_t* tile_act;               // (ceil(T/128), Tp/64): 1 = the tile pair has an allowed pair
  void* o; int64_t o_rs, o_hs;
  int p_format;
};

// Backward of scan + attention. Path-frame tensors are (B, H, Tp, Dp) row-major
// ("_t": 64-row tiles stored transposed, (B, H, Tp/64, Dp, 64)).
struct BwdArgs {
  int B, H, d, nb, Dp, gen_mode;
  int64_t T, Tp, nch;
  float scale, scale_log2, edge_scale;
  // saved forward state
  const void* gq; int64_t gq_rs, gq_hs;
  const void* gk; int64_t gk_rs, gk_hs;
  const void* qh; const void* kh; const void* vh_t; const float* P; const float* lse;
  const void* o; int64_t o_rs, o_hs;
  // incoming gradient of o
  const void* dout; int64_t do_rs, do_hs;
  // workspace
  void* doh; void* doh_t; void* qh_t; void* kh_t; void* vh;   // io dtype; the _t layouts fp32 only
  float* delta;                                               // (B, H, Tp): rowsum(do * o)
  float* dqh; float* dkh; float* dvh;                         // fp32, path frame
  float* carry;                                               // (B, H, nch, nb, 4) chained suffix sums
  unsigned* ticket;
  // outputs
  void* dq; int64_t dq_rs, dq_hs;
  void* dk; int64_t dk_rs, dk_hs;
  void* dv; int64_t dv_rs, dv_hs;
  float* dgq; int64_t dgq_rs, dgq_hs;
  float* dgk; int64_t dgk_rs, dgk_hs;
};

// Attention dropout of the exact path's training pair: pair (i, j) of head bh
// is kept when word j % 4 of Philox4x32-10 at counter (i, j / 4, bh, offset)
// under key (k0, k1) is >= thr; kept weights are multiplied by scale.
struct DropParams {
  uint32_t thr;                          // round(p 2^32), capped at 2^32 - 1
  float scale;                           // 1 / (1 - p)
  uint32_t k0, k1;                       // the seed's low and high words
  uint32_t offset;                       // the counter's fourth word
};

// The exact path's forward for training: MaskedArgs and the per-row
// log2-domain log-sum-exp of the scaled scores (m + log2 l over both
// branches), which its backward recomputes the probabilities from; with
// dropout on, the output weights are the softmax weights times keep * scale
// (the LSE stays that of the softmax).
struct MaskedLseArgs : MaskedArgs {
  float* lse;                            // (B, H, Tp)
  int dropout;                           // 1: apply `drop`
  DropParams drop;
};
template <bool LSE> struct MaskedArgsOf { typedef MaskedLseArgs type; };
template <> struct MaskedArgsOf<false> { typedef MaskedArgs type; };

// Backward of the exact path (any mask; causal mode with the wrap branch
// through the holonomy, or inert mode). The base fields keep their meaning;
// in inert mode qh, kh, vh_t, doh hold the primed values u' = P u.
struct MaskedBwdArgs : BwdArgs {
  int mode;                              // 0 causal (wrap through hol), 1 inert
  const float* hol;                      // (B, H, nb, 4) holonomy quaternions (causal)
  const uint64_t* mask_bits;             // (Tp, Tp/64) as for MaskedArgs; null = every pair
  const uint8_t* tile_act;               // (ceil(T/128), Tp/64) open-tile map as for MaskedArgs; null = all
  void* qw; void* dow;                   // Hol^T qh, Hol^T doh (io dtype, (B, H, Tp, Dp); causal)
  void* qw_t; void* dow_t;               // their transposed tiles (fp32 only)
  float* dqw; float* dkw; float* dvw;    // wrap-branch gradients, path frame (fp32, causal)
  float* hol_torque;                     // (B, H, nb, 4): the holonomy's cross sum (causal)
  int dropout;                           // 1: the forward applied `drop`
  DropParams drop;
};
// kernel variants of the backward: 0 the causal + tril path, 1 the exact
// path in causal mode, 2 the exact path in inert mode
template <int EX> struct BwdArgsOf { typedef MaskedBwdArgs type; };
template <> struct BwdArgsOf<0> { typedef BwdArgs type; };

struct DecodeGeomArgs {
  int B, H, d, nb, Dp, gen_mode;
  int64_t t, cap;                  // new token's position, cache capacity (multiple of 64)
  float edge_scale;
  const void* gq; int64_t gq_bs, gq_hs;   // link parameters of token t-1 (unused when t == 0)
  const void* gk; int64_t gk_bs, gk_hs;   // gk of token t (additive mode)
  const void* q; int64_t q_bs, q_hs;
  const void* k; int64_t k_bs, k_hs;
  const void* v; int64_t v_bs, v_hs;
  float* P;                        // (B, H, nb, 4) fp32: P_{t-1} in, P_t out
  void* qh;                        // (B, H, Dp)
  void* kc; void* vc;              // caches (B, H, cap, Dp) and (B, H, cap/64, Dp, 64)
};

struct DecodeAttnArgs {
  int B, H, d, nb, Dp;
  int64_t t, cap, nsplit;          // keys 0..t are attended
  float scale_log2;
  const void* qh; const void* kc; const void* vc; const float* P;
  void* o; int64_t o_bs, o_hs;
  float* ws;                       // (B, H, nsplit, Dp + 2) partials
};

// residual add + LayerNorm over rows of d (d a multiple of 16 bytes, at most 1024 such chunks)
struct AddNormArgs {
  int64_t n; int d; float eps;
  const void* x; int64_t x_rs;
  const void* delta; int64_t delta_rs;
  const void* w; const void* b;
  void* h; int64_t h_rs;
  void* y; int64_t y_rs;
};

// q/k/v projection and additive link generator in one GEMM (bf16 in, fp32
// accumulation): qkv (M, n_qkv) bf16 = x W_qkv^T and g (M, n_gen) fp32 =
// x_t W_gq^T + x_{t+1} W_gk^T, t+1 wrapping inside each sequence of T rows.
struct QkvgArgs {
  int64_t M;                 // B*T token rows
  int64_t T;                 // tokens per sequence
  int K;                     // d_model, a multiple of 64
  int n_qkv, n_gen;          // output columns (multiples of 4)
  int tm, tnq, tng;          // tiles: M blocks of 256, q/k/v and generator N blocks of 256
  const bf16* x; int64_t ldx;                  // (M, K), row stride ldx
  const bf16* wq;                              // (n_qkv, K) contiguous
  const bf16* wg0; const bf16* wg1;            // (n_gen, K) contiguous: gq and gk weights
  bf16* qkv; int64_t ldq;                      // (M, n_qkv)
  float* g; int64_t ldg;                       // (M, n_gen)
  int group_m;               // M-blocks per L2 group within an XCD's range of tiles
};
hipError_t launch_qkvg(const QkvgArgs& a, hipStream_t s);

// The interaction generator's edge MLP (core/attention_fast_chunked.py:56-60,
// 73-79) on the same GEMM: the hidden layer GELU([x_t ; x_{t+1}] W1^T + b1)
// reads W1 (n_gen, 2K) as two K segments, W1[:, :K] on the token rows t and
// W1[:, K:] on the rows t+1 (wg0 = W1, wg1 = W1 + K, weight row stride
// ldw = 2K), and writes bf16 `hid`; q/k/v tiles (n_qkv > 0) run in the same
// launch. The second layer is a plain GEMM with an fp32 output (g = hid W2^T,
// one K segment; the scan adds its bias per head).
struct EdgeGemmArgs : QkvgArgs {
  int64_t ldw;               // row stride of the generator weight (elements)
  const bf16* bias;          // (n_gen) hidden-layer bias (hidden layer only)
  bf16* hid; int64_t ldh;    // (M, n_gen) hidden output (hidden layer only)
};
hipError_t launch_edge_hidden(const EdgeGemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f32out(const EdgeGemmArgs& a, hipStream_t s);

template <typename IO, typename OP, typename GT> hipError_t launch_scan(const ScanArgs& a, hipStream_t s);
template <typename T> hipError_t launch_add_layernorm(const AddNormArgs& a, hipStream_t s);
hipError_t launch_pack_mask(const uint8_t* mask, int64_t mask_rs, int64_t T, int64_t Tp, uint64_t* bits,
                            uint8_t* tile_act, hipStream_t s);
template <typename T> hipError_t launch_attn_masked(const MaskedArgs& a, hipStream_t s);
template <typename T> hipError_t launch_attn_masked_lse(const MaskedLseArgs& a, hipStream_t s);
template <typename IO, typename GT> hipError_t launch_decode_geom(const DecodeGeomArgs& a, hipStream_t s);
template <typename T> hipError_t launch_decode_attn(const DecodeAttnArgs& a, hipStream_t s);
int64_t decode_splits(int64_t t);
// OPT: operand type of qh, kh, vh_t (fp32, bf16, fp16); OT: type of o (fp32, bf16)
template <typename OPT, typename OT> hipError_t launch_attn(const AttnArgs& a, hipStream_t s);
hipError_t launch_quat_to_dense(int64_t n, int d, const float* q, float* out, hipStream_t s);
hipError_t launch_chain_reset(void* state, int64_t n_pairs, unsigned* ticket, hipStream_t s);
template <typename IO, typename GT> hipError_t launch_bwd(const BwdArgs& a, hipStream_t s);
template <typename IO, typename GT> hipError_t launch_masked_bwd(const MaskedBwdArgs& a, hipStream_t s);
// keep (B, H, T, T) uint8: 1 where attention dropout keeps pair (i, j)
hipError_t launch_dropout_keep(int B, int H, int64_t T, const DropParams& d, uint8_t* keep, hipStream_t s);

}  // namespace holo
