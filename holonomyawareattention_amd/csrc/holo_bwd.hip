// Backward of the path-ordered attention forward (scan + attention) on gfx950.
//
// Reference behaviour: gradients of core/attention_fast_chunked.py:63-173
// (its kernel path recomputes the backward through PyTorch autograd,
// kernel/attention_kernel.py:174-187). With qh = P^T q, kh = P^T k, vh = P^T v,
// oh = softmax(scale qh kh^T) vh and o = P oh, the gradient splits into
//   1. doh = P^T do and delta = rowsum(do * o) (= rowsum(doh * oh)),
//   2. the causal softmax-attention backward in the path frame:
//        dS = Pm * (doh vh^T - delta),  dqh = scale dS kh,  dkh = scale dS^T qh,
//        dvh = Pm^T doh                    (Pm recomputed from the saved LSE),
//   3. dq = P dqh, dk = P dkh, dv = P dvh, and the links: with
//        c_t = oh x doh + dqh x qh + dkh x kh + dvh x vh   (per 3-dim block),
//      the reverse recursion of P_{t+1} = G_t P_t reduces to a suffix sum
//      m_t = sum_{s >= t} c_s (P_t^T dL/dP_t summed along the path), and
//      vee(G_t^T dL/dG_t - transpose) = P_t m_{t+1}; through the right
//      Jacobian of exp on SO(3), dL/da_t = map(J_r(phi_t)^T P_t m_{t+1}).
//      The closing edge only enters the holonomy (zero gradient).
//
// Kernels, in launch order:
//   bwd_prep      one workgroup per (b, h, 64 tokens): doh, delta, vh
//                 row-major and, for fp32 only, the transposed operand
//                 layouts doh_t, qh_t, kh_t (the bf16 MFMA kernels read their
//                 transposed operands from row-major LDS tiles with
//                 ds_read_b64_tr_b16)
//   attn_bwd_dkdv one workgroup per (b, h, 128 keys); each wave keeps its 32
//                 keys' V rows as MFMA operands in registers (the K rows of
//                 the workgroup's keys sit in LDS) and sweeps the causal query
//                 tiles, the next fill's loads in flight while the current one
//                 is computed: S, dP, then dV += Pm^T dO and dK += dS^T Q with
//                 the probabilities already in the operand layout of the
//                 second product
//   attn_bwd_dq   one workgroup per (b, h, 128 queries), each wave 32 queries
//                 in registers, sweeping key tiles: dQ^T += K^T dS^T
//   link_bwd      chained suffix scan over 64-token chunks (reverse ticket
//                 order, the same bounded-wait protocol as the forward scan),
//                 then dq, dk, dv and the generator gradients
#include "holo_bwd_kernels.h"

namespace holo {

// ---------------------------------------------------------------------------
template <typename IO, typename GT, int DP>
static hipError_t launch_bwd_dp(const BwdArgs& a, hipStream_t s) {
  const int64_t nbh = (int64_t)a.B * a.H;
  const int64_t nblk = (a.Tp + 127) / 128;
  hipLaunchKernelGGL((bwd_prep<IO, DP>), dim3((unsigned)(nbh * a.nch)), dim3(kBwdThreads), 0, s, a);
  hipLaunchKernelGGL((attn_bwd_dkdv<IO, DP>), dim3((unsigned)(nbh * nblk)), dim3(kBwdThreads), 0, s, a);
  hipLaunchKernelGGL((attn_bwd_dq<IO, DP>), dim3((unsigned)(nbh * nblk)), dim3(kBwdThreads), 0, s, a);
  hipError_t e = launch_chain_reset(a.carry, nbh * a.nch * a.nb * 2, a.ticket, s);
  if (e != hipSuccess) return e;
  // 16-byte spans: 8 blocks (24 dims) per thread at d = 96, every row and
  // head stride of the token-major tensors a multiple of 16 bytes
  auto al = [](const void* ptr, int64_t rs, int64_t hs, size_t es) {
    return ptr == nullptr || ((reinterpret_cast<uintptr_t>(ptr) & 15) == 0 && (rs * (int64_t)es) % 16 == 0 &&
                              (hs * (int64_t)es) % 16 == 0);
  };
  const bool wide = DP == 96 && a.d == 96 && al(a.o, a.o_rs, a.o_hs, sizeof(IO)) &&
                    al(a.dout, a.do_rs, a.do_hs, sizeof(IO)) && al(a.dq, a.dq_rs, a.dq_hs, sizeof(IO)) &&
                    al(a.dk, a.dk_rs, a.dk_hs, sizeof(IO)) && al(a.dv, a.dv_rs, a.dv_hs, sizeof(IO)) &&
                    al(a.gq, a.gq_rs, a.gq_hs, sizeof(GT)) && al(a.gk, a.gk_rs, a.gk_hs, sizeof(GT)) &&
                    al(a.dgq, a.dgq_rs, a.dgq_hs, 4) && al(a.dgk, a.dgk_rs, a.dgk_hs, 4);
  if (wide)
    hipLaunchKernelGGL((link_bwd<IO, GT, DP, true>), dim3((unsigned)(nbh * a.nch)), dim3(kBwdThreads), 0, s, a);
  else
    hipLaunchKernelGGL((link_bwd<IO, GT, DP, false>), dim3((unsigned)(nbh * a.nch)), dim3(kBwdThreads), 0, s, a);
  return hipGetLastError();
}

template <typename IO, typename GT>
hipError_t launch_bwd(const BwdArgs& a, hipStream_t s) {
  switch (a.Dp) {
    case 32: return launch_bwd_dp<IO, GT, 32>(a, s);
    case 64: return launch_bwd_dp<IO, GT, 64>(a, s);
    case 96: return launch_bwd_dp<IO, GT, 96>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template hipError_t launch_bwd<float, float>(const BwdArgs&, hipStream_t);
template hipError_t launch_bwd<bf16, float>(const BwdArgs&, hipStream_t);

}  // namespace holo
