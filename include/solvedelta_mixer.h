/* SolveDelta mixer frontend and readout on MI355X (gfx950): C-ABI of
 * libsolvedelta_hip.so, next to the operator entry points of solvedelta.h.
 *
 * The reference runs these pieces through third-party CUDA/Triton code; each
 * entry point here replaces one call site:
 *   - sd_conv4_silu_fwd / _bwd  <- causal_conv1d_fn(x^T, conv_weight, initial_states,
 *                                  return_final_states, activation="silu") in
 *                                  causallsso/model.py:119-136 (CPU semantics :146-164);
 *   - sd_kda_gate_fwd / _bwd    <- fla.ops.kda.gate.fused_kda_gate in
 *                                  causallsso/model.py:375-383 (its CPU form :384-390);
 *   - sd_rmsnorm_gated_fwd/_bwd <- layer_norm_gated_fwd / _bwd (rms, sigmoid) in
 *                                  causallsso/ops/norm_gate.py:46-150 (definition :20-43).
 *
 * Layouts: bf16 activations, FP32 parameters and parameter gradients.  Entry
 * points enqueue on `stream`, never allocate or synchronise, and return 0 or an
 * SD_ERR_* code of solvedelta.h.  Parameter gradients are reduced in two
 * deterministic stages through the caller's workspace (*_workspace_bytes).
 */
#ifndef SOLVEDELTA_MIXER_H
#define SOLVEDELTA_MIXER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Causal depthwise conv4 + SiLU over T tokens of D channels:
 *   y[b,t,d] = silu(sum_k w[d,k] xs[b,t-3+k,d]), xs[b,-3..-1,:] = init[b,:,0..2] (or 0).
 * x: bf16, element (b,t,d) at x[b*x_sb + t*x_st + d]; w: fp32 [D][4];
 * init, final_state: bf16 [B][D][3], nullable; y: bf16 [B][T][D] contiguous.
 * final_state[b,d,m] = xs[b,T-3+m,d]. */
int sd_conv4_silu_fwd(int B, int T, int D, const void *x, int64_t x_sb, int64_t x_st,
                      const float *w, const void *init, void *y, void *final_state,
                      void *stream);
size_t sd_conv4_workspace_bytes(int B, int T, int D);
/* dy: bf16 [B][T][D]; dfinal: bf16 [B][D][3] nullable; dx: bf16 [B][T][D];
 * dw: fp32 [D][4]; dinit: fp32 [B][D][3] nullable. */
int sd_conv4_silu_bwd(int B, int T, int D, const void *x, int64_t x_sb, int64_t x_st,
                      const float *w, const void *init, const void *dy, const void *dfinal,
                      void *dx, float *dw, float *dinit, void *workspace,
                      size_t workspace_bytes, void *stream);

/* conv4 + SiLU under valid / reset masks (uint8 [B,T], element (b,t) at
 * m[b*m_sb + t*m_st], each nullable), the reference's CPU loop
 * (causallsso/model.py:146-164) that its varlen path reproduces by repacking
 * (model.py:166-220, packing.py:130-132): a reset on a valid token zeroes the
 * state first, an invalid token emits 0 and keeps the state, a valid token
 * emits silu(w . [state, x_t]) and shifts x_t in.  No repacking, no host sync.
 * Other arguments as sd_conv4_silu_fwd / _bwd; dx of invalid tokens is 0. */
int sd_conv4_silu_masked_fwd(int B, int T, int D, const void *x, int64_t x_sb, int64_t x_st,
                             const float *w, const void *init, const uint8_t *valid,
                             const uint8_t *reset, int64_t m_sb, int64_t m_st, void *y,
                             void *final_state, void *stream);
size_t sd_conv4_masked_workspace_bytes(int B, int D);
int sd_conv4_silu_masked_bwd(int B, int T, int D, const void *x, int64_t x_sb, int64_t x_st,
                             const float *w, const void *init, const uint8_t *valid,
                             const uint8_t *reset, int64_t m_sb, int64_t m_st, const void *dy,
                             const void *dfinal, void *dx, float *dw, float *dinit,
                             void *workspace, size_t workspace_bytes, void *stream);

/* KDA decay gate over N rows of H*r columns:
 *   out[n,h*r+c] = -exp(log_rate[h]) * softplus(raw[n*raw_row_stride + h*r+c] + bias[h*r+c])
 * (softplus(x) = x above 20).  raw: bf16; out: fp32 [N][H*r]. */
int sd_kda_gate_fwd(int N, int H, int r, const void *raw, int64_t raw_row_stride,
                    const float *log_rate, const float *bias, float *out, void *stream);
size_t sd_kda_gate_workspace_bytes(int N, int H, int r);
/* dout: fp32 [N][H*r]; draw: bf16 [N][H*r]; dlog_rate fp32 [H]; dbias fp32 [H*r]. */
int sd_kda_gate_bwd(int N, int H, int r, const void *raw, int64_t raw_row_stride,
                    const float *log_rate, const float *bias, const float *dout, void *draw,
                    float *dlog_rate, float *dbias, void *workspace, size_t workspace_bytes,
                    void *stream);

/* Sigmoid-gated RMSNorm over N rows of width D <= 256 (contiguous bf16):
 *   y = x * rsqrt(mean(x^2) + eps) * weight * sigmoid(gate);  rstd fp32 [N] nullable. */
int sd_rmsnorm_gated_fwd(int N, int D, float eps, const void *x, const void *gate,
                         const float *weight, void *y, float *rstd, void *stream);
size_t sd_rmsnorm_gated_workspace_bytes(int N, int D);
/* dy: bf16 [N][D]; dx, dgate: bf16 [N][D]; dweight fp32 [D];
 * y: bf16 [N][D] nullable, the recomputed forward output (for a following Linear). */
int sd_rmsnorm_gated_bwd(int N, int D, float eps, const void *x, const void *gate,
                         const float *weight, const void *dy, void *dx, void *dgate,
                         float *dweight, void *y, void *workspace, size_t workspace_bytes,
                         void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SOLVEDELTA_MIXER_H */
