/* SolveDelta chunked recurrence on MI355X (gfx950): C-ABI of libsolvedelta_hip.so.
 *
 * The library replaces the reference's native operator for this path:
 *   - sd_fwd      <- causallsso/ops/operator.py:13-55 (solvedelta_native forward) and
 *                    causallsso/ops/residual_frame/operator.py:154-304 (its composition:
 *                    L2 norms, predictor C solve, sources, exterior S memory);
 *   - sd_bwd      <- the autograd backward of that composition
 *                    (residual_frame/operator.py:74-138, predictor.py:130-282);
 *   - sd_decode   <- residual_frame/recurrent.py:188-327 (T = 1 recurrent inference).
 *
 * Conventions (identical to the reference's public operands):
 *   u,h,q [B,T,H,r], keys/erase_raw [B,T,H,1,r], values/write_raw [B,T,H,1,V]: bf16,
 *   arbitrary outer strides (in elements), unit innermost stride;
 *   associative_log_decay [B,T,H,r] fp32 (unit inner stride); geometry_write (gamma)
 *   fp32 addressed as gamma[b*sb + t*st + h*sh] (strides 0 broadcast [H] / [1,H]);
 *   initial / final states: C [B,H,r,r] (prediction = C u) and S [B,H,r,V], fp32,
 *   contiguous.  Erase/write gates are raw logits; the sigmoid is applied inside.
 *   Widths: 1 <= r, V <= 256, as the reference's state pass
 *   (residual_frame/common_left_h.py:139-140).  r, V <= 128 run on the main
 *   kernels (64-token chunks); a call with either width above 128 runs on the
 *   wide-width kernels (32-token chunks, FP32 panels) with their own workspace
 *   layout, which the *_workspace_bytes queries size from (r, V).  The Python
 *   operator cuts wider value axes into groups.  sd_decode takes r, V <= 128
 *   (wider T = 1 calls take the chunked path, as in the reference).
 *   Any T >= 1 (tails are neutrally padded inside).
 *
 * All entry points enqueue work on `stream` and never allocate or synchronise:
 * scratch comes from the caller's workspace, whose size the *_workspace_bytes
 * queries return.  Return value: 0 on success, SD_ERR_* otherwise.
 */
#ifndef SOLVEDELTA_H
#define SOLVEDELTA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SD_OK 0
#define SD_ERR_SHAPE 1    /* unsupported sizes (maps to ValueError)          */
#define SD_ERR_ARG 2      /* null pointer / bad stride (maps to ValueError)  */
#define SD_ERR_WORKSPACE 3 /* workspace too small (maps to ValueError)        */
#define SD_ERR_LAUNCH 4   /* HIP launch failure (maps to RuntimeError)       */

typedef struct {
  const void *data;   /* element (b,t,h,c) at data[b*sb + t*st + h*sh + c] */
  int64_t sb, st, sh; /* strides in elements */
} sd_view;

/* Token flags of sd_inputs.fresh, and the log-decay a reset token is read with. */
#define SD_TOK_FRESH 1u
#define SD_TOK_INVALID 2u
#define SD_TOK_RESET 4u
#define SD_RESET_LOG_DECAY (-20.0f)

typedef struct {
  int B, T, H, r, V;
  sd_view u, h, q, k, v, erase_raw, write_raw; /* bf16 */
  sd_view log_decay;                           /* fp32 */
  sd_view gamma;                               /* fp32, no channel axis */
  const float *C0, *S0;                        /* nullable initial state */
  sd_view fresh; /* uint8 [B,T] token flags at data[b*sb + t*st], nullable (no flags):
                  *  SD_TOK_FRESH: the token's predictor residual reads a zero state (the
                  *    predictor's erase read is dropped exactly);
                  *  SD_TOK_INVALID: the token is read as neutral -- its q, keys, gamma
                  *    and log-decay as 0 -- so it emits 0 and leaves both states as
                  *    they were (its u, h, values and gate logits must be finite);
                  *  SD_TOK_RESET: its log-decay is read as SD_RESET_LOG_DECAY.
                  * FRESH | RESET on a token is the reference's reset
                  * (reference.py:156-227) up to e^-20 ~ 2.1e-9 of both states before
                  * it, which the reference zeroes: a decay whose 16-token block total
                  * exceeds 60 takes the kernels' exact but slow per-coordinate path.
                  * Gradients are those of the operands as read: a caller that masks
                  * with these flags zeroes the gradients of invalid tokens' q, keys,
                  * gamma and log-decay and of reset tokens' log-decay itself
                  * (solvedelta_amd.masks does, with sd_mask_rows). */
} sd_inputs;

/* Forward. out: bf16 [B,T,H,V] contiguous. C_T / S_T nullable.
 * The workspace is two regions: the first sd_fwd_saved_bytes hold what sd_bwd
 * reads (pass that region, or the whole workspace, to sd_bwd and keep it alive
 * until then); the rest is forward-only scratch.  sd_fwd_split takes the two
 * regions as separate buffers, so a caller can release the scratch as soon as
 * the forward has run (the saved region is what an autograd graph holds). */
size_t sd_fwd_workspace_bytes(int B, int T, int H, int r, int V);
size_t sd_fwd_saved_bytes(int B, int T, int H, int r, int V);
size_t sd_fwd_scratch_bytes(int B, int T, int H, int r, int V);
int sd_fwd(const sd_inputs *in, void *out, float *C_T, float *S_T, void *workspace,
           size_t workspace_bytes, void *stream);
int sd_fwd_split(const sd_inputs *in, void *out, float *C_T, float *S_T, void *saved,
                 size_t saved_bytes, void *scratch, size_t scratch_bytes, void *stream);

/* Backward of sd_fwd with the same inputs and the forward's workspace.
 * dout: bf16 [B,T,H,V] contiguous (nullable = zero); dC_T, dS_T fp32 (nullable).
 * Gradient outputs, all contiguous: du,dh,dq,dk,dv,derase,dwrite bf16 in the
 * shapes of the inputs; dlog_decay fp32 [B,T,H,r]; dgamma fp32 [B,T,H];
 * dC0, dS0 fp32 (nullable). */
size_t sd_bwd_workspace_bytes(int B, int T, int H, int r, int V);
int sd_bwd(const sd_inputs *in, const void *fwd_workspace, const void *dout, const float *dC_T,
           const float *dS_T, void *du, void *dh, void *dq, void *dk, void *dv, void *derase,
           void *dwrite, float *dlog_decay, float *dgamma, float *dC0, float *dS0,
           void *workspace, size_t workspace_bytes, void *stream);

/* Row masking for masked batches on the dense layout (no counterpart in the
 * reference, whose masked path repacks valid tokens into segments with a host
 * sync, causallsso/ops/packing.py:43-150): one launch copies up to eight
 * [B,T,H,width] tensors into contiguous outputs, keeping the rows of valid
 * tokens and zeroing the others; on valid reset tokens rows with reset_fill
 * set take reset_value.  flags: uint8 [B,T] at flags[b*flags_sb + t*flags_st],
 * bit 0 valid, bit 1 reset.  solvedelta_amd.masks uses it on the gradients
 * (zero on invalid tokens, zero log-decay gradient on reset tokens; the kernels
 * read the operands masked through the token flags).  dst == src masks in place
 * (src must then be contiguous): only the rows that change are written.
 * Returns SD_ERR_ARG for dst == src with a non-contiguous src. */
typedef struct {
  const void *src; /* element (b,t,h,c) at src[b*sb + t*st + h*sh + c] */
  int64_t sb, st, sh;
  void *dst;       /* contiguous [B,T,H,width]; or src itself (in place) */
  int width, is_fp32, reset_fill;
  float reset_value;
} sd_mask_tensor;
int sd_mask_rows(int B, int T, int H, const uint8_t *flags, int64_t flags_sb, int64_t flags_st,
                 const sd_mask_tensor *tensors, int n, void *stream);

/* The flags sd_mask_rows and the operator's fresh input take, from bool
 * (one byte, 0 / 1) [B,T] masks, in one launch (no counterpart in the
 * reference; it replaces the host-side mask arithmetic of its packing step,
 * causallsso/ops/packing.py:43-60): element (b,t) of valid / reset at
 * mask[b*sb + t*st]; a null valid mask means every token is valid, a null reset
 * mask none resets.  Writes flags (uint8 [B,T] contiguous: bit 0 valid, bit 1
 * valid reset) for sd_mask_rows and the operator's token flags (uint8 [B,T]
 * contiguous, sd_inputs.fresh): SD_TOK_INVALID on invalid tokens,
 * SD_TOK_FRESH | SD_TOK_RESET on valid reset tokens, 0 otherwise. */
int sd_mask_flags(int B, int T, const uint8_t *valid, int64_t valid_sb, int64_t valid_st,
                  const uint8_t *reset, int64_t reset_sb, int64_t reset_st, uint8_t *flags,
                  uint8_t *fresh, void *stream);

/* One-token recurrent step (T must be 1). out: bf16 [B,1,H,V] contiguous.
 * C_T / S_T receive the advanced state; they may alias C0 / S0 (in place). */
int sd_decode(const sd_inputs *in, void *out, float *C_T, float *S_T, void *stream);

/* Opt-in per-kernel timing with HIP events on the launch stream (no
 * counterpart in the reference; used by bench.py).  sd_profile_enable(1)
 * clears the totals and starts recording; sd_profile_read writes lines
 * "kernel total_ms launches" into buf and returns the bytes needed. */
int sd_profile_enable(int on);
size_t sd_profile_read(char *buf, size_t len);

/* Library version string. */
const char *sd_version(void);

#ifdef __cplusplus
}
#endif
#endif
