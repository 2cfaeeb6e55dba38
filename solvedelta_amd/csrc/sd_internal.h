// Internal parameter blocks shared by the kernels and the host launcher.
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include "../../include/solvedelta.h"

namespace sd {

#ifdef __HIPCC__
// Fragment order of a per-chunk panel of R rows x C columns (C = 64 or
// 128): each 16-row x 32-column MFMA operand block is 512 consecutive
// elements, lane-major (lane = 16 * ((col % 32) / 8) + row % 16, 8 elements
// per lane), so the sequential state pass reads a fragment as one contiguous
// 1 KiB 16-byte-per-lane load instead of 16 half-used cache lines.
__device__ __forceinline__ long long frag_off(int row, int col, int C) {
  return ((long long)(row >> 4) * (C >> 5) + (col >> 5)) * 512 +
         ((((col & 31) >> 3) << 4) + (row & 15)) * 8 + (col & 7);
}

// Per-token flags (sd_inputs.fresh, bit-coded; include/solvedelta.h): bit 0
// fresh (the C op's erase read x = gamma u^ is dropped), bit 1 invalid (q,
// keys, gamma and the log-decay read as 0), bit 2 reset (the log-decay reads as
// SD_RESET_LOG_DECAY).  t must be a valid token index.
// The flag's address is selected, not branched on: a load under a branch would
// wait for every load issued before it.
static __device__ const uint8_t sd_no_fresh = 0;  // the flag read when no flags are given
__device__ __forceinline__ const uint8_t* tok_flag_row(const sd_inputs& in, int b) {
  return in.fresh.data ? (const uint8_t*)in.fresh.data + (long long)b * in.fresh.sb : &sd_no_fresh;
}
__device__ __forceinline__ long long tok_flag_st(const sd_inputs& in) {
  return in.fresh.data ? in.fresh.st : 0;
}
__device__ __forceinline__ unsigned tok_flags(const sd_inputs& in, int b, int t) {
  return tok_flag_row(in, b)[(long long)t * tok_flag_st(in)];
}
// operand_keep of token t; 1 without a load in a kernel built without flags (FL)
template <bool FL>
__device__ __forceinline__ float operand_keep_at(const sd_inputs& in, int b, int t) {
  if constexpr (FL) return (tok_flags(in, b, t) & SD_TOK_INVALID) ? 0.f : 1.f;
  return 1.f;
}
// 0 on a fresh token, 1 otherwise
__device__ __forceinline__ float erase_keep_f(unsigned f) { return (f & SD_TOK_FRESH) ? 0.f : 1.f; }
__device__ __forceinline__ float erase_keep(const sd_inputs& in, int b, int t) {
  return erase_keep_f(tok_flags(in, b, t));
}
// 0 on an invalid token (its q, keys and gamma read as 0), 1 otherwise
__device__ __forceinline__ float operand_keep(unsigned f) { return (f & SD_TOK_INVALID) ? 0.f : 1.f; }
// the log-decay a token's kernels read: 0 when invalid, the reset value on a reset
__device__ __forceinline__ float decay_eff(unsigned f, float g) {
  return (f & SD_TOK_INVALID) ? 0.f : ((f & SD_TOK_RESET) ? SD_RESET_LOG_DECAY : g);
}
#endif

// Chunk-boundary state slots saved for the backward, in a 2-byte type (the
// final states handed to the caller stay fp32).  Forward states X (C^T and S)
// are fp16: the log-decay gradient's closure needs its 11-bit mantissa (the
// reference keeps its per-chunk S states 16-bit too,
// residual_frame/common_left_h.py:157).  The reverse passes' cotangent states
// lambda are bf16, whose exponent range holds any cotangent scale.
typedef _Float16 xslot_t;
typedef __bf16 lslot_t;
// Forward token panels the backward reads (e, chi, delta, d and the S op's w):
// fp16, like the forward state panels.
typedef _Float16 fpan_t;
// Backward token panels (partial gradients passed between the backward kernels):
// bf16, whose exponent range holds any scale of the output cotangent.
typedef __bf16 bpan_t;

// Forward workspace: every buffer is [n][Tp][128] (token panels) or
// [n][NT][...] (per-chunk), n = B*H, Tp = NT*64.
struct FwdWs {
  // kept for the backward
  xslot_t* Xc;   // C-op chunk-entering states X = C^T     [n][NT+1][128][128] (slot NT = final)
  xslot_t* Xs;   // S-op chunk-entering states              [n][NT+1][128][128]
  float* Ac;     // C-op (I+L)^-1 per chunk                 [n][NT][64][64]
  float* As;     // S-op (I+L)^-1 per chunk                 [n][NT][64][64]
  fpan_t* e;      // dual erase source e                     [n][Tp][128]
  fpan_t* chi;    // dual query chi                          [n][Tp][128]
  fpan_t* delta;  // predictor write delta (C-op w)          [n][Tp][128]
  fpan_t* d;      // primal address d = k + C^T k            [n][Tp][128]
  fpan_t* wS;     // S-op w = z - S~^T e                     [n][Tp][128]
  float* Gam;     // chunk decay e^{G_C}                     [n][NT][128]
  _Float16* Ps;   // S readout's output pair P, fragment order [n][NT][64][64]
  // forward-only panels: the state passes' MFMA operands W (token-major) and
  // K^ (chunk-transposed), fp16 in fragment order, U (fp32), and the S
  // readout's Q~ (token-major, fp16 fragment order)
  _Float16* Wc; float* Uc; _Float16* Kc;
  _Float16* Ws; float* Us; _Float16* Ks; _Float16* Qs;
};

struct FwdParams {
  sd_inputs in;
  int H, T, r, V, NT, Tp;
  xslot_t* Xc;
  fpan_t *delta, *d, *e, *chi;
  float *Ac, *As;
  _Float16* Wc; float* Uc; _Float16* Kc; float* Gam;
  _Float16* Ws; float* Us; _Float16* Ks; _Float16* Qs; _Float16* Ps;
};

// Sequential chunk pass, forward (state X) or reverse (cotangent lambda, rev):
//   slot[ch] = X;  w = U + Wneg X;  X = Gamma X + Kt w (+ At1 B1 when rev)
// Wneg token-major [Tp][128], Kt and At1 chunk-transposed [128][64], B1
// chunk-transposed [128 cols][64 tokens], all in fragment order.  Wneg and Kt
// are fp16 in forward passes and bf16 in reverse passes; At1 and B1 are bf16.
struct StateParams {
  int H, T, NT, Tp, rows, cols, rev;
  const void* Wneg; const float* U; const void* Kt; const float* Gam;
  const __bf16* At1; const __bf16* B1;  // reverse-pass injection
  void* Xs;  // state slots: xslot_t (forward) or lslot_t (reverse)
  void* wout;  // w panel: fpan_t (forward) or bpan_t (reverse)
  const float* init; int init_transposed;
  float* fin; int fin_transposed;
  // forward S pass only: the readout o = Q~ X0 + P w of every chunk, formed
  // from the staged X0 and w tiles and written to out [B,T,H,V] (bf16)
  const _Float16* Q; const _Float16* P; __bf16* out;
  int out_vec;  // rows of out take 16-byte stores (V % 8 == 0, aligned base)
};

void prof_begin(const char* name, hipStream_t st);
void prof_end(hipStream_t st);
// Raises a kernel's dynamic-LDS limit once per device.  The attribute call is
// not a stream operation; doing it only on the first (eager) launch keeps it
// out of graph captures of later calls.
inline void set_smem_once(const void* fn, int bytes, unsigned char* done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    return;
  }
  if (!done[dev]) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    done[dev] = 1;
  }
}
#define SD_SMEM_ONCE(kern, bytes)                                  \
  do {                                                             \
    static unsigned char sd_smem_done_[64] = {};                   \
    ::sd::set_smem_once((const void*)(kern), (int)(bytes), sd_smem_done_); \
  } while (0)

#define SD_LAUNCH(name, kern, grid, block, smem, st, ...)                 \
  do {                                                                   \
    ::sd::prof_begin(name, st);                                          \
    hipLaunchKernelGGL(kern, grid, block, smem, st, __VA_ARGS__);        \
    ::sd::prof_end(st);                                                  \
  } while (0)

void launch_state(const char* name, const StateParams& sp, int nseq, hipStream_t st);
size_t prep_c_smem();
size_t prep_s_smem();

int launch_fwd(const sd_inputs* in, void* out, float* C_T, float* S_T, const FwdWs& w,
               hipStream_t st);
struct BwdWs {
  lslot_t* Lc;  // C-op chunk-end cotangents                [n][NT+1][128][128]
  lslot_t* Ls;  // S-op chunk-end cotangents
  // reverse-pass panels (reused by both ops), bf16 in fragment order
  float* dU; __bf16* Wk; __bf16* At1; __bf16* B1t; __bf16* Ant;
  bpan_t* dwS; bpan_t* dwC;         // dw of each op           [n][Tp][128]
  bpan_t* de; bpan_t* dchi; bpan_t* dd;
  bpan_t* ddelta;  // shares dw_S's storage (written in place by the sources transpose)
  float* rn;  // 1 / |u_t|, 1 / |k_t| of every token (0 past T)       [n][Tp][2]
  float* Pp;  // P'_li = sum_c dd_lc u_ic e^{G_lc - G_ic} (i <= l) of the C op  [n][NT][64][64]
};

int launch_bwd(const sd_inputs* in, const FwdWs& fw, const BwdWs& bw, const void* dout,
               const float* dC_T, const float* dS_T, void* du, void* dh, void* dq, void* dk,
               void* dv, void* derase, void* dwrite, float* dlog_decay, float* dgamma,
               float* dC0, float* dS0, hipStream_t st);
int launch_decode(const sd_inputs* in, void* out, float* C_T, float* S_T, hipStream_t st);

// Wide-width path (key or value width above 128, both <= 256): its own
// workspace layout and kernels (sd_wide.hip).
constexpr int kWideMax = 256;
inline bool is_wide(int r, int V) { return r > 128 || V > 128; }
void wide_fwd_sizes(int B, int T, int H, int r, int V, size_t* saved, size_t* scratch);
size_t wide_bwd_workspace_bytes(int B, int T, int H, int r, int V);
int launch_wide_fwd(const sd_inputs* in, void* out, float* C_T, float* S_T, void* saved,
                    void* scratch, hipStream_t st);
int launch_wide_bwd(const sd_inputs* in, const void* fws, void* bws, const void* dout,
                    const float* dC_T, const float* dS_T, void* du, void* dh, void* dq, void* dk,
                    void* dv, void* derase, void* dwrite, float* dlog_decay, float* dgamma,
                    float* dC0, float* dS0, hipStream_t st);

}  // namespace sd
