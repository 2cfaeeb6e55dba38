// Internal parameter blocks shared by the kernels and the host launcher.
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include "../../include/solvedelta.h"

namespace sd {

// Forward workspace: every buffer is [n][Tp][128] (token panels) or
// [n][NT][...] (per-chunk), n = B*H, Tp = NT*64.
struct FwdWs {
  // kept for the backward
  float* Xc;     // C-op chunk-entering states X = C^T     [n][NT][128][128]
  float* Xs;     // S-op chunk-entering states              [n][NT][128][128]
  float* delta;  // predictor write delta (C-op w)          [n][Tp][128]
  float* d;      // primal address d = k + C^T k            [n][Tp][128]
  float* wS;     // S-op w = z - S~^T e                     [n][Tp][128]
  // transient panels
  float* Wc; float* Uc; float* Kc; float* Gam;
  float* Ws; float* Us; float* Ks; float* Qs; float* Ps;
};

struct FwdParams {
  sd_inputs in;
  int H, T, r, V, NT, Tp;
  float *Xc, *delta, *d;
  float* Wc; float* Uc; float* Kc; float* Gam;
  float* Ws; float* Us; float* Ks; float* Qs; float* Ps;
};

struct StateParams {
  int H, T, NT, Tp, rows, cols;
  const float* Wneg; const float* U; const float* Kt; const float* Gam;
  const float* Q; const float* P;  // output operands (COL_OUT)
  float* Xs; float* wout; __bf16* out;
  const float* init; int init_transposed;
  float* fin; int fin_transposed;
};

size_t prep_c_smem();
size_t prep_s_smem();

int launch_fwd(const sd_inputs* in, void* out, float* C_T, float* S_T, const FwdWs& w,
               hipStream_t st);
int launch_decode(const sd_inputs* in, void* out, float* C_T, float* S_T, hipStream_t st);

}  // namespace sd
