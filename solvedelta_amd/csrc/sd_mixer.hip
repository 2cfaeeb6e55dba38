// Mixer frontend and readout of the SolveDelta layer on MI355X:
//   * causal depthwise conv4 + SiLU with initial / final state
//     (reference: causallsso/model.py:119-136, CPU semantics :146-164);
//   * the KDA decay gate  log_decay = -exp(log_rate[h]) * softplus(raw + bias[h, c])
//     (reference: causallsso/model.py:375-390);
//   * the sigmoid-gated RMSNorm feeding the output projection
//     (reference: causallsso/ops/norm_gate.py:20-43 definition, :46-150 owner).
// Forward and backward of each; parameter-gradient reductions are two-stage
// (per-workgroup partials in the caller's workspace, then one reduction kernel),
// so results are deterministic.  All arithmetic is FP32; bf16 in / out.
#include <hip/hip_runtime.h>

#include "sd_common.cuh"
#include "sd_internal.h"
#include "../../include/solvedelta_mixer.h"

namespace sd {

__device__ __forceinline__ float silu(float a) { return a / (1.f + __expf(-a)); }
__device__ __forceinline__ float sigm(float a) { return 1.f / (1.f + __expf(-a)); }
// torch.nn.functional.softplus with its default threshold 20
__device__ __forceinline__ float softplus20(float x) {
  return x > 20.f ? x : log1pf(__expf(x));
}

// ---------------------------------------------------------------------------
// conv4 + SiLU.  One thread per (channel, batch row, CONV_TC-token chunk): the
// chunk's inputs (plus the 3-token halo) are loaded into registers up front so
// the loads overlap, then the window slides through registers.  xs[-3..-1] is
// the initial state (zeros when absent); y_t = silu(sum_k w_k xs[t-3+k]).
// ---------------------------------------------------------------------------
constexpr int CONV_TC = 32;

struct ConvArgs {
  int B, T, D;
  const __bf16* __restrict__ x;
  long long sb, st;
  const float* __restrict__ w;       // [D][4]
  const __bf16* __restrict__ init;   // [B][D][3] or null
};

__device__ __forceinline__ float conv_x(const ConvArgs& a, int b, int t, int d) {
  if (t >= a.T) return 0.f;
  if (t >= 0) return bf2f(a.x[(long long)b * a.sb + (long long)t * a.st + d]);
  if (!a.init) return 0.f;
  return bf2f(a.init[((long long)b * a.D + d) * 3 + (t + 3)]);
}

// xs[t0 - 3 + j] for j < N: every load reads a clamped, valid token and is
// issued before the first use (a guarded load would branch and wait for the
// loads before it); tokens past T read 0, and the three halo tokens of the
// first chunk come from the initial state (zeros when absent).
template <int N>
__device__ __forceinline__ void conv_window(const ConvArgs& a, int b, int t0, int d, float (&xv)[N]) {
  const __bf16* xb = a.x + (long long)b * a.sb + d;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int t = t0 - 3 + j, tc = t < 0 ? 0 : (t < a.T ? t : a.T - 1);
    xv[j] = keep_if(t < a.T, bf2f(xb[(long long)tc * a.st]));
  }
  if (t0 == 0) {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      xv[j] = a.init ? bf2f(a.init[((long long)b * a.D + d) * 3 + j]) : 0.f;
  }
}

__global__ __launch_bounds__(NTHREADS) void k_conv_fwd(ConvArgs a, __bf16* __restrict__ y,
                                                       __bf16* __restrict__ fin) {
  const int d = blockIdx.x * NTHREADS + threadIdx.x, b = blockIdx.z;
  if (d >= a.D) return;
  const int t0 = blockIdx.y * CONV_TC;
  const float w0 = a.w[d * 4], w1 = a.w[d * 4 + 1], w2 = a.w[d * 4 + 2], w3 = a.w[d * 4 + 3];
  float xv[CONV_TC + 3];
  conv_window(a, b, t0, d, xv);
#pragma unroll
  for (int j = 0; j < CONV_TC; ++j) {
    const int t = t0 + j;
    const float acc = w0 * xv[j] + w1 * xv[j + 1] + w2 * xv[j + 2] + w3 * xv[j + 3];
    if (t < a.T) y[((long long)b * a.T + t) * a.D + d] = f2bf(silu(acc));
  }
  if (fin && t0 + CONV_TC >= a.T) {  // the chunk that holds the last token writes the state
    __bf16* f = fin + ((long long)b * a.D + d) * 3;
    f[0] = f2bf(conv_x(a, b, a.T - 3, d));
    f[1] = f2bf(conv_x(a, b, a.T - 2, d));
    f[2] = f2bf(conv_x(a, b, a.T - 1, d));
  }
}

// Backward.  da_t = dy_t silu'(a_t);  dx_s = sum_k w_k da_{s+3-k} (+ dfinal);
// dw_k = sum_t da_t xs[t-3+k];  dinit_j = sum_{k<=j} w_k da_{j-k} (+ dfinal).
// Thread (d, b, chunk) recomputes a_t for t in [t0, t0 + CONV_TC + 3) from
// register-resident inputs (zero beyond T), so every dx of its chunk is local.
__global__ __launch_bounds__(NTHREADS) void k_conv_bwd(ConvArgs a, const __bf16* __restrict__ dy,
                                                       const __bf16* __restrict__ dfin,
                                                       __bf16* __restrict__ dx,
                                                       float* __restrict__ dinit,
                                                       float* __restrict__ dw_part) {
  const int d = blockIdx.x * NTHREADS + threadIdx.x, b = blockIdx.z;
  if (d >= a.D) return;
  const int T = a.T, t0 = blockIdx.y * CONV_TC;
  const float w0 = a.w[d * 4], w1 = a.w[d * 4 + 1], w2 = a.w[d * 4 + 2], w3 = a.w[d * 4 + 3];
  constexpr int NX = CONV_TC + 6, NA = CONV_TC + 3;
  float xv[NX];   // xs[t0-3 .. t0+CONV_TC+2]
  float gv[NA];   // dy[t0 .. t0+CONV_TC+2]
  conv_window(a, b, t0, d, xv);
#pragma unroll
  for (int j = 0; j < NA; ++j) {  // clamped token, then select
    const int t = t0 + j;
    gv[j] = keep_if(t < T, bf2f(dy[((long long)b * T + (t < T ? t : T - 1)) * a.D + d]));
  }
  float df[3] = {0.f, 0.f, 0.f};  // dfinal_m is the cotangent of xs[T-3+m]
  if (dfin)
#pragma unroll
    for (int m = 0; m < 3; ++m) df[m] = bf2f(dfin[((long long)b * a.D + d) * 3 + m]);
  float da[NA];
  float g0 = 0.f, g1 = 0.f, g2 = 0.f, g3 = 0.f;
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const float acc = w0 * xv[j] + w1 * xv[j + 1] + w2 * xv[j + 2] + w3 * xv[j + 3];
    const float sg = sigm(acc);
    da[j] = gv[j] * sg * (1.f + acc * (1.f - sg));   // gv = 0 beyond T
    if (j < CONV_TC) {
      g0 += da[j] * xv[j]; g1 += da[j] * xv[j + 1]; g2 += da[j] * xv[j + 2];
      g3 += da[j] * xv[j + 3];
    }
  }
#pragma unroll
  for (int j = 0; j < CONV_TC; ++j) {
    const int s = t0 + j;
    if (s < T) {
      float v = w3 * da[j] + w2 * da[j + 1] + w1 * da[j + 2] + w0 * da[j + 3];
      if (s >= T - 3) v += df[s - (T - 3)];
      dx[((long long)b * T + s) * a.D + d] = f2bf(v);
    }
  }
  if (t0 == 0 && dinit) {
    // xs[-3+j] feeds a_t for t = j - k >= 0 with weight w_k (k <= j)
    float v0 = w0 * da[0];
    float v1 = w1 * da[0] + w0 * da[1];
    float v2 = w2 * da[0] + w1 * da[1] + w0 * da[2];
#pragma unroll
    for (int m = 0; m < 3; ++m) {  // final-state cotangents that land on the initial state (T < 3)
      const int j = T + m;
      if (j < 3) (j == 0 ? v0 : j == 1 ? v1 : v2) += df[m];
    }
    float* di = dinit + ((long long)b * a.D + d) * 3;
    di[0] = v0; di[1] = v1; di[2] = v2;
  }
  float* p = dw_part + (((long long)b * gridDim.y + blockIdx.y) * a.D + d) * 4;
  p[0] = g0; p[1] = g1; p[2] = g2; p[3] = g3;
}

// out[i] = sum_p part[p][i]: 32 columns x 8 partial rows per workgroup, the
// eight row sums combined through LDS.
__global__ __launch_bounds__(NTHREADS) void k_sum_parts(const float* __restrict__ part, int nparts,
                                                        int width, float* __restrict__ out) {
  __shared__ float red[8][33];
  const int cx = threadIdx.x & 31, ry = threadIdx.x >> 5;
  const int i = blockIdx.x * 32 + cx;
  float s = 0.f;
  if (i < width) {
#pragma unroll 4
    for (int p = ry; p < nparts; p += 8) s += part[(long long)p * width + i];
  }
  red[ry][cx] = s;
  __syncthreads();
  if (ry == 0 && i < width) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) t += red[k][cx];
    out[i] = t;
  }
}

// ---------------------------------------------------------------------------
// KDA decay gate.  raw [N][H*r] bf16 (row stride), bias [H*r], log_rate [H].
// ---------------------------------------------------------------------------
constexpr int GATE_TR = 16;  // rows per backward workgroup

__global__ __launch_bounds__(NTHREADS) void k_gate_fwd(int N, int H, int r, const __bf16* raw,
                                                       long long rs, const float* log_rate,
                                                       const float* bias, float* out) {
  const int HR = H * r;
  const long long i = (long long)blockIdx.x * NTHREADS + threadIdx.x;
  if (i >= (long long)N * HR) return;
  const int c = (int)(i % HR);
  const long long n = i / HR;
  const float x = bf2f(raw[n * rs + c]) + bias[c];
  out[i] = -__expf(log_rate[c / r]) * softplus20(x);
}

// draw = dout * (-exp(lr)) * sigmoid(raw + bias) (softplus' is 1 above the
// threshold); partials: dbias_c = sum draw, dlr_c = sum dout * out.
__global__ __launch_bounds__(NTHREADS) void k_gate_bwd(int N, int H, int r, const __bf16* raw,
                                                       long long rs, const float* log_rate,
                                                       const float* bias, const float* dout,
                                                       __bf16* draw, float* part) {
  const int HR = H * r;
  const int c = blockIdx.x * NTHREADS + threadIdx.x;
  if (c >= HR) return;
  const int n0 = blockIdx.y * GATE_TR, n1 = min(N, n0 + GATE_TR);
  const float rate = __expf(log_rate[c / r]), bc = bias[c];
  float db = 0.f, dl = 0.f;
#pragma unroll 4
  for (int n = n0; n < n1; ++n) {
    const float x = bf2f(raw[(long long)n * rs + c]) + bc;
    const float g = dout[(long long)n * HR + c];
    const float sp = softplus20(x);
    const float dx = -rate * g * (x > 20.f ? 1.f : sigm(x));
    draw[(long long)n * HR + c] = f2bf(dx);
    db += dx;
    dl += -rate * sp * g;
  }
  part[(long long)blockIdx.y * 2 * HR + c] = db;
  part[(long long)blockIdx.y * 2 * HR + HR + c] = dl;
}

// One workgroup per head: dbias[c] for the head's columns, dlog_rate[h], from
// nparts partial rows (the backward passes the one row of column sums).
__global__ __launch_bounds__(NTHREADS) void k_gate_reduce(int H, int r, int nparts,
                                                          const float* part, float* dbias,
                                                          float* dlog_rate) {
  __shared__ float red[NTHREADS / 64];
  const int h = blockIdx.x, HR = H * r;
  float acc = 0.f;
  for (int cc = threadIdx.x; cc < r; cc += NTHREADS) {
    const int c = h * r + cc;
    float db = 0.f, dl = 0.f;
    for (int p = 0; p < nparts; ++p) {
      db += part[(long long)p * 2 * HR + c];
      dl += part[(long long)p * 2 * HR + HR + c];
    }
    dbias[c] = db;
    acc += dl;
  }
  acc = wave_sum(acc);
  if (lane_id() == 0) red[wave_id()] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < NTHREADS / 64; ++w) s += red[w];
    dlog_rate[h] = s;
  }
}

// ---------------------------------------------------------------------------
// Sigmoid-gated RMSNorm: y = x rstd w sigmoid(g), rstd = 1/sqrt(mean(x^2) + eps).
// One wave per row of width D <= 256 (4 elements per lane).
// ---------------------------------------------------------------------------
constexpr int RMS_ROWS = 4;     // rows (waves) per workgroup
constexpr int RMS_PART = 64;    // rows per dweight partial

__device__ __forceinline__ void rms_row(const __bf16* x, const __bf16* g, const float* w, int D,
                                        float (&xv)[4], float (&gv)[4], float (&wv)[4]) {
  const int l = lane_id();
#pragma unroll
  for (int m = 0; m < 4; ++m) {  // clamped column, then select: no branch around the loads
    const int c = l + 64 * m, cc = c < D ? c : D - 1;
    const bool ok = c < D;
    xv[m] = keep_if(ok, bf2f(x[cc]));
    gv[m] = keep_if(ok, bf2f(g[cc]));
    wv[m] = keep_if(ok, w[cc]);
  }
}

__global__ __launch_bounds__(RMS_ROWS * 64) void k_rms_fwd(int N, int D, float eps,
                                                           const __bf16* x, const __bf16* g,
                                                           const float* w, __bf16* y,
                                                           float* rstd_out) {
  const int n = blockIdx.x * RMS_ROWS + wave_id();
  if (n >= N) return;
  float xv[4], gv[4], wv[4];
  rms_row(x + (long long)n * D, g + (long long)n * D, w, D, xv, gv, wv);
  const float ss = wave_sum(xv[0] * xv[0] + xv[1] * xv[1] + xv[2] * xv[2] + xv[3] * xv[3]);
  const float rs = rsqrtf(ss / D + eps);
  const int l = lane_id();
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = l + 64 * m;
    if (c < D) y[(long long)n * D + c] = f2bf(xv[m] * rs * wv[m] * sigm(gv[m]));
  }
  if (rstd_out && l == 0) rstd_out[n] = rs;
}

// dx = rstd (gy - xhat mean(gy xhat)), gy = dy w s;  dg = dy xhat w s (1 - s);
// dw_c = sum dy xhat s;  y (recomputed for the projection's weight gradient).
// Each wave takes RMS_U rows at a time, every row's loads issued before the
// first row's reductions (rows past N read row N - 1 and store nothing).
constexpr int RMS_U = 4;
static_assert(RMS_PART % (RMS_ROWS * RMS_U) == 0, "whole row groups per workgroup");

__global__ __launch_bounds__(RMS_ROWS * 64) void k_rms_bwd(int N, int D, float eps,
                                                           const __bf16* __restrict__ x,
                                                           const __bf16* __restrict__ g,
                                                           const float* __restrict__ w,
                                                           const __bf16* __restrict__ dy,
                                                           __bf16* __restrict__ dx,
                                                           __bf16* __restrict__ dg,
                                                           __bf16* __restrict__ y,
                                                           float* __restrict__ part) {
  __shared__ float pw[RMS_ROWS][256];
  const int l = lane_id(), wv_ = wave_id();
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float wv[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = l + 64 * m;
    wv[m] = keep_if(c < D, w[c < D ? c : D - 1]);
  }
  // a workgroup covers RMS_PART rows: each wave walks RMS_PART / RMS_ROWS of them
  const int base = blockIdx.x * RMS_PART;
  for (int r0 = wv_; r0 < RMS_PART; r0 += RMS_ROWS * RMS_U) {
    if (base + r0 >= N) break;
    float xv[RMS_U][4], gv[RMS_U][4], dv[RMS_U][4];
#pragma unroll
    for (int u = 0; u < RMS_U; ++u) {
      const int n = base + r0 + u * RMS_ROWS, nc = n < N ? n : N - 1;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int c = l + 64 * m, cc = c < D ? c : D - 1;
        const long long o = (long long)nc * D + cc;
        xv[u][m] = keep_if(c < D, bf2f(x[o]));
        gv[u][m] = keep_if(c < D, bf2f(g[o]));
        dv[u][m] = keep_if(c < D && n < N, bf2f(dy[o]));
      }
    }
#pragma unroll
    for (int u = 0; u < RMS_U; ++u) {
      const int n = base + r0 + u * RMS_ROWS;
      const float ss = wave_sum(xv[u][0] * xv[u][0] + xv[u][1] * xv[u][1] + xv[u][2] * xv[u][2] +
                                xv[u][3] * xv[u][3]);
      const float rs = rsqrtf(ss / D + eps);
      float gy[4], xh[4], sg[4], dot = 0.f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        sg[m] = sigm(gv[u][m]);
        xh[m] = xv[u][m] * rs;
        gy[m] = dv[u][m] * wv[m] * sg[m];
        dot += gy[m] * xh[m];
      }
      dot = wave_sum(dot) / D;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int c = l + 64 * m;
        acc[m] += dv[u][m] * xh[m] * sg[m];  // 0 on rows past N (dv = 0)
        if (c < D && n < N) {
          const long long o = (long long)n * D + c;
          dx[o] = f2bf(rs * (gy[m] - xh[m] * dot));
          dg[o] = f2bf(dv[u][m] * xh[m] * wv[m] * sg[m] * (1.f - sg[m]));
          if (y) y[o] = f2bf(xh[m] * wv[m] * sg[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) pw[wv_][l + 64 * m] = acc[m];
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += RMS_ROWS * 64) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < RMS_ROWS; ++k) s += pw[k][c];
    part[(long long)blockIdx.x * D + c] = s;
  }
}

static inline int cdiv(long long a, int b) { return (int)((a + b - 1) / b); }


// ---------------------------------------------------------------------------
// conv4 + SiLU under valid / reset masks, the CPU loop's semantics
// (model.py:146-164): a reset on a valid token zeroes the 3-token state first;
// an invalid token emits 0 and leaves the state; a valid token emits
// silu(w . [state, x_t]) and shifts x_t into the state.  One thread per
// (channel, batch row) walks the row, 8 tokens' loads issued at a time: the
// masks make each window depend on the row's whole history, so the row is not
// cut into chunks.
// ---------------------------------------------------------------------------
struct ConvMask {
  const uint8_t* __restrict__ valid;  // [B,T] at b*sb + t*st, nullable (all valid)
  const uint8_t* __restrict__ reset;  // nullable (no reset)
  long long sb, st;
};
constexpr int MCONV_U = 8;

__device__ __forceinline__ void conv_mask_at(const ConvMask& m, int b, int t, bool& v, bool& r) {
  const long long o = (long long)b * m.sb + (long long)t * m.st;
  v = m.valid ? m.valid[o] != 0 : true;
  r = v && m.reset && m.reset[o] != 0;
}

__global__ __launch_bounds__(NTHREADS) void k_conv_masked_fwd(ConvArgs a, ConvMask m,
                                                              __bf16* __restrict__ y,
                                                              __bf16* __restrict__ fin) {
  const int d = blockIdx.x * NTHREADS + threadIdx.x, b = blockIdx.y;
  if (d >= a.D) return;
  const int T = a.T;
  const float w0 = a.w[d * 4], w1 = a.w[d * 4 + 1], w2 = a.w[d * 4 + 2], w3 = a.w[d * 4 + 3];
  float s0 = conv_x(a, b, -3, d), s1 = conv_x(a, b, -2, d), s2 = conv_x(a, b, -1, d);
  for (int t0 = 0; t0 < T; t0 += MCONV_U) {
    float xv[MCONV_U];
    bool vv[MCONV_U], rr[MCONV_U];
#pragma unroll
    for (int j = 0; j < MCONV_U; ++j) {
      const int t = t0 + j < T ? t0 + j : T - 1;
      xv[j] = bf2f(a.x[(long long)b * a.sb + (long long)t * a.st + d]);
      conv_mask_at(m, b, t, vv[j], rr[j]);
    }
#pragma unroll
    for (int j = 0; j < MCONV_U; ++j) {
      const int t = t0 + j;
      if (t < T) {
        if (rr[j]) s0 = s1 = s2 = 0.f;
        const float acc = w0 * s0 + w1 * s1 + w2 * s2 + w3 * xv[j];
        y[((long long)b * T + t) * a.D + d] = f2bf(vv[j] ? silu(acc) : 0.f);
        if (vv[j]) {
          s0 = s1;
          s1 = s2;
          s2 = xv[j];
        }
      }
    }
  }
  if (fin) {
    __bf16* f = fin + ((long long)b * a.D + d) * 3;
    f[0] = f2bf(s0);
    f[1] = f2bf(s1);
    f[2] = f2bf(s2);
  }
}

// Backward in one forward walk.  Each window slot carries its owner (a token
// t >= 0, an initial-state slot -1..-3, or kNoOwner after a reset) and the
// cotangent gathered for it so far; a slot's cotangent is complete when its
// value leaves the window (shift, reset, or the end of the row, where the
// final-state cotangent joins it) and is written to dx / dinit then.  Invalid
// tokens get dx = 0.  dw partials per (row, channel) go to the workspace.
constexpr int kNoOwner = -1000;

__device__ __forceinline__ void conv_flush(int owner, float g, __bf16* __restrict__ dx,
                                           float* __restrict__ dinit, int b, int T, int D, int d) {
  if (owner >= 0) dx[((long long)b * T + owner) * D + d] = f2bf(g);
  else if (owner > kNoOwner && dinit) dinit[((long long)b * D + d) * 3 + (-owner - 1)] = g;
}

__global__ __launch_bounds__(NTHREADS) void k_conv_masked_bwd(ConvArgs a, ConvMask m,
                                                              const __bf16* __restrict__ dy,
                                                              const __bf16* __restrict__ dfin,
                                                              __bf16* __restrict__ dx,
                                                              float* __restrict__ dinit,
                                                              float* __restrict__ dw_part) {
  const int d = blockIdx.x * NTHREADS + threadIdx.x, b = blockIdx.y;
  if (d >= a.D) return;
  const int T = a.T, D = a.D;
  const float w0 = a.w[d * 4], w1 = a.w[d * 4 + 1], w2 = a.w[d * 4 + 2], w3 = a.w[d * 4 + 3];
  float s0 = conv_x(a, b, -3, d), s1 = conv_x(a, b, -2, d), s2 = conv_x(a, b, -1, d);
  int o0 = a.init ? -1 : kNoOwner, o1 = a.init ? -2 : kNoOwner, o2 = a.init ? -3 : kNoOwner;
  float p0 = 0.f, p1 = 0.f, p2 = 0.f;
  float g0 = 0.f, g1 = 0.f, g2 = 0.f, g3 = 0.f;
  for (int t0 = 0; t0 < T; t0 += MCONV_U) {
    float xv[MCONV_U], gv[MCONV_U];
    bool vv[MCONV_U], rr[MCONV_U];
#pragma unroll
    for (int j = 0; j < MCONV_U; ++j) {
      const int t = t0 + j < T ? t0 + j : T - 1;
      xv[j] = bf2f(a.x[(long long)b * a.sb + (long long)t * a.st + d]);
      gv[j] = bf2f(dy[((long long)b * T + t) * D + d]);
      conv_mask_at(m, b, t, vv[j], rr[j]);
    }
#pragma unroll
    for (int j = 0; j < MCONV_U; ++j) {
      const int t = t0 + j;
      if (t >= T) continue;
      if (!vv[j]) {
        dx[((long long)b * T + t) * D + d] = f2bf(0.f);
        continue;
      }
      if (rr[j]) {
        conv_flush(o0, p0, dx, dinit, b, T, D, d);
        conv_flush(o1, p1, dx, dinit, b, T, D, d);
        conv_flush(o2, p2, dx, dinit, b, T, D, d);
        s0 = s1 = s2 = 0.f;
        p0 = p1 = p2 = 0.f;
        o0 = o1 = o2 = kNoOwner;
      }
      const float acc = w0 * s0 + w1 * s1 + w2 * s2 + w3 * xv[j];
      const float sg = sigm(acc);
      const float da = gv[j] * sg * (1.f + acc * (1.f - sg));
      g0 += da * s0; g1 += da * s1; g2 += da * s2; g3 += da * xv[j];
      p0 += da * w0; p1 += da * w1; p2 += da * w2;
      conv_flush(o0, p0, dx, dinit, b, T, D, d);  // slot 0 leaves the window
      s0 = s1; o0 = o1; p0 = p1;
      s1 = s2; o1 = o2; p1 = p2;
      s2 = xv[j]; o2 = t; p2 = da * w3;
    }
  }
  if (dfin) {
    const __bf16* f = dfin + ((long long)b * D + d) * 3;
    p0 += bf2f(f[0]);
    p1 += bf2f(f[1]);
    p2 += bf2f(f[2]);
  }
  conv_flush(o0, p0, dx, dinit, b, T, D, d);
  conv_flush(o1, p1, dx, dinit, b, T, D, d);
  conv_flush(o2, p2, dx, dinit, b, T, D, d);
  float* wp = dw_part + ((long long)b * D + d) * 4;
  wp[0] = g0; wp[1] = g1; wp[2] = g2; wp[3] = g3;
}

}  // namespace sd

using namespace sd;

extern "C" {

size_t sd_conv4_workspace_bytes(int B, int T, int D) {
  if (B <= 0 || T <= 0 || D <= 0) return 0;
  return (size_t)B * cdiv(T, CONV_TC) * D * 4 * sizeof(float);
}

int sd_conv4_silu_fwd(int B, int T, int D, const void* x, int64_t x_sb, int64_t x_st,
                      const float* w, const void* init, void* y, void* final_state, void* stream) {
  if (B <= 0 || T <= 0 || D <= 0) return SD_ERR_SHAPE;
  if (!x || !w || !y) return SD_ERR_ARG;
  ConvArgs a{B, T, D, (const __bf16*)x, x_sb, x_st, w, (const __bf16*)init};
  dim3 grid(cdiv(D, NTHREADS), cdiv(T, CONV_TC), B);
  SD_LAUNCH("k_conv_fwd", k_conv_fwd, grid, dim3(NTHREADS), 0, (hipStream_t)stream, a,
            (__bf16*)y, (__bf16*)final_state);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

int sd_conv4_silu_bwd(int B, int T, int D, const void* x, int64_t x_sb, int64_t x_st,
                      const float* w, const void* init, const void* dy, const void* dfinal,
                      void* dx, float* dw, float* dinit, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (B <= 0 || T <= 0 || D <= 0) return SD_ERR_SHAPE;
  if (!x || !w || !dy || !dx || !dw || !workspace) return SD_ERR_ARG;
  if (workspace_bytes < sd_conv4_workspace_bytes(B, T, D)) return SD_ERR_WORKSPACE;
  ConvArgs a{B, T, D, (const __bf16*)x, x_sb, x_st, w, (const __bf16*)init};
  const int nch = cdiv(T, CONV_TC);
  hipStream_t st = (hipStream_t)stream;
  SD_LAUNCH("k_conv_bwd", k_conv_bwd, dim3(cdiv(D, NTHREADS), nch, B), dim3(NTHREADS), 0, st, a,
            (const __bf16*)dy, (const __bf16*)dfinal, (__bf16*)dx, dinit, (float*)workspace);
  SD_LAUNCH("k_sum_parts", k_sum_parts, dim3(cdiv(4LL * D, 32)), dim3(NTHREADS), 0, st,
            (const float*)workspace, B * nch, 4 * D, dw);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

size_t sd_conv4_masked_workspace_bytes(int B, int D) {
  if (B <= 0 || D <= 0) return 0;
  return (size_t)B * D * 4 * sizeof(float);
}

int sd_conv4_silu_masked_fwd(int B, int T, int D, const void* x, int64_t x_sb, int64_t x_st,
                             const float* w, const void* init, const uint8_t* valid,
                             const uint8_t* reset, int64_t m_sb, int64_t m_st, void* y,
                             void* final_state, void* stream) {
  if (B <= 0 || T <= 0 || D <= 0) return SD_ERR_SHAPE;
  if (!x || !w || !y) return SD_ERR_ARG;
  ConvArgs a{B, T, D, (const __bf16*)x, x_sb, x_st, w, (const __bf16*)init};
  ConvMask m{valid, reset, m_sb, m_st};
  SD_LAUNCH("k_conv_masked_fwd", k_conv_masked_fwd, dim3(cdiv(D, NTHREADS), B), dim3(NTHREADS), 0,
            (hipStream_t)stream, a, m, (__bf16*)y, (__bf16*)final_state);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

int sd_conv4_silu_masked_bwd(int B, int T, int D, const void* x, int64_t x_sb, int64_t x_st,
                             const float* w, const void* init, const uint8_t* valid,
                             const uint8_t* reset, int64_t m_sb, int64_t m_st, const void* dy,
                             const void* dfinal, void* dx, float* dw, float* dinit,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (B <= 0 || T <= 0 || D <= 0) return SD_ERR_SHAPE;
  if (!x || !w || !dy || !dx || !dw || !workspace) return SD_ERR_ARG;
  if (workspace_bytes < sd_conv4_masked_workspace_bytes(B, D)) return SD_ERR_WORKSPACE;
  ConvArgs a{B, T, D, (const __bf16*)x, x_sb, x_st, w, (const __bf16*)init};
  ConvMask m{valid, reset, m_sb, m_st};
  hipStream_t st = (hipStream_t)stream;
  SD_LAUNCH("k_conv_masked_bwd", k_conv_masked_bwd, dim3(cdiv(D, NTHREADS), B), dim3(NTHREADS), 0,
            st, a, m, (const __bf16*)dy, (const __bf16*)dfinal, (__bf16*)dx, dinit,
            (float*)workspace);
  SD_LAUNCH("k_sum_parts", k_sum_parts, dim3(cdiv(4LL * D, 32)), dim3(NTHREADS), 0, st,
            (const float*)workspace, B, 4 * D, dw);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

// Workspace: the [np][2][H*r] per-workgroup partials, then their [2][H*r] column sums.
size_t sd_kda_gate_workspace_bytes(int N, int H, int r) {
  if (N <= 0 || H <= 0 || r <= 0) return 0;
  return (size_t)(cdiv(N, GATE_TR) + 1) * 2 * H * r * sizeof(float);
}

int sd_kda_gate_fwd(int N, int H, int r, const void* raw, int64_t raw_row_stride,
                    const float* log_rate, const float* bias, float* out, void* stream) {
  if (N <= 0 || H <= 0 || r <= 0) return SD_ERR_SHAPE;
  if (!raw || !log_rate || !bias || !out) return SD_ERR_ARG;
  SD_LAUNCH("k_gate_fwd", k_gate_fwd, dim3(cdiv((long long)N * H * r, NTHREADS)), dim3(NTHREADS),
            0, (hipStream_t)stream, N, H, r, (const __bf16*)raw, raw_row_stride, log_rate, bias,
            out);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

int sd_kda_gate_bwd(int N, int H, int r, const void* raw, int64_t raw_row_stride,
                    const float* log_rate, const float* bias, const float* dout, void* draw,
                    float* dlog_rate, float* dbias, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (N <= 0 || H <= 0 || r <= 0) return SD_ERR_SHAPE;
  if (!raw || !log_rate || !bias || !dout || !draw || !dlog_rate || !dbias || !workspace)
    return SD_ERR_ARG;
  if (workspace_bytes < sd_kda_gate_workspace_bytes(N, H, r)) return SD_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const int np = cdiv(N, GATE_TR);
  SD_LAUNCH("k_gate_bwd", k_gate_bwd, dim3(cdiv(H * r, NTHREADS), np), dim3(NTHREADS), 0, st, N,
            H, r, (const __bf16*)raw, raw_row_stride, log_rate, bias, dout, (__bf16*)draw,
            (float*)workspace);
  // column sums over the partial rows spread over many workgroups (a per-head
  // walk over every partial row kept only H workgroups busy), then per head
  float* colsum = (float*)workspace + (size_t)np * 2 * H * r;
  SD_LAUNCH("k_sum_parts", k_sum_parts, dim3(cdiv(2 * H * r, 32)), dim3(NTHREADS), 0, st,
            (const float*)workspace, np, 2 * H * r, colsum);
  SD_LAUNCH("k_gate_reduce", k_gate_reduce, dim3(H), dim3(NTHREADS), 0, st, H, r, 1,
            (const float*)colsum, dbias, dlog_rate);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

size_t sd_rmsnorm_gated_workspace_bytes(int N, int D) {
  if (N <= 0 || D <= 0) return 0;
  return (size_t)cdiv(N, RMS_PART) * D * sizeof(float);
}

int sd_rmsnorm_gated_fwd(int N, int D, float eps, const void* x, const void* gate,
                         const float* weight, void* y, float* rstd, void* stream) {
  if (N <= 0 || D <= 0 || D > 256) return SD_ERR_SHAPE;
  if (!x || !gate || !weight || !y) return SD_ERR_ARG;
  SD_LAUNCH("k_rms_fwd", k_rms_fwd, dim3(cdiv(N, RMS_ROWS)), dim3(RMS_ROWS * 64), 0,
            (hipStream_t)stream, N, D, eps, (const __bf16*)x, (const __bf16*)gate, weight,
            (__bf16*)y, rstd);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

int sd_rmsnorm_gated_bwd(int N, int D, float eps, const void* x, const void* gate,
                         const float* weight, const void* dy, void* dx, void* dgate,
                         float* dweight, void* y, void* workspace, size_t workspace_bytes,
                         void* stream) {
  if (N <= 0 || D <= 0 || D > 256) return SD_ERR_SHAPE;
  if (!x || !gate || !weight || !dy || !dx || !dgate || !dweight || !workspace) return SD_ERR_ARG;
  if (workspace_bytes < sd_rmsnorm_gated_workspace_bytes(N, D)) return SD_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const int np = cdiv(N, RMS_PART);
  SD_LAUNCH("k_rms_bwd", k_rms_bwd, dim3(np), dim3(RMS_ROWS * 64), 0, st, N, D, eps,
            (const __bf16*)x, (const __bf16*)gate, weight, (const __bf16*)dy, (__bf16*)dx,
            (__bf16*)dgate, (__bf16*)y, (float*)workspace);
  SD_LAUNCH("k_sum_parts", k_sum_parts, dim3(cdiv(D, 32)), dim3(NTHREADS), 0, st,
            (const float*)workspace, np, D, dweight);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

}  // extern "C"
