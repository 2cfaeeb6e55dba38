// Wide-width path of the SolveDelta recurrence: key widths 128 < r <= 256 and
// value widths up to 256 (gfx950).
//
// The reference runs its state pass for head widths up to 256
// (causallsso/ops/residual_frame/common_left_h.py:139-151).  The main kernels
// hold a 64-token chunk's 128-wide panels in LDS; at 256 they would not fit, so
// this path states the same chunked algebra (the generic pre-decay-read delta
// op restated in tests/chunk_model.py) with 32-token chunks, runtime padded
// widths KP, VP (multiples of 32, <= 256), FP32 token panels and a 16-bit
// matrix-core state pass (its panels and the chunk states in fp16 / bf16):
//
//   k_w_tokens  (chunk-parallel)  in-chunk log-decay prefix G, L2 norms, gamma;
//   per op (predictor C: X = C^T, erase read before the token's decay, row
//   output; memory S: erase read after it, column output):
//     k_w_prep    decayed Gram L, (I+L)^-1, WY panels W, U, decayed keys,
//                 readout pair P (column output);
//     k_w_state   sequential chunk pass over one 32-column state tile;
//     k_w_out     chunk readout (row output also forms d = k^ + C^T k^);
//   k_w_sources (per token)  dual sources e, chi and gated values z;
// and backward, per op in reverse order:
//     k_w_bprep   dU = A^T (dW + pair^T dO), W' = -A^T K^, K' = -x~, injection;
//     k_w_state   reverse cotangent pass (lambda, dw);
//     k_w_grad    closed-form chunk gradients dk, dx, dq and the decay closure;
//   k_w_src_bwd, k_w_final (per token)  source and norm closures.
//
// Every decay factor is exp(a - b) with a <= b prefix sums inside one chunk (no
// reciprocal decays), formed per element; padding tokens and coordinates are
// zero and stay neutral.
#include <type_traits>

#include "sd_common.cuh"
#include "sd_internal.h"

namespace sd {
namespace wide {

constexpr int WBT = 32;    // chunk length
constexpr int WMAX = 256;  // widest padded width
constexpr int WT = 256;    // threads per workgroup
constexpr int MS = WBT + 1;  // row stride of 32 x 32 LDS matrices

// Chunk-boundary state slots in a 2-byte type, as in the main kernels: the
// forward states X (C^T and S) in fp16, the reverse passes' cotangent states
// lambda in bf16.  The final states handed to the caller stay FP32.
using xs_t = xslot_t;
using ls_t = lslot_t;
__device__ __forceinline__ float4 ld4s(const _Float16* p) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 v = *reinterpret_cast<const h4*>(p);
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}
__device__ __forceinline__ float4 ld4s(const __bf16* p) {
  typedef __bf16 b4 __attribute__((ext_vector_type(4)));
  const b4 v = *reinterpret_cast<const b4*>(p);
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

// Workgroup ids are dealt round-robin over the 8 XCDs (each with its own L2).
// Maps a linear id over (inner, outer) = (L % inner, L / inner) so that, when the
// outer count is a multiple of 8, the inner indices of one outer index run on
// one XCD in consecutive order: the state pass's column tiles of a sequence
// share its L2 copy of the chunk panels, and the chunk gradients of neighbouring
// chunks share the state slot between them.
__device__ __forceinline__ void xcd_map(int L, int inner, int outer, int& in, int& out) {
  if (outer % 8 == 0) {
    const int x = L % 8, j = L / 8;
    in = j % inner;
    out = (j / inner) * 8 + x;
  } else {
    in = L % inner;
    out = L / inner;
  }
}

__device__ __forceinline__ const __bf16* wrow(const sd_view& v, int b, int t, int h) {
  return (const __bf16*)v.data + (long long)b * v.sb + (long long)t * v.st + (long long)h * v.sh;
}
__device__ __forceinline__ float wgamma(const sd_view& g, int b, int t, int h) {
  return ((const float*)g.data)[(long long)b * g.sb + (long long)t * g.st + (long long)h * g.sh];
}

// ---------------------------------------------------------------------------
// Token preparation: G prefix, norms, gamma-scaled predictor operands.
// ---------------------------------------------------------------------------
struct TokParams {
  sd_inputs in;
  int NT, Tp, KP;
  float *G, *uh, *kh, *qh, *xC, *vC, *gam, *rs;
};

// Loads here are unconditional (indices clamped into the row, invalid values
// masked afterwards by a select): a load under a branch waits for every load
// issued before it, so guarded loads would run one round trip at a time.
__global__ __launch_bounds__(WT) void k_w_tokens(TokParams p) {
  const int ch = blockIdx.x, s = blockIdx.y;
  const int H = p.in.H, T = p.in.T, r = p.in.r, KP = p.KP;
  const int b = s / H, h = s % H, t0 = ch * WBT;
  const long long pb = (long long)s * p.Tp;
  // in-chunk inclusive log-decay prefix, one coordinate per thread: the chunk's
  // 32 values are loaded first, then summed
  const int c = threadIdx.x;
  // token flags (invalid: the log-decay reads 0; reset: the reset value): lane l
  // holds token t0 + l % 32's, read across lanes below (loaded by every lane)
  const int fl = tok_flag_row(p.in, b)[(long long)min(t0 + (int)(threadIdx.x & 31), T - 1) *
                                       tok_flag_st(p.in)];
  if (c < KP) {
    const float* g = (const float*)p.in.log_decay.data + (long long)b * p.in.log_decay.sb +
                     (long long)h * p.in.log_decay.sh + min(c, r - 1);
    float gv[WBT];
#pragma unroll
    for (int i = 0; i < WBT; ++i) gv[i] = g[(long long)min(t0 + i, T - 1) * p.in.log_decay.st];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < WBT; ++i) {
      acc += (t0 + i < T && c < r) ? decay_eff(__builtin_amdgcn_readlane(fl, i), gv[i]) : 0.f;
      p.G[(pb + t0 + i) * KP + c] = acc;
    }
  }
  // per token: norms and the gamma-scaled predictor operands, two tokens per
  // wave at a time with all their loads in flight together
  constexpr int NW = WT / 64, TU = 2;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  static_assert(WBT % (NW * TU) == 0, "tokens per wave");
  for (int i0 = w; i0 < WBT; i0 += NW * TU) {
    float uu[TU][4], kk[TU][4], qq[TU][4], hv[TU][4], gm[TU], ek[TU], om[TU];
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      const int tc = min(t0 + i0 + u * NW, T - 1);
      const unsigned f = tok_flags(p.in, b, tc);
      gm[u] = wgamma(p.in.gamma, b, tc, h);
      ek[u] = erase_keep_f(f);
      om[u] = operand_keep(f);  // an invalid token's q, keys and gamma read 0
      const __bf16* ur = wrow(p.in.u, b, tc, h);
      const __bf16* kr = wrow(p.in.k, b, tc, h);
      const __bf16* qr = wrow(p.in.q, b, tc, h);
      const __bf16* hr = wrow(p.in.h, b, tc, h);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cc = min(l + 64 * j, r - 1);
        uu[u][j] = bf2f(ur[cc]);
        kk[u][j] = bf2f(kr[cc]);
        qq[u][j] = bf2f(qr[cc]);
        hv[u][j] = bf2f(hr[cc]);
      }
    }
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      const int t = t0 + i0 + u * NW;
      const bool tv = t < T;
      const float g1 = tv ? gm[u] * om[u] : 0.f;
      const float gx = tv ? g1 * ek[u] : 0.f;  // erase side: 0 on fresh tokens
      float su = 0.f, sk = 0.f, sq = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = tv && l + 64 * j < r;
        uu[u][j] = ok ? uu[u][j] : 0.f;
        kk[u][j] = ok ? kk[u][j] * om[u] : 0.f;
        qq[u][j] = ok ? qq[u][j] * om[u] : 0.f;
        hv[u][j] = ok ? hv[u][j] : 0.f;
        su += uu[u][j] * uu[u][j];
        sk += kk[u][j] * kk[u][j];
        sq += qq[u][j] * qq[u][j];
      }
      const float ru = rsqrtf(wave_sum(su) + 1e-24f);
      const float rk = rsqrtf(wave_sum(sk) + 1e-24f);
      const float rq = rsqrtf(wave_sum(sq) + 1e-24f);
      const long long row = (pb + t) * KP;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cc = l + 64 * j;
        if (cc < KP) {
          p.uh[row + cc] = uu[u][j] * ru;
          p.kh[row + cc] = kk[u][j] * rk;
          p.qh[row + cc] = qq[u][j] * rq;
          p.xC[row + cc] = gx * uu[u][j] * ru;
          p.vC[row + cc] = g1 * hv[u][j];
        }
      }
      if (l == 0) {
        p.gam[pb + t] = g1;
        p.rs[(pb + t) * 3 + 0] = ru;
        p.rs[(pb + t) * 3 + 1] = rk;
        p.rs[(pb + t) * 3 + 2] = rq;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// One op (state X [kw x vw]) of the chunked recurrence.
// ---------------------------------------------------------------------------
struct OpParams {
  int NT, Tp, kw, vw, excl, colout;
  const float *k, *x, *v, *q, *G;  // k, x, G [Tp][kw]; v [Tp][vw]; q [Tp][kw] (col) / [Tp][vw] (row)
  float *A, *P;                    // [NT][32][32]
  _Float16 *Wneg, *Kt;             // state-pass panels: -W [Tp][kw] (fragment order), K^ transposed per chunk [NT][kw][32]
  float *U, *Qt, *Gam;             // Qt [Tp][kw]; U [Tp][vw] (accumulator order); Gam [NT][kw]
};

// G of the erase read for token i at coordinate c: the prefix before token i
// (predictor) or through it (memory).
__device__ __forceinline__ float gx_at(const float* Gs, int ld, int i, int c, int excl) {
  // branch-free: the read is unconditional (a branch around it would serialise
  // every operand behind its own LDS wait), the first token's value selected away
  const float v = Gs[(excl && i > 0 ? i - 1 : i) * ld + c];
  return excl && i == 0 ? 0.f : v;
}

// Decay factors of the matrix-core Grams and applies are factored per
// coordinate c as exp(Ga_i) * exp(-Gb_j), both prefixes inside the chunk.  That
// is exact up to rounding while the coordinate's decay over the chunk,
// -G_{31,c}, stays at most WILD (exp(WILD) is far inside FP32); "wild"
// coordinates beyond it are left out of the factored product and their terms
// added exactly.
// Accumulator order of a chunk's [32 tokens][C] FP32 panel (U, dU): the 16 x 16
// tile (token block tb, column block cb) is 64 lanes x 4 elements, lane (g, m)
// holding tokens 16 tb + 4 g .. + 3 of column 16 cb + m, as an MFMA writes it.
__device__ __forceinline__ unsigned acc_off(int tb, int cb, int lane, int C) {
  return (unsigned)(((tb * (C >> 4) + cb) * 64 + lane) * 4);
}

constexpr float WILD = 60.f;

// x * e^{g} for a factored decay operand, zero on a wild coordinate.  Both
// sides are evaluated (the operands are loaded unconditionally by the caller;
// a branch around them would serialise every operand behind its own memory
// wait), the exponent clamped so a wild coordinate's factor stays finite
// before the select drops it.
__device__ __forceinline__ float keep_exp(bool keep, float x, float g) {
  const float v = x * __expf(fminf(g, 80.f));
  return keep ? v : 0.f;
}

// v_mfma_f32_16x16x4f32: used with the sum index k = 4 g + e carried by MFMA e
// (e = 0..3) and lane group g = lane / 16, so an accumulator (lane (g, n)
// holding rows 4g..4g+3 of column n) is the B operand of a following product
// as it stands.
__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}


// The chunk's wild coordinates in increasing order (deterministic: wave
// ballots and a prefix over the four waves), from the last row of the in-chunk
// prefix G (row stride ld).  Every thread must call it; returns the count.
__device__ __forceinline__ int wild_list(const float* Gs, int ld, int kw, int* wl, int* cnt) {
  const int c = threadIdx.x, w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const bool f = c < kw && -Gs[(WBT - 1) * ld + c] > WILD;
  const unsigned long long mask = __ballot(f);
  if (l == 0) cnt[w] = __popcll(mask);
  __syncthreads();
  int off = 0;
  for (int v = 0; v < w; ++v) off += cnt[v];
  if (f) wl[off + __popcll(mask & ((1ull << l) - 1ull))] = c;
  const int total = cnt[0] + cnt[1] + cnt[2] + cnt[3];
  __syncthreads();
  return total;
}

// M[i][j] = sum_c A(i, c) B(j, c) exp(Ga(i, c) - Gb(j, c)) for i, j < 32, kept
// where keep(i, j), on FP32 matrix cores: wave w forms the 16 x 16 block
// (w >> 1, w & 1) from fa(i, c) = A e^{Ga} and fb(j, c) = B e^{-Gb} (zero on
// wild coordinates), then adds the wild coordinates' exact terms fx(i, j, c).
template <class FA, class FB, class FX, class KEEP>
__device__ __forceinline__ void gram_mfma(int kw, const int* wl, int nw, FA fa, FB fb, FX fx,
                                          KEEP keep, float* M) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15;
  const int bi = w >> 1, bj = w & 1;
  f4 acc = zero4();
#pragma unroll 4
  for (int kb = 0; kb < kw; kb += 16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = kb + 4 * g + e;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa(bi * 16 + m, c), fb(bj * 16 + m, c), acc, 0, 0, 0);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = bi * 16 + 4 * g + e, j = bj * 16 + m;
    float v = acc[e];
    for (int t = 0; t < nw; ++t) v += fx(i, j, wl[t]);
    M[i * MS + j] = keep(i, j) ? v : 0.f;
  }
}

// Stages NA [32][kw] FP32 token panels (rows from token tb) into LDS panels of
// row stride ld.  Every thread's 16-byte loads of all of them are issued before
// its first LDS write, so the staging costs one memory latency, not one per row.
template <int NA>
__device__ __forceinline__ void stage_panels(const float* const (&src)[NA], float* const (&dst)[NA],
                                             long long tb, int kw, int ld) {
  constexpr int PQ = WBT * WMAX / 4 / WT;  // 16-byte pieces per thread and panel at kw = 256
  const int npc = WBT * kw / 4;
  float4 v[NA][PQ];
#pragma unroll
  for (int q = 0; q < PQ; ++q) {
    const int idx = threadIdx.x + WT * q, i = (idx * 4) / kw, c = (idx * 4) % kw;
    if (idx < npc)
#pragma unroll
      for (int a = 0; a < NA; ++a) v[a][q] = *reinterpret_cast<const float4*>(src[a] + (tb + i) * kw + c);
  }
#pragma unroll
  for (int q = 0; q < PQ; ++q) {
    const int idx = threadIdx.x + WT * q, i = (idx * 4) / kw, c = (idx * 4) % kw;
    if (idx < npc)
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        float* d = dst[a] + i * ld + c;
        d[0] = v[a][q].x;
        d[1] = v[a][q].y;
        d[2] = v[a][q].z;
        d[3] = v[a][q].w;
      }
  }
}

__global__ __launch_bounds__(WT) void k_w_prep(OpParams p) {
  extern __shared__ __align__(16) float sm[];
  const int ch = blockIdx.x, s = blockIdx.y, kw = p.kw, vw = p.vw, ld = kw + 1;
  float* xs = sm;                 // x  [32][kw+1]
  float* ks = xs + WBT * ld;      // k
  float* Gs = ks + WBT * ld;      // G
  float* qs = Gs + WBT * ld;      // q (column output)
  float* Ls = qs + WBT * ld;      // L, then A  [32][33]
  float* Ps = Ls + WBT * MS;      // P
  const long long tb = (long long)s * p.Tp + ch * WBT;
  if (p.colout) {
    const float* const src[4] = {p.x, p.k, p.G, p.q};
    float* const dst[4] = {xs, ks, Gs, qs};
    stage_panels<4>(src, dst, tb, kw, ld);
  } else {
    const float* const src[3] = {p.x, p.k, p.G};
    float* const dst[3] = {xs, ks, Gs};
    stage_panels<3>(src, dst, tb, kw, ld);
  }
  // this lane's values for U = A v (the MFMA B operand: tokens kb * 16 + 4 g + e
  // of column block w + 4 j), loaded before any store of the kernel (a load
  // issued after a store waits for it: one counter retires both)
  const int c = threadIdx.x;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15;
  constexpr int NJ = WMAX / 16 / 4;
  float vb[NJ][2][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int nb = w + 4 * j;
        vb[j][kb][e] = nb * 16 < vw ? p.v[(tb + kb * 16 + 4 * g + e) * vw + nb * 16 + m] : 0.f;
      }
  __syncthreads();
  // L_ij = sum_c x_ic k_jc e^{Gx_ic - G_jc} (j < i); P_ij = sum_c q_ic k_jc e^{G_ic - G_jc} (j <= i)
  int* wl = reinterpret_cast<int*>(Ps + WBT * MS);
  const int nw = wild_list(Gs, ld, kw, wl, wl + WMAX);
  auto wild = [&](int c) { return -Gs[(WBT - 1) * ld + c] > WILD; };
  auto kb = [&](int j, int c) { return keep_exp(!wild(c), ks[j * ld + c], -Gs[j * ld + c]); };
  gram_mfma(
      kw, wl, nw,
      [&](int i, int c) { return xs[i * ld + c] * __expf(gx_at(Gs, ld, i, c, p.excl)); }, kb,
      [&](int i, int j, int c) {
        return xs[i * ld + c] * ks[j * ld + c] * __expf(gx_at(Gs, ld, i, c, p.excl) - Gs[j * ld + c]);
      },
      [](int i, int j) { return j < i; }, Ls);
  if (p.colout)
    gram_mfma(
        kw, wl, nw, [&](int i, int c) { return qs[i * ld + c] * __expf(Gs[i * ld + c]); }, kb,
        [&](int i, int j, int c) {
          return qs[i * ld + c] * ks[j * ld + c] * __expf(Gs[i * ld + c] - Gs[j * ld + c]);
        },
        [](int i, int j) { return j <= i; }, Ps);
  __syncthreads();
  // A = (I + L)^-1, one column per thread: a_i = [i == j] - sum_{m < i} L_im a_m
  float acol[WBT];
  if (threadIdx.x < WBT) {
    const int j = threadIdx.x;
#pragma unroll
    for (int i = 0; i < WBT; ++i) {
      float a = (i == j) ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) a -= Ls[i * MS + m] * acol[m];
      acol[i] = (i < j) ? 0.f : a;
    }
  }
  __syncthreads();
  if (threadIdx.x < WBT) {
#pragma unroll
    for (int i = 0; i < WBT; ++i) Ls[i * MS + threadIdx.x] = acol[i];
  }
  __syncthreads();
  const long long mb = ((long long)s * p.NT + ch) * WBT * WBT;
  for (int idx = threadIdx.x; idx < WBT * WBT; idx += WT) {
    p.A[mb + idx] = Ls[(idx >> 5) * MS + (idx & 31)];
    if (p.colout) p.P[mb + idx] = Ps[(idx >> 5) * MS + (idx & 31)];
  }
  // W = A x~ and U = A v on FP32 matrix cores (the sum index k = 4 g + e carried
  // by MFMA e and lane group g); -W stored fp16 for the state pass
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int nb = w + 4 * j;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      if (nb * 16 < kw) {
        f4 a = zero4();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int k = kb * 16 + 4 * g + e, cc = nb * 16 + m;
            a = mfma4(Ls[(t2 * 16 + m) * MS + k], xs[k * ld + cc] * __expf(gx_at(Gs, ld, k, cc, p.excl)), a);
          }
#pragma unroll
        for (int e = 0; e < 4; ++e) p.Wneg[tb * kw + frag_off(t2 * 16 + 4 * g + e, nb * 16 + m, kw)] = (_Float16)(-a[e]);
      }
      if (nb * 16 < vw) {
        f4 a = zero4();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) a = mfma4(Ls[(t2 * 16 + m) * MS + kb * 16 + 4 * g + e], vb[j][kb][e], a);
        *reinterpret_cast<f4*>(p.U + tb * vw + acc_off(t2, nb, l, vw)) = a;
      }
    }
  }
  // K^, Qt, Gam: one key coordinate per thread (K^ in fp16 for the state pass,
  // transposed per chunk: this thread's 32 tokens contiguous)
  if (c < kw) {
    _Float16* const kt = p.Kt + (((long long)s * p.NT + ch) * kw + c) * WBT;
    f16x8 kv;
    const float gl = Gs[(WBT - 1) * ld + c];
#pragma unroll
    for (int i = 0; i < WBT; ++i) {
      const long long o = (tb + i) * kw + c;
      kv[i & 7] = (_Float16)(ks[i * ld + c] * __expf(gl - Gs[i * ld + c]));
      if ((i & 7) == 7) *reinterpret_cast<f16x8*>(kt + i - 7) = kv;
      if (p.colout) p.Qt[o] = qs[i * ld + c] * __expf(Gs[i * ld + c]);
    }
    p.Gam[((long long)s * p.NT + ch) * kw + c] = __expf(gl);
  }
}

constexpr size_t prep_smem(int kw) {
  return (size_t)(4 * WBT * (kw + 1) + 2 * WBT * MS + WMAX + 4) * sizeof(float);  // + wild list
}

// ---------------------------------------------------------------------------
// Sequential chunk pass over a 32-column tile of X [kw x vw]:
//   slot[ch] = X;  w = U + Wneg X;  X = Gamma X + K^T w (+ At^T Ib)
// forward (chunks ascending; slot NT = final state) or reverse (descending).
// ---------------------------------------------------------------------------
struct WStateParams {
  int NT, Tp, kw, vw, rows, cols, rev;
  const void* Wneg;  // -W [Tp][kw] in fragment order (frag_off; fp16 forward, bf16 reverse)
  const void* Kt;    // K^T per chunk [NT][kw][32] (fp16 forward, bf16 reverse)
  const __bf16* At;  // injection A^T per chunk [NT][kw][32] (reverse only; nullable)
  const float *U, *Gam, *Ib;  // U [Tp][vw] (accumulator order), Ib [Tp][vw]; Gam [NT][kw]
  void* slots;  // xs_t (forward) or ls_t (reverse)
  float* wout;
  const float* init; int init_t;
  float* fin; int fin_t;
};

// Matrix-core form on 16-bit MFMAs (v_mfma_f32_16x16x32_{f16,bf16}), as the
// main kernels' state pass: a workgroup of 8 waves owns a 32-column tile of the
// state, wave w holding the 16-row blocks w and w + 8 of both 16-column halves
// in FP32 accumulators.  Per chunk step:
//   the state X0 is staged into LDS split into high and low 16-bit halves,
//   transposed ([column][row]), as the B operand of w = U + Wneg X0, which
//   waves 0-3 form (one 16-token x 16-column tile each, over all kw rows);
//   w is staged split the same way ([column][token]) as the B operand of
//   X = Gamma X + K^T w (+ At^T Ib, reverse), which every wave forms for its
//   own rows.
// The panels Wneg, K^T and At are stored 16-bit by the prep kernels in the
// order the MFMA operands read them, so each lane's fragment is one 16-byte
// load; they, U, Gamma and Ib are fetched SPF - 1 chunks ahead into a ring of
// registers (Ib as two FP32 elements per thread, staged split through LDS like
// w).  Forward: panels fp16 (W and K are bounded by construction), X
// and w split into fp16 halves (~22 bits).  Reverse: bf16 throughout (its
// exponent range keeps any scale of the cotangent), lambda, dw and Ib split
// into bf16 halves.  Two barriers per step: the next step writes the X0
// staging only after this step's second barrier (its readers, the w tiles,
// are done), and the w staging only after its own first barrier.
constexpr int WRB = WMAX / 16 / 4;   // row blocks per wave (four-wave kernels)
constexpr int SW = 8;                // state-pass waves: two per SIMD
constexpr int ST = SW * 64;
constexpr int SRB = WMAX / 16 / SW;  // state-pass row blocks per wave
constexpr int STILE = 32;            // state columns per workgroup
constexpr int NSUB = STILE / 16;
constexpr int WKS = WMAX / 32;       // K = 32 steps of the w product
constexpr int SPF = 2;               // prefetch ring depth (chunks)
constexpr int XLD = WMAX + 8;        // row stride (16-bit) of the staged X0
constexpr int WLD = WBT + 8;         // row stride (16-bit) of the staged w
constexpr int XRS = STILE + 8;       // row stride (16-bit) of the row-major slot copy
constexpr int WFS = WBT + 4;         // row stride (FP32) of the w tile
constexpr size_t state_smem() {
  return (size_t)(2 * STILE * XLD + 4 * STILE * WLD + WMAX * XRS) * 2 + (size_t)STILE * WFS * 4;
}

template <bool REV> struct WStateT;
template <> struct WStateT<false> {
  using E = _Float16;
  using V8 = f16x8;
  using V4 = f16x4;
  static __device__ __forceinline__ f4 mma(V8 a, V8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct WStateT<true> {
  using E = __bf16;
  using V8 = bf16x8;
  using V4 = bf16x4;
  static __device__ __forceinline__ f4 mma(V8 a, V8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <bool REV>
struct WFrags {
  using V8 = typename WStateT<REV>::V8;
  V8 W[WKS];                      // Wneg rows of token block w & 1
  V8 K[SRB];                      // K^T rows of this wave's row blocks, the chunk's 32 tokens
  bf16x8 A[REV ? SRB : 1];        // At rows (reverse)
  float2 ib;                      // reverse: this thread's two elements of the Ib tile
  f4 U;                           // U tile (C-operand layout)
  float4 G[SRB];                  // Gamma of this wave's rows 16 rb + 4 g .. + 3
};

// Chunk-uniform bases with 32-bit lane offsets throughout: 64-bit per-lane
// addresses for the ~20 fragment loads of a chunk would not fit in registers
// beside the prefetch ring.  Every load is unconditional (indices clamped into
// the panel; a null At replaced by a panel of the same shape): a memory
// operation under a branch gives the two paths different counts of
// operations in flight, and the compiler then waits for all of them (the
// ring's prefetches included) wherever the paths meet.  Waves 4-7 fetch the
// W and U fragments waves 0-3 use, for the same reason.
template <bool REV>
__device__ __forceinline__ void wstate_load(const WStateParams& p, int s, int ch, int c0,
                                            WFrags<REV>& f) {
  using E = typename WStateT<REV>::E;
  using V8 = typename WStateT<REV>::V8;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15, kq = g * 8;
  const int kw = p.kw, vw = p.vw, nrb = kw / 16;
  const long long tb = (long long)s * p.Tp + (long long)ch * WBT;
  const long long cb = ((long long)s * p.NT + ch) * kw;  // chunk base of [kw][32] and [kw] panels
  {
    const int tbk = w & 1, hh = (w >> 1) & 1, nks = kw >> 5;
    const E* Wc = static_cast<const E*>(p.Wneg) + tb * kw;
    // fragment order: a K = 32 step of a 16-token block is 1 KiB, lane-contiguous
    const unsigned wo = (unsigned)(tbk * nks * 512 + l * 8);
#pragma unroll
    for (int ks = 0; ks < WKS; ++ks)
      f.W[ks] = *reinterpret_cast<const V8*>(Wc + wo + min(ks, nks - 1) * 512);
    f.U = *reinterpret_cast<const f4*>(p.U + tb * vw + acc_off(tbk, (c0 >> 4) + hh, l, vw));
  }
  const E* Kc = static_cast<const E*>(p.Kt) + cb * WBT;
  const float* Gc = p.Gam + cb;
#pragma unroll
  for (int q = 0; q < SRB; ++q) {
    const int rb = min(w + SW * q, nrb - 1);
    const unsigned ko = (unsigned)((rb * 16 + m) * WBT + kq);
    f.K[q] = *reinterpret_cast<const V8*>(Kc + ko);
    f.G[q] = *reinterpret_cast<const float4*>(Gc + (unsigned)(rb * 16 + 4 * g));
    if constexpr (REV) {
      const __bf16* Ap = p.At ? p.At : static_cast<const __bf16*>(p.Kt);
      f.A[q] = *reinterpret_cast<const bf16x8*>(Ap + cb * WBT + ko);
    }
  }
  if constexpr (REV) {
    static_assert(WBT * STILE == 2 * ST, "two Ib elements per thread");
    const float* Ip = p.At ? p.Ib : p.U;  // both [Tp][vw]
    const int tok = threadIdx.x / (STILE / 2), col = (threadIdx.x % (STILE / 2)) * 2;
    f.ib = *reinterpret_cast<const float2*>(Ip + tb * vw + c0 + (unsigned)(tok * vw + col));
  }
}

// Four 16-bit values split from an FP32 accumulator fragment, stored as two
// 8-byte pieces (high and low halves).
template <class E, class V4>
__device__ __forceinline__ void wsplit4(E* hi, E* lo, f4 v) {
  V4 h, o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const E a = (E)v[e];
    h[e] = a;
    o[e] = (E)(v[e] - (float)a);
  }
  *reinterpret_cast<V4*>(hi) = h;
  *reinterpret_cast<V4*>(lo) = o;
}

template <bool REV>
__device__ __forceinline__ void wstate_step(const WStateParams& p, int s, int ch, int c0,
                                            const WFrags<REV>& f, f4 (&X)[SRB][NSUB], unsigned char* sm) {
  using T = WStateT<REV>;
  using E = typename T::E;
  using V8 = typename T::V8;
  using V4 = typename T::V4;
  using S = typename std::conditional<REV, ls_t, xs_t>::type;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15, kq = g * 8;
  const int kw = p.kw, vw = p.vw, nrb = kw / 16;
  const long long tb = (long long)s * p.Tp + (long long)ch * WBT;
  E* Xh = reinterpret_cast<E*>(sm);  // X0 [32 columns][XLD], high and low halves
  E* Xl = Xh + STILE * XLD;
  E* wh = Xl + STILE * XLD;          // w [32 columns][WLD]
  E* wl = wh + STILE * WLD;
  E* ih = wl + STILE * WLD;          // reverse: the injection's Ib tile [32 columns][WLD]
  E* il = ih + STILE * WLD;
  E* Xr = il + STILE * WLD;          // X0 row-major [rows][XRS]: the slot, written back below
  float* wf = reinterpret_cast<float*>(Xr + WMAX * XRS);  // w FP32 [32 columns][WFS]
  static_assert(std::is_same<S, E>::value, "the slot holds the staged high half");
  // X0 staged split and transposed for the w product, and row-major for the slot
#pragma unroll
  for (int q = 0; q < SRB; ++q) {
    const int rb = w + SW * q;
    if (rb >= nrb) continue;
#pragma unroll
    for (int h = 0; h < NSUB; ++h) {
      const int col = h * 16 + m, row = rb * 16 + 4 * g;
      wsplit4<E, V4>(Xh + col * XLD + row, Xl + col * XLD + row, X[q][h]);
#pragma unroll
      for (int e = 0; e < 4; ++e) Xr[(row + e) * XRS + col] = (E)X[q][h][e];
    }
  }
  if constexpr (REV) {
    if (p.At) {  // the Ib tile staged split and transposed ([column][token])
      const int tok = threadIdx.x / (STILE / 2), col = (threadIdx.x % (STILE / 2)) * 2;
      const float v2[2] = {f.ib.x, f.ib.y};
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const E hi = (E)v2[j];
        ih[(col + j) * WLD + tok] = hi;
        il[(col + j) * WLD + tok] = (E)(v2[j] - (float)hi);
      }
    }
  }
  __syncthreads();
  {  // slot[ch] = X0: 16 columns of one row per thread, two 16-byte pieces
    static_assert(WMAX * 2 == ST && STILE == 32, "one half row of the slot tile per thread");
    // (rows past kw repeat row kw - 1: same values, and no store under a branch)
    const int row = min(threadIdx.x >> 1, kw - 1), c = (threadIdx.x & 1) * 16;
    typedef E E8 __attribute__((ext_vector_type(8)));
    const E8 v0 = *reinterpret_cast<const E8*>(Xr + row * XRS + c);
    const E8 v1 = *reinterpret_cast<const E8*>(Xr + row * XRS + c + 8);
    S* dst = static_cast<S*>(p.slots) + ((long long)s * (p.NT + 1) + ch) * kw * vw + c0 +
             (unsigned)(row * vw + c);
    *reinterpret_cast<E8*>(dst) = v0;
    *reinterpret_cast<E8*>(dst + 8) = v1;
  }
  // w = U + Wneg X0 (waves 0-3, one 16 x 16 tile each; high and low halves of
  // X0 in two accumulators so the two dependent chains interleave)
  if (w < 4) {
    const int tbk = w & 1, hh = w >> 1;
    f4 a0 = f.U, a1 = zero4();
    const E* bh = Xh + (hh * 16 + m) * XLD + kq;
    const E* bl = Xl + (hh * 16 + m) * XLD + kq;
#pragma unroll
    for (int ks = 0; ks < WKS; ++ks)
      if (ks * 32 < kw) {
        a1 = T::mma(f.W[ks], *reinterpret_cast<const V8*>(bl + ks * 32), a1);
        a0 = T::mma(f.W[ks], *reinterpret_cast<const V8*>(bh + ks * 32), a0);
      }
    f4 wv;
#pragma unroll
    for (int e = 0; e < 4; ++e) wv[e] = a0[e] + a1[e];
    const int col = hh * 16 + m, tok = tbk * 16 + 4 * g;
    wsplit4<E, V4>(wh + col * WLD + tok, wl + col * WLD + tok, wv);
    *reinterpret_cast<f4*>(wf + col * WFS + tok) = wv;
  }
  // X = Gamma X (+ At^T Ib): independent of w, so it overlaps the w tiles
#pragma unroll
  for (int q = 0; q < SRB; ++q) {
    const int rb = w + SW * q;
    if (rb >= nrb) continue;
    const float gv[4] = {f.G[q].x, f.G[q].y, f.G[q].z, f.G[q].w};
#pragma unroll
    for (int h = 0; h < NSUB; ++h) {
#pragma unroll
      for (int e = 0; e < 4; ++e) X[q][h][e] *= gv[e];
      if constexpr (REV) {
        if (p.At) {
          const bf16x8 bh = *reinterpret_cast<const bf16x8*>(ih + (h * 16 + m) * WLD + kq);
          const bf16x8 bl = *reinterpret_cast<const bf16x8*>(il + (h * 16 + m) * WLD + kq);
          X[q][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.A[q], bl, X[q][h], 0, 0, 0);
          X[q][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.A[q], bh, X[q][h], 0, 0, 0);
        }
      }
    }
  }
  __syncthreads();
  {  // w to global memory, two elements per thread
    static_assert(WBT * STILE == 2 * ST, "two w elements per thread");
    const int tok = threadIdx.x / (STILE / 2), col = (threadIdx.x % (STILE / 2)) * 2;
    const float2 v = make_float2(wf[col * WFS + tok], wf[(col + 1) * WFS + tok]);
    *reinterpret_cast<float2*>(p.wout + tb * vw + c0 + (unsigned)(tok * vw + col)) = v;
  }
  // X += K^T w
#pragma unroll
  for (int h = 0; h < NSUB; ++h) {
    const V8 whv = *reinterpret_cast<const V8*>(wh + (h * 16 + m) * WLD + kq);
    const V8 wlv = *reinterpret_cast<const V8*>(wl + (h * 16 + m) * WLD + kq);
#pragma unroll
    for (int q = 0; q < SRB; ++q) {
      const int rb = w + SW * q;
      if (rb >= nrb) continue;
      X[q][h] = T::mma(f.K[q], wlv, X[q][h]);
      X[q][h] = T::mma(f.K[q], whv, X[q][h]);
    }
  }
}

template <bool REV>
__global__ __launch_bounds__(ST) void k_w_state(WStateParams p) {
  extern __shared__ __align__(16) unsigned char wsm[];
  int tile, s;
  xcd_map(blockIdx.x, p.vw / STILE, gridDim.x / (p.vw / STILE), tile, s);
  const int kw = p.kw, c0 = tile * STILE, NT = p.NT;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15;
  const int nrb = kw / 16;
  f4 X[SRB][NSUB];
#pragma unroll
  for (int q = 0; q < SRB; ++q) {
    const int rb = w + SW * q;
#pragma unroll
    for (int h = 0; h < NSUB; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = rb * 16 + 4 * g + e, col = c0 + h * 16 + m;
        float v = 0.f;
        if (rb < nrb && p.init && row < p.rows && col < p.cols)
          v = p.init_t ? p.init[((long long)s * p.cols + col) * p.rows + row]
                       : p.init[((long long)s * p.rows + row) * p.cols + col];
        X[q][h][e] = v;
      }
  }
  auto chunk_of = [&](int it) { return REV ? NT - 1 - it : it; };
  auto clampc = [&](int it) { return chunk_of(it < NT ? it : NT - 1); };
  // Straight-line ring (no breaks; clamped, unconditional prefetches) so the
  // compiler's wait counts only cover the buffer being consumed; the last
  // SPF - 1 or fewer chunks run after the loop.
  WFrags<REV> f[SPF];
#pragma unroll
  for (int j = 0; j < SPF - 1; ++j) wstate_load<REV>(p, s, clampc(j), c0, f[j]);
  int it = 0;
  for (; it + SPF - 1 < NT; it += SPF) {
#pragma unroll
    for (int j = 0; j < SPF; ++j) {
      wstate_load<REV>(p, s, clampc(it + j + SPF - 1), c0, f[(j + SPF - 1) % SPF]);
      wstate_step<REV>(p, s, chunk_of(it + j), c0, f[j], X, wsm);
    }
  }
#pragma unroll
  for (int j = 0; j < SPF - 1; ++j)
    if (it + j < NT) wstate_step<REV>(p, s, chunk_of(it + j), c0, f[j], X, wsm);
  // final state (forward: also slot NT for the backward)
  using S = typename std::conditional<REV, ls_t, xs_t>::type;
#pragma unroll
  for (int q = 0; q < SRB; ++q) {
    const int rb = w + SW * q;
    if (rb >= nrb) continue;
#pragma unroll
    for (int h = 0; h < NSUB; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = rb * 16 + 4 * g + e, col = c0 + h * 16 + m;
        if (!REV)
          static_cast<S*>(p.slots)[((long long)s * (p.NT + 1) + p.NT) * kw * p.vw + (long long)row * p.vw + col] =
              (S)X[q][h][e];
        if (p.fin && row < p.rows && col < p.cols) {
          if (p.fin_t) p.fin[((long long)s * p.cols + col) * p.rows + row] = X[q][h][e];
          else p.fin[((long long)s * p.rows + row) * p.cols + col] = X[q][h][e];
        }
      }
  }
}

struct OutParams {
  int NT, Tp, kw, vw, colout, H, T, V;
  const xs_t* slots;
  const float *w, *Qt, *P, *q, *k, *G, *base;
  float *o, *d;
  __bf16* out;
};

__global__ __launch_bounds__(WT) void k_w_out(OutParams p) {
  extern __shared__ __align__(16) float sm[];
  const int ch = blockIdx.x, s = blockIdx.y, kw = p.kw, vw = p.vw;
  const long long tb = (long long)s * p.Tp + ch * WBT;
  const xs_t* X0 = p.slots + ((long long)s * (p.NT + 1) + ch) * kw * vw;
  if (p.colout) {
    // Column output on matrix cores: o = Q~ X0 + P w.
    //   Q~ X0 on v_mfma_f32_16x16x32_f16: Q~ (|Q~| <= 1) split into fp16 high and
    //   low halves, X0 exact in its fp16 slot; the slot is row-major, so each
    //   32-row block is staged transposed ([column][row]) through LDS, the
    //   next block's loads in flight while the current one is used;
    //   P w (32 tokens) on v_mfma_f32_16x16x4f32 from FP32 P and w.
    // Wave w owns output tiles (token block t2, column block w + 4 j).
    using h8 = f16x8;
    constexpr int QLD = WMAX + 8, XTL = WBT + 8, PLD = WBT + 4, NJ = WMAX / 16 / 4;
    _Float16* Qh = reinterpret_cast<_Float16*>(sm);  // Q~ high / low [32][QLD]
    _Float16* Qo = Qh + WBT * QLD;
    _Float16* Xt = Qo + WBT * QLD;                   // X0 row block, transposed [vw][XTL]
    float* Pl = reinterpret_cast<float*>(Xt + WMAX * XTL);  // P [32][PLD]
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15, kq = g * 8;
    const int nvb = vw / 16;
    // this lane's w values for the P w product: B[k = 4 g + e][n = m] of token block kb
    float wb[NJ][2][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int nb = w + 4 * j;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          wb[j][kb][e] = nb < nvb ? p.w[(tb + kb * 16 + 4 * g + e) * vw + nb * 16 + m] : 0.f;
    }
    // X0 row-block staging: task (column c, 8-row group rg), 8 rows of one column
    constexpr int XQ = WMAX * 4 / WT;  // tasks per thread at vw = 256
    h8 xr[XQ];
    auto fetch = [&](int rb) {
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        const int task = threadIdx.x + WT * q, c = task % vw, rg = task / vw;
        if (task < vw * 4)
#pragma unroll
          for (int j = 0; j < 8; ++j) xr[q][j] = X0[(long long)(rb + rg * 8 + j) * vw + c];
      }
    };
    fetch(0);
    // Q~ split into LDS; P into LDS
    {
      const long long mb = ((long long)s * p.NT + ch) * WBT * WBT;
      for (int idx = threadIdx.x; idx < WBT * WBT; idx += WT) Pl[(idx >> 5) * PLD + (idx & 31)] = p.P[mb + idx];
      constexpr int PQ = WBT * WMAX / 4 / WT;
      float4 qv[PQ];
#pragma unroll
      for (int q = 0; q < PQ; ++q) {
        const int idx = threadIdx.x + WT * q, i = (idx * 4) / kw, c = (idx * 4) % kw;
        if (idx < WBT * kw / 4) qv[q] = *reinterpret_cast<const float4*>(p.Qt + (tb + i) * kw + c);
      }
#pragma unroll
      for (int q = 0; q < PQ; ++q) {
        const int idx = threadIdx.x + WT * q, i = (idx * 4) / kw, c = (idx * 4) % kw;
        if (idx < WBT * kw / 4) {
          f4 v = {qv[q].x, qv[q].y, qv[q].z, qv[q].w};
          f16x4 hi, lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            hi[e] = (_Float16)v[e];
            lo[e] = (_Float16)(v[e] - (float)hi[e]);
          }
          *reinterpret_cast<f16x4*>(Qh + i * QLD + c) = hi;
          *reinterpret_cast<f16x4*>(Qo + i * QLD + c) = lo;
        }
      }
    }
    f4 acc[2][NJ];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[t2][j] = zero4();
    for (int rb = 0; rb < kw; rb += 32) {
      __syncthreads();  // the previous block's readers are done
#pragma unroll
      for (int q = 0; q < XQ; ++q) {
        const int task = threadIdx.x + WT * q, c = task % vw, rg = task / vw;
        if (task < vw * 4) *reinterpret_cast<h8*>(Xt + c * XTL + rg * 8) = xr[q];
      }
      __syncthreads();
      if (rb + 32 < kw) fetch(rb + 32);
      h8 ah[2], al[2];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        ah[t2] = *reinterpret_cast<const h8*>(Qh + (t2 * 16 + m) * QLD + rb + kq);
        al[t2] = *reinterpret_cast<const h8*>(Qo + (t2 * 16 + m) * QLD + rb + kq);
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int nb = w + 4 * j;
        if (nb >= nvb) continue;
        const h8 bx = *reinterpret_cast<const h8*>(Xt + (nb * 16 + m) * XTL + kq);
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          acc[t2][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t2], bx, acc[t2][j], 0, 0, 0);
          acc[t2][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[t2], bx, acc[t2][j], 0, 0, 0);
        }
      }
    }
    // + P w, then the bf16 output
    const int b = s / p.H, h = s % p.H;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int nb = w + 4 * j;
      if (nb >= nvb) continue;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const float4 a4 = *reinterpret_cast<const float4*>(Pl + (t2 * 16 + m) * PLD + kb * 16 + 4 * g);
          acc[t2][j] = mfma4(a4.x, wb[j][kb][0], acc[t2][j]);
          acc[t2][j] = mfma4(a4.y, wb[j][kb][1], acc[t2][j]);
          acc[t2][j] = mfma4(a4.z, wb[j][kb][2], acc[t2][j]);
          acc[t2][j] = mfma4(a4.w, wb[j][kb][3], acc[t2][j]);
        }
        const int c = nb * 16 + m;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = ch * WBT + t2 * 16 + 4 * g + e;
          if (t < p.T && c < p.V) p.out[(((long long)b * p.T + t) * p.H + h) * p.V + c] = f2bf(acc[t2][j][e]);
        }
      }
    }
    return;
  }
  // row output on matrix cores: M = q w^T (j <= i), then
  //   o_ir = e^{G_ir} ((q X0^T)_ir + (M k~)_ir),  k~_jr = k_jr e^{-G_jr}
  // with the decay factored per state row r (wild rows: exact per-term sum).
  // q X0^T runs on v_mfma_f32_16x16x32_f16: q (unit rows) split into fp16 high
  // and low halves in LDS, X0 exact in its fp16 slot (the contraction runs
  // along the slot's rows, so each lane's fragment is one 16-byte load).
  constexpr int QLD = WMAX + 8;
  float* Ml = sm;  // [32][33]
  _Float16* Qh = reinterpret_cast<_Float16*>(Ml + WBT * MS);  // q high / low [32][QLD]
  _Float16* Qo = Qh + WBT * QLD;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15, kq = g * 8;
  {
    constexpr int PQ = WBT * WMAX / 4 / WT;
    float4 qv[PQ];
#pragma unroll
    for (int q = 0; q < PQ; ++q) {
      const int idx = threadIdx.x + WT * q, i = (idx * 4) / vw, c = (idx * 4) % vw;
      if (idx < WBT * vw / 4) qv[q] = *reinterpret_cast<const float4*>(p.q + (tb + i) * vw + c);
    }
#pragma unroll
    for (int q = 0; q < PQ; ++q) {
      const int idx = threadIdx.x + WT * q, i = (idx * 4) / vw, c = (idx * 4) % vw;
      if (idx < WBT * vw / 4) {
        f4 v = {qv[q].x, qv[q].y, qv[q].z, qv[q].w};
        f16x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hi[e] = (_Float16)v[e];
          lo[e] = (_Float16)(v[e] - (float)hi[e]);
        }
        *reinterpret_cast<f16x4*>(Qh + i * QLD + c) = hi;
        *reinterpret_cast<f16x4*>(Qo + i * QLD + c) = lo;
      }
    }
  }
  {
    const int bi = w >> 1, bj = w & 1;
    f4 acc = zero4();
    for (int cb = 0; cb < vw; cb += 16) {
      const float4 a4 = *reinterpret_cast<const float4*>(p.q + (tb + bi * 16 + m) * vw + cb + 4 * g);
      const float4 b4 = *reinterpret_cast<const float4*>(p.w + (tb + bj * 16 + m) * vw + cb + 4 * g);
      acc = mfma4(a4.x, b4.x, acc);
      acc = mfma4(a4.y, b4.y, acc);
      acc = mfma4(a4.z, b4.z, acc);
      acc = mfma4(a4.w, b4.w, acc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = bi * 16 + 4 * g + e, j = bj * 16 + m;
      Ml[i * MS + j] = j <= i ? acc[e] : 0.f;
    }
  }
  __syncthreads();
  const int nrb = kw / 16;
  float ro[WRB][2][4], rbase[WRB][2][4];
#pragma unroll
  for (int q = 0; q < WRB; ++q) {
    const int rb = w + 4 * q;
    if (rb >= nrb) continue;
    const int rr = rb * 16 + m;
    const bool wild = -p.G[(tb + WBT - 1) * kw + rr] > WILD;
    f4 acc[2] = {zero4(), zero4()};
#pragma unroll 4
    for (int cb = 0; cb < vw; cb += 32) {
      const f16x8 bx = *reinterpret_cast<const f16x8*>(X0 + (long long)rr * vw + cb + kq);
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const f16x8 ah = *reinterpret_cast<const f16x8*>(Qh + (t2 * 16 + m) * QLD + cb + kq);
        const f16x8 al = *reinterpret_cast<const f16x8*>(Qo + (t2 * 16 + m) * QLD + cb + kq);
        acc[t2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bx, acc[t2], 0, 0, 0);
        acc[t2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bx, acc[t2], 0, 0, 0);
      }
    }
    float kt[2][4];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const long long o = (tb + jb * 16 + 4 * g + e) * kw + rr;
        kt[jb][e] = keep_exp(!wild, p.k[o], -p.G[o]);
      }
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      f4 a = acc[t2];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 4; ++e) a = mfma4(Ml[(t2 * 16 + m) * MS + jb * 16 + 4 * g + e], kt[jb][e], a);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = t2 * 16 + 4 * g + e;
        const long long o = (tb + i) * kw + rr;
        const float gi = p.G[o];
        float v = __expf(gi) * a[e];
        if (wild)
          for (int j = 0; j <= i; ++j)
            v += Ml[i * MS + j] * p.k[(tb + j) * kw + rr] * __expf(gi - p.G[(tb + j) * kw + rr]);
        ro[q][t2][e] = v;
        rbase[q][t2][e] = p.base[o];
      }
    }
  }
  // stores after every row block's loads (a load issued after a store waits for it)
#pragma unroll
  for (int q = 0; q < WRB; ++q) {
    const int rb = w + 4 * q;
    if (rb >= nrb) continue;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const long long o = (tb + t2 * 16 + 4 * g + e) * kw + rb * 16 + m;
        p.o[o] = ro[q][t2][e];
        p.d[o] = rbase[q][t2][e] + ro[q][t2][e];
      }
  }
}

constexpr size_t out_smem(int kw, int vw, int colout) {
  // column output: Q~ high / low [32][WMAX+8] and X0 block [WMAX][40] fp16, P [32][36]
  if (colout) return (size_t)(2 * WBT * (WMAX + 8) + WMAX * (WBT + 8)) * 2 + WBT * (WBT + 4) * sizeof(float);
  return (size_t)(WBT * MS) * sizeof(float) + (size_t)2 * WBT * (WMAX + 8) * 2;  // M; q high / low
}

// ---------------------------------------------------------------------------
// Dual sources (per token): phi, den, e, chi, z.
// ---------------------------------------------------------------------------
struct SrcParams {
  sd_inputs in;
  int Tp, KP, VP;
  const float *uh, *delta, *kh, *qh;
  float *e, *chi, *z;
};

__global__ __launch_bounds__(WT) void k_w_sources(SrcParams p) {
  const int s = blockIdx.y, H = p.in.H, T = p.in.T, r = p.in.r, V = p.in.V;
  const int b = s / H, h = s % H;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int t = blockIdx.x * (WT / 64) + w;
  if (t >= p.Tp) return;
  const bool tv = t < T;
  const long long row = ((long long)s * p.Tp + t) * p.KP, vrow_ = ((long long)s * p.Tp + t) * p.VP;
  // every load first, at clamped indices (masked below): no load under a branch
  const int tc = min(t, T - 1);
  const __bf16 *err = wrow(p.in.erase_raw, b, tc, h), *vr = wrow(p.in.v, b, tc, h),
               *wrr = wrow(p.in.write_raw, b, tc, h);
  float u[4], dl[4], k[4], q[4], er[4], vv[4], wr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j, ck = min(c, p.KP - 1);
    u[j] = p.uh[row + ck];
    dl[j] = p.delta[row + ck];
    k[j] = p.kh[row + ck];
    q[j] = p.qh[row + ck];
    er[j] = bf2f(err[min(c, r - 1)]);
    vv[j] = bf2f(vr[min(c, V - 1)]);
    wr[j] = bf2f(wrr[min(c, V - 1)]);
  }
  float usq = 0.f, dsq = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j;
    const bool in = c < p.KP;
    u[j] = in ? u[j] : 0.f;
    dl[j] = in ? dl[j] : 0.f;
    k[j] = in ? k[j] : 0.f;
    q[j] = in ? q[j] : 0.f;
    er[j] = (tv && c < r) ? er[j] : 0.f;
    usq += u[j] * u[j];
    dsq += dl[j] * dl[j];
  }
  usq = wave_sum(usq);
  dsq = wave_sum(dsq);
  const float sc = RHO / sqrtf(RHO * RHO + usq * dsq);
  float phi[4], bb[4];
  float pu = 0.f, ub = 0.f, uq = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    phi[j] = sc * dl[j];
    bb[j] = k[j] / (1.f + __expf(-er[j]));
    pu += phi[j] * u[j];
    ub += u[j] * bb[j];
    uq += u[j] * q[j];
  }
  const float den = 1.f + wave_sum(pu);
  const float sb = wave_sum(ub) / den, sq = wave_sum(uq) / den;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j;
    if (c < p.KP) {
      p.e[row + c] = bb[j] - phi[j] * sb;
      p.chi[row + c] = q[j] - phi[j] * sq;
    }
    if (c < p.VP) {
      const bool ok = tv && c < V;
      p.z[vrow_ + c] = ok ? vv[j] / (1.f + __expf(-wr[j])) : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward preparation of one op's reverse pass.
//   column output: rhs = dW + P^T dO, injection Ia = q e^G, Ib = dO
//   row output:    Pp_ij = sum_r dO_ir k_jr e^{G_ir - G_jr} (j <= i), rhs = dW + Pp^T q,
//                  Ia = dO e^G, Ib = q
//   dU = A^T rhs,  Wn = -A^T Kh,  Kn = -x~  (Wn, Kn, Ia stored bf16 for the
//   reverse pass: -Wn token-major, Kn and Ia transposed per chunk)
// ---------------------------------------------------------------------------
struct BprepParams {
  int NT, Tp, kw, vw, excl, colout;
  const float *k, *x, *q, *G, *A, *P, *dO, *dW;
  float *dU, *Pp;  // dU [Tp][vw] in accumulator order (acc_off)
  __bf16 *Wneg, *Kt, *At;  // reverse-pass panels: -Wn [Tp][kw] (fragment order); Kn, Ia transposed per chunk [NT][kw][32]
};

__global__ __launch_bounds__(WT) void k_w_bprep(BprepParams p) {
  extern __shared__ __align__(16) float sm[];
  const int ch = blockIdx.x, s = blockIdx.y, kw = p.kw, vw = p.vw, ld = kw + 1;
  const long long tb = (long long)s * p.Tp + ch * WBT;
  const long long mb = ((long long)s * p.NT + ch) * WBT * WBT;
  float* Al = sm;              // A [32][33]
  float* Pl = Al + WBT * MS;   // P or Pp [32][33]
  float* dOl = Pl + WBT * MS;  // row output: dO, k, G [32][kw+1]
  float* kl = dOl + WBT * ld;
  float* Gl = kl + WBT * ld;
  // column vectors [32][256] (element i of column t at i*256+t), over the
  // row-output panels once the Pp Gram is done with them
  float* cv = dOl;
  const int tid = threadIdx.x;
  for (int idx = threadIdx.x; idx < WBT * WBT; idx += WT) {
    Al[(idx >> 5) * MS + (idx & 31)] = p.A[mb + idx];
    if (p.colout) Pl[(idx >> 5) * MS + (idx & 31)] = p.P[mb + idx];
  }
  if (!p.colout) {
    {
      const float* const src[3] = {p.dO, p.k, p.G};
      float* const dst[3] = {dOl, kl, Gl};
      stage_panels<3>(src, dst, tb, kw, ld);
    }
    __syncthreads();
    int* wl = reinterpret_cast<int*>(Gl + WBT * ld);
    const int nw = wild_list(Gl, ld, kw, wl, wl + WMAX);
    gram_mfma(
        kw, wl, nw, [&](int i, int c) { return dOl[i * ld + c] * __expf(Gl[i * ld + c]); },
        [&](int j, int c) {
          return keep_exp(-Gl[(WBT - 1) * ld + c] <= WILD, kl[j * ld + c], -Gl[j * ld + c]);
        },
        [&](int i, int j, int c) {
          return dOl[i * ld + c] * kl[j * ld + c] * __expf(Gl[i * ld + c] - Gl[j * ld + c]);
        },
        [](int i, int j) { return j <= i; }, Pl);
    __syncthreads();
    for (int idx = threadIdx.x; idx < WBT * WBT; idx += WT)
      p.Pp[mb + idx] = Pl[(idx >> 5) * MS + (idx & 31)];
  }
  __syncthreads();
  // The key side's inputs are loaded first, before any store of the value
  // side: a load issued after a store waits for it (one counter retires both).
  const int c = threadIdx.x;
  float kg[WBT], kk[WBT], kx[WBT], ks2[WBT];
  if (c < kw)
#pragma unroll
    for (int i = 0; i < WBT; ++i) {
      const long long o = (tb + i) * kw + c;
      kg[i] = p.G[o];
      kk[i] = p.k[o];
      kx[i] = p.x[o];
      ks2[i] = p.colout ? p.q[o] : p.dO[o];
    }
  // value side: rhs = dW + P^T Y and dU = A^T rhs on FP32 matrix cores (the sum
  // index k = 4 g + e carried by MFMA e and lane group g, so the rhs
  // accumulators are the B operands of the dU product as they stand); Y's
  // columns are staged in LDS by one thread per value column
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, m = l & 15;
  constexpr int NJ = WMAX / 16 / 4;  // column blocks per wave
  if (c < vw)
    for (int i = 0; i < WBT; ++i)
      cv[i * WT + tid] = p.colout ? p.dO[(tb + i) * vw + c] : p.q[(tb + i) * vw + c];
  f4 rhs[2][NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int nb = w + 4 * j;
        rhs[t2][j][e] = (p.dW && nb * 16 < vw) ? p.dW[(tb + t2 * 16 + 4 * g + e) * vw + nb * 16 + m] : 0.f;
      }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int nb = w + 4 * j;
    if (nb * 16 >= vw) continue;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rhs[t2][j] = mfma4(Pl[(kb * 16 + 4 * g + e) * MS + t2 * 16 + m],
                             cv[(kb * 16 + 4 * g + e) * WT + nb * 16 + m], rhs[t2][j]);
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      f4 du = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          du = mfma4(Al[(kb * 16 + 4 * g + e) * MS + t2 * 16 + m], rhs[kb][j][e], du);
      *reinterpret_cast<f4*>(p.dU + tb * vw + acc_off(t2, nb, l, vw)) = du;
    }
  }
  __syncthreads();  // cv is reused for the decayed keys
  // key side: Kn, Ia (transposed per chunk, one key coordinate per thread) and
  // the decayed keys' columns for Wn = -A^T K^ (matrix cores, as dU)
  if (c < kw) {
    const float gl = kg[WBT - 1];
    const long long cb = (((long long)s * p.NT + ch) * kw + c) * WBT;
    bf16x8 kv, av;
#pragma unroll
    for (int i = 0; i < WBT; ++i) {
      const float gi = kg[i];
      cv[i * WT + tid] = kk[i] * __expf(gl - gi);
      const float gx = p.excl ? (i > 0 ? kg[i - 1] : 0.f) : gi;
      kv[i & 7] = (__bf16)(-kx[i] * __expf(gx));
      av[i & 7] = (__bf16)(ks2[i] * __expf(gi));
      if ((i & 7) == 7) {
        *reinterpret_cast<bf16x8*>(p.Kt + cb + i - 7) = kv;
        *reinterpret_cast<bf16x8*>(p.At + cb + i - 7) = av;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int nb = w + 4 * j;
    if (nb * 16 >= kw) continue;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      f4 a = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          a = mfma4(Al[(kb * 16 + 4 * g + e) * MS + t2 * 16 + m],
                    cv[(kb * 16 + 4 * g + e) * WT + nb * 16 + m], a);
#pragma unroll
      for (int e = 0; e < 4; ++e) p.Wneg[tb * kw + frag_off(t2 * 16 + 4 * g + e, nb * 16 + m, kw)] = (__bf16)a[e];
    }
  }
}

constexpr size_t bprep_smem(int kw) {
  const size_t panels = 3 * WBT * (size_t)(kw + 1) + WMAX + 4, cols = (size_t)WBT * WT;
  return (2 * WBT * MS + (panels > cols ? panels : cols)) * sizeof(float);
}

// ---------------------------------------------------------------------------
// Closed-form chunk gradients of one op (tests/chunk_model.py Op.backward):
//   M1_ij = dw_i.w_j (j < i);  M2_lj = Y_l.w_j (j <= l), Y = dO (column) / q (row)
//   dx = -(e^{Gx} (dw X0^T) + apply(M1, k, Gx, G))
//   dk = e^{G_C - G} (w lam^T) + apply_t(M2, Yk, G, G) - apply_t(M1, x, Gx, G)
//        with Yk = q (column) / dO (row)
//   dq = e^{G} (dO X0^T) + apply(M2, k, G, G)          (column)
//   dq = (dO e^G) X0 + Pp w                             (row)
//   dG = q dq - k dk (column) / o dO - k dk (row), + x dx (shifted one token
//   earlier when the erase reads before the decay), last row + rowsum(X_C lam);
//   dg = in-chunk reverse cumulative sum of dG.
// ---------------------------------------------------------------------------
struct GradParams {
  int NT, Tp, kw, vw, excl, colout;
  const float *k, *x, *q, *G, *dO, *o, *w, *dw, *Pp;
  const xs_t* Xslots;
  const ls_t* Lslots;
  float *dk, *dx, *dq, *dg;
};

// Eight waves (two per SIMD, so one wave's loads overlap another's matrix
// work), each owning the 16-row blocks rb = wave + 8 q of the state.
constexpr int GW = 8;
constexpr int GT = GW * 64;
constexpr int GRB = WMAX / 16 / GW;

__global__ __launch_bounds__(GT) void k_w_grad(GradParams p) {
  extern __shared__ __align__(16) float sm[];
  int ch, s;
  xcd_map(blockIdx.x, p.NT, gridDim.x / p.NT, ch, s);
  const int kw = p.kw, vw = p.vw;
  const long long tb = (long long)s * p.Tp + ch * WBT;
  const long long slot = (long long)s * (p.NT + 1) + ch;
  const xs_t* X0 = p.Xslots + slot * kw * vw;
  const xs_t* XC = X0 + (long long)kw * vw;
  const ls_t* Lm = p.Lslots + slot * kw * vw;
  // LDS: the token Grams M1, M2 [32][33]; the rows dw, w, Y [3][32][vw+4]
  // (first pass), then for the row output dO e^G [32][kw+4]
  float* M1 = sm;
  float* M2 = M1 + WBT * MS;
  float* TR = M2 + WBT * MS;
  float* DG = TR;
  const int r = threadIdx.x;
  const int wv_ = r >> 6, l = r & 63, g = l >> 4, m = l & 15;
  const int nrb = kw / 16, nvb = vw / 16;
  const float* Y = p.colout ? p.dO : p.q;  // [Tp][vw]
  // phase 1 on matrix cores: the row products dwX = dw X0^T, wL = w lam^T, dOX = dO X0^T
  // (column output) over this wave's 16-row blocks of the state, kept in
  // accumulators (lane (g, n): tokens 4g..4g+3 of state row 16 rb + n) for
  // phase 3, and the token Grams M1 = dw w^T, M2 = Y w^T (one 16 x 16 block of
  // each per wave of the first four); the rows from LDS, the state slots by
  // 16-byte global loads.
  f4 aX[GRB][2], aL[GRB][2], aO[GRB][2];
  float rs[GRB];  // partial rowsum(X_C (.) lam) of state row 16 rb + m over this lane's columns
#pragma unroll
  for (int q = 0; q < GRB; ++q) {
    rs[q] = 0.f;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) aX[q][t2] = aL[q][t2] = aO[q][t2] = zero4();
  }
  // the chunk's dw, w, Y rows staged once into LDS (every wave reads all of them)
  const int lt = vw + 4;
#pragma unroll
  for (int q = 0; q < WBT * WMAX / 4 / GT; ++q) {
    const int idx = threadIdx.x + GT * q, i = (idx * 4) / vw, c = (idx * 4) % vw;
    if (idx < WBT * vw / 4) {
      const long long o = (tb + i) * vw + c;
      const float4 a0 = *reinterpret_cast<const float4*>(p.dw + o);
      const float4 a1 = *reinterpret_cast<const float4*>(p.w + o);
      const float4 a2 = *reinterpret_cast<const float4*>(Y + o);
      *reinterpret_cast<float4*>(TR + i * lt + c) = a0;
      *reinterpret_cast<float4*>(TR + (WBT + i) * lt + c) = a1;
      *reinterpret_cast<float4*>(TR + (2 * WBT + i) * lt + c) = a2;
    }
  }
  __syncthreads();
  {
    f4 m1a = zero4(), m2a = zero4();
    const int bi = (wv_ >> 1) & 1, bj = wv_ & 1;
    const bool gram = wv_ < 4;  // one 16 x 16 block of M1 and M2 per wave of the first four
    const int kq = g * 8;
    // 16-bit matrix cores over K = 32 columns per step (bf16: the cotangents
    // may take any scale).  The FP32 rows dw, w, Y and the fp16 state X0 enter
    // split into bf16 high and low halves (three MFMAs per product: hi.hi,
    // hi.lo, lo.hi); lambda is exact in its bf16 slot (two MFMAs).
    auto split8 = [](const float* v, bf16x8& hi, bf16x8& lo) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const __bf16 h = (__bf16)v[j];
        hi[j] = h;
        lo[j] = (__bf16)(v[j] - (float)h);
      }
    };
    auto mma = [](bf16x8 a, bf16x8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); };
#pragma unroll 2
    for (int cb = 0; cb < vw; cb += 32) {
      bf16x8 dwh[2], dwl[2], wh[2], wl[2], yh[2], yl[2];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const int o = (t2 * 16 + m) * lt + cb + kq;
        float v[8];
        *reinterpret_cast<float4*>(v) = *reinterpret_cast<const float4*>(TR + o);
        *reinterpret_cast<float4*>(v + 4) = *reinterpret_cast<const float4*>(TR + o + 4);
        split8(v, dwh[t2], dwl[t2]);
        *reinterpret_cast<float4*>(v) = *reinterpret_cast<const float4*>(TR + WBT * lt + o);
        *reinterpret_cast<float4*>(v + 4) = *reinterpret_cast<const float4*>(TR + WBT * lt + o + 4);
        split8(v, wh[t2], wl[t2]);
        *reinterpret_cast<float4*>(v) = *reinterpret_cast<const float4*>(TR + 2 * WBT * lt + o);
        *reinterpret_cast<float4*>(v + 4) = *reinterpret_cast<const float4*>(TR + 2 * WBT * lt + o + 4);
        split8(v, yh[t2], yl[t2]);
      }
#pragma unroll
      for (int q = 0; q < GRB; ++q) {
        const int rb = wv_ + GW * q;
        if (rb < nrb) {
          const long long o = (long long)(rb * 16 + m) * vw + cb + kq;
          const f16x8 x8 = *reinterpret_cast<const f16x8*>(X0 + o);
          const f16x8 c8 = *reinterpret_cast<const f16x8*>(XC + o);
          const bf16x8 lb = *reinterpret_cast<const bf16x8*>(Lm + o);
          float xv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            xv[j] = (float)x8[j];
            rs[q] += (float)c8[j] * (float)lb[j];
          }
          bf16x8 xh, xl;
          split8(xv, xh, xl);
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2) {
            aX[q][t2] = mma(dwl[t2], xh, aX[q][t2]);
            aX[q][t2] = mma(dwh[t2], xl, aX[q][t2]);
            aX[q][t2] = mma(dwh[t2], xh, aX[q][t2]);
            aL[q][t2] = mma(wl[t2], lb, aL[q][t2]);
            aL[q][t2] = mma(wh[t2], lb, aL[q][t2]);
            if (p.colout) {
              aO[q][t2] = mma(yl[t2], xh, aO[q][t2]);
              aO[q][t2] = mma(yh[t2], xl, aO[q][t2]);
              aO[q][t2] = mma(yh[t2], xh, aO[q][t2]);
            }
          }
        }
      }
      if (gram) {  // selects, not indexing: a runtime index would put the arrays in scratch
        const bf16x8 dah = bi ? dwh[1] : dwh[0], dal = bi ? dwl[1] : dwl[0];
        const bf16x8 yah = bi ? yh[1] : yh[0], yal = bi ? yl[1] : yl[0];
        const bf16x8 wbh = bj ? wh[1] : wh[0], wbl = bj ? wl[1] : wl[0];
        m1a = mma(dal, wbh, m1a);
        m1a = mma(dah, wbl, m1a);
        m1a = mma(dah, wbh, m1a);
        m2a = mma(yal, wbh, m2a);
        m2a = mma(yah, wbl, m2a);
        m2a = mma(yah, wbh, m2a);
      }
    }
    if (gram)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = bi * 16 + 4 * g + e, j = bj * 16 + m;
        M1[i * MS + j] = j < i ? m1a[e] : 0.f;
        M2[i * MS + j] = j <= i ? m2a[e] : 0.f;
      }
  }
  // rowsum(X_C (.) lam): the four lane groups' partials of each state row
  // (every lane of the row ends with the total)
#pragma unroll
  for (int q = 0; q < GRB; ++q) {
    rs[q] += __shfl_xor(rs[q], 16);
    rs[q] += __shfl_xor(rs[q], 32);
  }
  // phase 2 (row output): dq = (dO e^G) X0 + Pp w on matrix cores, this wave's
  // 16-column blocks of the value axis; dO e^G is formed once into LDS
  if (!p.colout) {
    const long long mb = ((long long)s * p.NT + ch) * WBT * WBT;
    const int la = kw + 4;
    __syncthreads();  // every wave is done reading the rows DG overwrites
#pragma unroll
    for (int q = 0; q < WBT * WMAX / 4 / GT; ++q) {
      const int idx = threadIdx.x + GT * q, i = (idx * 4) / kw, c = (idx * 4) % kw;
      if (idx < WBT * kw / 4) {
        const float4 d4 = *reinterpret_cast<const float4*>(p.dO + (tb + i) * kw + c);
        const float4 g4 = *reinterpret_cast<const float4*>(p.G + (tb + i) * kw + c);
        *reinterpret_cast<float4*>(DG + i * la + c) =
            make_float4(d4.x * __expf(g4.x), d4.y * __expf(g4.y), d4.z * __expf(g4.z), d4.w * __expf(g4.w));
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < GRB; ++q) {
      const int nb = wv_ + GW * q;
      if (nb >= nvb) continue;
      f4 acc[2] = {zero4(), zero4()};
#pragma unroll 4
      for (int rb = 0; rb < nrb; ++rb) {
        float bx[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bx[e] = (float)X0[(long long)(rb * 16 + 4 * g + e) * vw + nb * 16 + m];
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const float4 a4 = *reinterpret_cast<const float4*>(DG + (t2 * 16 + m) * la + rb * 16 + 4 * g);
          acc[t2] = mfma4(a4.x, bx[0], acc[t2]);
          acc[t2] = mfma4(a4.y, bx[1], acc[t2]);
          acc[t2] = mfma4(a4.z, bx[2], acc[t2]);
          acc[t2] = mfma4(a4.w, bx[3], acc[t2]);
        }
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float bw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bw[e] = p.w[(tb + kb * 16 + 4 * g + e) * vw + nb * 16 + m];
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const float4 a4 = *reinterpret_cast<const float4*>(p.Pp + mb + (t2 * 16 + m) * WBT + kb * 16 + 4 * g);
          acc[t2] = mfma4(a4.x, bw[0], acc[t2]);
          acc[t2] = mfma4(a4.y, bw[1], acc[t2]);
          acc[t2] = mfma4(a4.z, bw[2], acc[t2]);
          acc[t2] = mfma4(a4.w, bw[3], acc[t2]);
        }
      }
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int e = 0; e < 4; ++e) p.dq[(tb + t2 * 16 + 4 * g + e) * vw + nb * 16 + m] = acc[t2][e];
    }
  }
  __syncthreads();  // M1, M2 complete
  // phase 3: the in-chunk applies on matrix cores, decay factored per state
  // row r as e^{Ga_i} e^{-Gb_j} (exact while r's decay over the chunk is at
  // most WILD; wild rows take the exact per-term sums):
  //   dx = -e^{Gx} (dwX + M1 k~),               k~_jr = k_jr e^{-G_jr}
  //   dk = e^{-G} (e^{G_C} wL + M2^T Y~ - M1^T x~),  Y~ = Yk e^{G}, x~ = x e^{Gx}
  //   dq = e^{G} (dOX + M2 k~)                   (column output)
  const float* Yk = p.colout ? p.q : p.dO;  // [Tp][kw]
  auto gx_g = [&](int i, int rr) {  // branch-free, as gx_at
    const float v = p.G[(tb + (p.excl && i > 0 ? i - 1 : i)) * kw + rr];
    return p.excl && i == 0 ? 0.f : v;
  };
  float rdx[GRB][2][4], rdk[GRB][2][4], rdq[GRB][2][4], rdg[GRB][2][4];
#pragma unroll
  for (int q = 0; q < GRB; ++q) {
    const int rb = wv_ + GW * q;
    if (rb >= nrb) continue;
    const int rr = rb * 16 + m;  // this lane's state row (output column)
    const float gl = p.G[(tb + WBT - 1) * kw + rr];
    const bool wild = -gl > WILD;
    // the lane's operands at tokens jb * 16 + 4 g + e of row rr: the same
    // tokens its outputs (t2 = jb) cover, so the decay closure below needs no
    // further loads
    float kt[2][4], yt[2][4], xt[2][4], kr[2][4], yr[2][4], xr[2][4], orw[2][4];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = jb * 16 + 4 * g + e;
        const long long o = (tb + j) * kw + rr;
        const float gj = p.G[o];
        kr[jb][e] = p.k[o];
        yr[jb][e] = Yk[o];
        xr[jb][e] = p.x[o];
        orw[jb][e] = p.colout ? 0.f : p.o[o];
        kt[jb][e] = keep_exp(!wild, kr[jb][e], -gj);
        yt[jb][e] = keep_exp(!wild, yr[jb][e], gj);
        xt[jb][e] = keep_exp(!wild, xr[jb][e], gx_g(j, rr));
      }
    const float egl = __expf(gl);
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      f4 ax = aX[q][t2], aq = aO[q][t2], ak;
#pragma unroll
      for (int e = 0; e < 4; ++e) ak[e] = egl * aL[q][t2][e];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int jj = jb * 16 + 4 * g + e, ii = t2 * 16 + m;
          ax = mfma4(M1[ii * MS + jj], kt[jb][e], ax);
          ak = mfma4(M2[jj * MS + ii], yt[jb][e], ak);
          ak = mfma4(-M1[jj * MS + ii], xt[jb][e], ak);
          if (p.colout) aq = mfma4(M2[ii * MS + jj], kt[jb][e], aq);
        }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = t2 * 16 + 4 * g + e;
        const long long o = (tb + i) * kw + rr;
        const float gi = p.G[o], gxi = gx_g(i, rr);
        float dx, dk, dq = 0.f;
        if (!wild) {
          dx = -__expf(gxi) * ax[e];
          dk = __expf(-gi) * ak[e];
          dq = __expf(gi) * aq[e];
        } else {
          float a = __expf(gxi) * aX[q][t2][e];
          for (int j = 0; j < i; ++j)
            a += M1[i * MS + j] * p.k[(tb + j) * kw + rr] * __expf(gxi - p.G[(tb + j) * kw + rr]);
          dx = -a;
          float b = __expf(gl - gi) * aL[q][t2][e];
          for (int j = i; j < WBT; ++j)
            b += M2[j * MS + i] * Yk[(tb + j) * kw + rr] * __expf(p.G[(tb + j) * kw + rr] - gi);
          for (int j = i + 1; j < WBT; ++j)
            b -= M1[j * MS + i] * p.x[(tb + j) * kw + rr] * __expf(gx_g(j, rr) - gi);
          dk = b;
          if (p.colout) {
            float c2 = __expf(gi) * aO[q][t2][e];
            for (int j = 0; j <= i; ++j)
              c2 += M2[i * MS + j] * p.k[(tb + j) * kw + rr] * __expf(gi - p.G[(tb + j) * kw + rr]);
            dq = c2;
          }
        }
        rdx[q][t2][e] = dx;
        rdk[q][t2][e] = dk;
        rdq[q][t2][e] = dq;
      }
    }
    // decay closure of row rr: dG = q dq - k dk (column) / o dO - k dk (row)
    // + x dx (of the next token when the erase reads before the decay), and
    // dg = rowsum(X_C lam) + the in-chunk reverse cumulative sum of dG.  The
    // lane holds tokens t2 * 16 + 4 g + e; the next token of e = 3 sits in lane
    // group g + 1 (g = 3, t2 = 0: group 0 of t2 = 1).
    float dG[2][4], xd[2][4];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dG[t2][e] = -kr[t2][e] * rdk[q][t2][e] +
                    (p.colout ? yr[t2][e] * rdq[q][t2][e] : orw[t2][e] * yr[t2][e]);
        xd[t2][e] = xr[t2][e] * rdx[q][t2][e];
      }
    if (p.excl) {
      const int src = g < 3 ? l + 16 : l - 48;
      const float n0 = __shfl(xd[0][0], src), n1 = __shfl(xd[1][0], src);
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int e = 0; e < 3; ++e) dG[t2][e] += xd[t2][e + 1];
      dG[0][3] += g < 3 ? n0 : n1;
      dG[1][3] += g < 3 ? n1 : 0.f;
    } else {
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int e = 0; e < 4; ++e) dG[t2][e] += xd[t2][e];
    }
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 2; e >= 0; --e) dG[t2][e] += dG[t2][e + 1];  // suffix within the lane
    float later[2], total1 = 0.f;  // sums of the later lane groups' tokens, per t2
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      const float s1 = __shfl(dG[t2][0], (l + 16) & 63), s2 = __shfl(dG[t2][0], (l + 32) & 63),
                  s3 = __shfl(dG[t2][0], (l + 48) & 63);
      later[t2] = (g < 3 ? s1 : 0.f) + (g < 2 ? s2 : 0.f) + (g < 1 ? s3 : 0.f);
      if (t2 == 1) total1 = dG[1][0] + s1 + s2 + s3;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      rdg[q][1][e] = rs[q] + dG[1][e] + later[1];
      rdg[q][0][e] = rs[q] + dG[0][e] + later[0] + total1;
    }
  }
  // stores after every row block's loads (a load issued after a store waits for it)
#pragma unroll
  for (int q = 0; q < GRB; ++q) {
    const int rb = wv_ + GW * q;
    if (rb >= nrb) continue;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const long long o = (tb + t2 * 16 + 4 * g + e) * kw + rb * 16 + m;
        p.dx[o] = rdx[q][t2][e];
        p.dk[o] = rdk[q][t2][e];
        if (p.colout) p.dq[o] = rdq[q][t2][e];
        p.dg[o] = rdg[q][t2][e];
      }
  }
}

constexpr size_t grad_smem(int w) { return (2 * WBT * MS + 3 * WBT * (w + 4)) * sizeof(float); }

// ---------------------------------------------------------------------------
// Source closure (per token): cotangents of e, chi, z back to u^, delta, k^, q^,
// the raw gates and the values (tests/chunk_model.py sources_bwd).
// ---------------------------------------------------------------------------
struct SrcBwdParams {
  sd_inputs in;
  int Tp, KP, VP;
  const float *uh, *delta, *kh, *qh, *de, *dchi, *dz;
  float *duh, *ddelta, *dkh, *dqh;
  __bf16 *derase, *dwrite, *dv;
};

__global__ __launch_bounds__(WT) void k_w_src_bwd(SrcBwdParams p) {
  const int s = blockIdx.y, H = p.in.H, T = p.in.T, r = p.in.r, V = p.in.V;
  const int b = s / H, h = s % H;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int t = blockIdx.x * (WT / 64) + w;
  if (t >= p.Tp) return;
  const bool tv = t < T;
  const long long row = ((long long)s * p.Tp + t) * p.KP, vr = ((long long)s * p.Tp + t) * p.VP;
  // every load first, at clamped indices (masked below): no load under a branch
  const int tc = min(t, T - 1);
  const __bf16 *err = wrow(p.in.erase_raw, b, tc, h), *vrow = wrow(p.in.v, b, tc, h),
               *wrr = wrow(p.in.write_raw, b, tc, h);
  float u[4], dl[4], k[4], q[4], er[4], de[4], dc[4], vv[4], wr[4], dzv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j, ck = min(c, p.KP - 1), cv = min(c, V - 1);
    u[j] = p.uh[row + ck];
    dl[j] = p.delta[row + ck];
    k[j] = p.kh[row + ck];
    q[j] = p.qh[row + ck];
    de[j] = p.de[row + ck];
    dc[j] = p.dchi[row + ck];
    er[j] = bf2f(err[min(c, r - 1)]);
    vv[j] = bf2f(vrow[cv]);
    wr[j] = bf2f(wrr[cv]);
    dzv[j] = p.dz[vr + cv];
  }
  float usq = 0.f, dsq = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j;
    const bool in = c < p.KP;
    u[j] = in ? u[j] : 0.f;
    dl[j] = in ? dl[j] : 0.f;
    k[j] = in ? k[j] : 0.f;
    q[j] = in ? q[j] : 0.f;
    de[j] = in ? de[j] : 0.f;
    dc[j] = in ? dc[j] : 0.f;
    er[j] = (tv && c < r) ? er[j] : 0.f;
    usq += u[j] * u[j];
    dsq += dl[j] * dl[j];
  }
  usq = wave_sum(usq);
  dsq = wave_sum(dsq);
  const float N = sqrtf(RHO * RHO + usq * dsq), sc = RHO / N;
  float phi[4], se[4], bb[4];
  float pu = 0.f, ub = 0.f, uq = 0.f, pde = 0.f, pdc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    phi[j] = sc * dl[j];
    se[j] = 1.f / (1.f + __expf(-er[j]));
    bb[j] = se[j] * k[j];
    pu += phi[j] * u[j];
    ub += u[j] * bb[j];
    uq += u[j] * q[j];
    pde += phi[j] * de[j];
    pdc += phi[j] * dc[j];
  }
  const float den = 1.f + wave_sum(pu);
  const float sb = wave_sum(ub) / den, sqv = wave_sum(uq) / den;
  const float dsb = -wave_sum(pde), dsqv = -wave_sum(pdc);
  const float dub = dsb / den, duq = dsqv / den;
  const float dden = -(dsb * sb + dsqv * sqv) / den;
  float dphi[4], duh[4], dqh[4], db[4];
  float ds = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    dphi[j] = -sb * de[j] - sqv * dc[j] + dden * u[j];
    duh[j] = dub * bb[j] + duq * q[j] + dden * phi[j];
    db[j] = de[j] + dub * u[j];
    dqh[j] = dc[j] + duq * u[j];
    ds += dphi[j] * dl[j];
  }
  ds = wave_sum(ds);
  const float dN2 = (-RHO * ds / (N * N)) / (2.f * N);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j;
    if (c < p.KP) {
      p.duh[row + c] = duh[j] + 2.f * dN2 * dsq * u[j];
      p.ddelta[row + c] = sc * dphi[j] + 2.f * dN2 * usq * dl[j];
      p.dkh[row + c] = db[j] * se[j];
      p.dqh[row + c] = dqh[j];
    }
    const long long obase = ((long long)b * T + t) * H + h;
    if (tv && c < r) p.derase[obase * r + c] = f2bf(db[j] * k[j] * se[j] * (1.f - se[j]));
    if (tv && c < V) {
      const float sw = 1.f / (1.f + __expf(-wr[j]));
      p.dv[obase * V + c] = f2bf(sw * dzv[j]);
      p.dwrite[obase * V + c] = f2bf(dzv[j] * vv[j] * sw * (1.f - sw));
    }
  }
}

// ---------------------------------------------------------------------------
// Final closure (per token): norms, gamma, and the two ops' decay gradients.
// ---------------------------------------------------------------------------
struct FinalParams {
  sd_inputs in;
  int Tp, KP;
  const float *uh, *kh, *qh, *gam, *rs;
  const float *duh, *dkh, *dqh, *dd, *dkC, *dxC, *dvC, *dqC, *dgS, *dgC;
  __bf16 *du, *dh, *dq, *dk;
  float *dlog_decay, *dgamma;
};

__global__ __launch_bounds__(WT) void k_w_final(FinalParams p) {
  const int s = blockIdx.y, H = p.in.H, T = p.in.T, r = p.in.r;
  const int b = s / H, h = s % H;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int t = blockIdx.x * (WT / 64) + w;
  if (t >= T) return;
  const long long tok = (long long)s * p.Tp + t, row = tok * p.KP;
  const float gm = p.gam[tok];
  const float xk = erase_keep(p.in, b, t);  // fresh tokens: dx reaches neither u nor gamma
  // every load first, at clamped indices (masked below): no load under a branch,
  // and none issued after a store
  const __bf16* hr = wrow(p.in.h, b, t, h);
  const float ru = p.rs[tok * 3], rk = p.rs[tok * 3 + 1], rq = p.rs[tok * 3 + 2];
  float u[4], k[4], q[4], dxc[4], dvc[4], gu[4], gk[4], gq[4], hv[4], dgl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j, ck = min(c, p.KP - 1);
    u[j] = p.uh[row + ck];
    k[j] = p.kh[row + ck];
    q[j] = p.qh[row + ck];
    dxc[j] = p.dxC[row + ck];
    dvc[j] = p.dvC[row + ck];
    gu[j] = p.duh[row + ck] + p.dkC[row + ck];
    gk[j] = p.dkh[row + ck] + p.dd[row + ck] + p.dqC[row + ck];
    gq[j] = p.dqh[row + ck];
    hv[j] = bf2f(hr[min(c, r - 1)]);
    dgl[j] = p.dgS[row + ck] + p.dgC[row + ck];
  }
  float su = 0.f, sk = 0.f, sq = 0.f, sg = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j;
    const bool in = c < p.KP;
    u[j] = in ? u[j] : 0.f;
    k[j] = in ? k[j] : 0.f;
    q[j] = in ? q[j] : 0.f;
    dxc[j] = in ? xk * dxc[j] : 0.f;
    dvc[j] = in ? dvc[j] : 0.f;
    gu[j] = in ? gu[j] + gm * dxc[j] : 0.f;
    gk[j] = in ? gk[j] : 0.f;
    gq[j] = in ? gq[j] : 0.f;
    hv[j] = c < r ? hv[j] : 0.f;
    su += gu[j] * u[j];
    sk += gk[j] * k[j];
    sq += gq[j] * q[j];
    sg += u[j] * dxc[j] + hv[j] * dvc[j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j;
    if (c < r) {
      const long long o = (((long long)b * T + t) * H + h) * r + c;
      p.dh[o] = f2bf(gm * dvc[j]);
      p.dlog_decay[o] = dgl[j];
    }
  }
  su = wave_sum(su);
  sk = wave_sum(sk);
  sq = wave_sum(sq);
  sg = wave_sum(sg);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = l + 64 * j;
    if (c < r) {
      const long long o = (((long long)b * T + t) * H + h) * r + c;
      p.du[o] = f2bf((gu[j] - su * u[j]) * ru);
      p.dk[o] = f2bf((gk[j] - sk * k[j]) * rk);
      p.dq[o] = f2bf((gq[j] - sq * q[j]) * rq);
    }
  }
  if (l == 0) p.dgamma[((long long)b * T + t) * H + h] = sg;
}

// Output cotangent as an FP32 panel (zero when absent and on padded entries).
struct DoutParams {
  int H, T, V, Tp, VP;
  const __bf16* dout;
  float* dO;
};
__global__ __launch_bounds__(WT) void k_w_dout(DoutParams p) {
  const int s = blockIdx.y, b = s / p.H, h = s % p.H;
  const long long n = (long long)p.Tp * p.VP;
  for (long long idx = (long long)blockIdx.x * WT + threadIdx.x; idx < n; idx += (long long)gridDim.x * WT) {
    const int t = (int)(idx / p.VP), c = (int)(idx % p.VP);
    float v = 0.f;
    if (p.dout && t < p.T && c < p.V) v = bf2f(p.dout[(((long long)b * p.T + t) * p.H + h) * p.V + c]);
    p.dO[(long long)s * n + idx] = v;
  }
}

}  // namespace wide

// ---------------------------------------------------------------------------
// Host side: workspace layout and launch sequences.
// ---------------------------------------------------------------------------
namespace {

using namespace wide;

int pad32(int x) { return (x + 31) / 32 * 32; }

struct WideDims {
  int n, NT, Tp, KP, VP;
};
WideDims wide_dims(int B, int T, int H, int r, int V) {
  WideDims d;
  d.n = B * H;
  d.NT = (T + WBT - 1) / WBT;
  d.Tp = d.NT * WBT;
  d.KP = pad32(r);
  d.VP = pad32(V);
  return d;
}

struct WCarver {
  char* base;
  size_t off = 0;
  template <class T = float>
  T* take(size_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

struct WideFwd {
  float *G, *uh, *kh, *qh, *xC, *vC, *gam, *rs;
  float *delta, *oC, *d, *e, *chi, *z, *wS;
  float *AC, *AS, *PS;
  xs_t *XC, *XS;
  _Float16 *Wneg, *Kt;
  float *U, *Qt, *Gam;
};

// saved: what the backward reads; scratch: the forward-only panels (the C op's
// gamma h, the S op's z, and both ops' W, U, K^, Q~).
WideFwd carve_wide_fwd(void* saved, void* scratch, const WideDims& d, size_t* saved_bytes,
                       size_t* scratch_bytes) {
  WCarver c{(char*)saved};
  const size_t tok = (size_t)d.n * d.Tp, pk = tok * d.KP, pv = tok * d.VP;
  const size_t mat = (size_t)d.n * d.NT * WBT * WBT;
  WideFwd w;
  w.G = c.take(pk); w.uh = c.take(pk); w.kh = c.take(pk); w.qh = c.take(pk);
  w.xC = c.take(pk); w.gam = c.take(tok); w.rs = c.take(tok * 3);
  w.delta = c.take(pk); w.oC = c.take(pk); w.d = c.take(pk); w.e = c.take(pk);
  w.chi = c.take(pk); w.wS = c.take(pv);
  w.AC = c.take(mat); w.AS = c.take(mat); w.PS = c.take(mat);
  w.XC = c.take<xs_t>((size_t)d.n * (d.NT + 1) * d.KP * d.KP);
  w.XS = c.take<xs_t>((size_t)d.n * (d.NT + 1) * d.KP * d.VP);
  w.Gam = c.take((size_t)d.n * d.NT * d.KP);
  if (saved_bytes) *saved_bytes = c.off + 256;
  WCarver t{(char*)scratch};
  const size_t pm = d.KP > d.VP ? pk : pv;
  w.vC = t.take(pk); w.z = t.take(pv);
  w.Wneg = t.take<_Float16>(pk); w.U = t.take(pm); w.Kt = t.take<_Float16>(pk); w.Qt = t.take(pk);
  if (scratch_bytes) *scratch_bytes = t.off + 256;
  return w;
}

struct WideBwd {
  float* dO;
  ls_t *LC, *LS;
  float *dU, *Pp;
  __bf16 *Wneg, *Kt, *At;
  float *dwS, *dwC, *dd, *de, *dchi, *dgS;
  float *duh, *ddelta, *dkh, *dqh, *dkC, *dxC, *dqC, *dgC;
};

WideBwd carve_wide_bwd(void* base, const WideDims& d, size_t* total) {
  WCarver c{(char*)base};
  const size_t tok = (size_t)d.n * d.Tp, pk = tok * d.KP, pv = tok * d.VP;
  const size_t pm = d.KP > d.VP ? pk : pv;
  WideBwd w;
  w.dO = c.take(pv);
  w.LC = c.take<ls_t>((size_t)d.n * (d.NT + 1) * d.KP * d.KP);
  w.LS = c.take<ls_t>((size_t)d.n * (d.NT + 1) * d.KP * d.VP);
  w.dU = c.take(pm); w.Wneg = c.take<__bf16>(pk); w.Kt = c.take<__bf16>(pk); w.At = c.take<__bf16>(pk);
  w.Pp = c.take((size_t)d.n * d.NT * WBT * WBT);
  w.dwS = c.take(pv); w.dwC = c.take(pk);
  w.dd = c.take(pk); w.de = c.take(pk); w.dchi = c.take(pk); w.dgS = c.take(pk);
  w.duh = c.take(pk); w.ddelta = c.take(pk); w.dkh = c.take(pk); w.dqh = c.take(pk);
  w.dkC = c.take(pk); w.dxC = c.take(pk); w.dqC = c.take(pk); w.dgC = c.take(pk);
  if (total) *total = c.off + 256;
  return w;
}

constexpr size_t kMaxLds = 160 * 1024;  // LDS of one gfx950 CU
static_assert(prep_smem(WMAX) <= kMaxLds && state_smem() <= kMaxLds && out_smem(WMAX, WMAX, 0) <= kMaxLds &&
                  out_smem(WMAX, WMAX, 1) <= kMaxLds && bprep_smem(WMAX) <= kMaxLds &&
                  grad_smem(WMAX) <= kMaxLds,
              "a wide kernel's LDS exceeds the CU");

void launch_wprep(const OpParams& op, int n, hipStream_t st) {
  const size_t sm = prep_smem(op.kw);
  SD_SMEM_ONCE(k_w_prep, (int)prep_smem(WMAX));
  SD_LAUNCH("k_w_prep", k_w_prep, dim3(op.NT, n), dim3(WT), sm, st, op);
}

void launch_wstate(const char* name, const WStateParams& sp, int n, hipStream_t st) {
  const dim3 grid(sp.vw / STILE * n), blk(ST);
  if (sp.rev)
    SD_LAUNCH(name, k_w_state<true>, grid, blk, state_smem(), st, sp);
  else
    SD_LAUNCH(name, k_w_state<false>, grid, blk, state_smem(), st, sp);
}

}  // namespace

void wide_fwd_sizes(int B, int T, int H, int r, int V, size_t* saved, size_t* scratch) {
  carve_wide_fwd(nullptr, nullptr, wide_dims(B, T, H, r, V), saved, scratch);
}

size_t wide_bwd_workspace_bytes(int B, int T, int H, int r, int V) {
  size_t total = 0;
  carve_wide_bwd(nullptr, wide_dims(B, T, H, r, V), &total);
  return total;
}

int launch_wide_fwd(const sd_inputs* in, void* out, float* C_T, float* S_T, void* saved,
                    void* scratch, hipStream_t st) {
  const WideDims d = wide_dims(in->B, in->T, in->H, in->r, in->V);
  const WideFwd w = carve_wide_fwd(saved, scratch, d, nullptr, nullptr);

  TokParams tp{};
  tp.in = *in; tp.NT = d.NT; tp.Tp = d.Tp; tp.KP = d.KP;
  tp.G = w.G; tp.uh = w.uh; tp.kh = w.kh; tp.qh = w.qh; tp.xC = w.xC; tp.vC = w.vC;
  tp.gam = w.gam; tp.rs = w.rs;
  SD_LAUNCH("k_w_tokens", k_w_tokens, dim3(d.NT, d.n), dim3(WT), 0, st, tp);

  // predictor C: X = C^T, k = u^, x = gamma u^, v = gamma h, q = k^, row output
  OpParams oc{};
  oc.NT = d.NT; oc.Tp = d.Tp; oc.kw = d.KP; oc.vw = d.KP; oc.excl = 1; oc.colout = 0;
  oc.k = w.uh; oc.x = w.xC; oc.v = w.vC; oc.q = w.kh; oc.G = w.G;
  oc.A = w.AC; oc.P = w.PS; oc.Wneg = w.Wneg; oc.U = w.U; oc.Kt = w.Kt; oc.Qt = w.Qt; oc.Gam = w.Gam;
  launch_wprep(oc, d.n, st);
  WStateParams sc{};
  sc.NT = d.NT; sc.Tp = d.Tp; sc.kw = d.KP; sc.vw = d.KP; sc.rows = in->r; sc.cols = in->r;
  sc.Wneg = w.Wneg; sc.U = w.U; sc.Kt = w.Kt; sc.Gam = w.Gam;
  sc.slots = w.XC; sc.wout = w.delta;
  sc.init = in->C0; sc.init_t = 1; sc.fin = C_T; sc.fin_t = 1;
  launch_wstate("w_state_c_fwd", sc, d.n, st);
  OutParams orow{};
  orow.NT = d.NT; orow.Tp = d.Tp; orow.kw = d.KP; orow.vw = d.KP; orow.colout = 0;
  orow.slots = w.XC; orow.w = w.delta; orow.q = w.kh; orow.k = w.uh; orow.G = w.G;
  orow.base = w.kh; orow.o = w.oC; orow.d = w.d;
  SD_SMEM_ONCE(k_w_out, (int)(out_smem(WMAX, WMAX, 0) > out_smem(WMAX, WMAX, 1) ? out_smem(WMAX, WMAX, 0) : out_smem(WMAX, WMAX, 1)));
  SD_LAUNCH("k_w_out_c", k_w_out, dim3(d.NT, d.n), dim3(WT), out_smem(d.KP, d.KP, 0), st, orow);

  SrcParams sp{};
  sp.in = *in; sp.Tp = d.Tp; sp.KP = d.KP; sp.VP = d.VP;
  sp.uh = w.uh; sp.delta = w.delta; sp.kh = w.kh; sp.qh = w.qh;
  sp.e = w.e; sp.chi = w.chi; sp.z = w.z;
  SD_LAUNCH("k_w_sources", k_w_sources, dim3(d.Tp / (WT / 64), d.n), dim3(WT), 0, st, sp);

  // memory S: k = d, x = e, v = z, q = chi, column output
  OpParams os{};
  os.NT = d.NT; os.Tp = d.Tp; os.kw = d.KP; os.vw = d.VP; os.excl = 0; os.colout = 1;
  os.k = w.d; os.x = w.e; os.v = w.z; os.q = w.chi; os.G = w.G;
  os.A = w.AS; os.P = w.PS; os.Wneg = w.Wneg; os.U = w.U; os.Kt = w.Kt; os.Qt = w.Qt; os.Gam = w.Gam;
  launch_wprep(os, d.n, st);
  WStateParams ss{};
  ss.NT = d.NT; ss.Tp = d.Tp; ss.kw = d.KP; ss.vw = d.VP; ss.rows = in->r; ss.cols = in->V;
  ss.Wneg = w.Wneg; ss.U = w.U; ss.Kt = w.Kt; ss.Gam = w.Gam;
  ss.slots = w.XS; ss.wout = w.wS;
  ss.init = in->S0; ss.init_t = 0; ss.fin = S_T; ss.fin_t = 0;
  launch_wstate("w_state_s_fwd", ss, d.n, st);
  OutParams ocol{};
  ocol.NT = d.NT; ocol.Tp = d.Tp; ocol.kw = d.KP; ocol.vw = d.VP; ocol.colout = 1;
  ocol.H = in->H; ocol.T = in->T; ocol.V = in->V;
  ocol.slots = w.XS; ocol.w = w.wS; ocol.Qt = w.Qt; ocol.P = w.PS; ocol.out = (__bf16*)out;
  SD_LAUNCH("k_w_out_s", k_w_out, dim3(d.NT, d.n), dim3(WT), out_smem(d.KP, d.VP, 1), st, ocol);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

int launch_wide_bwd(const sd_inputs* in, const void* fws, void* bws, const void* dout,
                    const float* dC_T, const float* dS_T, void* du, void* dh, void* dq, void* dk,
                    void* dv, void* derase, void* dwrite, float* dlog_decay, float* dgamma,
                    float* dC0, float* dS0, hipStream_t st) {
  const WideDims d = wide_dims(in->B, in->T, in->H, in->r, in->V);
  const WideFwd f = carve_wide_fwd((void*)fws, nullptr, d, nullptr, nullptr);
  const WideBwd w = carve_wide_bwd(bws, d, nullptr);
  // The forward's Gam panel holds exp(G_C) of the last op it ran; both ops share
  // the log-decay, so it serves both reverse passes.

  DoutParams dp{};
  dp.H = in->H; dp.T = in->T; dp.V = in->V; dp.Tp = d.Tp; dp.VP = d.VP;
  dp.dout = (const __bf16*)dout; dp.dO = w.dO;
  SD_LAUNCH("k_w_dout", k_w_dout, dim3(64, d.n), dim3(WT), 0, st, dp);

  SD_SMEM_ONCE(k_w_bprep, (int)bprep_smem(WMAX));
  SD_SMEM_ONCE(k_w_grad, (int)grad_smem(WMAX));

  // ---- memory S op ----
  BprepParams bs{};
  bs.NT = d.NT; bs.Tp = d.Tp; bs.kw = d.KP; bs.vw = d.VP; bs.excl = 0; bs.colout = 1;
  bs.k = f.d; bs.x = f.e; bs.q = f.chi; bs.G = f.G; bs.A = f.AS; bs.P = f.PS;
  bs.dO = w.dO; bs.dW = nullptr;
  bs.dU = w.dU; bs.Wneg = w.Wneg; bs.Kt = w.Kt; bs.At = w.At; bs.Pp = w.Pp;
  SD_LAUNCH("k_w_bprep_s", k_w_bprep, dim3(d.NT, d.n), dim3(WT), bprep_smem(d.KP), st, bs);
  WStateParams rs{};
  rs.NT = d.NT; rs.Tp = d.Tp; rs.kw = d.KP; rs.vw = d.VP; rs.rows = in->r; rs.cols = in->V; rs.rev = 1;
  rs.Wneg = w.Wneg; rs.U = w.dU; rs.Kt = w.Kt; rs.Gam = f.Gam; rs.At = w.At; rs.Ib = w.dO;
  rs.slots = w.LS; rs.wout = w.dwS;
  rs.init = dS_T; rs.init_t = 0; rs.fin = dS0; rs.fin_t = 0;
  launch_wstate("w_state_s_bwd", rs, d.n, st);
  GradParams gs{};
  gs.NT = d.NT; gs.Tp = d.Tp; gs.kw = d.KP; gs.vw = d.VP; gs.excl = 0; gs.colout = 1;
  gs.k = f.d; gs.x = f.e; gs.q = f.chi; gs.G = f.G; gs.dO = w.dO; gs.o = nullptr;
  gs.w = f.wS; gs.dw = w.dwS; gs.Xslots = f.XS; gs.Lslots = w.LS; gs.Pp = nullptr;
  gs.dk = w.dd; gs.dx = w.de; gs.dq = w.dchi; gs.dg = w.dgS;
  SD_LAUNCH("k_w_grad_s", k_w_grad, dim3(d.NT * d.n), dim3(GT), grad_smem(d.KP > d.VP ? d.KP : d.VP), st, gs);

  SrcBwdParams sb{};
  sb.in = *in; sb.Tp = d.Tp; sb.KP = d.KP; sb.VP = d.VP;
  sb.uh = f.uh; sb.delta = f.delta; sb.kh = f.kh; sb.qh = f.qh;
  sb.de = w.de; sb.dchi = w.dchi; sb.dz = w.dwS;
  sb.duh = w.duh; sb.ddelta = w.ddelta; sb.dkh = w.dkh; sb.dqh = w.dqh;
  sb.derase = (__bf16*)derase; sb.dwrite = (__bf16*)dwrite; sb.dv = (__bf16*)dv;
  SD_LAUNCH("k_w_src_bwd", k_w_src_bwd, dim3(d.Tp / (WT / 64), d.n), dim3(WT), 0, st, sb);

  // ---- predictor C op: output cotangent dd (d = k^ + o_C), dW = ddelta ----
  BprepParams bc{};
  bc.NT = d.NT; bc.Tp = d.Tp; bc.kw = d.KP; bc.vw = d.KP; bc.excl = 1; bc.colout = 0;
  bc.k = f.uh; bc.x = f.xC; bc.q = f.kh; bc.G = f.G; bc.A = f.AC; bc.P = nullptr;
  bc.dO = w.dd; bc.dW = w.ddelta;
  bc.dU = w.dU; bc.Wneg = w.Wneg; bc.Kt = w.Kt; bc.At = w.At; bc.Pp = w.Pp;
  SD_LAUNCH("k_w_bprep_c", k_w_bprep, dim3(d.NT, d.n), dim3(WT), bprep_smem(d.KP), st, bc);
  WStateParams rc{};
  rc.NT = d.NT; rc.Tp = d.Tp; rc.kw = d.KP; rc.vw = d.KP; rc.rows = in->r; rc.cols = in->r; rc.rev = 1;
  rc.Wneg = w.Wneg; rc.U = w.dU; rc.Kt = w.Kt; rc.Gam = f.Gam; rc.At = w.At; rc.Ib = f.kh;
  rc.slots = w.LC; rc.wout = w.dwC;
  rc.init = dC_T; rc.init_t = 1; rc.fin = dC0; rc.fin_t = 1;
  launch_wstate("w_state_c_bwd", rc, d.n, st);
  GradParams gc{};
  gc.NT = d.NT; gc.Tp = d.Tp; gc.kw = d.KP; gc.vw = d.KP; gc.excl = 1; gc.colout = 0;
  gc.k = f.uh; gc.x = f.xC; gc.q = f.kh; gc.G = f.G; gc.dO = w.dd; gc.o = f.oC;
  gc.w = f.delta; gc.dw = w.dwC; gc.Xslots = f.XC; gc.Lslots = w.LC; gc.Pp = w.Pp;
  gc.dk = w.dkC; gc.dx = w.dxC; gc.dq = w.dqC; gc.dg = w.dgC;
  SD_LAUNCH("k_w_grad_c", k_w_grad, dim3(d.NT * d.n), dim3(GT), grad_smem(d.KP > d.VP ? d.KP : d.VP), st, gc);

  FinalParams fp{};
  fp.in = *in; fp.Tp = d.Tp; fp.KP = d.KP;
  fp.uh = f.uh; fp.kh = f.kh; fp.qh = f.qh; fp.gam = f.gam; fp.rs = f.rs;
  fp.duh = w.duh; fp.dkh = w.dkh; fp.dqh = w.dqh; fp.dd = w.dd;
  fp.dkC = w.dkC; fp.dxC = w.dxC; fp.dvC = w.dwC; fp.dqC = w.dqC; fp.dgS = w.dgS; fp.dgC = w.dgC;
  fp.du = (__bf16*)du; fp.dh = (__bf16*)dh; fp.dq = (__bf16*)dq; fp.dk = (__bf16*)dk;
  fp.dlog_decay = dlog_decay; fp.dgamma = dgamma;
  SD_LAUNCH("k_w_final", k_w_final, dim3(d.Tp / (WT / 64), d.n), dim3(WT), 0, st, fp);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

}  // namespace sd
