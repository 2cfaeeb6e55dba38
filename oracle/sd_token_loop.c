/* CPU token-loop restatement of the SolveDelta forward (test infrastructure
 * and CPU baseline only; never linked into the product library).
 *
 * Follows causallsso/reference.py:147-227 (the FP64 oracle's token loop) with
 * raw gate logits, as the native entry takes them
 * (causallsso/ops/operator.py:13-26, sources.py:87-88,119-120).
 * OpenMP parallelises over the B*H independent (batch, head) sequences.
 *
 * All inputs are contiguous FP32 arrays:
 *   u,h,q,k,erase_raw [B,T,H,r]; v,write_raw [B,T,H,V]; g (log decay) [B,T,H,r];
 *   gamma [B,T,H]; C [B,H,r,r] (prediction = C u); S [B,H,r,V] (updated in place);
 *   out [B,T,H,V].
 * The arithmetic type is REAL (double for sd_cpu_forward_f64, float for _f32).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define RHO (5.0 / 8.0)

#define DEFINE_FORWARD(NAME, REAL, SQRT, EXP)                                          \
  int NAME(int B, int T, int H, int r, int V, const float *u, const float *h,        \
           const float *q, const float *k, const float *v, const float *g,             \
           const float *erase_raw, const float *write_raw, const float *gamma,        \
           float *C, float *S, float *out) {                                          \
    int ok = 0;                                                                        \
    _Pragma("omp parallel for schedule(dynamic)")                                      \
    for (int bh = 0; bh < B * H; ++bh) {                                               \
      int b = bh / H, hh = bh % H;                                                     \
      REAL *Cs = (REAL *)malloc(sizeof(REAL) * r * r);                                 \
      REAL *Ss = (REAL *)malloc(sizeof(REAL) * r * V);                                 \
      REAL *w = (REAL *)malloc(sizeof(REAL) * (8 * r + 2 * V));                        \
      if (!Cs || !Ss || !w) { ok = -1; free(Cs); free(Ss); free(w); continue; }        \
      REAL *un = w, *kn = w + r, *qn = w + 2 * r, *dl = w + 3 * r, *ph = w + 4 * r;    \
      REAL *dd = w + 5 * r, *e = w + 6 * r, *chi = w + 7 * r, *pred = w + 8 * r;       \
      REAL *z = pred + V;                                                              \
      float *Cg = C + (size_t)bh * r * r, *Sg = S + (size_t)bh * r * V;                \
      for (int i = 0; i < r * r; ++i) Cs[i] = Cg[i];                                   \
      for (int i = 0; i < r * V; ++i) Ss[i] = Sg[i];                                   \
      for (int t = 0; t < T; ++t) {                                                    \
        size_t tok = ((size_t)b * T + t) * H + hh;                                     \
        const float *ut = u + tok * r, *kt = k + tok * r, *qt = q + tok * r;           \
        const float *ht = h + tok * r, *gt = g + tok * r, *et = erase_raw + tok * r;   \
        const float *vt = v + tok * V, *wt = write_raw + tok * V;                      \
        REAL su = 0, sk = 0, sq = 0;                                                   \
        for (int i = 0; i < r; ++i) {                                                  \
          su += (REAL)ut[i] * ut[i]; sk += (REAL)kt[i] * kt[i];                        \
          sq += (REAL)qt[i] * qt[i];                                                   \
        }                                                                              \
        /* F.normalize: x / max(|x|, 1e-12) */                                        \
        REAL nu = SQRT(su), nk = SQRT(sk), nq = SQRT(sq);                              \
        nu = nu > 1e-12 ? nu : 1e-12; nk = nk > 1e-12 ? nk : 1e-12;                    \
        nq = nq > 1e-12 ? nq : 1e-12;                                                  \
        REAL usq = 0;                                                                  \
        for (int i = 0; i < r; ++i) {                                                  \
          un[i] = ut[i] / nu; kn[i] = kt[i] / nk; qn[i] = qt[i] / nq;                  \
          usq += un[i] * un[i];                                                        \
        }                                                                              \
        REAL gm = gamma[tok], dsq = 0;                                                 \
        for (int i = 0; i < r; ++i) {                                                  \
          REAL acc = 0;                                                                \
          for (int j = 0; j < r; ++j) acc += Cs[i * r + j] * un[j];                    \
          dl[i] = gm * ((REAL)ht[i] - acc);                                            \
          dsq += dl[i] * dl[i];                                                        \
        }                                                                              \
        for (int i = 0; i < r; ++i)                                                    \
          for (int j = 0; j < r; ++j)                                                  \
            Cs[i * r + j] = Cs[i * r + j] * EXP((REAL)gt[j]) + dl[i] * un[j];          \
        REAL sc = (REAL)RHO / SQRT((REAL)(RHO * RHO) + usq * dsq), den = 1, ub = 0,    \
             uq = 0;                                                                   \
        for (int i = 0; i < r; ++i) { ph[i] = sc * dl[i]; den += ph[i] * un[i]; }      \
        for (int j = 0; j < r; ++j) dd[j] = kn[j];                                     \
        for (int i = 0; i < r; ++i)                                                    \
          for (int j = 0; j < r; ++j) dd[j] += Cs[i * r + j] * kn[i];                  \
        for (int i = 0; i < r; ++i) {                                                  \
          REAL bi = kn[i] / (1 + EXP(-(REAL)et[i]));                                   \
          e[i] = bi; ub += un[i] * bi; uq += un[i] * qn[i];                            \
        }                                                                              \
        for (int i = 0; i < r; ++i) {                                                  \
          e[i] -= ph[i] * (ub / den);                                                  \
          chi[i] = qn[i] - ph[i] * (uq / den);                                         \
        }                                                                              \
        for (int c = 0; c < V; ++c) {                                                  \
          pred[c] = 0; z[c] = (REAL)vt[c] / (1 + EXP(-(REAL)wt[c]));                   \
        }                                                                              \
        for (int i = 0; i < r; ++i) {                                                  \
          REAL dec = EXP((REAL)gt[i]);                                                 \
          for (int c = 0; c < V; ++c) {                                                \
            Ss[i * V + c] *= dec;                                                      \
            pred[c] += Ss[i * V + c] * e[i];                                           \
          }                                                                            \
        }                                                                              \
        for (int c = 0; c < V; ++c) pred[c] = z[c] - pred[c];                          \
        float *ot = out + tok * V;                                                     \
        for (int c = 0; c < V; ++c) ot[c] = 0;                                         \
        REAL *oacc = z; /* reuse: z no longer needed */                                \
        for (int c = 0; c < V; ++c) oacc[c] = 0;                                       \
        for (int i = 0; i < r; ++i)                                                    \
          for (int c = 0; c < V; ++c) {                                                \
            Ss[i * V + c] += dd[i] * pred[c];                                          \
            oacc[c] += Ss[i * V + c] * chi[i];                                         \
          }                                                                            \
        for (int c = 0; c < V; ++c) ot[c] = (float)oacc[c];                            \
      }                                                                                \
      for (int i = 0; i < r * r; ++i) Cg[i] = (float)Cs[i];                            \
      for (int i = 0; i < r * V; ++i) Sg[i] = (float)Ss[i];                            \
      free(Cs); free(Ss); free(w);                                                     \
    }                                                                                  \
    return ok;                                                                         \
  }

DEFINE_FORWARD(sd_cpu_forward_f64, double, sqrt, exp)
DEFINE_FORWARD(sd_cpu_forward_f32, float, sqrtf, expf)
