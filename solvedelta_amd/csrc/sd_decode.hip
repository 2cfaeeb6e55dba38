// One-token recurrent step (T = 1), the recurrent-cache path
// (reference: causallsso/ops/residual_frame/recurrent.py:33-185 and FLA's
// fused recurrent DPLR step it delegates to).
//
// One 256-thread workgroup per (batch, head).  C is staged through LDS so the
// row reductions (C u) and column reductions (C'^T k) both read it once from
// HBM; S is streamed column-wise (two threads per value column, 64 rows each).
// State traffic per (b,h): read C and S once, write C' and S' once.
#include "sd_common.cuh"
#include "sd_internal.h"

namespace sd {

struct DecodeSmem {
  float C[KD][KD + 1];
  float u[KD], k[KD], q[KD], g[KD], hh[KD], er[KD];
  float delta[KD], d[KD], e[KD], chi[KD], z[VD], pred[VD];
  float red[8];
};

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(NTHREADS) void k_decode(sd_inputs in, __bf16* out, float* C_T,
                                                     float* S_T) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  DecodeSmem& s = *reinterpret_cast<DecodeSmem*>(smem_raw);
  const int n = blockIdx.x, b = n / in.H, hd = n % in.H;
  const int r = in.r, V = in.V, tid = threadIdx.x;
  auto ld = [&](const sd_view& v, int c, int w) -> float {
    if (c >= w) return 0.f;
    return bf2f(((const __bf16*)v.data)[(long long)b * v.sb + (long long)hd * v.sh + c]);
  };
  float uu = 0.f, kk = 0.f, qq = 0.f;
  if (tid < KD) {
    const int c = tid;
    uu = ld(in.u, c, r); kk = ld(in.k, c, r); qq = ld(in.q, c, r);
    s.hh[c] = ld(in.h, c, r);
    s.er[c] = ld(in.erase_raw, c, r);
    s.g[c] = c < r ? ((const float*)in.log_decay.data)[(long long)b * in.log_decay.sb +
                                                       (long long)hd * in.log_decay.sh + c]
                   : 0.f;
    s.z[c] = ld(in.v, c, V) / (1.f + __expf(-ld(in.write_raw, c, V)));
  }
  const float su = block_sum(uu * uu, s.red);
  const float sk = block_sum(kk * kk, s.red);
  const float sq = block_sum(qq * qq, s.red);
  if (tid < KD) {
    s.u[tid] = uu * rsqrtf(su + 1e-24f);
    s.k[tid] = kk * rsqrtf(sk + 1e-24f);
    s.q[tid] = qq * rsqrtf(sq + 1e-24f);
  }
  const float gam = ((const float*)in.gamma.data)[(long long)b * in.gamma.sb +
                                                  (long long)hd * in.gamma.sh];
  // stage C (zero when no initial state)
  const float* C0 = in.C0 ? in.C0 + (long long)n * r * r : nullptr;
  for (int idx = tid; idx < KD * KD; idx += NTHREADS) {
    const int i = idx / KD, j = idx % KD;
    s.C[i][j] = (C0 && i < r && j < r) ? C0[(long long)i * r + j] : 0.f;
  }
  __syncthreads();
  // delta_i = gamma (h_i - sum_j C_ij u_j): two threads per row
  {
    const int i = tid >> 1, half = tid & 1;
    float acc = 0.f;
    for (int j = half * 64; j < half * 64 + 64; ++j) acc += s.C[i][j] * s.u[j];
    acc += __shfl_xor(acc, 1, 64);
    if (half == 0) s.delta[i] = gam * (s.hh[i] - acc);
  }
  __syncthreads();
  // C' = C diag(e^g) + delta u^T
  for (int idx = tid; idx < KD * KD; idx += NTHREADS) {
    const int i = idx / KD, j = idx % KD;
    s.C[i][j] = s.C[i][j] * __expf(s.g[j]) + s.delta[i] * s.u[j];
  }
  __syncthreads();
  if (C_T) {
    float* Cn = C_T + (long long)n * r * r;
    for (int idx = tid; idx < r * r; idx += NTHREADS) Cn[idx] = s.C[idx / r][idx % r];
  }
  // d_j = k_j + sum_i C'_ij k_i: two threads per column
  {
    const int j = tid >> 1, half = tid & 1;
    float acc = 0.f;
    for (int i = half * 64; i < half * 64 + 64; ++i) acc += s.C[i][j] * s.k[i];
    acc += __shfl_xor(acc, 1, 64);
    if (half == 0) s.d[j] = s.k[j] + acc;
  }
  // sources
  const float dl = tid < KD ? s.delta[tid] : 0.f;
  const float uv = tid < KD ? s.u[tid] : 0.f;
  const float usq = block_sum(uv * uv, s.red);
  const float dsq = block_sum(dl * dl, s.red);
  const float sc = RHO / sqrtf(RHO * RHO + usq * dsq);
  const float phi = sc * dl;
  const float den = 1.f + block_sum(phi * uv, s.red);
  const float bb = tid < KD ? s.k[tid] / (1.f + __expf(-s.er[tid])) : 0.f;
  const float qv = tid < KD ? s.q[tid] : 0.f;
  const float ub = block_sum(uv * bb, s.red) / den;
  const float uq = block_sum(uv * qv, s.red) / den;
  if (tid < KD) {
    s.e[tid] = bb - phi * ub;
    s.chi[tid] = qv - phi * uq;
  }
  __syncthreads();
  // S: two threads per value column v, rows split in halves
  {
    const int v = tid >> 1, half = tid & 1;
    const float* S0 = in.S0 ? in.S0 + (long long)n * r * V : nullptr;
    float sv[64];
    float pr = 0.f;
#pragma unroll
    for (int a = 0; a < 64; ++a) {
      const int i = half * 64 + a;
      float x = (S0 && i < r && v < V) ? S0[(long long)i * V + v] : 0.f;
      x *= __expf(s.g[i]);
      sv[a] = x;
      pr += x * s.e[i];
    }
    pr += __shfl_xor(pr, 1, 64);
    const float upd = s.z[v] - pr;
    float o = 0.f;
#pragma unroll
    for (int a = 0; a < 64; ++a) {
      const int i = half * 64 + a;
      sv[a] += s.d[i] * upd;
      o += sv[a] * s.chi[i];
    }
    o += __shfl_xor(o, 1, 64);
    if (S_T && v < V) {
      float* Sn = S_T + (long long)n * r * V;
#pragma unroll
      for (int a = 0; a < 64; ++a) {
        const int i = half * 64 + a;
        if (i < r) Sn[(long long)i * V + v] = sv[a];
      }
    }
    if (half == 0 && v < V) out[(long long)n * V + v] = f2bf(o);
  }
}

int launch_decode(const sd_inputs* in, void* out, float* C_T, float* S_T, hipStream_t st) {
  (void)hipFuncSetAttribute((const void*)k_decode, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)sizeof(DecodeSmem));
  SD_LAUNCH("k_decode", k_decode, dim3(in->B * in->H), dim3(NTHREADS), sizeof(DecodeSmem), st, *in,
                     (__bf16*)out, C_T, S_T);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

}  // namespace sd
