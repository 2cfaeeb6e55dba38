// One-token recurrent step (T = 1), the recurrent-cache path
// (reference: causallsso/ops/residual_frame/recurrent.py:33-185 and FLA's
// fused recurrent DPLR step it delegates to).
//
// One 256-thread workgroup per (batch, head), two resident per CU (the register
// budget is capped for it: at one per CU a 64-stream step ran as two rounds).  Every thread owns a 16-row x
// 4-column patch of C and of S (columns 4*(tid & 31), rows 16*(tid >> 5)).  It
// issues the token's vector loads, then all 32 of its 16-byte state loads (C
// first) before any arithmetic, so the whole 128 KiB of state per (b,h) is in
// flight at once and the norms and the C phase overlap the S loads.  The
// r = V = 128 instantiation has no per-element guards: guarded loads compile
// to branches that each wait for the previous load.  Row reductions of C (C u) go through an LDS copy of C; column
// reductions (C'^T k, S'^T e, S^T chi) reduce the patches across the eight row
// groups (lane xor 32, then the four waves through LDS).  The new states are
// written back from registers with 16-byte stores.
// State traffic per (b,h): read C and S once, write C' and S' once.  In place
// (C_T == C0, S_T == S0) is allowed: a workgroup reads its state before it
// writes it and touches no other workgroup's.
#include "sd_common.cuh"
#include "sd_internal.h"

namespace sd {

constexpr int DCS = KD + 4;  // LDS row stride of C (16-byte aligned rows)

struct DecodeSmem {
  float C[KD][DCS];
  float u[KD], k[KD], q[KD], eg[KD], hh[KD];
  float delta[KD], d[KD], e[KD], chi[KD], z[VD];
  float4 part[4][32];
  float red[4][8];
};

// Sum of up to eight per-thread values over the workgroup (one barrier pair).
template <int N>
__device__ __forceinline__ void block_sums(float (&v)[N], float (&red)[4][8]) {
  static_assert(N <= 8, "eight sums at most");
#pragma unroll
  for (int m = 0; m < N; ++m) v[m] = wave_sum(v[m]);
  __syncthreads();
  if (lane_id() == 0)
#pragma unroll
    for (int m = 0; m < N; ++m) red[wave_id()][m] = v[m];
  __syncthreads();
#pragma unroll
  for (int m = 0; m < N; ++m) v[m] = red[0][m] + red[1][m] + red[2][m] + red[3][m];
}

// Column sums of the per-thread float4 partials over the 8 row groups: the
// result for columns 4*(tid & 31) .. +3 is returned to every thread.
__device__ __forceinline__ float4 col_sums(float4 v, float4 (&part)[4][32]) {
  v.x += __shfl_xor(v.x, 32, 64);
  v.y += __shfl_xor(v.y, 32, 64);
  v.z += __shfl_xor(v.z, 32, 64);
  v.w += __shfl_xor(v.w, 32, 64);
  __syncthreads();
  if (lane_id() < 32) part[wave_id()][lane_id()] = v;
  __syncthreads();
  const int cg = threadIdx.x & 31;
  float4 r = part[0][cg];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    const float4 t = part[w][cg];
    r.x += t.x; r.y += t.y; r.z += t.z; r.w += t.w;
  }
  return r;
}

// FULL: r = V = 128, 16-byte aligned states: unguarded 16-byte accesses (no
// per-element branches, so all loads stay in flight together).
template <bool FULL>
__device__ __forceinline__ float4 ld4(const float* base, int row, int col, int ld, int nrow,
                                      int ncol) {
  if constexpr (FULL) return *reinterpret_cast<const float4*>(base + (long long)row * ld + col);
  if (!base || row >= nrow) return make_float4(0.f, 0.f, 0.f, 0.f);
  const float* p = base + (long long)row * ld + col;
  float t[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) t[m] = col + m < ncol ? p[m] : 0.f;
  return make_float4(t[0], t[1], t[2], t[3]);
}

template <bool FULL>
__device__ __forceinline__ void st4(float* base, int row, int col, int ld, int nrow, int ncol,
                                    float4 v) {
  if constexpr (FULL) {
    *reinterpret_cast<float4*>(base + (long long)row * ld + col) = v;
    return;
  }
  if (row >= nrow) return;
  float* p = base + (long long)row * ld + col;
  const float t[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int m = 0; m < 4; ++m)
    if (col + m < ncol) p[m] = t[m];
}

__device__ __forceinline__ float f4get(const float4& v, int m) {
  return m == 0 ? v.x : m == 1 ? v.y : m == 2 ? v.z : v.w;
}

template <bool FULL>
__global__ __launch_bounds__(NTHREADS, 2) void k_decode(sd_inputs in, __bf16* out, float* C_T,
                                                     float* S_T) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  DecodeSmem& s = *reinterpret_cast<DecodeSmem*>(smem_raw);
  const int n = blockIdx.x, b = n / in.H, hd = n % in.H;
  const int r = in.r, V = in.V, tid = threadIdx.x;
  const int cg = tid & 31, c0 = cg * 4, rg = tid >> 5, i0 = rg * 16;
  auto ld = [&](const sd_view& v, int c, int w) -> float {
    if (!FULL && c >= w) return 0.f;
    return bf2f(((const __bf16*)v.data)[(long long)b * v.sb + (long long)hd * v.sh + c]);
  };
  // ---- the token's vectors, then every state load (C before S), all issued
  // before any of them is consumed; the norms and the C phase proceed while
  // the S loads are still in flight
  // every thread loads channel tid & 127 (branch-free, so the loads stay in
  // flight); threads >= 128 drop their copies after the barrier below
  float uu, kk, qq, er, hv, gl = 0.f, vv, wr;
  {
    const int c = tid & (KD - 1);
    uu = ld(in.u, c, r); kk = ld(in.k, c, r); qq = ld(in.q, c, r);
    er = ld(in.erase_raw, c, r);
    hv = ld(in.h, c, r);
    if (FULL || c < r)
      gl = ((const float*)in.log_decay.data)[(long long)b * in.log_decay.sb +
                                             (long long)hd * in.log_decay.sh + c];
    vv = ld(in.v, c, V);
    wr = ld(in.write_raw, c, V);
  }
  const float gam_raw = ((const float*)in.gamma.data)[(long long)b * in.gamma.sb +
                                                      (long long)hd * in.gamma.sh];
  const unsigned tf = tok_flags(in, b, 0);
  const float* C0 = in.C0 ? in.C0 + (long long)n * r * r : nullptr;
  const float* S0 = in.S0 ? in.S0 + (long long)n * r * V : nullptr;
  float4 cv[16], sv[16];
#pragma unroll
  for (int a = 0; a < 16; ++a) cv[a] = ld4<FULL>(C0, i0 + a, c0, r, r, r);
#pragma unroll
  for (int a = 0; a < 16; ++a) sv[a] = ld4<FULL>(S0, i0 + a, c0, V, r, V);
  __builtin_amdgcn_sched_barrier(0);  // keep every load above the first use
  // token flags: an invalid token reads q, keys, gamma and the log-decay as 0, a
  // reset reads the log-decay as the reset value
  const float om = operand_keep(tf);
  kk *= om;
  qq *= om;
  const float gam = gam_raw * om;
  if (FULL || (tid & (KD - 1)) < r) gl = decay_eff(tf, gl);
  if (tid >= KD) uu = kk = qq = er = 0.f;
  if (tid < KD) {
    const int c = tid;
    s.hh[c] = hv;
    s.eg[c] = (FULL || c < r) ? __expf(gl) : 0.f;
    s.z[c] = vv / (1.f + __expf(-wr));
  }
  // Every token-vector sum the step needs, in one reduction: the three norms
  // and the two dual-source products u.b and u.q (b = k sigmoid(erase)), taken
  // on the raw vectors and rescaled by the norms.
  float usq, ub, uq, bb;
  {
    const float sig = tid < KD ? 1.f / (1.f + __expf(-er)) : 0.f;
    float sums[5] = {uu * uu, kk * kk, qq * qq, uu * kk * sig, uu * qq};
    block_sums(sums, s.red);
    const float ru = rsqrtf(sums[0] + 1e-24f), rk = rsqrtf(sums[1] + 1e-24f),
                rq = rsqrtf(sums[2] + 1e-24f);
    usq = sums[0] * ru * ru;
    ub = sums[3] * ru * rk;
    uq = sums[4] * ru * rq;
    uu *= ru;
    kk *= rk;
    qq *= rq;
    bb = kk * sig;
  }
  if (tid < KD) {
    s.u[tid] = uu;
    s.k[tid] = kk;
  }
#pragma unroll
  for (int a = 0; a < 16; ++a) *reinterpret_cast<float4*>(&s.C[i0 + a][c0]) = cv[a];
  __syncthreads();
  // delta_i = gamma (h_i - sum_j C_ij u_j): two threads per row
  {
    const int i = tid >> 1, half = tid & 1;
    float acc = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int j = half * 64 + m * 4;
      const float4 c = *reinterpret_cast<const float4*>(&s.C[i][j]);
      acc += c.x * s.u[j] + c.y * s.u[j + 1] + c.z * s.u[j + 2] + c.w * s.u[j + 3];
    }
    acc += __shfl_xor(acc, 1, 64);
    if (half == 0) s.delta[i] = gam * (s.hh[i] - erase_keep_f(tf) * acc);
  }
  __syncthreads();
  // C' = C diag(e^g) + delta u^T in registers; d_j = k_j + sum_i C'_ij k_i
  {
    float egc[4], uc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      egc[m] = s.eg[c0 + m];
      uc[m] = s.u[c0 + m];
    }
    float4 dp = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const float dl = s.delta[i0 + a], ki = s.k[i0 + a];
      float4& c = cv[a];
      c = *reinterpret_cast<const float4*>(&s.C[i0 + a][c0]);  // from LDS: cv is not held across the delta phase
      c.x = c.x * egc[0] + dl * uc[0];
      c.y = c.y * egc[1] + dl * uc[1];
      c.z = c.z * egc[2] + dl * uc[2];
      c.w = c.w * egc[3] + dl * uc[3];
      dp.x += c.x * ki; dp.y += c.y * ki; dp.z += c.z * ki; dp.w += c.w * ki;
    }
    if (C_T) {
      float* Cn = C_T + (long long)n * r * r;
#pragma unroll
      for (int a = 0; a < 16; ++a) st4<FULL>(Cn, i0 + a, c0, r, r, r, cv[a]);
    }
    dp = col_sums(dp, s.part);
    if (rg == 0) {
#pragma unroll
      for (int m = 0; m < 4; ++m) s.d[c0 + m] = s.k[c0 + m] + f4get(dp, m);
    }
  }
  // sources: phi = rho delta / sqrt(rho^2 + |u|^2 |delta|^2), den = 1 + phi.u
  // (|delta|^2 and delta.u in one reduction)
  const float dl = tid < KD ? s.delta[tid] : 0.f;
  float dsum[2] = {dl * dl, dl * uu};
  block_sums(dsum, s.red);
  const float sc = RHO / sqrtf(RHO * RHO + usq * dsum[0]);
  const float phi = sc * dl;
  const float den = 1.f + sc * dsum[1];
  if (tid < KD) {
    s.e[tid] = bb - phi * (ub / den);
    s.chi[tid] = qq - phi * (uq / den);
  }
  __syncthreads();
  // S' = D S + d (z - (D S)^T e)^T ;  o = S'^T chi
  {
    float4 pr = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const float g = s.eg[i0 + a], ei = s.e[i0 + a];
      float4& x = sv[a];
      x.x *= g; x.y *= g; x.z *= g; x.w *= g;
      pr.x += x.x * ei; pr.y += x.y * ei; pr.z += x.z * ei; pr.w += x.w * ei;
    }
    pr = col_sums(pr, s.part);
    float upd[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) upd[m] = s.z[c0 + m] - f4get(pr, m);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const float di = s.d[i0 + a], ci = s.chi[i0 + a];
      float4& x = sv[a];
      x.x += di * upd[0]; x.y += di * upd[1]; x.z += di * upd[2]; x.w += di * upd[3];
      o.x += x.x * ci; o.y += x.y * ci; o.z += x.z * ci; o.w += x.w * ci;
    }
    if (S_T) {
      float* Sn = S_T + (long long)n * r * V;
#pragma unroll
      for (int a = 0; a < 16; ++a) st4<FULL>(Sn, i0 + a, c0, V, r, V, sv[a]);
    }
    o = col_sums(o, s.part);
    if (rg == 0) {
#pragma unroll
      for (int m = 0; m < 4; ++m)
        if (FULL || c0 + m < V) out[(long long)n * V + c0 + m] = f2bf(f4get(o, m));
    }
  }
}

int launch_decode(const sd_inputs* in, void* out, float* C_T, float* S_T, hipStream_t st) {
  SD_SMEM_ONCE(k_decode<true>, (int)sizeof(DecodeSmem));
  SD_SMEM_ONCE(k_decode<false>, (int)sizeof(DecodeSmem));
  auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool full = in->r == KD && in->V == VD && in->C0 && in->S0 && C_T && S_T && al(in->C0) &&
                    al(in->S0) && al(C_T) && al(S_T);
  if (full)
    SD_LAUNCH("k_decode", k_decode<true>, dim3(in->B * in->H), dim3(NTHREADS), sizeof(DecodeSmem),
              st, *in, (__bf16*)out, C_T, S_T);
  else
    SD_LAUNCH("k_decode", k_decode<false>, dim3(in->B * in->H), dim3(NTHREADS), sizeof(DecodeSmem),
              st, *in, (__bf16*)out, C_T, S_T);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

}  // namespace sd
