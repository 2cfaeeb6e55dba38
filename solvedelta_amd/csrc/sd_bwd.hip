// Backward (VJP) chunk kernels of the SolveDelta recurrence (gfx950).
//
// Mirror of the forward, in reverse order, recomputing nothing per token that
// the forward workspace keeps (chunk states, (I+L)^-1, WY/key panels, delta,
// d, e, chi, w).  For each op (S memory first, then C predictor):
//   k_bprep_*   chunk-parallel: dU = (P A)^T rhs (+ A^T ext), Wk = A^T K^,
//               and the reverse-pass injection panels;
//   k_state<true, true> (rev = 1): lambda <- Gamma lambda + A1 B1 - x~^T dw,
//               dw = dU + Wk lambda, storing the chunk-end cotangents;
//   k_grad_*    chunk-parallel closed-form gradients of (k, x, v, q) and the
//               in-chunk reverse cumulative sum that closes the decay gradient
//               (k_grad_s writes the S side's log-decay gradient to the output,
//               k_grad_c adds the C side's).
// Between the ops k_src_bwd transposes the dual sources (phi, den, e, chi, z
// and the q / erase / write / value gates); the C chunk gradient closes with u,
// k, h and gamma.
// The closed forms are the ones checked against FP64 autograd in
// tests/chunk_model.py (Op.backward, sources_bwd, backward_seq).
#include "sd_common.cuh"
#include "sd_internal.h"

namespace sd {

struct BwdParams {
  sd_inputs in;
  int H, T, r, V, NT, Tp;
  FwdWs f;
  BwdWs g;
  const __bf16* dout;  // nullable
  __bf16 *du, *dh, *dq, *dk, *dv, *der, *dwr;
  float *dg, *dgam;
};

__device__ __forceinline__ const __bf16* brow(const sd_view& v, int b, int t, int h) {
  return (const __bf16*)v.data + (long long)b * v.sb + (long long)t * v.st + (long long)h * v.sh;
}


// dout_at split into a raw load (clamped address) and its use.
struct DoutRaw {
  __bf16 x;
  bool ok;
};
// A missing cotangent reads this zero element instead (pointer select, no branch).
__device__ const __bf16 sd_zero_bf16[1] = {};
__device__ __align__(16) const __bf16 sd_zero_bf16x8[8] = {};
__device__ __forceinline__ DoutRaw dout_raw(const BwdParams& p, int b, int t, int h, int c) {
  const bool has = p.dout != nullptr;
  const bool ok = has && t < p.T && c < p.V;
  const __bf16* base = has ? (const __bf16*)p.dout : sd_zero_bf16;
  const long long i = (((long long)b * p.T + (t < p.T ? t : p.T - 1)) * p.H + h) * p.V +
                      (c < p.V ? c : p.V - 1);
  return {base[has ? i : 0], ok};
}
__device__ __forceinline__ float dout_val(DoutRaw r) { return keep_if(r.ok, bf2f(r.x)); }

// Stages the chunk's output cotangent (bf16, read in place; padded tokens and
// columns read 0) as a split LDS panel, in two steps: the raw 16-bit loads (two
// elements per word), issued early, then the split written to LDS.  All CT threads.
struct DoutPanelRaw { unsigned w[BT * KD / 4 / CT][2]; };
__device__ __forceinline__ void dout_panel_load(const BwdParams& p, int b, int t0, int hh,
                                                DoutPanelRaw& o) {
  constexpr int PER = BT * KD / 4 / CT;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 4, i = idx / KD, c = idx % KD;
    unsigned short v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = __builtin_bit_cast(unsigned short, dout_raw(p, b, t0 + i, hh, c + e).x);
    o.w[q][0] = (unsigned)v[0] | (unsigned)v[1] << 16;
    o.w[q][1] = (unsigned)v[2] | (unsigned)v[3] << 16;
  }
}
// dO is exact in bf16: it is staged as it is (no low half) into the rows of
// dst, a [BT][LPS] bf16 array.
__device__ __forceinline__ void dout_panel_store(__bf16 (*dst)[LPS], const BwdParams& p, int t0,
                                                 const DoutPanelRaw& raw) {
  constexpr int PER = BT * KD / 4 / CT;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 4, i = idx / KD, c = idx % KD;
    bf16x4 hh4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned wd = raw.w[q][e >> 1];
      const float x = __uint_as_float((e & 1) ? wd & 0xffff0000u : wd << 16);
      const bool ok = p.dout != nullptr && t0 + i < p.T && c + e < p.V;
      hh4[e] = (__bf16)keep_if(ok, x);
    }
    *reinterpret_cast<bf16x4*>(&dst[i][c]) = hh4;
  }
}

// Branch-free row load: out-of-range tokens and coordinates read a valid element
// and are selected to 0 (a guarded load would branch and wait).
__device__ __forceinline__ void ldrow2(const sd_view& v, int b, int t, int h, int T, int w,
                                       float& x0, float& x1) {
  const int l = lane_id();
  const bool tv = t < T;
  const __bf16* q = brow(v, b, tv ? t : T - 1, h);
  const float a0 = bf2f(q[l < w ? l : w - 1]), a1 = bf2f(q[l + 64 < w ? l + 64 : w - 1]);
  x0 = keep_if(tv && l < w, a0);
  x1 = keep_if(tv && l + 64 < w, a1);
}

__device__ __forceinline__ float norm2(float& x0, float& x1) {
  const float rs = rsqrtf(wave_sum(x0 * x0 + x1 * x1) + 1e-24f);
  x0 *= rs;
  x1 *= rs;
  return rs;
}

__device__ __forceinline__ const float* gptr(const sd_inputs& in, int b, int h) {
  return (const float*)in.log_decay.data + (long long)b * in.log_decay.sb +
         (long long)h * in.log_decay.sh;
}

// A wave's 64 x 16 output column block (MFMA layout, block Jb in v[Jb]) stored
// after the loop that made it: a store between the loop's gathers would hold
// every later gather behind it.
__device__ __forceinline__ void store_du_slab(float* base, const f4 (&v)[NB]) {
  const int c = wave_id() * 16 + out_col();
#pragma unroll
  for (int Jb = 0; Jb < NB; ++Jb)
#pragma unroll
    for (int e = 0; e < 4; ++e) base[(unsigned)((Jb * BS + out_row(e)) * KD + c)] = v[Jb][e];
}

// 64x64 N = P A (both 64 x LS in LDS) -> N (64 x LS)
// N = P A for lower-triangular P and A (block lower): N is block lower too,
// and block (I, J) sums only K in [16 J, 16 I + 16).
__device__ void mat64_mul(const float* P, const float* A, float* N) {
  for (int tt = wave_id(); tt < NB * NB; tt += CW) {
    const int I = tt / NB, J = tt % NB;
    f4 acc = zero4();
    if (J <= I)
      acc = mma_k32([&](int m, int k) { return P[(I * BS + m) * LS + k]; },
                    [&](int k, int nn) { return A[k * LS + J * BS + nn]; }, (I + 1) * BS, zero4(),
                    J * BS);
#pragma unroll
    for (int e = 0; e < 4; ++e) N[(I * BS + out_row(e)) * LS + J * BS + out_col()] = acc[e];
  }
}

// ---------------------------------------------------------------------------
// S memory
// ---------------------------------------------------------------------------
// A 64 x 64 operand split into bf16 hi / lo, row-major with K contiguous.
constexpr int SPS = BT + 8;  // row stride (bf16 elements), keeps 16-byte alignment
struct SPanel64 {
  __bf16 h[BT][SPS];
  __bf16 l[BT][SPS];
};

// Eight fp32 values (one lane's K slice of an MFMA operand) split into bf16 hi / lo.
__device__ __forceinline__ Frag split8(const float (&v)[8]) {
  Frag f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    __bf16 a, b2;
    split_bf(v[e], a, b2);
    f.h[e] = a;
    f.l[e] = b2;
  }
  return f;
}

struct BprepSSmem {
  ChunkDecay cd;
  float A[BT * LS];
  float P[BT * LS];  // P and N are contiguous: reused as a 64 x 128 staging panel
  float N[BT * LS];
  SPanel64 At, Nt;   // A^T and N^T split once: the MFMA A operands of Wk and dU
  __bf16 dO[BT][LPS]; // the chunk's output cotangent rows (exact bf16; zero past T, V)
};

// The chunk's output cotangent rows into LDS, two 8-column pieces per thread:
// with VEC (V a multiple of 8; rows are then 16-byte aligned) one 16-byte load
// per piece, otherwise element by element (clamped address + mask).  A missing
// cotangent stages zeros.
template <bool VEC>
__device__ __forceinline__ void stage_dout_rows(const BwdParams& p, int b, int t0, int hh,
                                                __bf16 (*dst)[LPS]) {
  constexpr int PER = BT * KD / 8 / CT;
  bf16x8 v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 8, i = idx / KD, c = idx % KD, t = t0 + i;
    if constexpr (VEC) {
      const bool ok = p.dout != nullptr && t < p.T && c < p.V;
      const __bf16* base = p.dout ? p.dout : sd_zero_bf16x8;
      const long long o = p.dout ? (((long long)b * p.T + (t < p.T ? t : p.T - 1)) * p.H + hh) *
                                           p.V + (c < p.V ? c : p.V - 8)
                                 : 0;
      const bf16x8 raw = *reinterpret_cast<const bf16x8*>(base + o);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[q][e] = (__bf16)keep_if(ok, bf2f(raw[e]));
    } else {
      DoutRaw r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = dout_raw(p, b, t, hh, c + e);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[q][e] = (__bf16)dout_val(r[e]);
    }
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 8;
    *reinterpret_cast<bf16x8*>(&dst[idx / KD][idx % KD]) = v[q];
  }
}

// A fragment of an fp16 panel, re-split into bf16 high + low halves (exact:
// fp16's 11-bit significand fits the two bf16 halves) for the 3-term product.
__device__ __forceinline__ Frag ldfrag_h(const _Float16* p, long long off) {
  const f16x8 v = *reinterpret_cast<const f16x8*>(p + off);
  Frag f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    __bf16 a, b;
    split_bf((float)v[e], a, b);
    f.h[e] = a;
    f.l[e] = b;
  }
  return f;
}
static_assert(2 * BT * LS >= BT * KD, "P + N hold a 64 x 128 panel");

template <bool VEC, bool FL>  // FL: the call has token flags (sd_inputs.fresh)
__global__ __launch_bounds__(CT) void k_bprep_s(BwdParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  BprepSSmem& s = *reinterpret_cast<BprepSSmem*>(smem_raw);
  // chunk-major dispatch, first chunk first: the last chunk, where the reverse
  // state pass starts right after this kernel, is written last
  const int n = blockIdx.x, ch = blockIdx.y, b = n / p.H, hh = n % p.H, t0 = ch * BT;
  float xdec[BS];  // the decay column's loads go out first: their latency overlaps dO's
  decay_load(gptr(p.in, b, hh), p.in.log_decay.st, t0, p.T, p.r, xdec, FL ? tok_flag_row(p.in, b) : nullptr,
             tok_flag_st(p.in));
  stage_dout_rows<VEC>(p, b, t0, hh, s.dO);  // read below after the first barrier
  decay_build(s.cd, xdec);
  const ChunkDecay& cd = s.cd;
  const long long cidx = (long long)n * p.NT + ch, rowbase = (long long)n * p.Tp + t0;
  {
    constexpr int PA = BT * BT / CT;
    float av[PA];
    _Float16 pv[PA];
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      av[q] = p.f.As[cidx * BT * BT + threadIdx.x + q * CT];
      const int idx = threadIdx.x + q * CT;
      pv[q] = p.f.Ps[cidx * BT * BT + frag_off(idx / BT, idx % BT, BT)];
    }
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      const int idx = threadIdx.x + q * CT;
      s.A[(idx / BT) * LS + idx % BT] = av[q];
      s.P[(idx / BT) * LS + idx % BT] = (float)pv[q];
    }
  }
  __syncthreads();
  mat64_mul(s.P, s.A, s.N);
  __syncthreads();
  {  // A^T, N^T split once (each wave would otherwise split all of them)
    constexpr int PER = BT * BT / CT;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int idx = threadIdx.x + q * CT, j = idx / BT, k = idx % BT;
      __bf16 a, b2;
      split_bf(s.A[k * LS + j], a, b2);
      s.At.h[j][k] = a;
      s.At.l[j][k] = b2;
      split_bf(s.N[k * LS + j], a, b2);
      s.Nt.h[j][k] = a;
      s.Nt.l[j][k] = b2;
    }
  }
  __syncthreads();
  const int w = wave_id(), l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
  const long long kbase = cidx * KD * BT;
  f4 wks[NB], dus[NB];
  {
    const int cb = w;
    // B operands, shared by the four output blocks: dO (exact in bf16, so its
    // split has no low part) gathered over the chunk's tokens, and the stored
    // split key panel K^ read as ready-made fragments.
    bf16x8 db[2];
    Frag kf[2];
    const fpan_t* const dp = p.f.d + rowbase * KD;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float kv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        db[ks][e] = s.dO[ks * 32 + kq + e][cb * 16 + m];
        kv[e] = (float)dp[(ks * 32 + kq + e) * KD + cb * 16 + m];
      }
      // the decayed keys K^_i = d_i e^{G_C - G_i} of the forward's S pass, formed
      // again from the saved d (the exponent is <= 0)
      const int c = cb * 16 + m;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        kv[e] *= __expf(cd.G[BT - 1][c] - cd.G[ks * 32 + kq + e][c]);
      kf[ks] = split8(kv);
    }
#pragma unroll
    for (int Jb = 0; Jb < NB; ++Jb) {
      // dU_j = sum_l N_lj dO_l ;  Wk_j = sum_i A_ij K^_i
      f4 du = zero4(), wk = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 nh = *reinterpret_cast<const bf16x8*>(&s.Nt.h[Jb * BS + m][ks * 32 + kq]);
        const bf16x8 nl = *reinterpret_cast<const bf16x8*>(&s.Nt.l[Jb * BS + m][ks * 32 + kq]);
        du = __builtin_amdgcn_mfma_f32_16x16x32_bf16(nl, db[ks], du, 0, 0, 0);
        du = __builtin_amdgcn_mfma_f32_16x16x32_bf16(nh, db[ks], du, 0, 0, 0);
        Frag af;
        af.h = *reinterpret_cast<const bf16x8*>(&s.At.h[Jb * BS + m][ks * 32 + kq]);
        af.l = *reinterpret_cast<const bf16x8*>(&s.At.l[Jb * BS + m][ks * 32 + kq]);
        wk = mma3f(af, kf[ks], wk);
      }
      dus[Jb] = du;
      wks[Jb] = wk;
    }
  }
  // The chunk-transposed panels' loads are issued before the dU and Wk stores
  // below (a load issued after a store waits for it: one counter retires both).
  // Fragment order: a thread's two pieces are (state row c, tokens i0 .. i0+7).
  constexpr int NPC = KD * BT / 8 / CT;
  float ev[NPC][8];
  _Float16 qv[NPC][8];
#pragma unroll
  for (int q = 0; q < NPC; ++q) {
    const int pc = threadIdx.x + q * CT, block = pc >> 6, lane = pc & 63;
    const int c = (block / (BT / 32)) * 16 + (lane & 15);
    const int i0 = (block % (BT / 32)) * 32 + (lane >> 4) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = i0 + e;
      ev[q][e] = (float)p.f.e[(rowbase + i) * KD + c];
      qv[q][e] = p.f.chi[(rowbase + i) * KD + c];  // Q~ = chi e^G, scaled below
    }
  }
  store_du_slab(p.g.dU + rowbase * KD, dus);
  // Wk staged in the free P / N rows, then stored in fragment order
  __syncthreads();
  {
    float* Wst = s.P;  // 64 x 128 fits in P and N
#pragma unroll
    for (int Jb = 0; Jb < NB; ++Jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) Wst[(Jb * BS + out_row(e)) * KD + w * 16 + out_col()] = wks[Jb][e];
    __syncthreads();
    store_frag_panel1<BT, KD>(p.g.Wk, rowbase * KD,
                             [&](int i, int c) { return Wst[i * KD + c]; });
  }
  {
#pragma unroll
    for (int q = 0; q < NPC; ++q) {
      const int pc = threadIdx.x + q * CT, block = pc >> 6, lane = pc & 63;
      const int c = (block / (BT / 32)) * 16 + (lane & 15);
      const int i0 = (block % (BT / 32)) * 32 + (lane >> 4) * 8;
      bf16x8 ah, qh, dh;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float eg = __expf(cd.G[i0 + e][c]);
        ah[e] = (__bf16)(-ev[q][e] * eg);
        qh[e] = (__bf16)((float)qv[q][e] * eg);  // Q~ = chi e^G, transposed, bf16
        dh[e] = s.dO[i0 + e][c];  // exact in bf16
      }
      const long long ot = cidx * KD * BT + (long long)pc * 8;
      *reinterpret_cast<bf16x8*>(p.g.Ant + ot) = ah;
      *reinterpret_cast<bf16x8*>(p.g.At1 + ot) = qh;
      *reinterpret_cast<bf16x8*>(p.g.B1t + ot) = dh;
    }
  }
}

// Lambda-block load for the key product, fused with the decay closure's row
// sums: wave cb loads rows cb*16 .. cb*16+15 of lambda (split for the MFMA) and
// the same elements of X_C, and leaves rowsum_c(X_C (.) lambda) partials (one
// per 32-column lane group) in rsum[g][c], so the closure need not read either
// 64 KiB block again.
__device__ __forceinline__ void lam_rowsum(const Blk& rl, const Blk& rx, int cb, BlkS& BL,
                                           float (*rsum)[KD]) {
  float acc = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      acc += rl.v[ks][h].x * rx.v[ks][h].x + rl.v[ks][h].y * rx.v[ks][h].y +
             rl.v[ks][h].z * rx.v[ks][h].z + rl.v[ks][h].w * rx.v[ks][h].w;
  const int l = lane_id();
  rsum[l >> 4][cb * 16 + (l & 15)] = acc;
  split_blk(rl, BL);
}

__device__ __forceinline__ void load_lam_rowsum(const lslot_t* lam, const xslot_t* XC, int cb, BlkS& BL,
                                                float (*rsum)[KD]) {
  Blk rl, rx;
  load_blk(rl, lam + cb * 16 * KD, KD);
  load_blk(rx, XC + cb * 16 * KD, KD);
  lam_rowsum(rl, rx, cb, BL, rsum);
}

// Decay-gradient closure for this wave's 16 columns, in registers: v holds the
// un-summed decay cotangent of column c = cb*16 + (l & 15) at rows
// 16 I + 4 (l >> 4) + e; it becomes the reverse cumulative sum over the chunk's
// rows plus rowsum_c(X_C (.) lambda) (from the partials load_lam_rowsum left in
// rsum).  The four lane groups exchange their block sums with shuffles.
__device__ __forceinline__ void close_decay_column(float (&v)[NB][4], const float (*rsum)[KD], int cb) {
  const int l = lane_id(), g = l >> 4, c = cb * 16 + (l & 15);
  float later[NB], tot[NB];
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    const float t = v[I][0] + v[I][1] + v[I][2] + v[I][3];
    const float s1 = __shfl(t, (l + 16) & 63), s2 = __shfl(t, (l + 32) & 63),
                s3 = __shfl(t, (l + 48) & 63);
    later[I] = keep_if(g < 3, s1) + keep_if(g < 2, s2) + keep_if(g < 1, s3);  // groups after g
    tot[I] = (t + s1) + (s2 + s3);
  }
  float acc = rsum[0][c] + rsum[1][c] + rsum[2][c] + rsum[3][c];  // carry from later blocks
#pragma unroll
  for (int I = NB - 1; I >= 0; --I) {
    float run = acc + later[I];
#pragma unroll
    for (int e = 3; e >= 0; --e) {
      run += v[I][e];
      v[I][e] = run;
    }
    acc += tot[I];
  }
}

struct GradSmem {
  ChunkDecay cd;
  float M1[BT * LS];
  float M2[BT * LS];
  float rsum[4][KD];  // rowsum(X_C (.) lambda) partials
  LPanel PA;  // dw, then dO
  LPanel PW;  // w
};

template <bool FL>
__global__ __launch_bounds__(CT) void k_grad_s(BwdParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  GradSmem& s = *reinterpret_cast<GradSmem*>(smem_raw);
  const int ch = blockIdx.x, n = blockIdx.y, b = n / p.H, hh = n % p.H, t0 = ch * BT;
  const long long rowbase = (long long)n * p.Tp + t0;
  const long long sidx = (long long)n * (p.NT + 1) + ch;
  const bpan_t* dw = p.g.dwS + rowbase * KD;
  const fpan_t* wv = p.f.wS + rowbase * KD;
  const fpan_t* dd_ = p.f.d + rowbase * KD;
  const fpan_t* ee = p.f.e + rowbase * KD;
  const fpan_t* chi = p.f.chi + rowbase * KD;
  const xslot_t* X0 = p.f.Xs + sidx * KD * KD;
  const xslot_t* XC = X0 + KD * KD;
  const lslot_t* lam = p.g.Ls + sidx * KD * KD;
  DoutPanelRaw doraw;  // the output cotangent's loads go out first
  dout_panel_load(p, b, t0, hh, doraw);
  // dw and dO are exact in bf16: PA holds dw in its high rows and dO in its low
  // rows (neither has a low half), so both Grams with w run in one pass
  stage_panel_bf(s.PA.h, dw);
  stage_panel(s.PW, wv);
  dout_panel_store(s.PA.l, p, t0, doraw);
  build_decay(s.cd, gptr(p.in, b, hh), p.in.log_decay.st, t0, p.T, p.r, FL ? tok_flag_row(p.in, b) : nullptr,
              tok_flag_st(p.in));  // ends with a barrier
  const ChunkDecay& cd = s.cd;
  const int w = wave_id(), l = lane_id(), cb = w, c = cb * 16 + (l & 15), r4 = (l >> 4) * 4;
  // this wave's X0 row block: loads issued ahead of the M1 Gram so their latency
  // overlaps it
  Blk bX0;
  load_blk(bX0, X0 + cb * 16 * KD, KD);
  // M1_ij = dw_i . w_j (j < i) and M2_li = dO_l . w_i (l >= i), one pass
  lds_pair2_h(s.PA, s.PW, s.M1, s.M2);
  // a = dw X0^T, bq = dO X0^T for this wave's column block (K = 128);  kl = w lam^T
  f4 a[NB], bq[NB], kl[NB];
  BlkS BX;
  split_blk(bX0, BX);
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    BlkH A;
    lblk_h(s.PA, I * BS, A);
    a[I] = mma_blks_h(A, BX, zero4());
  }
  {
    BlkS BL;
    load_lam_rowsum(lam, XC, cb, BL, s.rsum);
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      BlkH Ah;
      lblk_l(s.PA, I * BS, Ah);
      bq[I] = mma_blks_h(Ah, BX, zero4());
      BlkS A;
      lblk(s.PW, I * BS, A);
      kl[I] = mma_blks_bh(A, BL, zero4());  // lambda is a bf16 slot
    }
  }
  // kl is consumed only by pass B: park it in the dead PA panel (lane-private
  // slots) so it holds no registers through pass A.
  float* const kl_park = reinterpret_cast<float*>(&s.PA);
  static_assert(sizeof(LPanel) >= NB * 4 * CT * sizeof(float), "kl park slot");
  __syncthreads();  // every wave is done reading PA
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int e = 0; e < 4; ++e) kl_park[(I * 4 + e) * CT + threadIdx.x] = kl[I][e];
  auto D = [&](int j, int cc) { return (float)dd_[j * KD + cc]; };
  auto E = [&](int j, int cc) { return (float)ee[j * KD + cc]; };
  auto Q = [&](int j, int cc) { return (float)chi[j * KD + cc]; };
  Tab1 t1;
  RowF rf;
  ColF cf;
  make_tab1(cd, cb, t1);
  make_rowf<false>(cd, cb, rf);
  make_colf(cd, cb, cf);
  // This wave's d, e, chi slabs, loaded once for both passes (no global loads
  // between the passes' stores, which would wait for them).
  float Sd[NB][4], Se[NB][4], Sq[NB][4], pdg[NB][4];
  load_slab(Sd, dd_, cb);
  load_slab(Se, ee, cb);
  load_slab(Sq, chi, cb);
  // Pass A: de = -(e^G (dw X0^T) + apply(M1, d)),  dchi = e^G (dO X0^T) + apply(M2, d);
  // the decay terms chi.dchi + e.de of dg
  // Chunk-uniform output bases with 32-bit lane offsets: 64-bit per-row
  // addresses would not fit in registers beside the slabs.
  bpan_t* const de_b = p.g.de + rowbase * KD;
  bpan_t* const dchi_b = p.g.dchi + rowbase * KD;
  bpan_t* const dd_b = p.g.dd + rowbase * KD;
  {
    __syncthreads();  // M1, M2 complete
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      f4 ap, bp;
      apply2_tab<false>(cd, s.M1, s.M2, Sd, I, cb, t1, rf, cf, D, ap, bp);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = I * BS + r4 + e;
        const float eg = __expf(cd.G[i][c]);
        const float dev = -(eg * a[I][e] + ap[e]), dcv = eg * bq[I][e] + bp[e];
        a[I][e] = dev;  // results take the registers of the products they consume
        bq[I][e] = dcv;
        pdg[I][e] = Sq[I][e] * dcv + Se[I][e] * dev;
      }
    }
    // Stores after the pass: a store issued before a register reload would make
    // the reload wait for it (loads and stores share one counter).
#pragma unroll
    for (int I = 0; I < NB; ++I)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned o = (unsigned)((I * BS + r4 + e) * KD + c);
        de_b[o] = a[I][e];
        dchi_b[o] = bq[I][e];
      }
  }
  // Pass B: dd = e^{G_C - G} (w lam^T) + apply_t(M2, chi) - apply_t(M1, e); dg -= d.dd
  {
#pragma unroll
    for (int I = 0; I < NB; ++I)
#pragma unroll
      for (int e = 0; e < 4; ++e) kl[I][e] = kl_park[(I * 4 + e) * CT + threadIdx.x];
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      f4 k2, k3;
      apply_t2_tab<false>(cd, s.M2, Sq, s.M1, Se, I, cb, t1, rf, cf, Q, E, k2, k3);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = I * BS + r4 + e;
        const float ddv = __expf(cd.G[BT - 1][c] - cd.G[i][c]) * kl[I][e] + k2[e] - k3[e];
        kl[I][e] = ddv;
        pdg[I][e] -= Sd[I][e] * ddv;
      }
    }
    close_decay_column(pdg, s.rsum, cb);
    // the S side's log-decay gradient goes straight to the output; the C side's
    // chunk gradient adds its own part to it
    float* const dgo = p.dg + ((long long)b * p.T * p.H + hh) * p.r + c;
    const long long tstride = (long long)p.H * p.r;
#pragma unroll
    for (int I = 0; I < NB; ++I)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = I * BS + r4 + e, t = t0 + i;
        dd_b[(unsigned)(i * KD + c)] = kl[I][e];
        if (t < p.T && c < p.r) dgo[t * tstride] = pdg[I][e];
      }
  }
}

// ---------------------------------------------------------------------------
// Row pieces: in the per-token closures lane cl = l & 15 of DPP row l >> 4
// holds the eight consecutive columns 8 cl .. 8 cl + 7 of its token's rows, so
// a wave takes four tokens and each row reduction is four in-row DPP adds.
// With VEC (the width a multiple of 8 and every row 16-byte aligned: the
// launcher checks) a piece is one 16-byte load or store; otherwise the same
// eight columns move element by element (clamped address + mask), so both
// variants compute bitwise the same.  Workspace panels are always aligned.
// ---------------------------------------------------------------------------
template <bool VEC>
__device__ __forceinline__ void ld_piece(const __bf16* row, bool tv, int w, float (&x)[8]) {
  const int c0 = 8 * (lane_id() & 15);
  if constexpr (VEC) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(row + (c0 < w ? c0 : w - 8));
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = keep_if(tv && c0 < w, bf2f(v[e]));
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = c0 + e;
      x[e] = keep_if(tv && c < w, bf2f(row[c < w ? c : w - 1]));
    }
  }
}
template <class E>
__device__ __forceinline__ void ld_panel_piece(const E* row, float keep, float (&x)[8]) {
  typedef E V8 __attribute__((ext_vector_type(8)));
  const V8 v = *reinterpret_cast<const V8*>(row + 8 * (lane_id() & 15));
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = keep * (float)v[e];
}
// The same piece selected (not scaled) by tv: rows that were never written read as 0.
template <class E>
__device__ __forceinline__ void ld_panel_piece_sel(const E* row, bool tv, float (&x)[8]) {
  typedef E V8 __attribute__((ext_vector_type(8)));
  const V8 v = *reinterpret_cast<const V8*>(row + 8 * (lane_id() & 15));
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = keep_if(tv, (float)v[e]);
}
template <class E>
__device__ __forceinline__ void st_panel_piece(E* row, const float (&x)[8]) {
  typedef E V8 __attribute__((ext_vector_type(8)));
  V8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (E)x[e];
  *reinterpret_cast<V8*>(row + 8 * (lane_id() & 15)) = v;
}
// A bf16 output row of width w (columns past w are not written).
template <bool VEC>
__device__ __forceinline__ void st_piece(__bf16* row, int w, const float (&x)[8]) {
  const int c0 = 8 * (lane_id() & 15);
  if constexpr (VEC) {
    if (c0 < w) st_panel_piece(row, x);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (c0 + e < w) row[c0 + e] = f2bf(x[e]);
  }
}

// ---------------------------------------------------------------------------
// Sources transpose (row pieces, four waves of four tokens per workgroup, no
// LDS): phi, den, e, chi, z and the q / erase / write / value gates closed
// against the S side's cotangents de, dchi, dw, dd (the closed forms of
// tests/chunk_model.py::sources_bwd).  Writes dq, derase, dv, dwrite, the
// partial du / dk into the du / dk gradients (closed in place by the C chunk
// gradient's tail) and ddelta over dw (read by the C op's backward prep).  A
// padded token reads the last valid token's (finite) panel rows and masks
// them, and its own dw row selected to zero: its ddelta row comes out zero.
// ---------------------------------------------------------------------------
template <bool VEC, bool FL>
__global__ __launch_bounds__(NTHREADS) void k_src_bwd(BwdParams p) {
  // No multiply-add contraction: left to the compiler, the two row layouts'
  // instantiations fused different products and their partial du differed in
  // the last bit on rare inputs; unfused, both compute bitwise the same.
#pragma clang fp contract(off)
  const int n = blockIdx.y, b = n / p.H, hh = n % p.H;
  const int t = blockIdx.x * 16 + wave_id() * 4 + (lane_id() >> 4);
  const int r = p.r, V = p.V, T = p.T, c0 = 8 * (lane_id() & 15);
  const bool tv = t < T;
  const int tc = tv ? t : T - 1;
  const long long row = ((long long)n * p.Tp + (t < p.Tp ? t : p.Tp - 1)) * KD;
  // a padded token's panel rows may hold anything: it reads the last valid
  // token's (finite) rows and masks them
  const long long vrow = ((long long)n * p.Tp + tc) * KD;
  const float keep = tv ? 1.f : 0.f;
  float u[8], k[8], q[8], er[8], wr[8], v[8], d[8], de[8], dc[8], dz[8], dd[8];
  ld_piece<VEC>(brow(p.in.u, b, tc, hh), tv, r, u);
  ld_piece<VEC>(brow(p.in.k, b, tc, hh), tv, r, k);
  ld_piece<VEC>(brow(p.in.q, b, tc, hh), tv, r, q);
  const float om = operand_keep_at<FL>(p.in, b, tc);  // invalid tokens' q and keys read 0
  ld_piece<VEC>(brow(p.in.erase_raw, b, tc, hh), tv, r, er);
  ld_piece<VEC>(brow(p.in.write_raw, b, tc, hh), tv, V, wr);
  ld_piece<VEC>(brow(p.in.v, b, tc, hh), tv, V, v);
  ld_panel_piece(p.f.delta + vrow, keep, d);
  ld_panel_piece(p.g.de + vrow, keep, de);
  ld_panel_piece(p.g.dchi + vrow, keep, dc);
  // dw_S from this token's own row: ddelta is written over it below
  ld_panel_piece_sel(p.g.dwS + row, tv, dz);
  ld_panel_piece(p.g.dd + vrow, keep, dd);
  if (t >= p.Tp) return;  // past the padded chunk: nothing to write
  auto rsum = [](float (&x)[8], const float (&y)[8]) {
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) a += x[e] * y[e];
    return row16_sum(a);
  };
  auto normalise = [&](float (&x)[8]) {
    const float rs = rsqrtf(rsum(x, x) + 1e-24f);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= rs;
    return rs;
  };
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    k[e] *= om;
    q[e] *= om;
  }
  normalise(u);
  normalise(k);
  const float rq = normalise(q);
  const float usq = rsum(u, u);
  const float dsq = rsum(d, d);
  const float N = sqrtf(RHO * RHO + usq * dsq);
  const float sc = RHO / N;
  float pv[8], se[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pv[e] = sc * d[e];
    se[e] = 1.f / (1.f + __expf(-er[e]));
    bv[e] = se[e] * k[e];
  }
  const float den = 1.f + rsum(pv, u);
  const float sb = rsum(u, bv) / den;
  const float sq = rsum(u, q) / den;
  // e = b - phi sb ; chi = q - phi sq
  const float dsb = -rsum(pv, de);
  const float dsq_ = -rsum(pv, dc);
  const float dub = dsb / den, duq = dsq_ / den;
  const float dden = -(dsb * sb + dsq_ * sq) / den;
  float dph[8], duh[8], dqh[8], der[8], dkh[8], dvv[8], dwr[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dph[e] = -sb * de[e] - sq * dc[e] + dden * u[e];
    duh[e] = dub * bv[e] + duq * q[e] + dden * pv[e];
    const float db = de[e] + dub * u[e];
    dqh[e] = dc[e] + duq * u[e];
    dkh[e] = db * se[e] + dd[e];
    der[e] = db * k[e] * se[e] * (1.f - se[e]);
    // z = sigmoid(wr) v
    const float sw = 1.f / (1.f + __expf(-wr[e]));
    dvv[e] = sw * dz[e];
    dwr[e] = dz[e] * v[e] * sw * (1.f - sw);
  }
  // phi = rho delta / N,  N^2 = rho^2 + usq dsq
  const float ds = rsum(dph, d);
  const float qd = rsum(dqh, q);
  const float dN = -RHO * ds / (N * N);
  const float dN2 = dN / (2.f * N);
  float ddl[8], dq[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    ddl[e] = c0 + e < r ? sc * dph[e] + 2.f * dN2 * usq * d[e] : 0.f;
    duh[e] += 2.f * dN2 * dsq * u[e];
    // q L2 norm transpose
    dq[e] = (dqh[e] - qd * q[e]) * rq;
  }
  st_panel_piece(p.g.ddelta + row, ddl);
  if (!tv) return;
  const long long tok = ((long long)b * T + t) * p.H + hh;
  // partial du / dk, closed in place by the C chunk gradient's tail
  st_piece<VEC>(p.du + tok * r, r, duh);
  st_piece<VEC>(p.dk + tok * r, r, dkh);
  st_piece<VEC>(p.dq + tok * r, r, dq);
  st_piece<VEC>(p.der + tok * r, r, der);
  st_piece<VEC>(p.dv + tok * V, V, dvv);
  st_piece<VEC>(p.dwr + tok * V, V, dwr);
}

// ---------------------------------------------------------------------------
// C predictor
// ---------------------------------------------------------------------------
struct BprepCSmem {
  ChunkDecay cd;
  float A[BT * LS];
  float P[BT * LS];
  float N[BT * LS];
  float Uh[BT][GS];
  float Kh[BT][GS];
  float gam[BT];   // erase-side gamma: 0 on fresh tokens
  float krs[BT];  // 1 / |k_i|
};

template <bool FL>
__global__ __launch_bounds__(CT) void k_bprep_c(BwdParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  BprepCSmem& s = *reinterpret_cast<BprepCSmem*>(smem_raw);
  // chunk-major dispatch, first chunk first: the last chunk, where the reverse
  // state pass starts right after this kernel, is written last
  const int n = blockIdx.x, ch = blockIdx.y, b = n / p.H, hh = n % p.H, t0 = ch * BT;
  const ChunkDecay& cd = s.cd;
  const long long cidx = (long long)n * p.NT + ch, rowbase = (long long)n * p.Tp + t0;
  const int w = wave_id(), l = lane_id();
{
    // every load of the opening phase first (the decay column, then every
    // row's u and k), then the decay table's build
    const int cl = l & 15;  // 16-lane rows: every row's loads before the first reduction
    // the chunk's (I+L)^-1 (its LDS copy is written after the decay build)
    static_assert(BT * BT == 2 * 4 * CT, "two 16-byte pieces of (I+L)^-1 per thread");
    const float4 av0 = *reinterpret_cast<const float4*>(p.f.Ac + cidx * BT * BT + threadIdx.x * 4);
    const float4 av1 = *reinterpret_cast<const float4*>(p.f.Ac + cidx * BT * BT + (threadIdx.x + CT) * 4);
    float xdec[BS];
    decay_load(gptr(p.in, b, hh), p.in.log_decay.st, t0, p.T, p.r, xdec, FL ? tok_flag_row(p.in, b) : nullptr,
             tok_flag_st(p.in));
    float ux[2][RQ], kx[2][RQ], km[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int t = t0 + row16(w, g);
      ld_row16(brow(p.in.u, b, t < p.T ? t : p.T - 1, hh), t < p.T, p.r, ux[g]);
      ld_row16(brow(p.in.k, b, t < p.T ? t : p.T - 1, hh), t < p.T, p.r, kx[g]);
      km[g] = operand_keep_at<FL>(p.in, b, t < p.T ? t : p.T - 1);  // invalid: keys read 0
    }
    if (threadIdx.x < BT) {  // clamped token, then select (a guarded load would branch and wait)
      const int t = t0 + threadIdx.x;
      const float gv = ((const float*)p.in.gamma.data)[(long long)b * p.in.gamma.sb +
                                                      (long long)(t < p.T ? t : p.T - 1) * p.in.gamma.st +
                                                      (long long)hh * p.in.gamma.sh];
      const unsigned f = tok_flags(p.in, b, t < p.T ? t : p.T - 1);
      s.gam[threadIdx.x] = keep_if(t < p.T, gv) * operand_keep(f) * erase_keep_f(f);
    }
    decay_build(s.cd, xdec);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int i = row16(w, g);
#pragma unroll
      for (int q = 0; q < RQ; ++q) kx[g][q] *= km[g];
      const float ru = l2norm16(ux[g]);
      const float rk = l2norm16(kx[g]);
      if ((l & 15) == 0) {
        // 0 for an invalid token: the injection and the C chunk gradient pair
        // these with the raw (unmasked) key rows
        s.krs[i] = rk * km[g];
        // the C chunk gradient scales the raw rows by these (0 past T)
        const bool tv = t0 + i < p.T;
        *reinterpret_cast<float2*>(p.g.rn + (rowbase + i) * 2) =
            make_float2(tv ? ru : 0.f, tv ? rk * km[g] : 0.f);
      }
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        s.Uh[i][cl + 16 * q] = ux[g][q];
        s.Kh[i][cl + 16 * q] = kx[g][q];
      }
    }
    {
      const int i0 = threadIdx.x * 4, i1 = (threadIdx.x + CT) * 4;
      *reinterpret_cast<float4*>(&s.A[(i0 / BT) * LS + i0 % BT]) = av0;
      *reinterpret_cast<float4*>(&s.A[(i1 / BT) * LS + i1 % BT]) = av1;
    }
  }
  __syncthreads();
  const bpan_t* ddp = p.g.dd + rowbase * KD;
  // P'_li = sum_c dd_lc u_ic e^{G_lc - G_ic}, i <= l
  static_assert(sizeof(bpan_t) == 2, "dd is a bf16 panel");
  decayed_gram_gx<false>(cd, ddp, [&](int j, int c) { return s.Uh[j][c]; }, false, s.P);
  mat64_mul(s.P, s.A, s.N);
  __syncthreads();
  const bpan_t* ddl = p.g.ddelta + rowbase * KD;
  const long long kbase = cidx * KD * BT;
  f4 wks[NB], dus[NB];
  {
    const int cb = w, m = l & 15, kq = (l >> 4) * 8;
    // B operands, shared by the four output blocks: ddelta (global) and the
    // normalised keys (LDS) split once, the stored split key panel K^ read as
    // ready-made fragments.
    Frag bd[2], bk[2], kf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float vd[8], vk[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vd[e] = ddl[(ks * 32 + kq + e) * KD + cb * 16 + m];
        vk[e] = s.Kh[ks * 32 + kq + e][cb * 16 + m];
      }
      bd[ks] = split8(vd);
      bk[ks] = split8(vk);
      // the C op's decayed keys K^_i = u^_i e^{G_C - G_i} (exponent <= 0), formed
      // from the normalised u in LDS instead of a saved forward panel
      float vu[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vu[e] = s.Uh[ks * 32 + kq + e][cb * 16 + m] *
                __expf(cd.G[BT - 1][cb * 16 + m] - cd.G[ks * 32 + kq + e][cb * 16 + m]);
      kf[ks] = split8(vu);
    }
#pragma unroll
    for (int Jb = 0; Jb < NB; ++Jb) {
      // dU_j = sum_i A_ij ddelta_i + sum_l N_lj k_l ;  Wk_j = sum_i A_ij K^_i
      f4 du = zero4(), wk = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks == 0 && Jb >= 2) continue;  // A and N are lower: tokens < 32 reach only j < 32
        float va[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) va[e] = s.A[(ks * 32 + kq + e) * LS + Jb * BS + m];
        const Frag fa = split8(va);
        du = mma2f_bh(fa, bd[ks], du);  // ddelta is a bf16 panel
        wk = mma3f(fa, kf[ks], wk);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks == 0 && Jb >= 2) continue;
        float vn[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vn[e] = s.N[(ks * 32 + kq + e) * LS + Jb * BS + m];
        du = mma3f(split8(vn), bk[ks], du);
      }
      dus[Jb] = du;
      wks[Jb] = wk;
    }
  }
  // The global inputs of the chunk-transposed panels below (dd for At1, the
  // raw keys for B1t) are loaded before this kernel's stores: a load issued
  // after a store waits for it (one counter retires both).  Fragment order: a
  // thread's pieces are (state row c, tokens i0 .. i0+7).
  constexpr int PIECES = KD * BT / 8, PER = PIECES / CT;
  static_assert(PIECES % CT == 0, "whole pieces per thread");
  float ddv[PER][8];
  __bf16 kr[PER][8];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int pc = threadIdx.x + q * CT, block = pc >> 6, lane = pc & 63;
    const int c = (block / (BT / 32)) * 16 + (lane & 15);
    const int i0 = (block % (BT / 32)) * 32 + (lane >> 4) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {  // clamped address + mask: no guarded load
      const int t = t0 + i0 + e;
      ddv[q][e] = (float)ddp[(i0 + e) * KD + c];
      const float v = bf2f(brow(p.in.k, b, t < p.T ? t : p.T - 1, hh)[c < p.r ? c : p.r - 1]);
      kr[q][e] = (__bf16)keep_if(t < p.T && c < p.r, v);
    }
  }
  // P' is also the C chunk gradient's dq operand: stored once here (upper
  // blocks zero) instead of formed again there, after every load of the kernel
  for (int idx = threadIdx.x * 4; idx < BT * BT; idx += CT * 4) {
    const int i = idx / BT, j = idx % BT;
    const float4 v = *reinterpret_cast<const float4*>(&s.P[i * LS + j]);
    *reinterpret_cast<float4*>(p.g.Pp + cidx * BT * BT + idx) =
        (j / BS > i / BS) ? make_float4(0.f, 0.f, 0.f, 0.f) : v;
  }
  store_du_slab(p.g.dU + rowbase * KD, dus);
  __syncthreads();
  {
    float* Wst = s.P;  // 64 x 128 fits in P and N
#pragma unroll
    for (int Jb = 0; Jb < NB; ++Jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) Wst[(Jb * BS + out_row(e)) * KD + w * 16 + out_col()] = wks[Jb][e];
    __syncthreads();
    store_frag_panel1<BT, KD>(p.g.Wk, rowbase * KD,
                             [&](int i, int c) { return Wst[i * KD + c]; });
  }
  // chunk-transposed panels, fragment order
  // The reverse pass's injection sum_i At1_ci Kh_i,col is formed as
  // sum_i (At1_ci / |k_i|) k_i,col: its B operand is then the raw key input,
  // exact in bf16, so only a high half is stored (and read).
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int pc = threadIdx.x + q * CT, block = pc >> 6, lane = pc & 63;
    const int c = (block / (BT / 32)) * 16 + (lane & 15);
    const int i0 = (block % (BT / 32)) * 32 + (lane >> 4) * 8;
    bf16x8 a, h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = (__bf16)(ddv[q][e] * __expf(cd.G[i0 + e][c]) * s.krs[i0 + e]);
      h[e] = kr[q][e];
    }
    *reinterpret_cast<bf16x8*>(p.g.At1 + cidx * KD * BT + (long long)pc * 8) = a;
    *reinterpret_cast<bf16x8*>(p.g.B1t + cidx * KD * BT + (long long)pc * 8) = h;
  }
  store_frag_panel1<KD, BT>(p.g.Ant, cidx * KD * BT, [&](int c, int i) {
    return -s.gam[i] * s.Uh[i][c] * __expf(gx_excl(cd, i, c));
  });
}

// ---------------------------------------------------------------------------
// Final closure of a four-token group (16-lane row layout, rows i = row16(w, g)):
// u, k, h and gamma, from the C chunk gradient's dx, dk, dq rows (bf16, in its
// LDS, row stride KD), the C reverse pass's dw and the sources transpose's
// partial du / dk.  All of the group's global loads are issued first.
// ---------------------------------------------------------------------------
struct FinRows {
  float u[RQ], k[RQ], h[RQ], dv[RQ], us[RQ], ks[RQ];
  float gm, xk, om;  // gamma, erase keep (0 on fresh tokens), operand keep (0 on invalid)
};

template <bool VEC>
__device__ __forceinline__ void final_load(const BwdParams& p, int b, int hh, long long rowbase,
                                           int i, int t, FinRows& x) {
  const int T = p.T;
  const bool tv = t < T;
  const int tc = tv ? t : T - 1;
  ld_piece<VEC>(brow(p.in.u, b, tc, hh), tv, p.r, x.u);
  ld_piece<VEC>(brow(p.in.k, b, tc, hh), tv, p.r, x.k);
  ld_piece<VEC>(brow(p.in.h, b, tc, hh), tv, p.r, x.h);
  x.gm = ((const float*)p.in.gamma.data)[(long long)b * p.in.gamma.sb +
                                         (long long)tc * p.in.gamma.st +
                                         (long long)hh * p.in.gamma.sh];
  // the erase read x = gamma u^ is dropped on fresh tokens: its cotangent dx
  // reaches neither u nor gamma there; an invalid token's keys and gamma read 0
  const unsigned f = tok_flags(p.in, b, tc);
  x.xk = erase_keep_f(f);
  x.om = operand_keep(f);
  const long long prow = (rowbase + (tc - (t - i))) * KD;
  ld_panel_piece(p.g.dwC + prow, 1.f, x.dv);
  // the sources transpose's partial du / dk, in the gradients this tail overwrites
  const long long tok = ((long long)b * T + tc) * p.H + hh;
  ld_piece<VEC>(p.du + tok * p.r, tv, p.r, x.us);
  ld_piece<VEC>(p.dk + tok * p.r, tv, p.r, x.ks);
}

template <bool VEC>
__device__ __forceinline__ void final_close(const BwdParams& p, int b, int hh, int t,
                                            FinRows& x, const __bf16* dx_row,
                                            const __bf16* dk_row, const __bf16* dq_row) {
  // no multiply-add contraction: both row layouts' instantiations compute the
  // same bits (see k_src_bwd)
#pragma clang fp contract(off)
  const int r = p.r, c0 = 8 * (lane_id() & 15);
  const bool tv = t < p.T;
  float dx[RQ], du[RQ], dk[RQ];
  x.gm *= x.om;
#pragma unroll
  for (int q = 0; q < RQ; ++q) x.k[q] *= x.om;
  {
    const bf16x8 vx = *reinterpret_cast<const bf16x8*>(dx_row + c0);
    const bf16x8 vk = *reinterpret_cast<const bf16x8*>(dk_row + c0);
    const bf16x8 vq = *reinterpret_cast<const bf16x8*>(dq_row + c0);
#pragma unroll
    for (int q = 0; q < RQ; ++q) {
      dx[q] = x.xk * bf2f(vx[q]);
      du[q] = x.us[q] + bf2f(vk[q]) + x.gm * dx[q];
      dk[q] = x.ks[q] + bf2f(vq[q]);
    }
  }
  const float ru = l2norm16(x.u);
  const float rk = l2norm16(x.k);
  float g = 0.f, ud = 0.f, kd = 0.f;
#pragma unroll
  for (int q = 0; q < RQ; ++q) {
    g += x.u[q] * dx[q] + x.h[q] * x.dv[q];
    ud += du[q] * x.u[q];
    kd += dk[q] * x.k[q];
  }
  const float dgam = row16_sum(g);
  ud = row16_sum(ud);
  kd = row16_sum(kd);
  if (!tv) return;
  const long long tok = ((long long)b * p.T + t) * p.H + hh;
  float ou[RQ], ok[RQ], oh[RQ];
#pragma unroll
  for (int q = 0; q < RQ; ++q) {
    ou[q] = (du[q] - ud * x.u[q]) * ru;
    ok[q] = (dk[q] - kd * x.k[q]) * rk;
    oh[q] = x.gm * x.dv[q];
  }
  st_piece<VEC>(p.du + tok * r, r, ou);
  st_piece<VEC>(p.dk + tok * r, r, ok);
  st_piece<VEC>(p.dh + tok * r, r, oh);
  if ((lane_id() & 15) == 0) p.dgam[tok] = dgam;
}

struct GradCSmem {
  ChunkDecay cd;
  float M1[BT * LS];
  float M2[BT * LS];
  float gam[BT];      // erase-side gamma: 0 on fresh tokens
  float rn[BT][2];    // 1 / |u_i|, 1 / |k_i| (0 past T)
  float rsum[4][KD];  // rowsum(X_C (.) lambda) partials
  LPanel PA;  // dw, then dd e^G
  LPanel PW;  // delta
};

// Normalised u / k of the C chunk gradient, from the raw inputs and the norms
// the backward prep stored: one element (row j of the chunk, column c), and
// the 16 x 128 block of rows j0 .. j0+15 as split MFMA fragments (VEC: 16-byte
// row pieces; the element form reads the same values one by one).
__device__ __forceinline__ float norm_elem(const sd_view& v, int b, int hh, int t, int T, int r,
                                          int c, float rn) {
  const float x = bf2f(brow(v, b, t < T ? t : T - 1, hh)[c < r ? c : r - 1]);
  return keep_if(t < T && c < r, x) * rn;
}

// The raw rows t0 .. t0+63 of a bf16 input view copied into dst ([BT][LPS]
// rows, exact in bf16; padded tokens and columns >= r read 0), 16-byte row
// pieces with VEC, element by element otherwise (the same values).
template <bool VEC>
__device__ __forceinline__ void stage_raw_rows(__bf16 (*dst)[LPS], const sd_view& v, int b, int hh, int t0,
                                               int T, int r) {
  constexpr int PER = BT * KD / 8 / CT;
  bf16x8 x[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int pc = threadIdx.x + q * CT, i = pc / (KD / 8), c0 = (pc % (KD / 8)) * 8, t = t0 + i;
    const __bf16* row = brow(v, b, t < T ? t : T - 1, hh);
    if constexpr (VEC) {
      const bf16x8 pv = *reinterpret_cast<const bf16x8*>(row + (c0 < r ? c0 : r - 8));
      x[q] = (t < T && c0 < r) ? pv : bf16x8{};
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = c0 + e;
        const __bf16 val = row[c < r ? c : r - 1];
        x[q][e] = (t < T && c < r) ? val : (__bf16)0.f;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int pc = threadIdx.x + q * CT, i = pc / (KD / 8), c0 = (pc % (KD / 8)) * 8;
    *reinterpret_cast<bf16x8*>(&dst[i][c0]) = x[q];
  }
}

template <bool VEC, bool FL>
__global__ __launch_bounds__(CT) void k_grad_c(BwdParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  GradCSmem& s = *reinterpret_cast<GradCSmem*>(smem_raw);
  const int ch = blockIdx.x, n = blockIdx.y, b = n / p.H, hh = n % p.H, t0 = ch * BT;
  const long long rowbase = (long long)n * p.Tp + t0;
  const long long sidx = (long long)n * (p.NT + 1) + ch;
  const int w = wave_id(), l = lane_id(), cb = w, c = cb * 16 + (l & 15), r4 = (l >> 4) * 4;
  const bpan_t* dw = p.g.dwC + rowbase * KD;
  const fpan_t* wv = p.f.delta + rowbase * KD;
  const bpan_t* ddp = p.g.dd + rowbase * KD;  // cotangent of the C-op output
  const fpan_t* dprim = p.f.d + rowbase * KD;  // d = k + output
  const xslot_t* X0 = p.f.Xc + sidx * KD * KD;
  const xslot_t* XC = X0 + KD * KD;
  const lslot_t* lam = p.g.Lc + sidx * KD * KD;
  if (threadIdx.x < BT) {
    const int t = t0 + threadIdx.x;
    {  // clamped token, then select (a guarded load would branch and wait)
      const float gv = ((const float*)p.in.gamma.data)[(long long)b * p.in.gamma.sb +
                                                      (long long)(t < p.T ? t : p.T - 1) * p.in.gamma.st +
                                                      (long long)hh * p.in.gamma.sh];
      const unsigned f = tok_flags(p.in, b, t < p.T ? t : p.T - 1);
      s.gam[threadIdx.x] = keep_if(t < p.T, gv) * operand_keep(f) * erase_keep_f(f);
    }
    *reinterpret_cast<float2*>(s.rn[threadIdx.x]) =
        *reinterpret_cast<const float2*>(p.g.rn + (rowbase + threadIdx.x) * 2);
  }
  // dw and the raw keys are exact in bf16: PA holds dw in its high rows and the
  // raw keys in its low rows, so the M1 and M2 Grams run in one pass
  stage_panel_bf(s.PA.h, dw);
  stage_raw_rows<VEC>(s.PA.l, p.in.k, b, hh, t0, p.T, p.r);
  stage_panel(s.PW, wv);
  build_decay(s.cd, gptr(p.in, b, hh), p.in.log_decay.st, t0, p.T, p.r, FL ? tok_flag_row(p.in, b) : nullptr,
              tok_flag_st(p.in));  // ends with a barrier
  const ChunkDecay& cd = s.cd;
  // this wave's X0, lambda and X_C row blocks: loads issued ahead of the two
  // LDS Grams so their latency overlaps them
  Blk bX0, bLam, bXC;
  load_blk(bX0, X0 + cb * 16 * KD, KD);
  load_blk(bLam, lam + cb * 16 * KD, KD);
  load_blk(bXC, XC + cb * 16 * KD, KD);
  // M1_ij = dw_i . delta_j (j < i);  M2_li = k^_l . delta_i = (k_l . delta_i) / |k_l|
  // (l >= i): the raw keys are exact bf16 A operands, the norm scales the rows
  // afterwards (rn is read after build_decay's barrier)
  lds_pair2_h(s.PA, s.PW, s.M1, s.M2, [&](int i) { return s.rn[i][1]; });
  f4 a[NB], kl[NB];
  {
    BlkS BX, BL;
    split_blk(bX0, BX);
    lam_rowsum(bLam, bXC, cb, BL, s.rsum);
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      BlkH Ah;  // dw_C is a bf16 panel
      lblk_h(s.PA, I * BS, Ah);
      a[I] = mma_blks_h(Ah, BX, zero4());
      BlkS A;
      lblk(s.PW, I * BS, A);
      kl[I] = mma_blks_bh(A, BL, zero4());  // lambda is a bf16 slot
    }
  }
  // normalised u / k at row j of the chunk, column cc
  auto U = [&](int j, int cc) { return norm_elem(p.in.u, b, hh, t0 + j, p.T, p.r, cc, s.rn[j][0]); };
  float Su[NB][4], Sdd[NB][4], Sod[NB][4];
#pragma unroll
  for (int J = 0; J < NB; ++J)
#pragma unroll
    for (int e = 0; e < 4; ++e) Su[J][e] = U(J * BS + r4 + e, c);
  load_slab(Sdd, ddp, cb);
  {  // the C-op output o = d - k enters only as o (.) dd: formed at once, so
     // neither slab stays live through the applies
    float Sk[NB][4];
    load_slab(Sod, dprim, cb);
#pragma unroll
    for (int J = 0; J < NB; ++J)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // the raw keys staged in PA's low rows (0 past T and past r), normalised
        const int j = J * BS + r4 + e;
        Sk[J][e] = (float)s.PA.l[j][c] * s.rn[j][1];
      }
#pragma unroll
    for (int J = 0; J < NB; ++J)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Sod[J][e] = (Sod[J][e] - Sk[J][e]) * Sdd[J][e];
        // formed here: left to the compiler, the subtraction sank to its last use
        // and kept both fp16 slabs live (and spilled) through the applies
        asm volatile("" : "+v"(Sod[J][e]));
      }
  }
  Tab1 t1;
  RowF rx, ri;  // exclusive / inclusive row factors
  ColF cf;
  make_tab1(cd, cb, t1);
  make_rowf<true>(cd, cb, rx);
  make_rowf<false>(cd, cb, ri);
  make_colf(cd, cb, cf);
  // PA <- dd e^G for the dq product (staged once PA is free, consumed after the
  // applies): dd's row pieces are loaded before the barrier
  constexpr int DPC = BT * KD / 8 / CT;  // 16-byte dd pieces per thread
  bf16x8 ddr[DPC];
#pragma unroll
  for (int q = 0; q < DPC; ++q) ddr[q] = *reinterpret_cast<const bf16x8*>(ddp + (threadIdx.x + q * CT) * 8);
  __syncthreads();  // M1, M2 complete; PA free
#pragma unroll
  for (int q = 0; q < DPC; ++q) {
    const int idx = (threadIdx.x + q * CT) * 8, i = idx / KD, cc = idx % KD;
    bf16x8 hh, ll;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      __bf16 a2, b2;
      split_bf((float)ddr[q][e] * __expf(cd.G[i][cc + e]), a2, b2);
      hh[e] = a2;
      ll[e] = b2;
    }
    *reinterpret_cast<bf16x8*>(&s.PA.h[i][cc]) = hh;
    *reinterpret_cast<bf16x8*>(&s.PA.l[i][cc]) = ll;
  }
  auto Xg = [&](int j, int cc) { return s.gam[j] * U(j, cc); };
  auto DO = [&](int j, int cc) { return (float)ddp[j * KD + cc]; };
  float Sx[NB][4];
#pragma unroll
  for (int J = 0; J < NB; ++J)
#pragma unroll
    for (int e = 0; e < 4; ++e) Sx[J][e] = s.gam[J * BS + r4 + e] * Su[J][e];
  // P' (formed by the C chunk's backward prep): loaded now, written into M1 as
  // soon as every apply below has read it, and used by the dq product at the end
  constexpr int PPC = BT * BT / 4 / CT;
  float4 ppv[PPC];
  {
    const float* const pp = p.g.Pp + ((long long)n * p.NT + ch) * BT * BT;
#pragma unroll
    for (int q = 0; q < PPC; ++q) ppv[q] = *reinterpret_cast<const float4*>(pp + (threadIdx.x + q * CT) * 4);
  }
  // dx and dk stay in the workgroup for the closure tail, rounded to bf16 as the
  // panels between kernels were: once the applies are done, dx goes into M2 and
  // dk into the decay tables' storage (nothing reads the decay tables after the
  // applies)
  __bf16 dxr[NB][4], dkr[NB][4];
  // decay cotangent: dg_i = o_i dd_i - u_i dk_i plus the shifted gamma u (.) dx
  // term, closed in registers below (v = dg + xdx, then dg = suffix(v) - xdx)
  float vv[NB][4], xs[NB][4];
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    const f4 ap = apply_tab<true>(cd, s.M1, Su, I, cb, t1, rx, cf, U);
    const f4 k2 = apply_t_tab<false>(cd, s.M2, Sdd, I, cb, t1, ri, cf, DO);
    const f4 k3 = apply_t_tab<true>(cd, s.M1, Sx, I, cb, t1, rx, cf, Xg);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = I * BS + r4 + e;
      const float dx = -(__expf(gx_excl(cd, i, c)) * a[I][e] + ap[e]);
      const float dk = __expf(cd.G[BT - 1][c] - cd.G[i][c]) * kl[I][e] + k2[e] - k3[e];
      dxr[I][e] = f2bf(dx);
      dkr[I][e] = f2bf(dk);
      xs[I][e] = Sx[I][e] * dx;
      vv[I][e] = Sod[I][e] - Su[I][e] * dk + xs[I][e];
    }
  }
  // the dq product's X0 column block (K = 128 rows of X0): gathered now so the
  // latency overlaps the stores and the decay closure below (issued before the
  // applies, the gathers were held through them and spilled)
  __builtin_amdgcn_sched_barrier(0);
  Blk x0raw;
  {
    const int kq = (l >> 4) * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (float)X0[(ks * 32 + kq + e) * KD + c];
      x0raw.v[ks][0] = make_float4(v[0], v[1], v[2], v[3]);
      x0raw.v[ks][1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  __syncthreads();  // every apply has read M1 and M2
#pragma unroll
  for (int q = 0; q < PPC; ++q) {
    const int idx = (threadIdx.x + q * CT) * 4;
    *reinterpret_cast<float4*>(&s.M1[(idx / BT) * LS + idx % BT]) = ppv[q];
  }
  __bf16* const dxl = reinterpret_cast<__bf16*>(s.M2);  // [64][128] bf16 fits M2's 64 x 68 floats
  __bf16* const dkl = reinterpret_cast<__bf16*>(&s.cd);  // and the decay tables' 37 KB
  static_assert(sizeof(ChunkDecay) >= BT * KD * sizeof(__bf16), "dk fits the decay tables");
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dxl[(I * BS + r4 + e) * KD + c] = dxr[I][e];
      dkl[(I * BS + r4 + e) * KD + c] = dkr[I][e];
    }
  // dg_i = rowsum + sum_{i' >= i} dg_i' + sum_{i' > i} xdx_i'
  close_decay_column(vv, s.rsum, cb);
  // the C side's part of the log-decay gradient, added to the S side's (written
  // by the S chunk gradient) with a return-free atomic: the add happens in L2, so
  // nothing is loaded here, and with exactly one add per element on top of one
  // store the sum is deterministic
  {
    float* const dgo = p.dg + ((long long)b * p.T * p.H + hh) * p.r + c;
    const long long tstride = (long long)p.H * p.r;
#pragma unroll
    for (int I = 0; I < NB; ++I)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = t0 + I * BS + r4 + e;
        if (t < p.T && c < p.r) unsafeAtomicAdd(&dgo[t * tstride], vv[I][e] - xs[I][e]);
      }
  }
  __syncthreads();  // P' in M1; PA (dd e^G) staged
  // dq = (dd e^G) X0 + P' delta, from the X0 column block gathered above
  f4 dqs[NB];
  {
    BlkS BX;
    split_blk(x0raw, BX);
    // P' delta: the delta column block's stored hi / lo halves are the B operand
    // as they are (gathered once for the four row blocks)
    Frag pw[2];
    {
      const int m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pw[ks].h[e] = s.PW.h[ks * 32 + kq + e][cb * 16 + m];
          pw[ks].l[e] = s.PW.l[ks * 32 + kq + e][cb * 16 + m];
        }
    }
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      BlkS A;
      lblk(s.PA, I * BS, A);
      f4 dq = mma_blks(A, BX, zero4());
      const int m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks == 1 && I < 2) break;  // P' is lower triangular: rows < 32 reach tokens < 32
        float va[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) va[e] = s.M1[(I * BS + m) * LS + ks * 32 + kq + e];
        dq = mma3f(split8(va), pw[ks], dq);
      }
      dqs[I] = dq;
    }
  }
  __syncthreads();  // PA, PW and M1 read by every wave: dq takes PA's low half
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int e = 0; e < 4; ++e) s.PA.l[I * BS + r4 + e][c] = f2bf(dqs[I][e]);
  // closure of u, k, h and gamma: this wave's two four-token groups
  FinRows f0, f1;
  final_load<VEC>(p, b, hh, rowbase, row16(w, 0), t0 + row16(w, 0), f0);
  final_load<VEC>(p, b, hh, rowbase, row16(w, 1), t0 + row16(w, 1), f1);
  __syncthreads();
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int i = row16(w, g);
    final_close<VEC>(p, b, hh, t0 + i, g ? f1 : f0, dxl + i * KD, dkl + i * KD, s.PA.l[i]);
  }
}

// ---------------------------------------------------------------------------
int launch_bwd(const sd_inputs* in, const FwdWs& fw, const BwdWs& bw, const void* dout,
               const float* dC_T, const float* dS_T, void* du, void* dh, void* dq, void* dk,
               void* dv, void* derase, void* dwrite, float* dlog_decay, float* dgamma,
               float* dC0, float* dS0, hipStream_t st) {
  const int n = in->B * in->H, NT = (in->T + BT - 1) / BT, Tp = NT * BT;
  // the sources transpose takes whole 16-byte row pieces when every row allows it
  auto al16 = [](const sd_view& v) {
    return ((uintptr_t)v.data & 15) == 0 && v.sb % 8 == 0 && v.st % 8 == 0 && v.sh % 8 == 0;
  };
  const bool src_vec = in->r % 8 == 0 && in->V % 8 == 0 && al16(in->u) && al16(in->k) &&
                       al16(in->q) && al16(in->erase_raw) && al16(in->write_raw) && al16(in->v) &&
                       ((uintptr_t)dq & 15) == 0 && ((uintptr_t)derase & 15) == 0 &&
                       ((uintptr_t)dv & 15) == 0 && ((uintptr_t)dwrite & 15) == 0 &&
                       ((uintptr_t)du & 15) == 0 && ((uintptr_t)dk & 15) == 0;
  // so does the C chunk gradient's closure tail
  const bool fin_vec = in->r % 8 == 0 && al16(in->u) && al16(in->k) && al16(in->h) &&
                       ((uintptr_t)du & 15) == 0 && ((uintptr_t)dk & 15) == 0 &&
                       ((uintptr_t)dh & 15) == 0;
  BwdParams p{};
  p.in = *in;
  p.H = in->H; p.T = in->T; p.r = in->r; p.V = in->V; p.NT = NT; p.Tp = Tp;
  p.f = fw;
  p.g = bw;
  p.dout = (const __bf16*)dout;
  p.du = (__bf16*)du; p.dh = (__bf16*)dh; p.dq = (__bf16*)dq; p.dk = (__bf16*)dk;
  p.dv = (__bf16*)dv; p.der = (__bf16*)derase; p.dwr = (__bf16*)dwrite;
  p.dg = dlog_decay; p.dgam = dgamma;
  // kernels that read token flags are separate instantiations (FL): a call
  // without flags runs no flag code at all
  const bool fl = in->fresh.data != nullptr;
#define SD_BWD_LAUNCH(name, K, grid, blk, smem)  \
  do {                                            \
    SD_SMEM_ONCE(K, (int)(smem));                 \
    SD_LAUNCH(name, K, grid, blk, smem, st, p);   \
  } while (0)
#define SD_BWD_LAUNCH_FL(name, K, grid, blk, smem)                  \
  do {                                                              \
    if (fl) SD_BWD_LAUNCH(name, (K<true>), grid, blk, smem);        \
    else SD_BWD_LAUNCH(name, (K<false>), grid, blk, smem);          \
  } while (0)
#define SD_BWD_LAUNCH_VFL(name, K, vec, grid, blk, smem)                  \
  do {                                                                    \
    if (vec) {                                                            \
      if (fl) SD_BWD_LAUNCH(name, (K<true, true>), grid, blk, smem);      \
      else SD_BWD_LAUNCH(name, (K<true, false>), grid, blk, smem);        \
    } else {                                                              \
      if (fl) SD_BWD_LAUNCH(name, (K<false, true>), grid, blk, smem);     \
      else SD_BWD_LAUNCH(name, (K<false, false>), grid, blk, smem);       \
    }                                                                     \
  } while (0)
  const dim3 chunks(NT, n), blk(NTHREADS), cblk(CT);
  // S memory
  const dim3 chunks_cm(n, NT);  // chunk-major grid of the backward preps
  SD_BWD_LAUNCH_VFL("k_bprep_s", k_bprep_s, in->V % 8 == 0, chunks_cm, cblk, sizeof(BprepSSmem));
  StateParams ss{};
  ss.H = in->H; ss.T = in->T; ss.NT = NT; ss.Tp = Tp; ss.rows = in->r; ss.cols = in->V;
  ss.rev = 1;
  ss.Wneg = bw.Wk; ss.U = bw.dU; ss.Kt = bw.Ant; ss.Gam = fw.Gam;
  ss.At1 = bw.At1; ss.B1 = bw.B1t;  // B1t = dO, exact in bf16
  ss.Xs = bw.Ls; ss.wout = bw.dwS;
  ss.init = dS_T; ss.init_transposed = 0;
  ss.fin = dS0; ss.fin_transposed = 0;
  launch_state("state_s_bwd", ss, n, st);
  SD_BWD_LAUNCH_FL("k_grad_s", k_grad_s, chunks, cblk, sizeof(GradSmem));
  SD_BWD_LAUNCH_VFL("k_src_bwd", k_src_bwd, src_vec, dim3(Tp / 16, n), blk, 0);
  // C predictor
  SD_BWD_LAUNCH_FL("k_bprep_c", k_bprep_c, chunks_cm, cblk, sizeof(BprepCSmem));
  StateParams sc{};
  sc.H = in->H; sc.T = in->T; sc.NT = NT; sc.Tp = Tp; sc.rows = in->r; sc.cols = in->r;
  sc.rev = 1;
  sc.Wneg = bw.Wk; sc.U = bw.dU; sc.Kt = bw.Ant; sc.Gam = fw.Gam;
  sc.At1 = bw.At1; sc.B1 = bw.B1t;  // B1t = raw keys, exact in bf16
  sc.Xs = bw.Lc; sc.wout = bw.dwC;
  sc.init = dC_T; sc.init_transposed = 1;
  sc.fin = dC0; sc.fin_transposed = 1;
  launch_state("state_c_bwd", sc, n, st);
  SD_BWD_LAUNCH_VFL("k_grad_c", k_grad_c, fin_vec, chunks, cblk, sizeof(GradCSmem));
#undef SD_BWD_LAUNCH_VFL
#undef SD_BWD_LAUNCH_FL
#undef SD_BWD_LAUNCH
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

}  // namespace sd
