// Forward chunk kernels of the SolveDelta recurrence (gfx950).
//
// Pipeline for one call (n = b*H + h sequences, NT chunks of 64 tokens):
//   k_prep_c   (chunk-parallel) predictor C: norms, decayed Gram L_C, (I+L_C)^-1,
//              WY panels W_C, U_C, decayed keys, chunk decay;
//   k_state<false, false> (sequential per sequence x 16-column tile) C state
//              pass: delta = U - W X0, X <- Gamma X + K^T delta (X = C^T);
//   k_prep_s   (chunk-parallel) primal d = k + C^T k, dual sources e, chi, z,
//              then the S memory's Gram, inverse, WY panels and output pair P;
//   k_state<false, true> S state pass: chunk-entering slots and w, and the
//              readout o = Q~ X0 + P w of each chunk from the same X0 and w.
// The algebra is the generic pre-decay-read delta op: see the SolveDelta
// chunk derivation restated in tests/chunk_model.py.
#include "sd_common.cuh"
#include "sd_internal.h"

namespace sd {

// ---------------------------------------------------------------------------
// helpers for strided bf16 inputs
// ---------------------------------------------------------------------------
__device__ __forceinline__ const __bf16* vrow(const sd_view& v, int b, int t, int h) {
  return (const __bf16*)v.data + (long long)b * v.sb + (long long)t * v.st + (long long)h * v.sh;
}
__device__ __forceinline__ float gamma_at(const sd_view& g, int b, int t, int h) {
  return ((const float*)g.data)[(long long)b * g.sb + (long long)t * g.st + (long long)h * g.sh];
}

// Branch-free row load (lane holds coords lane and lane+64): out-of-range tokens
// and coordinates read a valid element and are selected to 0, so unrolled loops
// can issue every load before the first use.
__device__ __forceinline__ void load_row2(const sd_view& v, int b, int t, int h, int T, int w,
                                          float& x0, float& x1) {
  const int l = lane_id();
  const bool tv = t < T;
  const __bf16* p = vrow(v, b, tv ? t : T - 1, h);
  const float a0 = bf2f(p[l < w ? l : w - 1]), a1 = bf2f(p[l + 64 < w ? l + 64 : w - 1]);
  x0 = keep_if(tv && l < w, a0);
  x1 = keep_if(tv && l + 64 < w, a1);
}

// Branch-free 16-lane row load (see load_row2), columns (l & 15) + 16 q.
__device__ __forceinline__ void load_row16(const sd_view& v, int b, int t, int h, int T, int w,
                                           float (&x)[RQ]) {
  ld_row16(vrow(v, b, t < T ? t : T - 1, h), t < T, w, x);
}

constexpr int PS = KD + 8;  // bf16 panel row stride

// ---------------------------------------------------------------------------
// k_prep_c
// ---------------------------------------------------------------------------
struct PrepCSmem {
  ChunkDecay cd;
  float M[BT * LS];
  float tmp[BT * LS];
  float Uh[BT][GS];   // normalised u
  __bf16 Hh[BT][PS];  // h (raw bf16, exact)
  float gam[BT];
  float xm[BT];       // 1, or 0 on fresh tokens (no erase read)
  LPanel Yt;          // the L Gram's Y side (u), transformed and split once
};

template <bool FL>  // FL: the call has token flags (sd_inputs.fresh)
__global__ __launch_bounds__(CT) void k_prep_c(FwdParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  PrepCSmem& s = *reinterpret_cast<PrepCSmem*>(smem_raw);
  // chunk-major dispatch, last chunk first (chunk 0, where the C state pass
  // starts, is written last)
  const int n = blockIdx.x, ch = gridDim.y - 1 - blockIdx.y;
  const int b = n / p.H, hh = n % p.H, t0 = ch * BT;
  const int T = p.T, r = p.r;
  const sd_inputs& in = p.in;
  const float* g = (const float*)in.log_decay.data + (long long)b * in.log_decay.sb +
                   (long long)hh * in.log_decay.sh;
  const int w = wave_id(), l = lane_id();
{
    // every load of the opening phase first (the decay column, then every row's
    // u and h): a row's reduction would otherwise hold the next row's loads
    // behind it, and the decay table's build would wait for its own
    const int cl = l & 15;
    float xdec[BS];
    decay_load(g, in.log_decay.st, t0, T, r, xdec, FL ? tok_flag_row(in, b) : nullptr, tok_flag_st(in));
    float ux[2][RQ], hx[2][RQ];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int t = t0 + row16(w, g);
      load_row16(in.u, b, t, hh, T, r, ux[g]);
      load_row16(in.h, b, t, hh, T, r, hx[g]);
    }
    if (threadIdx.x < BT) {  // branch-free: clamped token, then select
      const int t = t0 + threadIdx.x;
      const float gv = gamma_at(in.gamma, b, t < T ? t : T - 1, hh);
      const unsigned f = tok_flags(in, b, t < T ? t : T - 1);
      s.gam[threadIdx.x] = keep_if(t < T, gv) * operand_keep(f);  // 0 on invalid tokens
      s.xm[threadIdx.x] = erase_keep_f(f);
    }
    decay_build(s.cd, xdec);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int i = row16(w, g);
      l2norm16(ux[g]);
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        s.Uh[i][cl + 16 * q] = ux[g][q];
        s.Hh[i][cl + 16 * q] = f2bf(hx[g][q]);
      }
    }
  }
  __syncthreads();
  const ChunkDecay& cd = s.cd;
  // L_ij = gamma_i sum_c u_ic u_jc exp(G_{i-1,c} - G_jc), j < i
  stage_ytilde(s.Yt, cd, [&](int j, int c) { return s.Uh[j][c]; });
  decayed_gram_yt<true>(
      cd, [&](int i, int c) { return s.gam[i] * s.xm[i] * s.Uh[i][c]; }, s.Yt,
      [&](int j, int c) { return s.Uh[j][c]; }, true, s.M);
  unit_lower_inverse(s.M, s.tmp);
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT)
    p.Ac[((long long)n * p.NT + ch) * BT * BT + idx] = s.M[(idx / BT) * LS + idx % BT];
  // W = A diag(gamma) (u e^{Gexcl} masked on fresh tokens),  U = A diag(gamma) h
  const long long rowbase = (long long)n * p.Tp + t0;
  {
    const int cb = w;
    // B operands, the same for every row block I: formed and split once
    const int m = l & 15, kq = (l >> 4) * 8;
    bf16x8 bh[2], bl[2], hb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = ks * 32 + kq + e, c = cb * 16 + m;
        __bf16 h, lo;
        split_bf(s.xm[k] * s.Uh[k][c] * __expf(gx_excl(cd, k, c)), h, lo);
        bh[ks][e] = h;
        bl[ks][e] = lo;
        hb[ks][e] = s.Hh[k][c];  // h is the raw bf16 input: exact
      }
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      const int K = I < 2 ? 32 : 64;
      f4 aw = zero4(), au = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks * 32 >= K) break;
        bf16x8 ah, al;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = ks * 32 + kq + e;
          __bf16 h, lo;
          split_bf(s.M[(I * BS + m) * LS + k] * s.gam[k], h, lo);
          ah[e] = h;
          al[e] = lo;
        }
        aw = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh[ks], aw, 0, 0, 0);
        au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, hb[ks], au, 0, 0, 0);
        aw = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl[ks], aw, 0, 0, 0);
        aw = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh[ks], aw, 0, 0, 0);
        au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, hb[ks], au, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const long long row = rowbase + I * BS + out_row(e);
        const int c = cb * 16 + out_col();
        p.Wc[rowbase * KD + frag_off(I * BS + out_row(e), c, KD)] = (_Float16)(-aw[e]);
        p.Uc[row * KD + c] = au[e];
      }
    }
  }
  // decayed keys (transposed per chunk) and chunk decay
  const long long cbase = ((long long)n * p.NT + ch);
  store_frag_panel1<KD, BT>(p.Kc, cbase * KD * BT, [&](int c, int i) {
    return s.Uh[i][c] * __expf(cd.G[BT - 1][c] - cd.G[i][c]);
  });
  if (threadIdx.x < KD) p.Gam[cbase * KD + threadIdx.x] = __expf(cd.G[BT - 1][threadIdx.x]);
}

// ---------------------------------------------------------------------------
// k_state: sequential chunk pass over one 16-column tile of the state.
//   X <- state [KD x 16] in MFMA accumulators (wave w owns rows 32w..32w+31)
//   per chunk: slot[ch] = X;  w = U + Wneg X;
//              X = Gamma X + Kt w (+ At1 B1)
// Operand layouts (all fp32, K contiguous so each lane's 8-element fragment is
// two 16-byte loads): Wneg, Q, U token-major [Tp][128]; Kt, At1 chunk-transposed
// [128][64]; B1 chunk-transposed [128 cols][64 tokens]; P [64][64].
// The next chunk's fragments are loaded into registers while the current chunk
// computes, so the global latency leaves the sequential critical path.
// ---------------------------------------------------------------------------
// State workgroup geometry: 4 waves (one per SIMD) own a 128 x SCOLS state tile
// split into HALVES 16-column halves; wave w holds state rows 32w..32w+31 (SRB = 2
// row blocks) of every half in MFMA accumulators and computes the w / o tiles of
// token block w.  KD / SCOLS workgroups cover a sequence's state columns; every
// one of them reads the chunk's full W and K panels, so wider tiles mean less
// panel traffic per chunk step.
constexpr int SCOLS = 16;
constexpr int HALVES = SCOLS / 16;
constexpr int SWAVES = 4;
constexpr int SRB = KD / 16 / SWAVES;
constexpr int STHREADS = SWAVES * 64;
constexpr int STILES = KD / SCOLS;
// State-pass prefetch buffers (PF - 1 chunks ahead).  Deeper rings measured no
// faster on the forward passes and push the reverse passes past 512 registers.
constexpr int PF = 3;

// fp32 staging row stride: 16-byte aligned rows, and the four 16-lane groups of
// an MFMA output tile (rows 4 apart) land on distinct LDS banks.
constexpr int XFS = SCOLS + 4;

// Operand types of the two pass kinds.  Forward (REV false): the W and K panels
// are fp16 (11-bit mantissa; both are bounded by construction: W = -(I+L)^-1
// x~ and K = k e^{G_C - G} with unit-norm or decayed rows), the state X and w
// are split into fp16 high + low halves (~22 bits), two f16 MFMAs per product.
// Reverse (REV true): the panels are bf16 (the exponent range of bf16 keeps any
// scale of the output cotangent representable), the cotangent state lambda and
// dw split into bf16 halves, two bf16 MFMAs per product; the injection A1 B1 is
// one bf16 MFMA (B1 is exact in bf16).
template <bool REV> struct StateT;
template <> struct StateT<false> {
  using Slot = xslot_t;
  using Wout = fpan_t;
  using E = _Float16;
  using V8 = f16x8;
  using V4 = f16x4;
  static __device__ __forceinline__ f4 mma(V8 a, V8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct StateT<true> {
  using Slot = lslot_t;
  using Wout = bpan_t;
  using E = __bf16;
  using V8 = bf16x8;
  using V4 = bf16x4;
  static __device__ __forceinline__ f4 mma(V8 a, V8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <bool REV>
struct StateSmem {
  using E = typename StateT<REV>::E;
  E Xh[SCOLS][KD + 8];  // X0 tile, transposed [col][row], split high / low
  E Xl[SCOLS][KD + 8];
  E wh[SCOLS][BT + 8];  // w tile, transposed [col][token], split high / low
  E wl[SCOLS][BT + 8];
  // fp32 copies of the X0 slot and the w tile, row-major, written back to global
  // memory as 16-byte pieces: a wave may hold at most 63 memory operations in
  // flight, and the prefetch ring needs that budget more than scalar stores do.
  float Xf[KD][XFS];
  float wf[BT][XFS];
  float Uf[BT][XFS];  // U tile, staged from one 16-byte load per thread
  float of[BT][XFS];  // readout tile of the previous chunk (forward S pass), stored one step later
  float Gf[KD];       // chunk decay, staged from one 16-byte load per lane of wave 0
  // reverse passes: the injection's B1 fragments, loaded by wave 0 only and shared
  // (every wave multiplies its own At1 rows by the same B1 tile)
  bf16x8 B1s[REV ? HALVES : 1][2][64];
};

template <bool REV, bool OUT>
struct StateFrags {
  using V8 = typename StateT<REV>::V8;
  V8 W[4];
  V8 Q[OUT ? 4 : 1];  // readout operands (forward S pass): Q~ rows of this wave's token block
  V8 P[OUT ? 2 : 1];  // and the same rows of P
  V8 K[SRB][2];
  bf16x8 A1[REV ? SRB : 1][2];
  bf16x8 B1[REV ? HALVES : 1][2];
  float4 U4;  // U tile piece: token threadIdx / (SCOLS / 4), columns 4 (threadIdx % (SCOLS / 4))
  float4 G4;  // chunk decay, columns 4 threadIdx .. +3 (threads < 32: the only ones that stage it)
};

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ bf16x8 ldb8(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
template <class V8, class E>
__device__ __forceinline__ V8 ldv8(const E* p) { return *reinterpret_cast<const V8*>(p); }

// Fragment groups of a chunk, loaded by mask so a pass can spread its loads
// over a step (a burst of them stalls the wave at issue).
enum : unsigned { FW = 1, FUG = 2, FK = 4, FQ = 8, FP = 16, FA1 = 32, FB1 = 64, FALL = 127 };

template <bool REV, bool OUT>
__device__ __forceinline__ void load_state_frags(const StateParams& p, int n, int ch, int tile,
                                                 StateFrags<REV, OUT>& f, unsigned mask) {
  using E = typename StateT<REV>::E;
  using V8 = typename StateT<REV>::V8;
  const int w = wave_id(), l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
  const int tb = w;  // this wave's token block
  const long long cidx = (long long)n * p.NT + ch;
  const long long rowbase = (long long)n * p.Tp + (long long)ch * BT;
  const long long wb = rowbase * KD;
  const E* Wp = static_cast<const E*>(p.Wneg);
  const E* Kp = static_cast<const E*>(p.Kt);
  if (mask & FW)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) f.W[ks] = ldv8<V8>(Wp + wb + frag_off(tb * 16 + m, ks * 32 + kq, KD));
  if constexpr (OUT) {
    static_assert(!REV, "the readout runs in the forward S pass");
    if (mask & FQ)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) f.Q[ks] = ldv8<V8>(p.Q + wb + frag_off(tb * 16 + m, ks * 32 + kq, KD));
    if (mask & FP)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        f.P[ks] = ldv8<V8>(p.P + cidx * BT * BT + frag_off(tb * 16 + m, ks * 32 + kq, BT));
  }
  if (mask & FK)
#pragma unroll
    for (int q = 0; q < SRB; ++q)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        f.K[q][ks] = ldv8<V8>(Kp + cidx * KD * BT + frag_off((SRB * w + q) * 16 + m, ks * 32 + kq, BT));
  if (mask & FUG) {
    constexpr int C4 = SCOLS / 4;
    static_assert(BT * C4 == STHREADS, "one U piece per thread");
    f.U4 = ld4(p.U + (rowbase + threadIdx.x / C4) * KD + tile * SCOLS + (threadIdx.x % C4) * 4);
    if (threadIdx.x < KD / 4) f.G4 = ld4(p.Gam + cidx * KD + threadIdx.x * 4);
  }
  if constexpr (REV) {
    if (mask & FA1)
#pragma unroll
      for (int q = 0; q < SRB; ++q)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          f.A1[q][ks] = ldb8(p.At1 + cidx * KD * BT + frag_off((SRB * w + q) * 16 + m, ks * 32 + kq, BT));
    if ((mask & FB1) && threadIdx.x < 64)
#pragma unroll
      for (int h = 0; h < HALVES; ++h)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          f.B1[h][ks] =
              ldb8(p.B1 + cidx * KD * BT + frag_off(tile * SCOLS + h * 16 + m, ks * 32 + kq, BT));
  }
}

// Where a pass issues the next chunk's fragment groups: before the step
// (pre) and at its three phases (after its start, after the first barrier,
// after the second).  Measured per pass on MI355X.
template <bool REV, bool OUT> struct LoadPlan;
template <> struct LoadPlan<false, false> {  // C forward
  static constexpr unsigned pre = 0, part[3] = {FW | FUG, FK, 0};
};
template <> struct LoadPlan<false, true> {  // S forward with the readout: W, U and the
  // decay before the step, Q~ and K^ after its start, P after the first barrier
  static constexpr unsigned pre = FW | FUG, part[3] = {FQ | FK, FP, 0};
};
template <> struct LoadPlan<true, false> {  // reverse passes
  static constexpr unsigned pre = 0, part[3] = {FW | FUG, FK | FB1, FA1};
};

// Splits four fp32 values into high / low halves of type E and stores each as
// one 8-byte piece.
template <class E, class V4>
__device__ __forceinline__ void stage_split4(E* hi, E* lo, f4 v) {
  V4 h, l;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const E a = (E)v[e];
    h[e] = a;
    l[e] = (E)(v[e] - (float)a);
  }
  *reinterpret_cast<V4*>(hi) = h;
  *reinterpret_cast<V4*>(lo) = l;
}

// Stores the readout tile a step staged in s.of (chunk ch, 64 tokens x 16
// columns) as bf16: one 16-byte piece per thread of the first 128 when the
// output rows allow it (p.out_vec: V a multiple of 8 and a 16-byte aligned
// base), element by element otherwise.  Called after a barrier that follows
// the staging writes and precedes the next ones.
template <bool REV>
__device__ __forceinline__ void store_readout(const StateParams& p, const StateSmem<REV>& s, int n,
                                              int ch, int tile) {
  const int b = n / p.H, hh = n % p.H;
  if (threadIdx.x >= BT * 2) return;
  const int tok = threadIdx.x >> 1, c8 = (threadIdx.x & 1) * 8, t = ch * BT + tok;
  const int col = tile * SCOLS + c8;
  if (t >= p.T) return;
  __bf16* dst = p.out + (((long long)b * p.T + t) * p.H + hh) * p.cols + col;
  if (p.out_vec && col + 8 <= p.cols) {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = f2bf(s.of[tok][c8 + e]);
    *reinterpret_cast<bf16x8*>(dst) = v;
  } else {
    for (int e = 0; e < 8 && col + e < p.cols; ++e) dst[e] = f2bf(s.of[tok][c8 + e]);
  }
}

// One chunk of the sequential pass with its operand fragments already in registers.
// With OUT (forward S pass) the step also forms the chunk's readout
// o = Q~ X0 + P w for its 16 columns: wave w's token block, from the X0 and w
// fragments the recurrence loads anyway; o is off the recurrence's critical path.
template <bool REV, bool OUT, class Prefetch>
__device__ __forceinline__ void state_step(const StateParams& p, StateSmem<REV>& s, int n, int ch,
                                           int tile, const StateFrags<REV, OUT>& cur,
                                           f4 (&X)[SRB][HALVES], Prefetch&& prefetch) {
  prefetch(0);
  static_assert(!OUT || HALVES == 1, "readout tiles are 16 columns wide");
  using T = StateT<REV>;
  using E = typename T::E;
  using V8 = typename T::V8;
  using V4 = typename T::V4;
  const int NS = p.NT + 1;
  const int w = wave_id(), l = lane_id(), m = l & 15, kq = (l >> 4) * 8, r4 = (l >> 4) * 4;
  const int tb = w;
  const long long sidx = (long long)n * NS + ch;
  const long long rowbase = (long long)n * p.Tp + (long long)ch * BT;
  // save X0 and stage it split and transposed ([col][row]) for the B operand
#pragma unroll
  for (int q = 0; q < SRB; ++q)
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      const int row0 = (SRB * w + q) * 16 + r4;
#pragma unroll
      for (int e = 0; e < 4; ++e) s.Xf[row0 + e][h * 16 + m] = X[q][h][e];
      stage_split4<E, V4>(&s.Xh[h * 16 + m][row0], &s.Xl[h * 16 + m][row0], X[q][h]);
    }
  *reinterpret_cast<float4*>(&s.Uf[threadIdx.x / (SCOLS / 4)][(threadIdx.x % (SCOLS / 4)) * 4]) = cur.U4;
  if (threadIdx.x < KD / 4) *reinterpret_cast<float4*>(&s.Gf[threadIdx.x * 4]) = cur.G4;
  if constexpr (REV) {
    if (threadIdx.x < 64)
#pragma unroll
      for (int h = 0; h < HALVES; ++h)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) s.B1s[h][ks][threadIdx.x] = cur.B1[h][ks];
  }
  __syncthreads();
  prefetch(1);
  if (p.Xs) {  // slot write-back: 128 rows x SCOLS columns, four elements per piece
    using S = typename StateT<REV>::Slot;
    typedef S S4 __attribute__((ext_vector_type(4)));
    constexpr int C4 = SCOLS / 4;
#pragma unroll
    for (int j = 0; j < KD * C4 / STHREADS; ++j) {
      const int idx = threadIdx.x + j * STHREADS, row = idx / C4, c4 = idx % C4;
      const float4 v = *reinterpret_cast<const float4*>(&s.Xf[row][c4 * 4]);
      S4 o;
      o[0] = (S)v.x; o[1] = (S)v.y; o[2] = (S)v.z; o[3] = (S)v.w;
      *reinterpret_cast<S4*>(static_cast<S*>(p.Xs) + sidx * KD * KD + (long long)row * KD +
                             tile * SCOLS + c4 * 4) = o;
    }
  }
  if constexpr (OUT) {
    if (ch > 0) store_readout(p, s, n, ch - 1, tile);
  }
  // w = U + Wneg X0 (token block tb, each half).  The work that does not depend
  // on this chunk's w -- Gamma X (+ At1 B1) -- is issued alongside so the
  // independent MFMA chains overlap.
  f4 acc[HALVES], ao = zero4();
#pragma unroll
  for (int h = 0; h < HALVES; ++h)
    acc[h] = {s.Uf[tb * 16 + r4][h * 16 + m], s.Uf[tb * 16 + r4 + 1][h * 16 + m],
              s.Uf[tb * 16 + r4 + 2][h * 16 + m], s.Uf[tb * 16 + r4 + 3][h * 16 + m]};
  // every X0 fragment is read before the first product: left to itself the
  // scheduler interleaves the reads with the MFMA chain and exposes one LDS
  // latency per product
  V8 xh[HALVES][4], xl[HALVES][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      xh[h][ks] = ldv8<V8>(&s.Xh[h * 16 + m][ks * 32 + kq]);
      xl[h][ks] = ldv8<V8>(&s.Xl[h * 16 + m][ks * 32 + kq]);
    }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      acc[h] = T::mma(cur.W[ks], xl[h][ks], acc[h]);
      if constexpr (OUT) ao = T::mma(cur.Q[ks], xl[h][ks], ao);
      acc[h] = T::mma(cur.W[ks], xh[h][ks], acc[h]);
      if constexpr (OUT) ao = T::mma(cur.Q[ks], xh[h][ks], ao);
    }
#pragma unroll
  for (int q = 0; q < SRB; ++q) {
    const float4 g4 = *reinterpret_cast<const float4*>(&s.Gf[(SRB * w + q) * 16 + r4]);
    const float gv[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      for (int e = 0; e < 4; ++e) X[q][h][e] *= gv[e];
      if constexpr (REV) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          X[q][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.A1[q][ks], s.B1s[h][ks][l], X[q][h],
                                                           0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < HALVES; ++h) {
#pragma unroll
    for (int e = 0; e < 4; ++e) s.wf[tb * 16 + r4 + e][h * 16 + m] = acc[h][e];
    stage_split4<E, V4>(&s.wh[h * 16 + m][tb * 16 + r4], &s.wl[h * 16 + m][tb * 16 + r4], acc[h]);
  }
  __syncthreads();
  prefetch(2);
  {  // w write-back: 64 tokens x SCOLS columns as float4 pieces
    constexpr int C4 = SCOLS / 4;
    static_assert(BT * C4 == STHREADS, "one w piece per thread");
    const int tok = threadIdx.x / C4, c4 = threadIdx.x % C4;
    using WO = typename StateT<REV>::Wout;
    WO* dst = static_cast<WO*>(p.wout) + (rowbase + tok) * KD + tile * SCOLS + c4 * 4;
    const float4 v = *reinterpret_cast<const float4*>(&s.wf[tok][c4 * 4]);
    if constexpr (sizeof(WO) == 4) {
      *reinterpret_cast<float4*>(dst) = v;
    } else {
      typedef WO W4 __attribute__((ext_vector_type(4)));
      W4 o;
      o[0] = (WO)v.x; o[1] = (WO)v.y; o[2] = (WO)v.z; o[3] = (WO)v.w;
      *reinterpret_cast<W4*>(dst) = o;
    }
  }
  // X += Kt w: the recurrence's critical path
#pragma unroll
  for (int h = 0; h < HALVES; ++h) {
    V8 wh[2], wl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      wh[ks] = ldv8<V8>(&s.wh[h * 16 + m][ks * 32 + kq]);
      wl[ks] = ldv8<V8>(&s.wl[h * 16 + m][ks * 32 + kq]);
    }
    __builtin_amdgcn_sched_barrier(0);  // all w fragments in flight before the chain
#pragma unroll
    for (int q = 0; q < SRB; ++q)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        X[q][h] = T::mma(cur.K[q][ks], wl[ks], X[q][h]);
        X[q][h] = T::mma(cur.K[q][ks], wh[ks], X[q][h]);
      }
    if constexpr (OUT) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        ao = T::mma(cur.P[ks], wl[ks], ao);
        ao = T::mma(cur.P[ks], wh[ks], ao);
      }
    }
  }
  if constexpr (OUT) {  // o rows of token block tb, staged for the next step's store
#pragma unroll
    for (int e = 0; e < 4; ++e) s.of[tb * 16 + r4 + e][m] = ao[e];
  }
  // No closing barrier: the next step writes Xh / Xl / Xf / Uf / Gf, whose last
  // readers all ran before this step's second barrier, and writes wh / wl / wf
  // only after its own first barrier, which no wave passes before every wave
  // has finished this step's reads of them.
}

template <bool REV, bool OUT>
__global__ __launch_bounds__(STHREADS) void k_state(StateParams p) {
  __shared__ __align__(16) StateSmem<REV> s;
  const int NS = p.NT + 1;  // state slots per sequence
  // Workgroups are dispatched round-robin over the 8 XCDs by linear id; when the
  // sequence count allows, map ids so that the column tiles of a sequence run
  // on one XCD and share its L2 copy of the chunk panels.
  int tile, n;
  {
    const int L = blockIdx.x, nseq = gridDim.x / STILES;
    if (nseq % 8 == 0) {
      const int x = L % 8, j = L / 8;
      tile = j % STILES;
      n = (j / STILES) * 8 + x;
    } else {
      tile = L % STILES;
      n = L / STILES;
    }
  }
  const int w = wave_id(), l = lane_id(), m = l & 15, r4 = (l >> 4) * 4;
  f4 X[SRB][HALVES];
  for (int q = 0; q < SRB; ++q)
    for (int h = 0; h < HALVES; ++h)
      for (int e = 0; e < 4; ++e) {
        const int row = (SRB * w + q) * 16 + r4 + e, col = tile * SCOLS + h * 16 + m;
        float x = 0.f;
        if (p.init && row < p.rows && col < p.cols)
          x = p.init_transposed ? p.init[(long long)n * p.rows * p.cols + (long long)col * p.rows + row]
                                : p.init[(long long)n * p.rows * p.cols + (long long)row * p.cols + col];
        X[q][h][e] = x;
      }
  const int NT = p.NT;
  auto chunk_of = [&](int it) { return p.rev ? NT - 1 - it : it; };
  // Loaded latency of these panel fetches (several microseconds once the
  // producer's output has left the memory-side cache) exceeds a chunk step, so
  // fragments are prefetched PF - 1 chunks ahead in PF rotating register
  // buffers.  The loop body is straight-line (no breaks; clamped, unconditional
  // prefetches) so the compiler's wait counts only cover the buffer being
  // consumed; the last PF - 1 or fewer chunks run after the loop.
  auto clampc = [&](int it2) { return chunk_of(it2 < NT ? it2 : NT - 1); };
  StateFrags<REV, OUT> f[PF];
#pragma unroll
  for (int j = 0; j < PF - 1; ++j) load_state_frags<REV, OUT>(p, n, clampc(j), tile, f[j], FALL);
  int it = 0;
  for (; it + PF - 1 < NT; it += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      using LP = LoadPlan<REV, OUT>;
      const int nb = (j + PF - 1) % PF, nch = clampc(it + j + PF - 1);
      if constexpr (LP::pre != 0) load_state_frags<REV, OUT>(p, n, nch, tile, f[nb], LP::pre);
      state_step<REV, OUT>(p, s, n, chunk_of(it + j), tile, f[j], X, [&](int part) {
        if (LP::part[part] != 0) load_state_frags<REV, OUT>(p, n, nch, tile, f[nb], LP::part[part]);
      });
    }
  }
#pragma unroll
  for (int j = 0; j < PF - 1; ++j)
    if (it + j < NT) state_step<REV, OUT>(p, s, n, chunk_of(it + j), tile, f[j], X, [](int) {});
  if constexpr (OUT) {  // the last chunk's readout
    __syncthreads();
    store_readout(p, s, n, NT - 1, tile);
  }
  // final state (also kept as slot NT for the backward)
  for (int q = 0; q < SRB; ++q)
    for (int h = 0; h < HALVES; ++h)
      for (int e = 0; e < 4; ++e) {
        const int row = (SRB * w + q) * 16 + r4 + e, col = tile * SCOLS + h * 16 + m;
        if (p.Xs && !p.rev)
          static_cast<xslot_t*>(p.Xs)[((long long)n * NS + p.NT) * KD * KD + (long long)row * KD + col] =
              (xslot_t)X[q][h][e];
        if (p.fin && row < p.rows && col < p.cols) {
          const long long base = (long long)n * p.rows * p.cols;
          if (p.fin_transposed)
            p.fin[base + (long long)col * p.rows + row] = X[q][h][e];
          else
            p.fin[base + (long long)row * p.cols + col] = X[q][h][e];
        }
      }
}

void launch_state(const char* name, const StateParams& sp, int nseq, hipStream_t st) {
  const dim3 grid(STILES * nseq), blk(STHREADS);
  if (sp.rev)
    SD_LAUNCH(name, (k_state<true, false>), grid, blk, 0, st, sp);
  else if (sp.out)
    SD_LAUNCH(name, (k_state<false, true>), grid, blk, 0, st, sp);
  else
    SD_LAUNCH(name, (k_state<false, false>), grid, blk, 0, st, sp);
}

// ---------------------------------------------------------------------------
// k_prep_s: primal d, dual sources, S-memory WY panels
// LDS plan: Pa holds u then e, Pb holds k then chi, Pc holds d then serves as
// the inverse's scratch once d has been consumed.
// ---------------------------------------------------------------------------
// A 64 x 128 panel split into fp16 high / low halves: the A operand of the f16
// MFMA against fp16 panels (delta, the X0 slot), which enter exactly as they are.
struct HPanel {
  _Float16 h[BT][LPS];
  _Float16 l[BT][LPS];
};
__device__ __forceinline__ void hblk(const HPanel& P, int row0, f16x8 (&h)[4], f16x8 (&lo)[4]) {
  const int l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    h[ks] = *reinterpret_cast<const f16x8*>(&P.h[row0 + m][ks * 32 + kq]);
    lo[ks] = *reinterpret_cast<const f16x8*>(&P.l[row0 + m][ks * 32 + kq]);
  }
}
// A (split fp16) times B (fp16, exact): two f16 MFMAs per K slice.
__device__ __forceinline__ f4 mma_h16(const f16x8 (&ah)[4], const f16x8 (&al)[4],
                                      const f16x8 (&b)[4], f4 acc) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ks], b[ks], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ks], b[ks], acc, 0, 0, 0);
  }
  return acc;
}
// 16 rows of a row-major fp16 panel (row stride KD) as B fragments: lane m reads
// 8 consecutive K of its row.
__device__ __forceinline__ void load_f16_blk(const _Float16* rows, f16x8 (&b)[4]) {
  const int l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) b[ks] = *reinterpret_cast<const f16x8*>(rows + m * KD + ks * 32 + kq);
}

struct PrepSSmem {
  ChunkDecay cd;
  float M[BT * LS];
  float Pa[BT][GS];
  float Pb[BT][GS];
  union {
    float Pc[BT][GS];
    HPanel Kq;  // keys split once into fp16 halves for the M Gram and X0 k (before d)
    LPanel Kp;  // d's staged Gram form
  };
};

template <bool FL>  // FL: the call has token flags (sd_inputs.fresh)
__global__ __launch_bounds__(CT) void k_prep_s(FwdParams p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  PrepSSmem& s = *reinterpret_cast<PrepSSmem*>(smem_raw);
  // chunk-major dispatch, last chunk first: chunk 0 is written last, so the S
  // state pass that starts on it right after this kernel finds it in cache
  const int n = blockIdx.x, ch = gridDim.y - 1 - blockIdx.y;
  const int b = n / p.H, hh = n % p.H, t0 = ch * BT;
  const int T = p.T, r = p.r, V = p.V;
  const sd_inputs& in = p.in;
  const float* g = (const float*)in.log_decay.data + (long long)b * in.log_decay.sb +
                   (long long)hh * in.log_decay.sh;
  const int w = wave_id(), l = lane_id();
  {
    const int cl = l & 15;
    // the rows' u / k loads are issued first: their latency overlaps the decay build
    float ux[2][RQ], kx[2][RQ], km[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int t = t0 + row16(w, g);
      load_row16(in.u, b, t, hh, T, r, ux[g]);
      load_row16(in.k, b, t, hh, T, r, kx[g]);
      km[g] = operand_keep_at<FL>(in, b, t < T ? t : T - 1);  // invalid tokens' keys read 0
    }
    build_decay(s.cd, g, in.log_decay.st, t0, T, r, FL ? tok_flag_row(in, b) : nullptr, tok_flag_st(in));
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int i = row16(w, g);
#pragma unroll
      for (int q = 0; q < RQ; ++q) kx[g][q] *= km[g];
      l2norm16(ux[g]);
      l2norm16(kx[g]);
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        s.Pa[i][cl + 16 * q] = ux[g][q];
        s.Pb[i][cl + 16 * q] = kx[g][q];
      }
    }
  }
  __syncthreads();
  const ChunkDecay& cd = s.cd;
  const long long rowbase = (long long)n * p.Tp + t0;
  const long long cidx = (long long)n * p.NT + ch;
  const fpan_t* delta = p.delta + rowbase * KD;
  {  // keys split once into a shared panel (every wave would otherwise split all of them)
    constexpr int PER = BT * KD / 4 / CT;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int idx = (threadIdx.x + q * CT) * 4, i = idx / KD, c = idx % KD;
      const float4 v = *reinterpret_cast<const float4*>(&s.Pb[i][c]);
      const float x[4] = {v.x, v.y, v.z, v.w};
      f16x4 hh4, ll4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 a = (_Float16)x[e];
        hh4[e] = a;
        ll4[e] = (_Float16)(x[e] - (float)a);
      }
      *reinterpret_cast<f16x4*>(&s.Kq.h[i][c]) = hh4;
      *reinterpret_cast<f16x4*>(&s.Kq.l[i][c]) = ll4;
    }
  }
  __syncthreads();
  // M_ij = k_i . delta_j  (j <= i)
  for (int pp = w; pp < 10; pp += CW) {
    int I = 0, J = pp;
    while (J > I) { J -= I + 1; ++I; }
    f16x8 ah[4], al[4], dj[4];
    load_f16_blk(delta + J * BS * KD, dj);  // delta is an fp16 panel: exact as an f16 operand
    hblk(s.Kq, I * BS, ah, al);
    const f4 acc = mma_h16(ah, al, dj, zero4());
    for (int e = 0; e < 4; ++e) {
      const int i = I * BS + out_row(e), j = J * BS + out_col();
      s.M[i * LS + j] = j <= i ? acc[e] : 0.f;
    }
  }
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int i = idx / BT, j = idx % BT;
    if ((j / BS) > (i / BS)) s.M[i * LS + j] = 0.f;
  }
  __syncthreads();
  // d = k + e^G (X0 k) + sum_j M_ij u_j e^{G_i - G_j}  (this wave's column block)
  const xslot_t* X0 = p.Xc + ((long long)n * (p.NT + 1) + ch) * KD * KD;
  // The sources phase's rows (delta, q, erase, v, write_raw) are loaded before
  // the apply as raw 16-bit values (clamped addresses, masked when converted),
  // so their latency overlaps it.
  constexpr int RPW = BT / CW;
  // two 16-bit values per register: element q of a row in the low half of
  // word q / 2 (even q) or its high half (odd q)
  unsigned dq_r[2][RQ / 2], qq_r[2][RQ / 2], er_r[2][RQ / 2], vx_r[RPW], wx_r[RPW];
  {
    const int cb = w, c = cb * 16 + (l & 15), r4 = (l >> 4) * 4;
    f16x8 BX[4];  // the X0 slot is fp16: exact as an f16 operand
    load_f16_blk(X0 + cb * 16 * KD, BX);
    float Su[NB][4];
#pragma unroll
    for (int J = 0; J < NB; ++J)
#pragma unroll
      for (int e = 0; e < 4; ++e) Su[J][e] = s.Pa[J * BS + r4 + e][c];
    Tab1 t1;
    RowF rf;
    ColF cf;
    make_tab1(cd, cb, t1);
    make_rowf<false>(cd, cb, rf);
    make_colf(cd, cb, cf);
    auto Uw = [&](int j, int cc) { return s.Pa[j][cc]; };
    f4 a1[NB];  // X0 k for this wave's column block, from the shared split keys
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      f16x8 ah[4], al[4];
      hblk(s.Kq, I * BS, ah, al);
      a1[I] = mma_h16(ah, al, BX, zero4());
    }
    {
      const int cl = l & 15;
      auto raw = [](const void* base, long long idx) -> unsigned {
        return static_cast<const unsigned short*>(base)[idx];
      };
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int i = row16(w, g), t = t0 + i, tc = t < T ? t : T - 1;
        const __bf16* qrow = vrow(in.q, b, tc, hh);
        const __bf16* erow = vrow(in.erase_raw, b, tc, hh);
        // an invalid token's q reads as 0 (all bits of both packed halves cleared)
        const unsigned qkeep = operand_keep_at<FL>(in, b, tc) != 0.f ? ~0u : 0u;
#pragma unroll
        for (int q2 = 0; q2 < RQ / 2; ++q2) {
          const int c0 = cl + 32 * q2, c1 = c0 + 16;
          const int cc0 = c0 < r ? c0 : r - 1, cc1 = c1 < r ? c1 : r - 1;
          dq_r[g][q2] = raw(delta, i * KD + c0) | raw(delta, i * KD + c1) << 16;
          qq_r[g][q2] = (raw(qrow, cc0) | raw(qrow, cc1) << 16) & qkeep;
          er_r[g][q2] = raw(erow, cc0) | raw(erow, cc1) << 16;
        }
      }
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr) {
        const int t = t0 + w + rr * CW, tc = t < T ? t : T - 1;
        const __bf16* vr = vrow(in.v, b, tc, hh);
        const __bf16* wr = vrow(in.write_raw, b, tc, hh);
        vx_r[rr] = raw(vr, l < V ? l : V - 1) | raw(vr, l + 64 < V ? l + 64 : V - 1) << 16;
        wx_r[rr] = raw(wr, l < V ? l : V - 1) | raw(wr, l + 64 < V ? l + 64 : V - 1) << 16;
      }
    }
    __syncthreads();  // the split keys are dead: d is formed in their place
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      const f4 ap = apply_tab<false>(cd, s.M, Su, I, cb, t1, rf, cf, Uw);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = I * BS + r4 + e;
        const float dv = s.Pb[i][c] + __expf(cd.G[i][c]) * a1[I][e] + ap[e];
        s.Pc[i][c] = dv;
      }
    }
  }
  __syncthreads();
  // sources (16-lane row layout; e overwrites u, chi overwrites k), from the
  // rows loaded before the apply
  float zz[RPW][2];
  {
    const int cl = l & 15;
    float dq_[2][RQ], qq_[2][RQ], er_[2][RQ], vx[RPW][2], wx[RPW][2];
    // the half of a packed word as fp16 / bf16
    auto h2f = [](unsigned x, int hi) {
      return (float)__builtin_bit_cast(_Float16, (unsigned short)(hi ? x >> 16 : x));
    };
    auto b2f = [](unsigned x, int hi) { return __uint_as_float(hi ? x & 0xffff0000u : x << 16); };
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const bool tv = t0 + row16(w, g) < T;
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        const bool ok = tv && cl + 16 * q < r;
        dq_[g][q] = h2f(dq_r[g][q / 2], q & 1);
        qq_[g][q] = keep_if(ok, b2f(qq_r[g][q / 2], q & 1));
        er_[g][q] = keep_if(ok, b2f(er_r[g][q / 2], q & 1));
      }
    }
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      const bool tv = t0 + w + rr * CW < T;
      vx[rr][0] = keep_if(tv && l < V, b2f(vx_r[rr], 0));
      vx[rr][1] = keep_if(tv && l + 64 < V, b2f(vx_r[rr], 1));
      wx[rr][0] = keep_if(tv && l < V, b2f(wx_r[rr], 0));
      wx[rr][1] = keep_if(tv && l + 64 < V, b2f(wx_r[rr], 1));
    }
    {  // d to global memory only now, from this thread's own LDS entries: stored
       // before the loads above, it would have held them (one counter retires both)
      const int c = w * 16 + (l & 15), r4 = (l >> 4) * 4;
      fpan_t* const d_b = p.d + rowbase * KD;
#pragma unroll
      for (int I = 0; I < NB; ++I)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = I * BS + r4 + e;
          d_b[i * KD + c] = (fpan_t)s.Pc[i][c];
        }
    }
    fpan_t* const e_b = p.e + rowbase * KD;
    fpan_t* const chi_b = p.chi + rowbase * KD;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int i = row16(w, g);
      float u[RQ], k[RQ];
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        u[q] = s.Pa[i][cl + 16 * q];
        k[q] = s.Pb[i][cl + 16 * q];
      }
      l2norm16(qq_[g]);
      float usq = 0.f, dsq = 0.f;
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        usq += u[q] * u[q];
        dsq += dq_[g][q] * dq_[g][q];
      }
      usq = row16_sum(usq);
      dsq = row16_sum(dsq);
      const float sc = RHO / sqrtf(RHO * RHO + usq * dsq);
      float pv[RQ], bv[RQ], pu = 0.f, ubs = 0.f, uqs = 0.f;
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        pv[q] = sc * dq_[g][q];
        bv[q] = k[q] / (1.f + __expf(-er_[g][q]));
        pu += pv[q] * u[q];
        ubs += u[q] * bv[q];
        uqs += u[q] * qq_[g][q];
      }
      const float den = 1.f + row16_sum(pu);
      const float ub = row16_sum(ubs) / den;
      const float uq = row16_sum(uqs) / den;
#pragma unroll
      for (int q = 0; q < RQ; ++q) {
        const int c = cl + 16 * q;
        const bool in = c < r;
        const float ev = in ? bv[q] - pv[q] * ub : 0.f;
        const float xv = in ? qq_[g][q] - pv[q] * uq : 0.f;
        s.Pa[i][c] = ev;
        s.Pb[i][c] = xv;
        e_b[i * KD + c] = (fpan_t)ev;
        chi_b[i * KD + c] = (fpan_t)xv;
      }
    }
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      zz[rr][0] = vx[rr][0] / (1.f + __expf(-wx[rr][0]));
      zz[rr][1] = vx[rr][1] / (1.f + __expf(-wx[rr][1]));
    }
  }
  __syncthreads();
  // panels that read d and chi as they are, then d's Gram form staged once for
  // both decayed Grams below (in d's own storage; the wild fix-ups read the
  // global copy of d)
  // the decayed keys K^ = d e^{G_C - G} (chunk-transposed, fragment order) are
  // formed from d while it is still in LDS and stored after the P Gram
  constexpr int KPC = KD * BT / 8 / CT;  // pieces per thread
  f16x8 ksv[KPC];
#pragma unroll
  for (int q = 0; q < KPC; ++q) {
    const int pc = threadIdx.x + q * CT, block = pc >> 6, lane = pc & 63;
    const int c = (block / (BT / 32)) * 16 + (lane & 15);
    const int i0 = (block % (BT / 32)) * 32 + (lane >> 4) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      ksv[q][e] = (_Float16)(s.Pc[i0 + e][c] * __expf(cd.G[BT - 1][c] - cd.G[i0 + e][c]));
  }
  stage_ytilde(s.Kp, cd, [&](int j, int c) { return s.Pc[j][c]; });
  const fpan_t* const dg_ = p.d + rowbase * KD;
  auto Draw = [&](int j, int c) { return (float)dg_[j * KD + c]; };
  // output pair P_ij = sum_c chi_ic d_jc e^{G_ic - G_jc}, j <= i, into M, and the
  // S-memory Gram L_ij = sum_c e_ic d_jc e^{G_ic - G_jc}, j < i, in registers
  // until P is stored (one pass: both share d's staged form and the decay factors)
  auto Xchi = [&](int i, int c) { return s.Pb[i][c]; };
  auto Xe = [&](int i, int c) { return s.Pa[i][c]; };
  f4 lacc[2];
  decayed_gram2_yt(cd, Xchi, Xe, s.Kp, s.M, lacc);
  gram_wild_fixup<false>(cd, Xchi, Draw, false, s.M);
  store_frag_panel1<BT, BT>(p.Ps, cidx * BT * BT, [&](int i, int j) { return s.M[i * LS + j]; });
#pragma unroll
  for (int q = 0; q < KPC; ++q) {
    const long long o = cidx * KD * BT + (long long)(threadIdx.x + q * CT) * 8;
    *reinterpret_cast<f16x8*>(p.Ks + o) = ksv[q];
  }
  store_frag_panel1<BT, KD>(p.Qs, rowbase * KD,
                            [&](int i, int c) { return s.Pb[i][c] * __expf(cd.G[i][c]); });
  __syncthreads();
  gram2_second_store(lacc, s.M);
  gram_wild_fixup<false>(cd, Xe, Draw, true, s.M);
  unit_lower_inverse(s.M, &s.Pc[0][0]);
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT)
    p.As[cidx * BT * BT + idx] = s.M[(idx / BT) * LS + idx % BT];
  // WY operands staged once: Pa <- e e^G, Pb <- z = sigmoid(write_raw) v
  for (int idx = threadIdx.x; idx < BT * KD; idx += CT) {
    const int i = idx / KD, c = idx % KD;
    s.Pa[i][c] *= __expf(cd.G[i][c]);
  }
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    s.Pb[w + rr * CW][l] = zz[rr][0];
    s.Pb[w + rr * CW][l + 64] = zz[rr][1];
  }
  __syncthreads();
  // W = A (e e^G), U = A z
  {
    const int cb = w, m = l & 15, kq = (l >> 4) * 8;
    // B operands, the same for every row block I: split once
    bf16x8 ph[2], pl[2], zh[2], zl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = ks * 32 + kq + e, c = cb * 16 + m;
        __bf16 h, lo;
        split_bf(s.Pa[k][c], h, lo);
        ph[ks][e] = h;
        pl[ks][e] = lo;
        split_bf(s.Pb[k][c], h, lo);
        zh[ks][e] = h;
        zl[ks][e] = lo;
      }
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      const int K = I < 2 ? 32 : 64;
      f4 aw = zero4(), au = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks * 32 >= K) break;
        bf16x8 ah, al;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          __bf16 h, lo;
          split_bf(s.M[(I * BS + m) * LS + ks * 32 + kq + e], h, lo);
          ah[e] = h;
          al[e] = lo;
        }
        aw = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, ph[ks], aw, 0, 0, 0);
        au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, zh[ks], au, 0, 0, 0);
        aw = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, pl[ks], aw, 0, 0, 0);
        au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, zl[ks], au, 0, 0, 0);
        aw = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, ph[ks], aw, 0, 0, 0);
        au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, zh[ks], au, 0, 0, 0);
      }
      for (int e = 0; e < 4; ++e) {
        const long long row = rowbase + I * BS + out_row(e);
        const int c = cb * 16 + out_col();
        s.Pc[I * BS + out_row(e)][c] = -aw[e];  // staged for the fragment-order store
        p.Us[row * KD + c] = au[e];
      }
    }
  }
  __syncthreads();
  store_frag_panel1<BT, KD>(p.Ws, rowbase * KD, [&](int i, int c) { return s.Pc[i][c]; });
}

size_t prep_c_smem() { return sizeof(PrepCSmem); }
size_t prep_s_smem() { return sizeof(PrepSSmem); }

int launch_fwd(const sd_inputs* in, void* out, float* C_T, float* S_T, const FwdWs& w,
               hipStream_t st) {
  
  const int n = in->B * in->H, NT = (in->T + BT - 1) / BT, Tp = NT * BT;

  FwdParams fp{};
  fp.in = *in;
  fp.H = in->H; fp.T = in->T; fp.r = in->r; fp.V = in->V; fp.NT = NT; fp.Tp = Tp;
  fp.Xc = w.Xc; fp.delta = w.delta; fp.d = w.d;
  fp.Ac = w.Ac; fp.As = w.As; fp.e = w.e; fp.chi = w.chi;
  fp.Wc = w.Wc; fp.Uc = w.Uc; fp.Kc = w.Kc; fp.Gam = w.Gam;
  fp.Ws = w.Ws; fp.Us = w.Us; fp.Ks = w.Ks; fp.Qs = w.Qs; fp.Ps = w.Ps;

  // kernels that read token flags are separate instantiations: a call without
  // flags runs no flag code at all
  const bool fl = in->fresh.data != nullptr;
  if (fl) {
    SD_SMEM_ONCE(k_prep_c<true>, (int)prep_c_smem());
    SD_LAUNCH("k_prep_c", k_prep_c<true>, dim3(n, NT), dim3(CT), prep_c_smem(), st, fp);
  } else {
    SD_SMEM_ONCE(k_prep_c<false>, (int)prep_c_smem());
    SD_LAUNCH("k_prep_c", k_prep_c<false>, dim3(n, NT), dim3(CT), prep_c_smem(), st, fp);
  }

  StateParams sc{};
  sc.H = in->H; sc.T = in->T; sc.NT = NT; sc.Tp = Tp; sc.rows = in->r; sc.cols = in->r;
  sc.Wneg = w.Wc; sc.U = w.Uc; sc.Kt = w.Kc; sc.Gam = w.Gam;
  sc.Xs = w.Xc; sc.wout = w.delta;
  sc.init = in->C0; sc.init_transposed = 1;
  sc.fin = C_T; sc.fin_transposed = 1;
  launch_state("state_c_fwd", sc, n, st);

  if (fl) {
    SD_SMEM_ONCE(k_prep_s<true>, (int)prep_s_smem());
    SD_LAUNCH("k_prep_s", k_prep_s<true>, dim3(n, NT), dim3(CT), prep_s_smem(), st, fp);
  } else {
    SD_SMEM_ONCE(k_prep_s<false>, (int)prep_s_smem());
    SD_LAUNCH("k_prep_s", k_prep_s<false>, dim3(n, NT), dim3(CT), prep_s_smem(), st, fp);
  }

  StateParams ss{};
  ss.H = in->H; ss.T = in->T; ss.NT = NT; ss.Tp = Tp; ss.rows = in->r; ss.cols = in->V;
  ss.Wneg = w.Ws; ss.U = w.Us; ss.Kt = w.Ks; ss.Gam = w.Gam;
  ss.Xs = w.Xs; ss.wout = w.wS;
  ss.init = in->S0; ss.init_transposed = 0;
  ss.fin = S_T; ss.fin_transposed = 0;
  ss.Q = w.Qs; ss.P = w.Ps; ss.out = (__bf16*)out;
  ss.out_vec = in->V % 8 == 0 && ((uintptr_t)out & 15) == 0;
  launch_state("state_s_fwd", ss, n, st);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

}  // namespace sd
