// Shared device code for the SolveDelta chunk kernels (gfx950 / CDNA4).
//
// Every chunk kernel works on one (batch, head) sequence and one chunk of
// BT = 64 tokens, split into 4 blocks of BS = 16 tokens.  Widths are padded to
// KD = 128 (key / geometry width r) and VD = 128 (value width V); padding
// coordinates are zero and stay zero through the recurrence.
//
// Decay handling (no reciprocal decays are ever formed):
//   G_i   = in-chunk inclusive prefix of log-decay g (fp32),
//   R_J   = G at the row before block J (0 for block 0),
//   exp(Gx_i - G_j) = exp(Gx_i - R_J) * exp(R_J - G_j)   for j in block J, i >= J0.
// The first factor is <= 1.  The second lies in [1, exp(drop_J)] where drop_J is
// the decay accumulated inside block J; coordinates with drop_J > TAU ("wild")
// are removed from the factored product and added back exactly.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include "../../include/solvedelta.h"

namespace sd {

constexpr int BT = 64;     // chunk length
constexpr int BS = 16;     // block length inside a chunk
constexpr int NB = BT / BS;
constexpr int KD = 128;    // padded key width
constexpr int VD = 128;    // padded value width
// The block factor exp(R_J - G_j) stays below exp(TAU); a factor exp(Gx_i - R_J)
// that underflows FP32 (below exp(-87)) then drops a term below exp(TAU - 87)
// ~ 2e-12 of its operands' product, far under FP32 rounding of the terms kept.
constexpr float TAU = 60.f;
constexpr float RHO = 0.625f;
constexpr int NTHREADS = 256;  // sequential / per-token kernels
constexpr int CT = 512;        // chunk-parallel kernels: 8 waves, one 16-column block each
constexpr int CW = CT / 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// v where ok, else 0, for a value loaded from a clamped (always valid) address.
// A multiply rather than a select: with a wave-uniform condition the compiler
// turns `ok ? v : 0` back into a branch around the load that then waits for it,
// which serialises every load of an unrolled gather.  (v is finite data, so
// v * 0 == 0.)
__device__ __forceinline__ float keep_if(bool ok, float v) { return v * (ok ? 1.f : 0.f); }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float bf2f(__bf16 x) { return (float)x; }
__device__ __forceinline__ __bf16 f2bf(float x) { return (__bf16)x; }

// Sum over the 64 lanes of a wave, returned to every lane: DPP adds inside each
// 16-lane row (quad swaps, half-row and row mirrors), then the four row sums are
// read into scalar registers.  Avoids the LDS-permute round trips of shuffles.
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel) {
  int x = __float_as_int(v), y;
  switch (ctrl_sel) {
    case 0: y = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); break;   // quad [1,0,3,2]
    case 1: y = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); break;   // quad [2,3,0,1]
    case 2: y = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false); break;  // row half mirror
    default: y = __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false); break; // row mirror
  }
  return v + __int_as_float(y);
}

__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add(v, 0);
  v = dpp_add(v, 1);
  v = dpp_add(v, 2);
  v = dpp_add(v, 3);
  const int x = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(x, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(x, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(x, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(x, 48));
  return (r0 + r1) + (r2 + r3);
}

// Sum over each 16-lane DPP row, returned to all 16 lanes of that row (no
// readlane, so four token rows reduce at once in one wave).
__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_add(v, 0);
  v = dpp_add(v, 1);
  v = dpp_add(v, 2);
  return dpp_add(v, 3);
}

// 16-lane row layout for per-token row work: a wave covers four token rows at
// once, lane (l & 15) of DPP row (l >> 4) holding columns (l & 15) + 16 q, so a
// row's reductions are four in-row DPP adds.  A chunk's 64 rows take two such
// groups per wave: row16(w, g) = 8 w + 4 g + (l >> 4).
constexpr int RQ = KD / 16;
__device__ __forceinline__ int row16(int w, int g) { return w * 8 + g * 4 + (lane_id() >> 4); }

// One bf16 row (row pointer p of a clamped token; tv false selects zeros) in the
// 16-lane layout; columns >= w read a valid element and are selected to 0, so
// unrolled loops can issue every load before the first use.
__device__ __forceinline__ void ld_row16(const __bf16* p, bool tv, int w, float (&x)[RQ]) {
  const int cl = lane_id() & 15;
#pragma unroll
  for (int q = 0; q < RQ; ++q) {
    const int c = cl + 16 * q;
    x[q] = keep_if(tv && c < w, bf2f(p[c < w ? c : w - 1]));
  }
}

// Normalises one 16-lane row in place and returns its inverse norm.
__device__ __forceinline__ float l2norm16(float (&x)[RQ]) {
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < RQ; ++q) ss += x[q] * x[q];
  const float rs = rsqrtf(row16_sum(ss) + 1e-24f);
#pragma unroll
  for (int q = 0; q < RQ; ++q) x[q] *= rs;
  return rs;
}

__device__ __forceinline__ f4 zero4() { f4 z = {0.f, 0.f, 0.f, 0.f}; return z; }

// Split an fp32 value into a bf16 high part and a bf16 residual.
__device__ __forceinline__ void split_bf(float x, __bf16& hi, __bf16& lo) {
  hi = f2bf(x);
  lo = f2bf(x - bf2f(hi));
}

// D(16x16) += A(16xK) * B(Kx16), K a multiple of 32, operands produced by
// lambdas fa(m, k) and fb(k, n) as fp32 values.  Both operands are split into
// bf16 hi + lo parts and multiplied as hi*hi + hi*lo + lo*hi (three MFMAs), which
// keeps ~16 mantissa bits per product (the dropped lo*lo term is ~2^-16 relative).
// Output layout: lane holds D[(lane>>4)*4 + e][lane & 15], e = 0..3.  32-wide K slices
// wholly below K0 are skipped (the caller knows their products are zero).
template <class FA, class FB>
__device__ __forceinline__ f4 mma_k32(FA fa, FB fb, int K, f4 acc, int K0 = 0) {
  const int l = lane_id();
  const int m = l & 15, kq = (l >> 4) * 8;
  // Gather every operand first (K <= 128) so all loads are in flight together,
  // then split and multiply.
  float av[4][8], bv[4][8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks * 32 < K && ks * 32 + 32 > K0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        av[ks][e] = fa(m, ks * 32 + kq + e);
        bv[ks][e] = fb(ks * 32 + kq + e, m);
      }
    }
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks * 32 < K && ks * 32 + 32 > K0) {
      bf16x8 ah, al, bh, bl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        __bf16 h, lo;
        split_bf(av[ks][e], h, lo);
        ah[e] = h; al[e] = lo;
        split_bf(bv[ks][e], h, lo);
        bh[e] = h; bl[e] = lo;
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
    }
  }
  return acc;
}

// Two products sharing the A operand (A B1 and A B2): A is gathered and split once.
// B2_EXACT: fb2's values are exact in bf16 (no low half), so its product takes two
// MFMAs per K slice.
template <bool B2_EXACT = false, class FA, class FB1, class FB2>
__device__ __forceinline__ void mma_k32x2(FA fa, FB1 fb1, FB2 fb2, int K, f4& acc1, f4& acc2) {
  const int l = lane_id();
  const int m = l & 15, kq = (l >> 4) * 8;
  float av[4][8], b1[4][8], b2[4][8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks * 32 < K) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        av[ks][e] = fa(m, ks * 32 + kq + e);
        b1[ks][e] = fb1(ks * 32 + kq + e, m);
        b2[ks][e] = fb2(ks * 32 + kq + e, m);
      }
    }
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks * 32 < K) {
      bf16x8 ah, al, ch, cl, dh, dl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        __bf16 h, lo;
        split_bf(av[ks][e], h, lo);
        ah[e] = h; al[e] = lo;
        split_bf(b1[ks][e], h, lo);
        ch[e] = h; cl[e] = lo;
        split_bf(b2[ks][e], h, lo);
        dh[e] = h; dl[e] = lo;
      }
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, ch, acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, dh, acc2, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, cl, acc1, 0, 0, 0);
      if constexpr (!B2_EXACT) acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, dl, acc2, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, ch, acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, dh, acc2, 0, 0, 0);
    }
  }
}

// mma_k32 with the operand gathers split into a raw-load pass and a transform
// pass: la(m, k) / lb(k, n) fetch the raw values (for global operands, every
// load is issued before the first use), xa(m, k, x) / xb(k, n, x) turn them into
// the operand values.  A lambda that loads and computes per element makes each
// load wait for the previous one's use.
template <class LA, class XA, class LB, class XB>
__device__ __forceinline__ f4 mma_k32_lx(LA la, XA xa, LB lb, XB xb, int K, f4 acc) {
  const int l = lane_id();
  const int m = l & 15, kq = (l >> 4) * 8;
  using RA = decltype(la(0, 0));
  using RB = decltype(lb(0, 0));
  RA ar[4][8];
  RB br[4][8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks * 32 < K) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ar[ks][e] = la(m, ks * 32 + kq + e);
        br[ks][e] = lb(ks * 32 + kq + e, m);
      }
    }
  }
  float av[4][8], bv[4][8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks * 32 < K) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        av[ks][e] = xa(m, ks * 32 + kq + e, ar[ks][e]);
        bv[ks][e] = xb(ks * 32 + kq + e, m, br[ks][e]);
      }
    }
  }
  return mma_k32([&](int mm, int k) { return av[k >> 5][k & 7]; },
                 [&](int k, int nn) { return bv[k >> 5][k & 7]; }, K, acc);
}

// Writes a per-chunk R x C panel (C = 64 or 128) kept in one 2-byte type E
// (fp16, or bf16 with no low half) in fragment order (see frag_off): each piece
// is one lane's 16 bytes of one 16 x 32 operand block -- a fixed row and 8
// consecutive columns -- produced from val(row, col), rounded to E and stored
// with one 16-byte store, so a wave's stores are contiguous.  All CT threads of
// the workgroup take part.
template <int R, int C, class E, class F>
__device__ __forceinline__ void store_frag_panel1(E* dst, long long base, F val) {
  typedef E V8 __attribute__((ext_vector_type(8)));
  constexpr int PIECES = R * C / 8;
#pragma unroll
  for (int q = 0; q < (PIECES + CT - 1) / CT; ++q) {
    const int pc = threadIdx.x + q * CT;
    if (PIECES % CT != 0 && pc >= PIECES) break;
    const int block = pc >> 6, lane = pc & 63;
    const int row = (block / (C / 32)) * 16 + (lane & 15);
    const int col0 = (block % (C / 32)) * 32 + (lane >> 4) * 8;
    V8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (E)val(row, col0 + e);
    *reinterpret_cast<V8*>(dst + base + (long long)pc * 8) = h;
  }
}

__device__ __forceinline__ int out_row(int e) { return (lane_id() >> 4) * 4 + e; }
__device__ __forceinline__ int out_col() { return lane_id() & 15; }

// ---------------------------------------------------------------------------
// Chunk-local shared state
// ---------------------------------------------------------------------------
constexpr int GS = KD + 4;  // fp32 panel row stride (floats)
constexpr int LS = BT + 4;  // 64x64 fp32 matrix row stride (16-byte aligned rows)

struct ChunkDecay {
  float G[BT][GS];          // inclusive prefix
  float R[NB][KD];          // block references
  unsigned char wild[NB][KD];
  int nwild[NB];
  short wlist[NB][KD];
};

// Loads g (fp32, [B,T,H,r] strided, token stride st, row pointer base at
// token t0) and builds G, R and the wild lists.  Tokens >= T load 0 (neutral).
// The chunk's log-decays in registers: thread (J, c) = (tid / 128, tid % 128)
// holds rows J*16 .. J*16+15 of column c (clamped addresses + select: a guarded
// load would branch and wait).
// frow / fst: the batch row of the per-token flags (SD_TOK_INVALID: the
// log-decay reads as 0; SD_TOK_RESET: it reads as SD_RESET_LOG_DECAY), or null
// when there are none.  The two cases are separate branches that each issue
// all of their loads (a branch after the loads would wait for them all before
// it, in the calls without flags as well).  A wave's 128 threads share one
// block J, so each lane loads the flags of token J*16 + (lane % 16) and the 16
// values are read across lanes.
__device__ __forceinline__ void decay_load_rows(const float* g, long long st, int t0, int T, int r,
                                                float (&x)[BS]) {
  const int c = threadIdx.x & (KD - 1), J = threadIdx.x / KD;
#pragma unroll
  for (int i = 0; i < BS; ++i) {
    const int t = t0 + J * BS + i;
    const float v = g[(long long)(t < T ? t : T - 1) * st + (c < r ? c : r - 1)];
    x[i] = keep_if(t < T && c < r, v);
  }
}
__device__ __forceinline__ void decay_load(const float* g, long long st, int t0, int T, int r,
                                           float (&x)[BS], const uint8_t* frow, long long fst) {
  if (!frow) {
    decay_load_rows(g, st, t0, T, r, x);
    return;
  }
  const int c = threadIdx.x & (KD - 1), J = threadIdx.x / KD;
  const int tf = t0 + J * BS + (threadIdx.x & 15);
  const int fl = frow[(long long)(tf < T ? tf : T - 1) * fst];
  decay_load_rows(g, st, t0, T, r, x);
#pragma unroll
  for (int i = 0; i < BS; ++i) {
    const int f = __builtin_amdgcn_readlane(fl, i);
    x[i] = (f & SD_TOK_INVALID) ? 0.f
           : ((f & SD_TOK_RESET) ? keep_if(t0 + J * BS + i < T && c < r, SD_RESET_LOG_DECAY) : x[i]);
  }
}

// Prefix tables from decay_load's registers: each thread scans its 16 rows, the
// four block totals of a column give each block's offset.
__device__ __forceinline__ void decay_build(ChunkDecay& cd, float (&x)[BS]) {
  static_assert(CT == NB * KD, "one thread per (block, column)");
  const int tid = threadIdx.x, c = tid & (KD - 1), J = tid / KD;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < BS; ++i) {
    acc += x[i];
    x[i] = acc;
  }
  cd.R[J][c] = acc;  // block totals for now
  __syncthreads();
  float off = 0.f;
#pragma unroll
  for (int K = 0; K < NB - 1; ++K) off += K < J ? cd.R[K][c] : 0.f;
  __syncthreads();  // every total read
#pragma unroll
  for (int i = 0; i < BS; ++i) cd.G[J * BS + i][c] = off + x[i];
  cd.R[J][c] = off;
  cd.wild[J][c] = off - (off + x[BS - 1]) > TAU ? 1 : 0;
  __syncthreads();
  {  // wild lists: wave J scans block J's coordinates with ballots
    const int w = tid >> 6, l = tid & 63;
    if (w < NB) {
      const bool f0 = cd.wild[w][l] != 0, f1 = cd.wild[w][l + 64] != 0;
      const unsigned long long m0 = __ballot(f0), m1 = __ballot(f1);
      const unsigned long long below = (l == 0) ? 0ull : (~0ull >> (64 - l));
      const int n0 = __popcll(m0);
      if (f0) cd.wlist[w][__popcll(m0 & below)] = (short)l;
      if (f1) cd.wlist[w][n0 + __popcll(m1 & below)] = (short)(l + 64);
      if (l == 0) cd.nwild[w] = n0 + __popcll(m1);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void build_decay(ChunkDecay& cd, const float* g, long long st, int t0, int T,
                                            int r, const uint8_t* frow, long long fst) {
  float x[BS];
  decay_load(g, st, t0, T, r, x, frow, fst);
  decay_build(cd, x);
}

// exp(x) on a non-wild coordinate, 0 on a wild one, without a branch (a
// per-element branch around the exp serialises the gathers it sits among).  A
// wild coordinate's argument can exceed the fp32 exp range, so it is clamped
// before the mask; a non-wild argument is at most TAU and is left unchanged.
__device__ __forceinline__ float exp_unless_wild(bool wild, float x) {
  return keep_if(!wild, __expf(fminf(x, TAU)));
}

// Gx for the erase side: inclusive (G_i) or exclusive (G_{i-1} = G_i - g_i).
// The exclusive prefix is G[i-1] (0 for i = 0).
__device__ __forceinline__ float gx_excl(const ChunkDecay& cd, int i, int c) {
  return keep_if(i > 0, cd.G[i > 0 ? i - 1 : 0][c]);  // clamped read + mask: no branch
}

// Decayed Gram M_ij = sum_c X_ic Y_jc exp(Gx_ic - G_jc), j<i (strict) or j<=i,
// written to M (64 x LS, fp32); entries above the diagonal set to 0.
// X(i,c), Y(j,c) are lambdas returning fp32; EXCL selects Gx.
template <bool EXCL, class FX, class FY>
__device__ void decayed_gram(const ChunkDecay& cd, FX X, FY Y, bool strict, float* M,
                             int ldm = LS) {
  const int w = wave_id();
  // 10 lower block pairs (I >= J), distributed over 4 waves.
  for (int p = w; p < 10; p += CW) {
    int I = 0, J = p;
    while (J > I) { J -= I + 1; ++I; }  // p -> (I, J) with J <= I
    const int I0 = I * BS, J0 = J * BS;
    const float* RJ = cd.R[J];
    f4 acc = mma_k32_lx(
        [&](int m, int c) { return X(I0 + m, c); },
        [&](int m, int c, float x) {
          const int i = I0 + m;
          const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
          return x * __expf(gx - RJ[c]);
        },
        [&](int c, int n) { return Y(J0 + n, c); },
        [&](int c, int n, float y) {
          return y * exp_unless_wild(cd.wild[J][c] != 0, RJ[c] - cd.G[J0 + n][c]);
        },
        KD, zero4());
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = I0 + out_row(e), j = J0 + out_col();
      const bool keep = strict ? (j < i) : (j <= i);
      M[i * ldm + j] = keep ? acc[e] : 0.f;
    }
  }
  // Zero the strictly-upper block pairs.
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int i = idx / BT, j = idx % BT;
    if ((j / BS) > (i / BS)) M[i * ldm + j] = 0.f;
  }
  __syncthreads();
  // Exact fix-up for wild coordinates.
  for (int J = 0; J < NB; ++J) {
    const int nw = cd.nwild[J];
    if (nw == 0) continue;
    const int J0 = J * BS;
    const int npairs = (BT - J0) * BS;
    for (int idx = threadIdx.x; idx < npairs; idx += CT) {
      const int i = J0 + idx / BS, j = J0 + idx % BS;
      const bool keep = strict ? (j < i) : (j <= i);
      if (!keep) continue;
      float s = 0.f;
      for (int q = 0; q < nw; ++q) {
        const int c = cd.wlist[J][q];
        const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
        s += X(i, c) * Y(j, c) * __expf(fminf(gx - cd.G[j][c], 0.f));
      }
      M[i * ldm + j] += s;
    }
  }
  __syncthreads();
}

// decayed_gram with the X side a 64 x 128 bf16 panel in global memory (row
// stride KD): each lane's 8-column slice of its row is one 16-byte load, all
// four issued before the first use (the per-element form makes 32 two-byte
// loads per block pair).
template <bool EXCL, class FY>
__device__ void decayed_gram_gx(const ChunkDecay& cd, const __bf16* Xg, FY Y, bool strict, float* M,
                                int ldm = LS) {
  const int w = wave_id(), l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
  for (int p = w; p < 10; p += CW) {
    int I = 0, J = p;
    while (J > I) { J -= I + 1; ++I; }  // p -> (I, J) with J <= I
    const int I0 = I * BS, J0 = J * BS;
    const float* RJ = cd.R[J];
    bf16x8 xr[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      xr[ks] = *reinterpret_cast<const bf16x8*>(Xg + (I0 + m) * KD + ks * 32 + kq);
    f4 acc = mma_k32_lx(
        [&](int mm, int c) { return (float)xr[c >> 5][c & 7]; },
        [&](int mm, int c, float x) {
          const int i = I0 + mm;
          const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
          return x * __expf(gx - RJ[c]);
        },
        [&](int c, int n) { return Y(J0 + n, c); },
        [&](int c, int n, float y) {
          return y * exp_unless_wild(cd.wild[J][c] != 0, RJ[c] - cd.G[J0 + n][c]);
        },
        KD, zero4());
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = I0 + out_row(e), j = J0 + out_col();
      const bool keep = strict ? (j < i) : (j <= i);
      M[i * ldm + j] = keep ? acc[e] : 0.f;
    }
  }
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int i = idx / BT, j = idx % BT;
    if ((j / BS) > (i / BS)) M[i * ldm + j] = 0.f;
  }
  __syncthreads();
  for (int J = 0; J < NB; ++J) {  // exact fix-up for wild coordinates
    const int nw = cd.nwild[J];
    if (nw == 0) continue;
    const int J0 = J * BS;
    const int npairs = (BT - J0) * BS;
    for (int idx = threadIdx.x; idx < npairs; idx += CT) {
      const int i = J0 + idx / BS, j = J0 + idx % BS;
      const bool keep = strict ? (j < i) : (j <= i);
      if (!keep) continue;
      float s = 0.f;
      for (int q = 0; q < nw; ++q) {
        const int c = cd.wlist[J][q];
        const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
        s += (float)Xg[i * KD + c] * Y(j, c) * __expf(fminf(gx - cd.G[j][c], 0.f));
      }
      M[i * ldm + j] += s;
    }
  }
  __syncthreads();
}

// D(16x16) += A(16x16) B(16x16) with lane (g = l >> 4, m = l & 15) holding
// av[e] = A[m][4g + e] and bv[e] = B[4g + e][m]: four fp32 16x16x4 MFMAs, one per
// e, each summing over g.  Exact fp32 products and no operand conversions, which
// keeps these short products off the (busier) vector ALU.
__device__ __forceinline__ f4 mma16s(const float* av, const float* bv, f4 acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[e], acc, 0, 0, 0);
  return acc;
}

// (I + L)^{-1} for strictly-lower L (64x64, stride LS, upper blocks zero), in
// place -> A, with four barriers.  Diagonal 16x16 blocks D_B by forward
// substitution (one lane per column), written over L's diagonal blocks; then
// the 2x2 block recursion, one wave per 16x16 block on the K=16 MFMA:
//   level 1: A10 = -D1 L10 D0,  A32 = -D3 L32 D2            (over L10, L32)
//   level 2: X = L[23][01] Inv01:  X20 = L20 D0 + L21 A10, X21 = L21 D1,
//            X30 = L30 D0 + L31 A10, X31 = L31 D1            (staged in tmp)
//   level 3: A[23][01] = -Inv23 X: A20 = -D2 X20, A21 = -D2 X21,
//            A30 = -(A32 X20 + D3 X30), A31 = -(A32 X21 + D3 X31)
// A block a wave overwrites is read only by that wave, and its LDS reads are
// drained (lgkmcnt) before the write.  The MFMA output layout (lane: rows
// (lane>>4)*4+e, column lane&15) is the K=16 B-operand layout, so a product
// feeds the next one from registers.  tmp: 64 x LS scratch.
__device__ __forceinline__ void unit_lower_inverse(float* L, float* tmp) {
  const int tid = threadIdx.x;
  const int wv = tid >> 6, l = tid & 63, m = l & 15, r4 = (l >> 4) * 4;
  // rows m of block (I, K) of a matrix, columns r4..r4+3 (A operand) / rows
  // r4..r4+3 of block (K, J), column m (B operand)
  auto rowseg = [&](const float* X, int I, int K, float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = X[(I * BS + m) * LS + K * BS + r4 + e];
  };
  auto colseg = [&](const float* X, int K, int J, float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = X[(K * BS + r4 + e) * LS + J * BS + m];
  };
  auto put = [&](float* X, int I, int J, f4 v, float sign) {
#pragma unroll
    for (int e = 0; e < 4; ++e) X[(I * BS + r4 + e) * LS + J * BS + m] = sign * v[e];
  };
  auto drain = [] { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); };
  // diagonal blocks: thread (B, j), block B = tid / 16 (tid < 64), column j
  if (tid < NB * BS) {
    const int B = tid / BS, j = tid % BS, B0 = B * BS;
    float col[BS];
#pragma unroll
    for (int i = 0; i < BS; ++i) {  // compile-time indices keep col[] in registers
      float sum = (i == j) ? 1.f : 0.f;
#pragma unroll
      for (int q = 0; q < i; ++q) sum -= L[(B0 + i) * LS + B0 + q] * col[q];
      col[i] = (i >= j) ? sum : 0.f;
    }
    drain();
#pragma unroll
    for (int i = 0; i < BS; ++i) L[(B0 + i) * LS + B0 + j] = col[i];
  }
  __syncthreads();
  if (wv < 2) {  // level 1
    const int J = 2 * wv, I = J + 1;
    float av[4], bv[4];
    rowseg(L, I, J, av);
    colseg(L, J, J, bv);
    const f4 t = mma16s(av, bv, zero4());
    rowseg(L, I, I, av);
    const float tv[4] = {t[0], t[1], t[2], t[3]};
    const f4 a = mma16s(av, tv, zero4());
    drain();
    put(L, I, J, a, -1.f);
  }
  __syncthreads();
  if (wv < 4) {  // level 2: X(I, J) for I = 2 + wv / 2, J = wv % 2
    const int I = 2 + wv / 2, J = wv % 2;
    float av[4], bv[4];
    rowseg(L, I, J, av);
    colseg(L, J, J, bv);  // D_J
    f4 x = mma16s(av, bv, zero4());
    if (J == 0) {  // + L_I1 A10
      rowseg(L, I, 1, av);
      colseg(L, 1, 0, bv);
      x = mma16s(av, bv, x);
    }
    put(tmp, I, J, x, 1.f);
  }
  __syncthreads();
  if (wv < 4) {  // level 3: A(I, J) = -(A_I2 X2J [I = 3] + D_I X_IJ)
    const int I = 2 + wv / 2, J = wv % 2;
    float av[4], bv[4];
    f4 a = zero4();
    if (I == 3) {
      rowseg(L, 3, 2, av);  // A32
      colseg(tmp, 2, J, bv);
      a = mma16s(av, bv, a);
    }
    rowseg(L, I, I, av);  // D_I
    colseg(tmp, I, J, bv);
    a = mma16s(av, bv, a);
    put(L, I, J, a, -1.f);
  }
  __syncthreads();
}

}  // namespace sd

namespace sd {

}  // namespace sd

namespace sd {

// ---------------------------------------------------------------------------
// Register-fragment helpers for the chunk-parallel kernels.
// A "block" is 16 rows x 128 K-contiguous fp32 values; its MFMA A- and B-fragment
// addressing is identical (lane m = lane&15 owns row m, 8 consecutive K).
// A "slab" is one 16-column block of a token panel, held in the MFMA output /
// K=16 B-operand layout: slab[J][e] = P[J*16 + (lane>>4)*4 + e][cb*16 + (lane&15)].
// ---------------------------------------------------------------------------
struct Blk { float4 v[4][2]; };

__device__ __forceinline__ float4 ld4g(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Eight consecutive elements of a panel of element type E (fp32, or a 2-byte
// type: one 16-byte load) as two float4.
__device__ __forceinline__ void ld8f(const float* p, float4& a, float4& b) {
  a = ld4g(p);
  b = ld4g(p + 4);
}
template <class E>
__device__ __forceinline__ void ld8f(const E* p, float4& a, float4& b) {
  typedef E V8 __attribute__((ext_vector_type(8)));
  const V8 v = *reinterpret_cast<const V8*>(p);
  a = make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
  b = make_float4((float)v[4], (float)v[5], (float)v[6], (float)v[7]);
}
// Four consecutive elements as a float4.
__device__ __forceinline__ float4 ld4f(const float* p) { return ld4g(p); }
template <class E>
__device__ __forceinline__ float4 ld4f(const E* p) {
  typedef E V4 __attribute__((ext_vector_type(4)));
  const V4 v = *reinterpret_cast<const V4*>(p);
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

template <class E>
__device__ __forceinline__ void load_blk(Blk& b, const E* rows, int ld) {
  const int l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
  const E* a = rows + (long long)m * ld + kq;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ld8f(a + ks * 32, b.v[ks][0], b.v[ks][1]);
}

template <class E>
__device__ __forceinline__ void load_slab(float (&s)[NB][4], const E* panel, int cb) {
  const int l = lane_id(), c = cb * 16 + (l & 15), r4 = (l >> 4) * 4;
#pragma unroll
  for (int J = 0; J < NB; ++J)
#pragma unroll
    for (int e = 0; e < 4; ++e) s[J][e] = (float)panel[(J * BS + r4 + e) * KD + c];
}


}  // namespace sd

namespace sd {

// Pre-split (bf16 hi + lo) MFMA operand fragment and the 3-term product.
struct Frag { bf16x8 h, l; };

__device__ __forceinline__ f4 mma3f(const Frag& a, const Frag& b, f4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.l, b.h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.l, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.h, acc, 0, 0, 0);
}

struct BlkS { Frag f[4]; };

__device__ __forceinline__ void split_blk(const Blk& b, BlkS& o) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const float v[8] = {b.v[ks][0].x, b.v[ks][0].y, b.v[ks][0].z, b.v[ks][0].w,
                        b.v[ks][1].x, b.v[ks][1].y, b.v[ks][1].z, b.v[ks][1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      __bf16 h, l;
      split_bf(v[e], h, l);
      o.f[ks].h[e] = h;
      o.f[ks].l[e] = l;
    }
  }
}

// A B operand exact in bf16 (split from bf16 values: its low half is zero):
// two MFMAs per K slice (the B-low term is exactly 0).
__device__ __forceinline__ f4 mma2f_bh(const Frag& a, const Frag& b, f4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.l, b.h, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.h, acc, 0, 0, 0);
}
__device__ __forceinline__ f4 mma_blks_bh(const BlkS& A, const BlkS& B, f4 acc) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) acc = mma2f_bh(A.f[ks], B.f[ks], acc);
  return acc;
}

// An A operand exact in bf16 (staged from a bf16 panel: its low half is zero):
// the high halves only, two MFMAs per K slice (the A-low term is exactly 0).
struct BlkH { bf16x8 h[4]; };
__device__ __forceinline__ f4 mma_blks_h(const BlkH& A, const BlkS& B, f4 acc) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A.h[ks], B.f[ks].l, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A.h[ks], B.f[ks].h, acc, 0, 0, 0);
  }
  return acc;
}

__device__ __forceinline__ f4 mma_blks(const BlkS& A, const BlkS& B, f4 acc) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) acc = mma3f(A.f[ks], B.f[ks], acc);
  return acc;
}

// Per-lane decay factors for the slab applies of one 16-column block:
//   E1[J][e] = exp(R_J - G_j), j = J*16 + (lane>>4)*4 + e  (0 for wild coords),
// and exp(Gx_i - R_J) for the block pairs J <= I (RowF / ColF below).
__device__ __forceinline__ int pidx(int I, int J) { return I * (I + 1) / 2 + J; }

struct Tab1 {
  float E1[NB][4];
  unsigned wm;  // bit J: this lane's coordinate is wild in block J (read once, not per use)
};

__device__ __forceinline__ void make_tab1(const ChunkDecay& cd, int cb, Tab1& t) {
  const int l = lane_id(), c = cb * 16 + (l & 15), r4 = (l >> 4) * 4;
  t.wm = 0;
#pragma unroll
  for (int J = 0; J < NB; ++J) {
    const bool wild = cd.wild[J][c];
    t.wm |= (wild ? 1u : 0u) << J;
#pragma unroll
    for (int e = 0; e < 4; ++e) t.E1[J][e] = exp_unless_wild(wild, cd.R[J][c] - cd.G[J * BS + r4 + e][c]);
  }
}

// Block decay factors in factored form: exp(Gx_i - R_J) = RowF[I][e] * ColF[pidx(I, J)]
// (i = I*BS + r4 + e, J <= I) with RowF = exp(Gx_i - R_I), Gx the inclusive or
// exclusive prefix, and ColF = exp(R_I - R_J), for this lane's coordinate.  Every
// exponent is <= 0 (the prefix only falls), so neither factor overflows.
struct RowF { float f[NB][4]; };
struct ColF { float f[10]; };

template <bool EXCL>
__device__ __forceinline__ void make_rowf(const ChunkDecay& cd, int cb, RowF& t) {
  const int l = lane_id(), c = cb * 16 + (l & 15), r4 = (l >> 4) * 4;
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = I * BS + r4 + e;
      const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
      t.f[I][e] = __expf(gx - cd.R[I][c]);
    }
}

__device__ __forceinline__ void make_colf(const ChunkDecay& cd, int cb, ColF& t) {
  const int c = cb * 16 + (lane_id() & 15);
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int J = 0; J <= I; ++J) t.f[pidx(I, J)] = J == I ? 1.f : __expf(cd.R[I][c] - cd.R[J][c]);
}

// Slab applies with precomputed factors: R_I = sum_{J<=I} e^{Gx_i - R_J} (M_IJ (Y_J (.) E1_J))
// for this wave's 16 columns, and the transposed form; wild coordinates take the
// exact elementwise path.
template <bool EXCL, class FW>
__device__ f4 apply_tab(const ChunkDecay& cd, const float* M, const float (&Y)[NB][4], int I, int cb,
                        const Tab1& t1, const RowF& rf, const ColF& cf, FW Yw) {
  const int l = lane_id(), m = l & 15, r4 = (l >> 4) * 4, c = cb * 16 + m;
  f4 tot = zero4();
#pragma unroll
  for (int J = 0; J < NB; ++J) {
    if (J > I) break;
    const float4 mv = *reinterpret_cast<const float4*>(&M[(I * BS + m) * LS + J * BS + r4]);
    const float av[4] = {mv.x, mv.y, mv.z, mv.w};
    float bv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) bv[e] = Y[J][e] * t1.E1[J][e];
    const f4 a2 = mma16s(av, bv, zero4());
    if ((t1.wm >> J) & 1u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = I * BS + r4 + e;
        const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
        float add = 0.f;
        #pragma unroll 1  // rare wild path: keep it small and low-pressure
        for (int j = J * BS; j < J * BS + BS; ++j)
          add += M[i * LS + j] * Yw(j, c) * __expf(fminf(gx - cd.G[j][c], 0.f));
        tot[e] += add;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) tot[e] += rf.f[I][e] * cf.f[pidx(I, J)] * a2[e];
    }
  }
  return tot;
}

template <bool EXCL, class FW>
__device__ f4 apply_t_tab(const ChunkDecay& cd, const float* M, const float (&X)[NB][4], int Jb,
                          int cb, const Tab1& t1, const RowF& rf, const ColF& cf, FW Xw) {
  const int l = lane_id(), m = l & 15, r4 = (l >> 4) * 4, c = cb * 16 + m;
  f4 acc = zero4();
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    if (I < Jb) continue;
    float av[4], bv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      av[e] = M[(I * BS + r4 + e) * LS + Jb * BS + m];
      bv[e] = X[I][e] * (rf.f[I][e] * cf.f[pidx(I, Jb)]);
    }
    acc = mma16s(av, bv, acc);
  }
  f4 res;
  if ((t1.wm >> Jb) & 1u) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = Jb * BS + r4 + e;
      float s = 0.f;
      #pragma unroll 1  // rare wild path: keep it small and low-pressure
      for (int i = j; i < BT; ++i) {
        const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
        s += M[i * LS + j] * Xw(i, c) * __expf(fminf(gx - cd.G[j][c], 0.f));
      }
      res[e] = s;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) res[e] = t1.E1[Jb][e] * acc[e];
  }
  return res;
}


// Two applies sharing Y (and so every decay factor): R1 with M1, R2 with M2.
template <bool EXCL, class FW>
__device__ void apply2_tab(const ChunkDecay& cd, const float* M1, const float* M2,
                           const float (&Y)[NB][4], int I, int cb, const Tab1& t1, const RowF& rf,
                           const ColF& cf, FW Yw, f4& r1, f4& r2) {
  static_assert(!EXCL, "the factored block factors are inclusive");
  const int l = lane_id(), m = l & 15, r4 = (l >> 4) * 4, c = cb * 16 + m;
  r1 = zero4();
  r2 = zero4();
#pragma unroll
  for (int J = 0; J < NB; ++J) {
    if (J > I) break;
    const float4 m1 = *reinterpret_cast<const float4*>(&M1[(I * BS + m) * LS + J * BS + r4]);
    const float4 m2 = *reinterpret_cast<const float4*>(&M2[(I * BS + m) * LS + J * BS + r4]);
    const float a1[4] = {m1.x, m1.y, m1.z, m1.w}, a2v[4] = {m2.x, m2.y, m2.z, m2.w};
    float bv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) bv[e] = Y[J][e] * t1.E1[J][e];
    const f4 p1 = mma16s(a1, bv, zero4());
    const f4 p2 = mma16s(a2v, bv, zero4());
    if ((t1.wm >> J) & 1u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = I * BS + r4 + e;
        const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
        float s1 = 0.f, s2 = 0.f;
        #pragma unroll 1  // rare wild path: keep it small and low-pressure
        for (int j = J * BS; j < J * BS + BS; ++j) {
          const float f = Yw(j, c) * __expf(fminf(gx - cd.G[j][c], 0.f));
          s1 += M1[i * LS + j] * f;
          s2 += M2[i * LS + j] * f;
        }
        r1[e] += s1;
        r2[e] += s2;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float f = rf.f[I][e] * cf.f[pidx(I, J)];
        r1[e] += f * p1[e];
        r2[e] += f * p2[e];
      }
    }
  }
}

// Two transposed applies sharing the decay factors: R1 = M1 with X1, R2 = M2 with X2.
template <bool EXCL, class FW1, class FW2>
__device__ void apply_t2_tab(const ChunkDecay& cd, const float* M1, const float (&X1)[NB][4],
                             const float* M2, const float (&X2)[NB][4], int Jb, int cb,
                             const Tab1& t1, const RowF& rf, const ColF& cf, FW1 X1w, FW2 X2w,
                             f4& r1, f4& r2) {
  static_assert(!EXCL, "the factored block factors are inclusive");
  const int l = lane_id(), m = l & 15, r4 = (l >> 4) * 4, c = cb * 16 + m;
  f4 acc1 = zero4(), acc2 = zero4();
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    if (I < Jb) continue;
    float av1[4], av2[4], bv1[4], bv2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = (I * BS + r4 + e) * LS + Jb * BS + m;
      av1[e] = M1[row];
      av2[e] = M2[row];
      const float f = rf.f[I][e] * cf.f[pidx(I, Jb)];
      bv1[e] = X1[I][e] * f;
      bv2[e] = X2[I][e] * f;
    }
    acc1 = mma16s(av1, bv1, acc1);
    acc2 = mma16s(av2, bv2, acc2);
  }
  if ((t1.wm >> Jb) & 1u) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = Jb * BS + r4 + e;
      float s1 = 0.f, s2 = 0.f;
      #pragma unroll 1  // rare wild path: keep it small and low-pressure
      for (int i = j; i < BT; ++i) {
        const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
        const float f = __expf(fminf(gx - cd.G[j][c], 0.f));
        s1 += M1[i * LS + j] * X1w(i, c) * f;
        s2 += M2[i * LS + j] * X2w(i, c) * f;
      }
      r1[e] = s1;
      r2[e] = s2;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r1[e] = t1.E1[Jb][e] * acc1[e];
      r2[e] = t1.E1[Jb][e] * acc2[e];
    }
  }
}


// ---------------------------------------------------------------------------
// Pre-split LDS panels: a 64 x 128 fp32 chunk panel held as bf16 hi + bf16 lo,
// row-major with K contiguous, so every wave reads MFMA-ready fragments with
// 16-byte LDS loads instead of re-splitting fp32 operands on each use.
// ---------------------------------------------------------------------------
constexpr int LPS = KD + 8;  // row stride (bf16 elements), keeps 16-byte alignment

struct LPanel {
  __bf16 h[BT][LPS];
  __bf16 l[BT][LPS];
};

// All CT threads: src is a [64][128] fp32 panel (row stride KD) in global memory;
// optional scale(i, c) multiplies each element before the split.
template <class E, class FS>
__device__ __forceinline__ void stage_panel(LPanel& P, const E* src, FS scale) {
  constexpr int PER = BT * KD / 4 / CT;  // float4 per thread
  float4 v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) v[q] = ld4f(src + (threadIdx.x + q * CT) * 4);
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 4, i = idx / KD, c = idx % KD;
    const float x[4] = {v[q].x * scale(i, c), v[q].y * scale(i, c + 1), v[q].z * scale(i, c + 2),
                        v[q].w * scale(i, c + 3)};
    bf16x4 hh, ll;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      __bf16 a, b;
      split_bf(x[e], a, b);
      hh[e] = a;
      ll[e] = b;
    }
    *reinterpret_cast<bf16x4*>(&P.h[i][c]) = hh;
    *reinterpret_cast<bf16x4*>(&P.l[i][c]) = ll;
  }
}

template <class E>
__device__ __forceinline__ void stage_panel(LPanel& P, const E* src) {
  stage_panel(P, src, [](int, int) { return 1.f; });
}

// Fragments of the 16-row block starting at row0 (A or B operand layout).
__device__ __forceinline__ void lblk(const LPanel& P, int row0, BlkS& o) {
  const int l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    o.f[ks].h = *reinterpret_cast<const bf16x8*>(&P.h[row0 + m][ks * 32 + kq]);
    o.f[ks].l = *reinterpret_cast<const bf16x8*>(&P.l[row0 + m][ks * 32 + kq]);
  }
}

__device__ __forceinline__ void lblk_h(const LPanel& P, int row0, BlkH& o) {
  const int l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) o.h[ks] = *reinterpret_cast<const bf16x8*>(&P.h[row0 + m][ks * 32 + kq]);
}

// The low-half rows of a panel read as a bf16-exact A operand (a second exact
// panel staged there; see stage_panel_bf).
__device__ __forceinline__ void lblk_l(const LPanel& P, int row0, BlkH& o) {
  const int l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) o.h[ks] = *reinterpret_cast<const bf16x8*>(&P.l[row0 + m][ks * 32 + kq]);
}

// All CT threads: a [64][128] bf16 panel in global memory (row stride KD),
// exact in bf16, copied as it is into dst ([BT][LPS] rows).
__device__ __forceinline__ void stage_panel_bf(__bf16 (*dst)[LPS], const __bf16* src) {
  constexpr int PER = BT * KD / 8 / CT;  // 16-byte pieces per thread
  bf16x8 v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) v[q] = *reinterpret_cast<const bf16x8*>(src + (threadIdx.x + q * CT) * 8);
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 8, i = idx / KD, c = idx % KD;
    *reinterpret_cast<bf16x8*>(&dst[i][c]) = v[q];
  }
}

template <class E>
__device__ __forceinline__ void load_split_blk_g(const E* rows, BlkS& o) {
  Blk raw;
  load_blk(raw, rows, KD);
  split_blk(raw, o);
}



// Pair matrix M = A Y^T over K = 128 (strict: j < i, else j <= i) from two LDS
// panels, A exact in bf16 (staged from bf16 values: no low half).
__device__ __forceinline__ void lds_pair_h(const LPanel& A, const LPanel& Y, float* M, bool strict) {
  const int w = wave_id();
  for (int pp = w; pp < 10; pp += CW) {
    int I = 0, J = pp;
    while (J > I) { J -= I + 1; ++I; }
    BlkH a;
    BlkS y;
    lblk_h(A, I * BS, a);
    lblk(Y, J * BS, y);
    const f4 r = mma_blks_h(a, y, zero4());
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = I * BS + out_row(e), j = J * BS + out_col();
      M[i * LS + j] = (strict ? j < i : j <= i) ? r[e] : 0.f;
    }
  }
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int i = idx / BT, j = idx % BT;
    if ((j / BS) > (i / BS)) M[i * LS + j] = 0.f;
  }
}


// Two pair matrices against one Y panel in one pass: M1 = A.h Y^T (j < i) and
// M2 = diag(s2) A.l Y^T (j <= i), the high and low rows of A holding two
// bf16-exact panels and s2(i) a row scale of M2.  Ends without a barrier, as
// lds_pair_h.
struct NoScale { __device__ float operator()(int) const { return 1.f; } };
template <class S2 = NoScale>
__device__ __forceinline__ void lds_pair2_h(const LPanel& A, const LPanel& Y, float* M1, float* M2,
                                            S2 s2 = S2()) {
  const int w = wave_id();
  for (int pp = w; pp < 10; pp += CW) {
    int I = 0, J = pp;
    while (J > I) { J -= I + 1; ++I; }
    BlkH a1, a2;
    BlkS y;
    lblk_h(A, I * BS, a1);
    lblk_l(A, I * BS, a2);
    lblk(Y, J * BS, y);
    const f4 r1 = mma_blks_h(a1, y, zero4());
    const f4 r2 = mma_blks_h(a2, y, zero4());
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = I * BS + out_row(e), j = J * BS + out_col();
      M1[i * LS + j] = j < i ? r1[e] : 0.f;
      M2[i * LS + j] = j <= i ? r2[e] * s2(i) : 0.f;
    }
  }
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int i = idx / BT, j = idx % BT;
    if ((j / BS) > (i / BS)) {
      M1[i * LS + j] = 0.f;
      M2[i * LS + j] = 0.f;
    }
  }
}

// Y side of a decayed Gram staged once for all block pairs:
//   Yt[j][c] = Y(j, c) exp(R_J[c] - G[j][c])   (J = j / BS; 0 on a wild coordinate of J),
// split into bf16 hi / lo.  Every block J is used by 4 - J pairs, and each pair would
// otherwise recompute its transform.  All CT threads; every value is read before the
// first barrier, so Yt may share storage with what Y reads.
template <class FY>
__device__ void stage_ytilde(LPanel& Yt, const ChunkDecay& cd, FY Y) {
  constexpr int PER = BT * KD / 4 / CT;  // 4-column groups per thread
  float v[PER][4];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 4, j = idx / KD, c = idx % KD, J = j / BS;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[q][e] = Y(j, c + e) *
                exp_unless_wild(cd.wild[J][c + e] != 0, cd.R[J][c + e] - cd.G[j][c + e]);
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int idx = (threadIdx.x + q * CT) * 4, j = idx / KD, c = idx % KD;
    bf16x4 hh4, ll4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      __bf16 a, b2;
      split_bf(v[q][e], a, b2);
      hh4[e] = a;
      ll4[e] = b2;
    }
    *reinterpret_cast<bf16x4*>(&Yt.h[j][c]) = hh4;
    *reinterpret_cast<bf16x4*>(&Yt.l[j][c]) = ll4;
  }
  __syncthreads();
}

// Exact fix-up of a decayed Gram for wild coordinates (their terms were left
// out of the factored product), then a barrier.
template <bool EXCL, class FX, class FYR>
__device__ void gram_wild_fixup(const ChunkDecay& cd, FX X, FYR Yraw, bool strict, float* M,
                                int ldm = LS) {
  for (int J = 0; J < NB; ++J) {
    const int nw = cd.nwild[J];
    if (nw == 0) continue;
    const int J0 = J * BS;
    const int npairs = (BT - J0) * BS;
    for (int idx = threadIdx.x; idx < npairs; idx += CT) {
      const int ii = J0 + idx / BS, j = J0 + idx % BS;
      const bool keep = strict ? (j < ii) : (j <= ii);
      if (!keep) continue;
      float sacc = 0.f;
#pragma unroll 1
      for (int q = 0; q < nw; ++q) {
        const int c = cd.wlist[J][q];
        const float gx = EXCL ? gx_excl(cd, ii, c) : cd.G[ii][c];
        sacc += X(ii, c) * Yraw(j, c) * __expf(fminf(gx - cd.G[j][c], 0.f));
      }
      M[ii * ldm + j] += sacc;
    }
  }
  __syncthreads();
}

// decayed_gram with its Y side staged by stage_ytilde: per pair only the X side
// (X(i, c) exp(Gx_ic - R_J[c])) is transformed and split; Yraw(j, c) gives the
// untransformed Y for the exact wild-coordinate fix-up.
template <bool EXCL, class FX, class FYR>
__device__ void decayed_gram_yt(const ChunkDecay& cd, FX X, const LPanel& Yt, FYR Yraw, bool strict,
                                float* M, int ldm = LS) {
  const int w = wave_id(), l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
  for (int p = w; p < 10; p += CW) {
    int I = 0, J = p;
    while (J > I) { J -= I + 1; ++I; }  // p -> (I, J) with J <= I
    const int I0 = I * BS, J0 = J * BS, i = I0 + m;
    const float* RJ = cd.R[J];
    float xr[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) xr[ks][e] = X(i, ks * 32 + kq + e);
    BlkS A, B;
    lblk(Yt, J0, B);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = ks * 32 + kq + e;
        const float gx = EXCL ? gx_excl(cd, i, c) : cd.G[i][c];
        v[e] = xr[ks][e] * __expf(gx - RJ[c]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        __bf16 h, lo;
        split_bf(v[e], h, lo);
        A.f[ks].h[e] = h;
        A.f[ks].l[e] = lo;
      }
    }
    const f4 acc = mma_blks(A, B, zero4());
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ii = I0 + out_row(e), j = J0 + out_col();
      const bool keep = strict ? (j < ii) : (j <= ii);
      M[ii * ldm + j] = keep ? acc[e] : 0.f;
    }
  }
  // Zero the strictly-upper block pairs.
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int ii = idx / BT, j = idx % BT;
    if ((j / BS) > (ii / BS)) M[ii * ldm + j] = 0.f;
  }
  __syncthreads();
  gram_wild_fixup<EXCL>(cd, X, Yraw, strict, M, ldm);
}

// Two decayed Grams against one staged Y side, in one pass over the block
// pairs:  M1 = X1 Y~ (j <= i) into M, and M2 = X2 Y~ (j < i) returned in the
// caller's registers (the pairs p = wave, wave + CW of the 10, in that order)
// for gram2_second_store.  The two X sides share the decay factor
// exp(G_ic - R_J[c]) and the B fragments.  Ends with M1's zero blocks written
// and a barrier; M1's wild-coordinate fix-up is gram_wild_fixup's, as is M2's
// once it is stored.
template <class FX1, class FX2>
__device__ void decayed_gram2_yt(const ChunkDecay& cd, FX1 X1, FX2 X2, const LPanel& Yt, float* M,
                                 f4 (&acc2)[2]) {
  const int w = wave_id(), l = lane_id(), m = l & 15, kq = (l >> 4) * 8;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int p = w + it * CW;
    acc2[it] = zero4();
    if (p >= 10) break;
    int I = 0, J = p;
    while (J > I) { J -= I + 1; ++I; }
    const int I0 = I * BS, J0 = J * BS, i = I0 + m;
    const float* RJ = cd.R[J];
    float x1[4][8], x2[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x1[ks][e] = X1(i, ks * 32 + kq + e);
        x2[ks][e] = X2(i, ks * 32 + kq + e);
      }
    BlkS A1, A2, B;
    lblk(Yt, J0, B);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = ks * 32 + kq + e;
        const float f = __expf(cd.G[i][c] - RJ[c]);
        __bf16 h, lo;
        split_bf(x1[ks][e] * f, h, lo);
        A1.f[ks].h[e] = h;
        A1.f[ks].l[e] = lo;
        split_bf(x2[ks][e] * f, h, lo);
        A2.f[ks].h[e] = h;
        A2.f[ks].l[e] = lo;
      }
    const f4 r1 = mma_blks(A1, B, zero4());
    acc2[it] = mma_blks(A2, B, zero4());
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ii = I0 + out_row(e), j = J0 + out_col();
      M[ii * LS + j] = j <= ii ? r1[e] : 0.f;
    }
  }
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int ii = idx / BT, j = idx % BT;
    if ((j / BS) > (ii / BS)) M[ii * LS + j] = 0.f;
  }
  __syncthreads();
}

// The second Gram of decayed_gram2_yt written into M (strict: j < i; zero
// blocks included), then its barrier.  M must be free for writing.
__device__ __forceinline__ void gram2_second_store(const f4 (&acc2)[2], float* M) {
  const int w = wave_id();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int p = w + it * CW;
    if (p >= 10) break;
    int I = 0, J = p;
    while (J > I) { J -= I + 1; ++I; }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ii = I * BS + out_row(e), j = J * BS + out_col();
      M[ii * LS + j] = j < ii ? acc2[it][e] : 0.f;
    }
  }
  for (int idx = threadIdx.x; idx < BT * BT; idx += CT) {
    const int ii = idx / BT, j = idx % BT;
    if ((j / BS) > (ii / BS)) M[ii * LS + j] = 0.f;
  }
  __syncthreads();
}


}  // namespace sd
