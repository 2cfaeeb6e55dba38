// Row masking for the dense-batch masked operator (valid / reset masks without
// repacking): one launch copies up to eight [B,T,H,w] tensors, keeping the
// rows of valid tokens, zeroing the others, and giving the log-decay rows of
// reset tokens a fixed value.  The same kernel masks the gradients on the way
// back (zero on invalid tokens, zero log-decay gradient on reset tokens), in
// place when the destination is the (contiguous) source: then only the rows it
// changes are written and nothing is read but the flags.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include "../../include/solvedelta.h"
#include "sd_internal.h"

namespace sd {
namespace {

constexpr int kMaxMasked = 8;

struct MaskJob {
  int n;
  sd_mask_tensor t[kMaxMasked];
};

// One thread per 16 bytes of one row of one tensor when the tensor's rows are
// 16-byte aligned on both sides (vec), else per 4 elements.
struct MaskJobExt {
  MaskJob job;
  int vec[kMaxMasked];
  int inplace[kMaxMasked];
};

__global__ __launch_bounds__(256) void k_mask_rows(MaskJobExt jx, int B, int T, int H,
                                                   const uint8_t* __restrict__ flags,
                                                   long long f_sb, long long f_st) {
  const sd_mask_tensor& m = jx.job.t[blockIdx.y];
  const int esz = m.is_fp32 ? 4 : 2, w = m.width;
  const int per = jx.vec[blockIdx.y] ? 16 / esz : 4;  // elements per thread
  const int q = (w + per - 1) / per;
  const long long rows = (long long)B * T * H;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * q) return;
  const long long row = idx / q;
  const int c0 = (int)(idx % q) * per;
  const int hh = (int)(row % H), t = (int)((row / H) % T), b = (int)(row / ((long long)H * T));
  const uint8_t f = flags[(long long)b * f_sb + (long long)t * f_st];
  const bool valid = f & 1, reset = (f & 2) != 0;
  const bool fill = valid && reset && m.reset_fill;
  if (jx.inplace[blockIdx.y] && valid && !fill) return;  // the row keeps its values
  const long long so = (long long)b * m.sb + (long long)t * m.st + (long long)hh * m.sh;
  const long long dof = row * w;
  if (jx.vec[blockIdx.y]) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (valid && !fill) v = *reinterpret_cast<const uint4*>((const char*)m.src + (so + c0) * esz);
    if (fill) {
      if (m.is_fp32) {
        const unsigned r = __float_as_uint(m.reset_value);
        v = make_uint4(r, r, r, r);
      } else {
        const __bf16 r = (__bf16)m.reset_value;
        const unsigned short rb = *reinterpret_cast<const unsigned short*>(&r);
        const unsigned r2 = (unsigned)rb | ((unsigned)rb << 16);
        v = make_uint4(r2, r2, r2, r2);
      }
    }
    *reinterpret_cast<uint4*>((char*)m.dst + (dof + c0) * esz) = v;
    return;
  }
  for (int c = c0; c < c0 + per && c < w; ++c) {
    if (m.is_fp32) {
      float v = valid ? ((const float*)m.src)[so + c] : 0.f;
      if (valid && reset && m.reset_fill) v = m.reset_value;
      ((float*)m.dst)[dof + c] = v;
    } else {
      __bf16 v = valid ? ((const __bf16*)m.src)[so + c] : (__bf16)0.f;
      if (valid && reset && m.reset_fill) v = (__bf16)m.reset_value;
      ((__bf16*)m.dst)[dof + c] = v;
    }
  }
}

// In place (every tensor masked in its own contiguous storage): one wave per
// token reads the token's flag, and only the tokens whose rows change (invalid
// ones, and valid resets for tensors with reset_fill) write them; the others
// cost one flag read per wave instead of one per element.
__global__ __launch_bounds__(256) void k_mask_tokens_inplace(MaskJobExt jx, int B, int T, int H,
                                                             const uint8_t* __restrict__ flags,
                                                             long long f_sb, long long f_st) {
  const long long tok = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= (long long)B * T) return;
  const int b = (int)(tok / T), t = (int)(tok % T), l = threadIdx.x & 63;
  const uint8_t f = flags[(long long)b * f_sb + (long long)t * f_st];
  const bool valid = f & 1, reset = (f & 2) != 0;
  if (valid && !reset) return;
  for (int i = 0; i < jx.job.n; ++i) {
    const sd_mask_tensor& m = jx.job.t[i];
    const bool fill = valid && reset && m.reset_fill;
    if (valid && !fill) continue;
    const long long n = (long long)H * m.width, base = tok * n;
    if (m.is_fp32) {
      const float v = fill ? m.reset_value : 0.f;
      for (long long e = l; e < n; e += 64) ((float*)m.dst)[base + e] = v;
    } else {
      const __bf16 v = fill ? (__bf16)m.reset_value : (__bf16)0.f;
      for (long long e = l; e < n; e += 64) ((__bf16*)m.dst)[base + e] = v;
    }
  }
}

// Packed flags (bit 0 valid, bit 1 valid reset) and the fresh flags from the
// bool masks, one thread per token.
__global__ __launch_bounds__(256) void k_mask_flags(int B, int T, const uint8_t* valid,
                                                    long long v_sb, long long v_st,
                                                    const uint8_t* reset, long long r_sb,
                                                    long long r_st, uint8_t* flags, uint8_t* fresh) {
  const long long tok = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (tok >= (long long)B * T) return;
  const int b = (int)(tok / T), t = (int)(tok % T);
  const bool v = valid ? valid[(long long)b * v_sb + (long long)t * v_st] != 0 : true;
  const bool r = v && (reset ? reset[(long long)b * r_sb + (long long)t * r_st] != 0 : false);
  flags[tok] = (uint8_t)((v ? 1 : 0) | (r ? 2 : 0));
  fresh[tok] = (uint8_t)(!v ? SD_TOK_INVALID : r ? (SD_TOK_FRESH | SD_TOK_RESET) : 0u);
}

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" int sd_mask_rows(int B, int T, int H, const uint8_t* flags, int64_t flags_sb,
                            int64_t flags_st, const sd_mask_tensor* tensors, int n,
                            void* stream) {
  if (B < 1 || T < 1 || H < 1 || n < 1 || n > kMaxMasked) return SD_ERR_SHAPE;
  if (!flags || !tensors) return SD_ERR_ARG;
  MaskJobExt jx{};
  jx.job.n = n;
  long long work = 0;
  for (int i = 0; i < n; ++i) {
    const sd_mask_tensor& m = tensors[i];
    jx.job.t[i] = m;
    if (!m.src || !m.dst || m.width < 1) return SD_ERR_ARG;
    const long long esz = m.is_fp32 ? 4 : 2;
    const bool vec = ((uintptr_t)m.src % 16 == 0) && ((uintptr_t)m.dst % 16 == 0) &&
                     (m.width * esz) % 16 == 0 && (m.sb * esz) % 16 == 0 &&
                     (m.st * esz) % 16 == 0 && (m.sh * esz) % 16 == 0;
    jx.vec[i] = vec;
    // in place: the destination is the source itself, stored contiguously
    jx.inplace[i] = m.src == m.dst && m.sh == m.width && m.st == (int64_t)H * m.width &&
                    m.sb == (int64_t)T * H * m.width;
    if (m.src == m.dst && !jx.inplace[i]) return SD_ERR_ARG;
    const long long per = vec ? 16 / esz : 4;
    const long long items = (long long)B * T * H * ((m.width + per - 1) / per);
    work = items > work ? items : work;
  }
  bool all_inplace = true;
  for (int i = 0; i < n; ++i) all_inplace = all_inplace && jx.inplace[i];
  if (all_inplace) {
    const long long ntok = (long long)B * T;
    SD_LAUNCH("k_mask_rows", k_mask_tokens_inplace, dim3((unsigned)((ntok + 3) / 4)), dim3(256), 0,
              (hipStream_t)stream, jx, B, T, H, flags, (long long)flags_sb, (long long)flags_st);
    return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
  }
  const dim3 grid((unsigned)((work + 255) / 256), (unsigned)n);
  SD_LAUNCH("k_mask_rows", k_mask_rows, grid, dim3(256), 0, (hipStream_t)stream, jx, B, T, H,
            flags, (long long)flags_sb, (long long)flags_st);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}

extern "C" int sd_mask_flags(int B, int T, const uint8_t* valid, int64_t valid_sb,
                             int64_t valid_st, const uint8_t* reset, int64_t reset_sb,
                             int64_t reset_st, uint8_t* flags, uint8_t* fresh, void* stream) {
  if (B < 1 || T < 1) return SD_ERR_SHAPE;
  if (!flags || !fresh) return SD_ERR_ARG;
  const long long ntok = (long long)B * T;
  SD_LAUNCH("k_mask_flags", k_mask_flags, dim3((unsigned)((ntok + 255) / 256)), dim3(256), 0,
            (hipStream_t)stream, B, T, valid, (long long)valid_sb, (long long)valid_st, reset,
            (long long)reset_sb, (long long)reset_st, flags, fresh);
  return hipGetLastError() == hipSuccess ? SD_OK : SD_ERR_LAUNCH;
}
