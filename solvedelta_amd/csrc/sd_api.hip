// Host side of the C-ABI: validation, workspace layout and kernel launches.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include "../../include/solvedelta.h"
#include "sd_internal.h"

using namespace sd;

namespace {

constexpr int kBT = 64, kKD = 128;

struct Carver {
  char* base; size_t off = 0;
  template <class T> T* take(size_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

// The forward workspace is two regions: `saved` holds what sd_bwd reads (chunk
// states, inverses, forward token panels, the output pair P and the chunk
// decay); `scratch` holds the panels only the forward's state passes read (the
// decayed keys K^ and W, U of both ops, the readout's Q~), free once sd_fwd
// returns.  The backward forms K^ and Q~ again from d, chi and u.
FwdWs carve_fwd(void* saved, void* scratch, int B, int T, int H, size_t* saved_bytes,
                size_t* scratch_bytes) {
  const size_t n = (size_t)B * H, NT = (T + kBT - 1) / kBT, Tp = NT * kBT;
  const size_t panel = n * Tp * kKD, states = n * (NT + 1) * kKD * kKD, amat = n * NT * kBT * kBT;
  Carver c{(char*)saved};
  FwdWs w;
  w.Xc = c.take<xslot_t>(states);
  w.Xs = c.take<xslot_t>(states);
  w.Ac = c.take<float>(amat);
  w.As = c.take<float>(amat);
  w.e = c.take<fpan_t>(panel);
  w.chi = c.take<fpan_t>(panel);
  w.delta = c.take<fpan_t>(panel);
  w.d = c.take<fpan_t>(panel);
  w.wS = c.take<fpan_t>(panel);
  w.Gam = c.take<float>(n * NT * kKD);
  w.Ps = c.take<_Float16>(n * NT * kBT * kBT);
  if (saved_bytes) *saved_bytes = c.off + 256;
  Carver t{(char*)scratch};
  w.Kc = t.take<_Float16>(panel);
  w.Ks = t.take<_Float16>(panel);
  w.Qs = t.take<_Float16>(panel);
  w.Wc = t.take<_Float16>(panel);
  w.Uc = t.take<float>(panel);
  w.Ws = t.take<_Float16>(panel);
  w.Us = t.take<float>(panel);
  if (scratch_bytes) *scratch_bytes = t.off + 256;
  return w;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Saved / scratch sizes of either kernel family.
void fwd_sizes(int B, int T, int H, int r, int V, size_t* saved, size_t* scratch) {
  if (is_wide(r, V)) {
    wide_fwd_sizes(B, T, H, r, V, saved, scratch);
    return;
  }
  carve_fwd(nullptr, nullptr, B, T, H, saved, scratch);
}

int check_chunk_grid(const sd_inputs* in);

int fwd_launch(const sd_inputs* in, void* out, float* C_T, float* S_T, void* saved,
               void* scratch, hipStream_t st) {
  if (int rc = check_chunk_grid(in)) return rc;
  if (is_wide(in->r, in->V)) return launch_wide_fwd(in, out, C_T, S_T, saved, scratch, st);
  FwdWs w = carve_fwd(saved, scratch, in->B, in->T, in->H, nullptr, nullptr);
  return launch_fwd(in, out, C_T, S_T, w, st);
}

BwdWs carve_bwd(void* base, int B, int T, int H, size_t* total) {
  const size_t n = (size_t)B * H, NT = (T + kBT - 1) / kBT, Tp = NT * kBT;
  const size_t panel = n * Tp * kKD, states = n * (NT + 1) * kKD * kKD;
  Carver c{(char*)base};
  BwdWs w;
  // Buffers whose last reader runs before the first writer of another share
  // its storage (kernel order: bprep_s, state_s, grad_s, src_bwd, bprep_c,
  // state_c, grad_c (its tail closes u, k, h, gamma)): the C op's cotangent
  // slots take the S op's (last read by grad_s), grad_s's de / dchi take the
  // injection panels At1 / B1 (read by the S reverse pass, written again by
  // bprep_c after src_bwd has read de / dchi), and dw_S's storage holds dw_S,
  // then ddelta (src_bwd overwrites each row piece it has read; bprep_c reads
  // ddelta), then dw_C (written by the C reverse pass).  The sources
  // transpose's partial du / dk go to the du / dk gradients themselves, which
  // the C chunk gradient's tail reads and overwrites.
  w.Ls = c.take<lslot_t>(states);
  w.Lc = w.Ls;
  w.Wk = c.take<__bf16>(panel);
  w.At1 = c.take<__bf16>(panel);
  w.B1t = c.take<__bf16>(panel);
  w.Ant = c.take<__bf16>(panel);
  w.dU = c.take<float>(panel);
  static_assert(sizeof(bpan_t) == sizeof(__bf16), "de / dchi share the bf16 injection panels");
  w.de = reinterpret_cast<bpan_t*>(w.At1);
  w.dchi = reinterpret_cast<bpan_t*>(w.B1t);
  w.dwS = c.take<bpan_t>(panel);
  w.dd = c.take<bpan_t>(panel);
  w.ddelta = w.dwS;
  w.dwC = w.dwS;
  w.rn = c.take<float>(n * Tp * 2);
  w.Pp = c.take<float>(n * NT * kBT * kBT);
  if (total) *total = c.off + 256;
  return w;
}

bool view_ok(const sd_view& v) { return v.data != nullptr; }

int check_inputs(const sd_inputs* in) {
  if (!in) return SD_ERR_ARG;
  if (in->B < 1 || in->T < 1 || in->H < 1 || in->r < 1 || in->V < 1) return SD_ERR_SHAPE;
  if (in->r > kWideMax || in->V > kWideMax) return SD_ERR_SHAPE;
  if (!view_ok(in->u) || !view_ok(in->h) || !view_ok(in->q) || !view_ok(in->k) ||
      !view_ok(in->v) || !view_ok(in->erase_raw) || !view_ok(in->write_raw) ||
      !view_ok(in->log_decay) || !view_ok(in->gamma))
    return SD_ERR_ARG;
  return SD_OK;
}

// The chunked kernels' grids put B*H and the chunk count on axes capped at
// 65535 workgroups (the decode grid is one-dimensional and has no such cap).
int check_chunk_grid(const sd_inputs* in) {
  if ((long long)in->B * in->H > 65535 || (in->T + 31) / 32 > 65535) return SD_ERR_SHAPE;
  return SD_OK;
}

}  // namespace

extern "C" {

const char* sd_version(void) { return "solvedelta_amd 0.1 (gfx950)"; }

size_t sd_fwd_saved_bytes(int B, int T, int H, int r, int V) {
  size_t saved = 0, scratch = 0;
  fwd_sizes(B, T, H, r, V, &saved, &scratch);
  return saved;
}

size_t sd_fwd_scratch_bytes(int B, int T, int H, int r, int V) {
  size_t saved = 0, scratch = 0;
  fwd_sizes(B, T, H, r, V, &saved, &scratch);
  return scratch;
}

size_t sd_fwd_workspace_bytes(int B, int T, int H, int r, int V) {
  size_t saved = 0, scratch = 0;
  fwd_sizes(B, T, H, r, V, &saved, &scratch);
  return align256(saved) + scratch;
}

int sd_fwd(const sd_inputs* in, void* out, float* C_T, float* S_T, void* workspace,
           size_t workspace_bytes, void* stream) {
  int rc = check_inputs(in);
  if (rc) return rc;
  if (!out || !workspace) return SD_ERR_ARG;
  size_t saved = 0, scratch = 0;
  fwd_sizes(in->B, in->T, in->H, in->r, in->V, &saved, &scratch);
  if (workspace_bytes < align256(saved) + scratch) return SD_ERR_WORKSPACE;
  return fwd_launch(in, out, C_T, S_T, workspace, (char*)workspace + align256(saved),
                    (hipStream_t)stream);
}

int sd_fwd_split(const sd_inputs* in, void* out, float* C_T, float* S_T, void* saved,
                 size_t saved_bytes, void* scratch, size_t scratch_bytes, void* stream) {
  int rc = check_inputs(in);
  if (rc) return rc;
  if (!out || !saved || !scratch) return SD_ERR_ARG;
  size_t need_saved = 0, need_scratch = 0;
  fwd_sizes(in->B, in->T, in->H, in->r, in->V, &need_saved, &need_scratch);
  if (saved_bytes < need_saved || scratch_bytes < need_scratch) return SD_ERR_WORKSPACE;
  return fwd_launch(in, out, C_T, S_T, saved, scratch, (hipStream_t)stream);
}

int sd_decode(const sd_inputs* in, void* out, float* C_T, float* S_T, void* stream) {
  // the decode kernel holds r, V <= 128 (wider states take the chunked path)
  if (in && (in->T != 1 || in->r > kKD || in->V > kKD)) return SD_ERR_SHAPE;
  int rc = check_inputs(in);
  if (rc) return rc;
  if (!out) return SD_ERR_ARG;
  return launch_decode(in, out, C_T, S_T, (hipStream_t)stream);
}

size_t sd_bwd_workspace_bytes(int B, int T, int H, int r, int V) {
  if (is_wide(r, V)) return wide_bwd_workspace_bytes(B, T, H, r, V);
  size_t total = 0;
  carve_bwd(nullptr, B, T, H, &total);
  return total;
}

int sd_bwd(const sd_inputs* in, const void* fwd_workspace, const void* dout, const float* dC_T,
           const float* dS_T, void* du, void* dh, void* dq, void* dk, void* dv, void* derase,
           void* dwrite, float* dlog_decay, float* dgamma, float* dC0, float* dS0,
           void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_inputs(in);
  if (rc) return rc;
  if (!fwd_workspace || !workspace || !du || !dh || !dq || !dk || !dv || !derase || !dwrite ||
      !dlog_decay || !dgamma)
    return SD_ERR_ARG;
  if ((rc = check_chunk_grid(in))) return rc;
  size_t need = 0;
  if (is_wide(in->r, in->V)) {
    if (workspace_bytes < wide_bwd_workspace_bytes(in->B, in->T, in->H, in->r, in->V))
      return SD_ERR_WORKSPACE;
    return launch_wide_bwd(in, fwd_workspace, workspace, dout, dC_T, dS_T, du, dh, dq, dk, dv,
                           derase, dwrite, dlog_decay, dgamma, dC0, dS0, (hipStream_t)stream);
  }
  BwdWs bw = carve_bwd(workspace, in->B, in->T, in->H, &need);
  if (workspace_bytes < need) return SD_ERR_WORKSPACE;
  FwdWs fw = carve_fwd((void*)fwd_workspace, nullptr, in->B, in->T, in->H, nullptr, nullptr);
  return launch_bwd(in, fw, bw, dout, dC_T, dS_T, du, dh, dq, dk, dv, derase, dwrite, dlog_decay,
                    dgamma, dC0, dS0, (hipStream_t)stream);
}

}  // extern "C"
