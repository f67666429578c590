// ugk_formats.hip - the file formats an end-to-end run reads and writes: the
// token .bin files of the data loader (gpt2_kernels.cuh:898-930, 1318-1331)
// and the parameter checkpoints (:944-964, :1281-1316).
//
// Token file: 256 int32 header (header[0] = 20240520, header[2] = token
// count), then the tokens as uint16. The loader serves windows of BT tokens:
// inputs = tokens[pos, pos+BT), targets = tokens[pos+1, pos+BT+1), pos += BT,
// wrapping to 0 when the window (plus the one-token shift) would pass the end.
// The tokens are read once into host memory, as the reference does; the
// device form keeps a uint16 copy resident in HBM (2 bytes per token, made on
// first use) and widens each window to int32 on the GPU, so a step moves no
// tokens over PCIe.
//
// Checkpoint: 8 int32 header {20240520, n low word, C, L, V, NH, steps,
// n high word}, then n floats. Saving and loading stream the buffer through
// two pinned staging chunks, so the device copy of one chunk overlaps the file
// write (or read) of the other.
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/ugk.h"
#include "ugk_internal.h"

namespace ugk {
namespace {

constexpr int kTokenMagic = 20240520;
constexpr size_t kStageBytes = (size_t)64 << 20;  // per pinned staging chunk

__global__ __launch_bounds__(kBlock) void k_widen_window(int *__restrict__ inp, int *__restrict__ tgt,
                                                         const uint16_t *__restrict__ tok, int BT) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i < BT) {
    inp[i] = (int)tok[i];
    tgt[i] = (int)tok[i + 1];
  }
}

}  // namespace
}  // namespace ugk

using namespace ugk;

struct ugk_loader {
  uint16_t *host = nullptr;   // the tokens as read
  uint16_t *dev = nullptr;    // resident copy, made by the first device window
  long n = 0;
  long pos = 0;
};

namespace {
int fail(int code, const char *fmt, const char *a, long b = 0) { return set_error(code, fmt, a, b); }

// The shared window rule of gpt2_kernels.cuh:924-929: returns the start.
long take_window(ugk_loader *ld, int BT) {
  if (ld->pos + BT + 1 > ld->n) ld->pos = 0;
  const long start = ld->pos;
  ld->pos += BT;
  return start;
}

int read_token_header(FILE *f, const char *path, long *ntok) {
  int header[256];
  if (fread(header, sizeof(int), 256, f) != 256) return fail(UGK_EINVAL, "loader: bad header in %s", path);
  if (header[0] != kTokenMagic) return fail(UGK_EINVAL, "loader: bad magic in %s (%ld)", path, header[0]);
  if (header[2] < 0) return fail(UGK_EINVAL, "loader: negative token count in %s (%ld)", path, header[2]);
  *ntok = header[2];
  return UGK_OK;
}
}  // namespace

extern "C" {

int ugk_loader_count(const char *path, long *ntok) {
  if (!path || !ntok) return fail(UGK_EINVAL, "ugk_loader_count: %s", "NULL pointer");
  FILE *f = fopen(path, "rb");
  if (!f) return fail(UGK_EINVAL, "loader: cannot open %s", path);
  const int rc = read_token_header(f, path, ntok);
  fclose(f);
  return rc;
}

int ugk_loader_open(ugk_loader **out, const char *path) {
  if (!out || !path) return fail(UGK_EINVAL, "ugk_loader_open: %s", "NULL pointer");
  *out = nullptr;
  FILE *f = fopen(path, "rb");
  if (!f) return fail(UGK_EINVAL, "loader: cannot open %s", path);
  long ntok = 0;
  if (int rc = read_token_header(f, path, &ntok)) {
    fclose(f);
    return rc;
  }
  ugk_loader *ld = new ugk_loader;
  ld->n = ntok;
  ld->host = static_cast<uint16_t *>(malloc((size_t)(ntok > 0 ? ntok : 1) * sizeof(uint16_t)));
  if (!ld->host) {
    fclose(f);
    delete ld;
    return fail(UGK_ENOMEM, "loader: cannot hold %s (%ld tokens)", path, ntok);
  }
  if (fread(ld->host, sizeof(uint16_t), (size_t)ntok, f) != (size_t)ntok) {
    fclose(f);
    free(ld->host);
    delete ld;
    return fail(UGK_EINVAL, "loader: short read on %s (%ld tokens expected)", path, ntok);
  }
  fclose(f);
  *out = ld;
  set_error(UGK_OK, "%s", "");
  return UGK_OK;
}

long ugk_loader_tokens(const ugk_loader *ld) { return ld ? ld->n : -1; }
long ugk_loader_position(const ugk_loader *ld) { return ld ? ld->pos : -1; }

int ugk_loader_next(ugk_loader *ld, int *h_inp, int *h_tgt, int BT) {
  if (!ld || !h_inp || !h_tgt) return fail(UGK_EINVAL, "ugk_loader_next: %s", "NULL pointer");
  if (BT < 0 || (long)BT + 1 > ld->n)
    return set_error(UGK_EINVAL, "ugk_loader_next: a window of BT+1 = %ld tokens needs more than the %ld loaded",
                     (long)BT + 1, ld->n);
  const long start = take_window(ld, BT);
  for (int i = 0; i < BT; i++) {
    h_inp[i] = (int)ld->host[start + i];
    h_tgt[i] = (int)ld->host[start + 1 + i];
  }
  set_error(UGK_OK, "%s", "");
  return UGK_OK;
}

int ugk_loader_next_device(ugk_loader *ld, int *d_inp, int *d_tgt, int BT) {
  if (!ld || !d_inp || !d_tgt) return fail(UGK_EINVAL, "ugk_loader_next_device: %s", "NULL pointer");
  if (BT < 0 || (long)BT + 1 > ld->n)
    return set_error(UGK_EINVAL,
                     "ugk_loader_next_device: a window of BT+1 = %ld tokens needs more than the %ld loaded",
                     (long)BT + 1, ld->n);
  if (!ld->dev) {
    const size_t bytes = (size_t)ld->n * sizeof(uint16_t);
    if (hipMalloc(&ld->dev, bytes) != hipSuccess) {
      (void)hipGetLastError();
      ld->dev = nullptr;
      return set_error(UGK_ENOMEM, "loader: cannot place %ld tokens in device memory", ld->n);
    }
    if (hipMemcpy(ld->dev, ld->host, bytes, hipMemcpyHostToDevice) != hipSuccess)
      return set_error(UGK_EHIP, "loader: copy to device failed: %s", hipGetErrorString(hipGetLastError()));
  }
  const long start = take_window(ld, BT);
  if (BT == 0) return UGK_OK;
  hipLaunchKernelGGL(k_widen_window, dim3(grid_for((size_t)BT, kBlock)), dim3(kBlock), 0, stream(), d_inp, d_tgt,
                     ld->dev + start, BT);
  if (int rc = check_launch("ugk_loader_next_device")) return rc;
  set_error(UGK_OK, "%s", "");
  return UGK_OK;
}

int ugk_loader_close(ugk_loader *ld) {
  if (!ld) return UGK_OK;
  int rc = UGK_OK;
  if (ld->dev) {
    // a queued window may still read the resident copy
    if (hipStreamSynchronize(stream()) != hipSuccess || hipFree(ld->dev) != hipSuccess)
      rc = set_error(UGK_EHIP, "ugk_loader_close: %s", hipGetErrorString(hipGetLastError()));
  }
  free(ld->host);
  delete ld;
  return rc;
}

// gpt2_kernels.cuh:950-951 / :1289-1290
int ugk_ckpt_path(char *buf, size_t size, const char *arm, const char *what, ugk_config cfg, int steps) {
  if (!buf || !arm || !what) return fail(UGK_EINVAL, "ugk_ckpt_path: %s", "NULL pointer");
  const int w = snprintf(buf, size, "runs/%s_C%d_L%d_%dk_%s.bin", arm, cfg.C, cfg.L, steps / 1000, what);
  if (w < 0 || (size_t)w >= size) return fail(UGK_EINVAL, "ugk_ckpt_path: buffer too small for %s", arm);
  return UGK_OK;
}

int ugk_ckpt_save(const char *path, const float *d_buf, size_t n, ugk_config cfg, int steps) {
  if (!path || (!d_buf && n)) return fail(UGK_EINVAL, "ugk_ckpt_save: %s", "NULL pointer");
  FILE *f = fopen(path, "wb");
  if (!f) return fail(UGK_EINVAL, "ckpt: cannot write %s", path);
  const int hdr[8] = {kTokenMagic, (int)(n & 0xffffffffu), cfg.C, cfg.L, cfg.V, cfg.NH, steps, (int)(n >> 32)};
  int rc = fwrite(hdr, sizeof(int), 8, f) == 8 ? UGK_OK : fail(UGK_EINVAL, "ckpt: write failed on %s", path);
  float *stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  const size_t chunk = kStageBytes / sizeof(float);
  if (rc == UGK_OK && n) {
    for (int k = 0; k < 2 && rc == UGK_OK; k++) {
      if (hipHostMalloc(reinterpret_cast<void **>(&stage[k]), kStageBytes, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&done[k], hipEventDisableTiming) != hipSuccess)
        rc = set_error(UGK_ENOMEM, "ckpt: cannot allocate pinned staging for %s", path);
    }
    // copy chunk i+1 while chunk i is written to the file
    size_t nchunks = (n + chunk - 1) / chunk;
    for (size_t i = 0; rc == UGK_OK && i <= nchunks; i++) {
      if (i < nchunks) {
        const size_t off = i * chunk, cnt = n - off < chunk ? n - off : chunk;
        if (hipMemcpyAsync(stage[i & 1], d_buf + off, cnt * sizeof(float), hipMemcpyDeviceToHost, stream()) !=
                hipSuccess ||
            hipEventRecord(done[i & 1], stream()) != hipSuccess)
          rc = set_error(UGK_EHIP, "ckpt: device copy failed: %s", hipGetErrorString(hipGetLastError()));
      }
      if (rc == UGK_OK && i > 0) {
        const size_t j = i - 1, off = j * chunk, cnt = n - off < chunk ? n - off : chunk;
        if (hipEventSynchronize(done[j & 1]) != hipSuccess)
          rc = set_error(UGK_EHIP, "ckpt: device copy failed: %s", hipGetErrorString(hipGetLastError()));
        else if (fwrite(stage[j & 1], sizeof(float), cnt, f) != cnt)
          rc = fail(UGK_EINVAL, "ckpt: write failed on %s", path);
      }
    }
  }
  if (hipStreamSynchronize(stream()) != hipSuccess && rc == UGK_OK)
    rc = set_error(UGK_EHIP, "ckpt: %s", hipGetErrorString(hipGetLastError()));
  for (int k = 0; k < 2; k++) {
    if (done[k]) (void)hipEventDestroy(done[k]);
    if (stage[k]) (void)hipHostFree(stage[k]);
  }
  if (fclose(f) != 0 && rc == UGK_OK) rc = fail(UGK_EINVAL, "ckpt: write failed on %s", path);
  if (rc == UGK_OK) set_error(UGK_OK, "%s", "");
  return rc;
}

int ugk_ckpt_load(const char *path, float *d_buf, size_t n, ugk_config cfg, int *steps) {
  if (!path || (!d_buf && n)) return fail(UGK_EINVAL, "ugk_ckpt_load: %s", "NULL pointer");
  FILE *f = fopen(path, "rb");
  if (!f) return fail(UGK_EINVAL, "ckpt: cannot open %s", path);
  int hdr[8];
  int rc = UGK_OK;
  if (fread(hdr, sizeof(int), 8, f) != 8) rc = fail(UGK_EINVAL, "ckpt: short header in %s", path);
  else if (hdr[0] != kTokenMagic) rc = fail(UGK_EINVAL, "ckpt: bad magic in %s (%ld)", path, hdr[0]);
  if (rc == UGK_OK) {
    const size_t got = (size_t)(unsigned)hdr[1] | ((size_t)(unsigned)hdr[7] << 32);
    if (got != n || hdr[2] != cfg.C || hdr[3] != cfg.L || hdr[4] != cfg.V || hdr[5] != cfg.NH) {
      char msg[512];
      snprintf(msg, sizeof msg,
               "ckpt: shape mismatch in %s: file n=%zu C=%d L=%d V=%d NH=%d, run n=%zu C=%d L=%d V=%d NH=%d", path,
               got, hdr[2], hdr[3], hdr[4], hdr[5], n, cfg.C, cfg.L, cfg.V, cfg.NH);
      rc = set_error(UGK_EINVAL, "%s", msg);
    }
  }
  float *stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  const size_t chunk = kStageBytes / sizeof(float);
  if (rc == UGK_OK && n) {
    for (int k = 0; k < 2 && rc == UGK_OK; k++) {
      if (hipHostMalloc(reinterpret_cast<void **>(&stage[k]), kStageBytes, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&done[k], hipEventDisableTiming) != hipSuccess)
        rc = set_error(UGK_ENOMEM, "ckpt: cannot allocate pinned staging for %s", path);
    }
    // read chunk i into one stage while chunk i-1 is copied from the other
    const size_t nchunks = (n + chunk - 1) / chunk;
    for (size_t i = 0; rc == UGK_OK && i < nchunks; i++) {
      const size_t off = i * chunk, cnt = n - off < chunk ? n - off : chunk;
      if (i >= 2 && hipEventSynchronize(done[i & 1]) != hipSuccess) {
        rc = set_error(UGK_EHIP, "ckpt: device copy failed: %s", hipGetErrorString(hipGetLastError()));
        break;
      }
      if (fread(stage[i & 1], sizeof(float), cnt, f) != cnt) {
        rc = fail(UGK_EINVAL, "ckpt: short read on %s", path);
        break;
      }
      if (hipMemcpyAsync(d_buf + off, stage[i & 1], cnt * sizeof(float), hipMemcpyHostToDevice, stream()) !=
              hipSuccess ||
          hipEventRecord(done[i & 1], stream()) != hipSuccess)
        rc = set_error(UGK_EHIP, "ckpt: device copy failed: %s", hipGetErrorString(hipGetLastError()));
    }
  }
  if (hipStreamSynchronize(stream()) != hipSuccess && rc == UGK_OK)
    rc = set_error(UGK_EHIP, "ckpt: %s", hipGetErrorString(hipGetLastError()));
  for (int k = 0; k < 2; k++) {
    if (done[k]) (void)hipEventDestroy(done[k]);
    if (stage[k]) (void)hipHostFree(stage[k]);
  }
  fclose(f);
  if (rc == UGK_OK) {
    if (steps) *steps = hdr[6];
    set_error(UGK_OK, "%s", "");
  }
  return rc;
}

}  // extern "C"
