// ugk_encoder.hip - token + position encoder forward (a gather) and backward
// (a scatter-add), train_bnn.c:41-65 and :647-662.
//
// Forward: one wavefront per (b,t) row; it reads the token id once, then
// streams wte[token] and wpe[t] as float4 and writes their sum. One IEEE add
// per element, so the result is bit-identical to the CPU loop.
//
// Backward, made deterministic and bit-identical to the CPU loop, which adds
// the rows of dout into dwte[token] and dwpe[t] in ascending (b,t) order:
//
//   dwpe: thread per (t, 4 channels) adds dout[0,t], dout[1,t], ... in b order.
//
//   dwte: the (b,t) rows are bucketed by token, then each bucket is added in
//   ascending (b,t) order. The tokens are processed in chunks of at most
//   kChunk rows (chunk k+1 is queued after chunk k, preserving the order):
//     K1 insert  - open-addressing hash table keyed by token (2x the chunk,
//                  power of two, linear probing, atomicCAS). Each row gets its
//                  slot and an arrival rank from atomicAdd on the slot count.
//                  The same launch also runs the dwpe threads (first chunk).
//     K2 scan    - exclusive scan of the slot counts in blocks of 4096 slots
//                  (the bucket starts within a block, and block totals).
//     K2 place   - thread per row: bucket start = earlier blocks' totals +
//                  its start within the block; row i goes to start + rank
//                  together with its bucket's start, size and token.
//     K3 add     - (also clears the table for the next chunk or call)
//                  one wavefront per placed position. A bucket of n rows is
//                  handled by the wavefront at its first position when
//                  n <= 64: the n row ids are ranked by comparison (ids are
//                  distinct) and the rows added in ascending order, 4 channels
//                  per lane. For n > 64 the wavefronts at its first
//                  ceil(C/64) positions each take 64 channels (one per lane),
//                  so the long serial chains of a frequent token run 64-wide on
//                  12 wavefronts at C=768; each builds an LDS bitmap of the
//                  bucket's row ids and walks it in ascending order.
//   The arrival order inside a bucket depends on scheduling, but it is
//   discarded: only the set of row ids is used, always in ascending order.
#include "ugk_internal.h"

namespace ugk {
namespace {

constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kChunk = 65536;            // rows per bucketing pass
constexpr int kTableMax = 2 * kChunk;    // hash slots (power of two)
constexpr int kSmall = kWave;            // bucket size handled by one wave
constexpr int kEmpty = -1;

// ---- forward ---------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void k_enc_fwd_vec(float4 *__restrict__ out, const int *__restrict__ inp,
                                                        const float4 *__restrict__ wte,
                                                        const float4 *__restrict__ wpe, int BT, int T,
                                                        int C4) {
  const int lane = threadIdx.x & (kWave - 1);
  const int bt = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (bt >= BT) return;
  const int t = bt % T;
  const int ix = inp[bt];
  const float4 *a = wte + (size_t)ix * C4;
  const float4 *p = wpe + (size_t)t * C4;
  float4 *o = out + (size_t)bt * C4;
  for (int c = lane; c < C4; c += kWave) {
    const float4 x = a[c], y = p[c];
    st_nt(o + c, make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
  }
}

__global__ __launch_bounds__(kBlock) void k_enc_fwd_scalar(float *out, const int *inp, const float *wte,
                                                           const float *wpe, int BT, int T, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  const int bt = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (bt >= BT) return;
  const int t = bt % T;
  const int ix = inp[bt];
  for (int c = lane; c < C; c += kWave)
    out[(size_t)bt * C + c] = wte[(size_t)ix * C + c] + wpe[(size_t)t * C + c];
}

// ---- backward --------------------------------------------------------------

struct EncState {
  int *keys;       // [kTableMax] token per slot, kEmpty when free (kept clean between calls)
  int *cnt;        // [kTableMax] rows per slot (kept zero between calls)
  int *bstart;     // [kTableMax] bucket start of a slot within its scan block (valid during a call)
  int *slot_of;    // [kChunk] slot of row i of the chunk (-1: skipped)
  int *rank_of;    // [kChunk] arrival rank of row i within its slot
  int4 *meta;      // [kChunk] per placed position: {bucket start, bucket size, token, row}
  int *total;      // [1] number of placed rows
  int *btot;       // [kTableMax / kScanSpan] slot count of each scan block
};

__device__ __forceinline__ unsigned hash_slot(int tok, unsigned mask, int shift) {
  return ((unsigned)tok * 0x9E3779B1u) >> shift & mask;
}

// K1: insert the chunk's rows; blocks past the insert range run dwpe.
template <bool kVec>
__global__ __launch_bounds__(kBlock) void k_enc_bwd_insert(EncState s, const int *__restrict__ inp, int n,
                                                           unsigned mask, int shift, int ins_blocks,
                                                           float *dwpe, const float *dout, int B, int T,
                                                           int C) {
  if ((int)blockIdx.x < ins_blocks) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const int tok = inp[i];
    if (tok < 0) {
      s.slot_of[i] = -1;
      return;
    }
    // At most n distinct tokens occupy 2n or more slots, so a free or matching
    // slot is always found; the probe count is bounded all the same.
    unsigned h = hash_slot(tok, mask, shift);
    bool found = false;
    for (unsigned probe = 0; probe <= mask; probe++) {
      const int prev = atomicCAS(&s.keys[h], kEmpty, tok);
      if (prev == kEmpty || prev == tok) {
        found = true;
        break;
      }
      h = (h + 1) & mask;
    }
    if (!found) {
      s.slot_of[i] = -1;
      return;
    }
    s.slot_of[i] = (int)h;
    s.rank_of[i] = atomicAdd(&s.cnt[h], 1);
    return;
  }
  // dwpe[t, c] += dout[b, t, c] for b = 0..B-1, in order; 8 rows in flight.
  const size_t j = (size_t)(blockIdx.x - ins_blocks) * kBlock + threadIdx.x;
  constexpr int kB = 8;
  if (kVec) {
    const int C4 = C >> 2;
    if (j >= (size_t)T * C4) return;
    const int t = (int)(j / C4), c4 = (int)(j % C4);
    float4 *p = reinterpret_cast<float4 *>(dwpe) + j;
    const float4 *g = reinterpret_cast<const float4 *>(dout) + (size_t)t * C4 + c4;
    float4 acc = *p;
    for (int b0 = 0; b0 < B; b0 += kB) {
      float4 d[kB];
#pragma unroll
      for (int q = 0; q < kB; q++)
        if (b0 + q < B) d[q] = ld_nt(g + (size_t)(b0 + q) * T * C4);
#pragma unroll
      for (int q = 0; q < kB; q++)
        if (b0 + q < B) {
          acc.x += d[q].x; acc.y += d[q].y; acc.z += d[q].z; acc.w += d[q].w;
        }
    }
    *p = acc;
  } else {
    if (j >= (size_t)T * C) return;
    const int t = (int)(j / C), c = (int)(j % C);
    float acc = dwpe[j];
    for (int b0 = 0; b0 < B; b0 += kB) {
      float d[kB];
#pragma unroll
      for (int q = 0; q < kB; q++)
        if (b0 + q < B) d[q] = dout[((size_t)(b0 + q) * T + t) * C + c];
#pragma unroll
      for (int q = 0; q < kB; q++)
        if (b0 + q < B) acc += d[q];
    }
    dwpe[j] = acc;
  }
}

// K2a: exclusive scan of the slot counts within blocks of kScanSpan slots
// (1024 threads x 4 slots): bstart[h] = slots before h in its block,
// btot[b] = the block's total.
constexpr int kScanThreads = 1024;
constexpr int kScanSpan = 4 * kScanThreads;
__global__ __launch_bounds__(kScanThreads) void k_enc_bwd_scan(EncState s, int tsize) {
  __shared__ int wsum[kScanThreads / kWave];
  const int tid = threadIdx.x;
  const int h0 = blockIdx.x * kScanSpan + tid * 4;
  int4 c = make_int4(0, 0, 0, 0);
  if (h0 < tsize) c = *reinterpret_cast<const int4 *>(s.cnt + h0);  // tsize is a multiple of 64
  const int local = c.x + c.y + c.z + c.w;
  const int lane = tid & (kWave - 1), wave = tid >> 6;
  int inc = local;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(inc, off);
    if (lane >= off) inc += y;
  }
  if (lane == kWave - 1) wsum[wave] = inc;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; w++) before += wsum[w];
  if (tid == kScanThreads - 1) s.btot[blockIdx.x] = before + inc;
  const int e = before + inc - local;
  if (h0 < tsize)
    *reinterpret_cast<int4 *>(s.bstart + h0) = make_int4(e, e + c.x, e + c.x + c.y, e + c.x + c.y + c.z);
}

// K2b: place every row at (start of its bucket) + (its arrival rank), with its
// bucket's start, size and token. Bucket start = totals of the scan blocks
// before the slot's block + bstart[slot].
constexpr int kMaxScanBlocks = kTableMax / kScanSpan;
__global__ __launch_bounds__(kBlock) void k_enc_bwd_place(EncState s, int n, int nscan) {
  __shared__ int bpre[kMaxScanBlocks + 1];
  if (threadIdx.x == 0) {
    int run = 0;
    for (int b = 0; b < nscan; b++) {
      bpre[b] = run;
      run += s.btot[b];
    }
    bpre[nscan] = run;
    if (blockIdx.x == 0) s.total[0] = run;
  }
  __syncthreads();
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const int h = s.slot_of[i];
  if (h < 0) return;
  const int rk = s.rank_of[i];
  const int st = bpre[h / kScanSpan] + s.bstart[h];
  s.meta[st + rk] = make_int4(st, s.cnt[h], s.keys[h], i);
}

// K3: add the buckets, one wavefront per placed position. Dynamic LDS: per
// wave max(kSmall, words) 32-bit words.
template <bool kVec>
__global__ __launch_bounds__(kBlock) void k_enc_bwd_add(EncState s, float *__restrict__ dwte,
                                                        const float *__restrict__ dout, int n, int C,
                                                        int words, int tsize) {
  extern __shared__ unsigned lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  // K2b was the table's last reader: return the used slots to empty
  for (int h = blockIdx.x * kBlock + threadIdx.x; h < tsize; h += gridDim.x * kBlock) {
    s.keys[h] = kEmpty;
    s.cnt[h] = 0;
  }
  const int p = blockIdx.x * kWavesPerBlock + wave;
  if (p >= n || p >= s.total[0]) return;
  const int per_wave = words > kSmall ? words : kSmall;
  unsigned *mine = lds + (size_t)wave * per_wave;
  const int4 mt = s.meta[p];
  const int start = mt.x, cnt = mt.y, tok = mt.z;
  const int k = p - start;
  if (cnt <= kSmall) {
    if (k != 0) return;
    int nrow = 1;
    if (cnt == 1) {
      mine[0] = (unsigned)mt.w;
    } else {
      // rank the bucket's row ids; ids are distinct, so ranks are a permutation
      const int id = lane < cnt ? s.meta[start + lane].w : 0x7fffffff;
      int rank = 0;
      for (int j = 0; j < cnt; j++) {
        const int o = __shfl(id, j);
        rank += (o < id) ? 1 : 0;
      }
      if (lane < cnt) mine[rank] = (unsigned)id;
      nrow = cnt;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (kVec) {
      const int C4 = C >> 2;
      float4 *row = reinterpret_cast<float4 *>(dwte) + (size_t)tok * C4;
      const float4 *g = reinterpret_cast<const float4 *>(dout);
      for (int c4 = lane; c4 < C4; c4 += kWave) {
        float4 acc = row[c4];
        for (int q = 0; q < nrow; q++) {
          const float4 d = ld_nt(g + (size_t)mine[q] * C4 + c4);
          acc.x += d.x; acc.y += d.y; acc.z += d.z; acc.w += d.w;
        }
        row[c4] = acc;
      }
    } else {
      float *row = dwte + (size_t)tok * C;
      for (int c = lane; c < C; c += kWave) {
        float acc = row[c];
        for (int q = 0; q < nrow; q++) acc += dout[(size_t)mine[q] * C + c];
        row[c] = acc;
      }
    }
    return;
  }
  // large bucket: wave k takes channel slices k, k+cnt, ...
  const int nslices = (C + kWave - 1) / kWave;
  if (k >= nslices) return;
  for (int w = lane; w < words; w += kWave) mine[w] = 0u;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int j = lane; j < cnt; j += kWave) {
    const int id = s.meta[start + j].w;
    atomicOr(&mine[id >> 5], 1u << (id & 31));
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int sl = k; sl < nslices; sl += cnt) {
    const int c = sl * kWave + lane;
    const bool on = c < C;
    float acc = on ? dwte[(size_t)tok * C + c] : 0.0f;
    for (int w0 = 0; w0 < words; w0 += kWave) {
      const unsigned mw = (w0 + lane < words) ? mine[w0 + lane] : 0u;
      unsigned long long nz = __ballot(mw != 0u);
      while (nz) {
        const int j = __builtin_ctzll(nz);
        nz &= nz - 1;
        unsigned bits = __shfl(mw, j);
        const int base = (w0 + j) << 5;
        while (bits) {
          const int b = __builtin_ctz(bits);
          bits &= bits - 1;
          if (on) acc += dout[(size_t)(base + b) * C + c];
        }
      }
    }
    if (on) dwte[(size_t)tok * C + c] = acc;
  }
}

__global__ void k_enc_init(EncState s) {
  const int h = blockIdx.x * kBlock + threadIdx.x;
  if (h < kTableMax) {
    s.keys[h] = kEmpty;
    s.cnt[h] = 0;
  }
}

size_t state_bytes() {
  return ((size_t)3 * kTableMax + (size_t)2 * kChunk + 64 + kMaxScanBlocks) * sizeof(int) +
         (size_t)kChunk * sizeof(int4);
}

EncState carve(void *base) {
  int4 *m = static_cast<int4 *>(base);
  EncState s;
  s.meta = m;
  int *p = reinterpret_cast<int *>(m + kChunk);
  s.keys = p; p += kTableMax;
  s.cnt = p; p += kTableMax;
  s.bstart = p; p += kTableMax;
  s.slot_of = p; p += kChunk;
  s.rank_of = p; p += kChunk;
  s.total = p; p += 64;
  s.btot = p;
  return s;
}

// The table must start empty; K2 returns it to empty after each chunk. State
// is kept per device in the encoder's own allocation (not the shared scratch,
// which other ops overwrite).
struct DevState {
  void *mem = nullptr;
};
DevState g_state[64];

}  // namespace

size_t encoder_backward_scratch(int) { return state_bytes(); }

int launch_encoder_forward(float *out, const int *inp, const float *wte, const float *wpe, int B,
                           int T, int C) {
  const int BT = B * T;
  if (BT == 0 || C == 0) return 0;
  const dim3 grid(grid_for((size_t)BT, kWavesPerBlock)), block(kBlock);
  if ((C & 3) == 0 && aligned16(out) && aligned16(wte) && aligned16(wpe)) {
    hipLaunchKernelGGL(k_enc_fwd_vec, grid, block, 0, stream(), reinterpret_cast<float4 *>(out), inp,
                       reinterpret_cast<const float4 *>(wte), reinterpret_cast<const float4 *>(wpe), BT,
                       T, C >> 2);
  } else {
    hipLaunchKernelGGL(k_enc_fwd_scalar, grid, block, 0, stream(), out, inp, wte, wpe, BT, T, C);
  }
  return check_launch("encoder_forward");
}

int launch_encoder_backward(float *dwte, float *dwpe, const float *dout, const int *inp, int B,
                            int T, int C) {
  const int BT = B * T;
  if (BT == 0 || C == 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(2, "encoder_backward: hipGetDevice failed");
  DevState &ds = g_state[dev];
  if (!ds.mem) {
    if (hipMalloc(&ds.mem, state_bytes()) != hipSuccess) {
      ds.mem = nullptr;
      (void)hipGetLastError();
      return set_error(3, "encoder_backward: cannot allocate %zu bytes of bucket state", state_bytes());
    }
    hipLaunchKernelGGL(k_enc_init, dim3(grid_for(kTableMax, kBlock)), dim3(kBlock), 0, stream(),
                       carve(ds.mem));
  }
  const EncState s = carve(ds.mem);
  const bool vec = (C & 3) == 0 && aligned16(dwte) && aligned16(dwpe) && aligned16(dout);
  for (int c0 = 0; c0 < BT; c0 += kChunk) {
    const int n = BT - c0 < kChunk ? BT - c0 : kChunk;
    int tsize = 64, lg = 6;
    while (tsize < 2 * n) { tsize <<= 1; lg++; }
    const unsigned mask = (unsigned)tsize - 1u;
    const int shift = 32 - lg;
    const int ins_blocks = (int)grid_for((size_t)n, kBlock);
    int pe_blocks = 0;
    if (c0 == 0) pe_blocks = (int)grid_for((size_t)T * (vec ? C / 4 : C), kBlock);
    if (vec)
      hipLaunchKernelGGL(k_enc_bwd_insert<true>, dim3(ins_blocks + pe_blocks), dim3(kBlock), 0, stream(), s,
                         inp + c0, n, mask, shift, ins_blocks, dwpe, dout, B, T, C);
    else
      hipLaunchKernelGGL(k_enc_bwd_insert<false>, dim3(ins_blocks + pe_blocks), dim3(kBlock), 0, stream(), s,
                         inp + c0, n, mask, shift, ins_blocks, dwpe, dout, B, T, C);
    const int nscan = (tsize + kScanSpan - 1) / kScanSpan;
    hipLaunchKernelGGL(k_enc_bwd_scan, dim3(nscan), dim3(kScanThreads), 0, stream(), s, tsize);
    hipLaunchKernelGGL(k_enc_bwd_place, dim3(ins_blocks), dim3(kBlock), 0, stream(), s, n, nscan);
    const int words = (n + 31) / 32;
    const size_t lds = (size_t)kWavesPerBlock * (size_t)(words > kSmall ? words : kSmall) * sizeof(unsigned);
    const float *dchunk = dout + (size_t)c0 * C;
    if (vec)
      hipLaunchKernelGGL(k_enc_bwd_add<true>, dim3(grid_for((size_t)n, kWavesPerBlock)), dim3(kBlock), lds,
                         stream(), s, dwte, dchunk, n, C, words, tsize);
    else
      hipLaunchKernelGGL(k_enc_bwd_add<false>, dim3(grid_for((size_t)n, kWavesPerBlock)), dim3(kBlock), lds,
                         stream(), s, dwte, dchunk, n, C, words, tsize);
  }
  return check_launch("encoder_backward");
}

}  // namespace ugk
