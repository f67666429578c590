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
//   ascending (b,t) order. Rows are processed in chunks of at most kChunk
//   (chunk k+1 is queued after chunk k, preserving the order). Three launches
//   per chunk:
//     K1 insert  - each workgroup of 256 rows first groups its rows by
//                  token in an LDS hash table (local count, local rank), then
//                  one thread per distinct token probes the global open-
//                  addressing table (8x the chunk, at most kTableMax, power
//                  of two, linear probing). A slot is one 64-bit word, token and row count:
//                  a token's first workgroup claims a free slot with its
//                  count in one atomicCAS, later ones take a block of ranks
//                  with one atomicAdd. A frequent token thus costs one global
//                  atomic per workgroup, not one per row. The workgroup's
//                  distinct tokens are first listed, one per thread, so all
//                  their probes are in flight together. Every row records
//                  its slot; ranks below kCap also store the row id in the
//                  slot's own list. The slots a workgroup claims are listed
//                  in its 256-entry region of the slot list. The same launch
//                  runs the dwpe threads (first chunk).
//     K2 add     - one wavefront per slot-list entry (as many as rows, not
//                  as many as table slots). A bucket of at most kCap rows is
//                  ranked by comparison (row ids are distinct) and its rows
//                  added in ascending order, 4 channels per lane, 8 loads in
//                  flight. The same launch has one more workgroup per
//                  possible large bucket (K1 lists them with their slots):
//                  its 256 threads scan the rows' slots in row order, 6,144
//                  per round, and write the matching row ids, ascending, to a
//                  list for K3.
//     K3 large   - workgroups of 16 wavefronts, one per (large bucket, 64
//                  channels): one wavefront only adds staged rows in order,
//                  one channel per lane, from one half of a double-buffered
//                  LDS stage, while three groups of five loader wavefronts
//                  take turns staging the next round of 240 rows into the
//                  other half, each group loading its round three rounds
//                  ahead (one round of loads in flight per wavefront, so its
//                  waits are exact). A frequent token's serial chain of adds
//                  thus runs without waiting for its loads.
//   The table and its counters return to their cleared state within each
//   chunk, on the device: K2 frees each slot once it has read it (the
//   wavefront of its list entry, or the scan workgroup of a large bucket),
//   and the last K3 workgroup to finish zeroes the counters. No state stays
//   on the host between calls, so a captured HIP graph may replay any number
//   of calls.
//   The arrival order inside a bucket depends on scheduling, but it is
//   discarded: only the set of row ids is used, always in ascending order.
#include <atomic>
#include <mutex>

#include "ugk_internal.h"

namespace ugk {
namespace {

constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kChunk = 65536;            // rows per bucketing pass
constexpr int kTableMax = 2 * kChunk;    // hash slots (power of two)
// Table slots per row of a chunk (capped at kTableMax, which keeps at least
// 2): a sparse table shortens the atomicCAS probe chains of the insert and
// puts fewer claimed slots in one cache line. At 8,192 x 768 a quarter-full
// table was 3.9 us faster than a half-full one, and an eighth-full one another
// 1.2 us (no change at 16,384 rows, where the cap leaves it quarter-full).
constexpr int kLoadInv = 8;
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

// The same with the row held in registers: V float4 per lane (C/4 <= 64 V),
// every load of the row issued before the first store (columns past the row
// load the last one again and are not stored).
template <int V>
__global__ __launch_bounds__(kBlock) void k_enc_fwd_row(float4 *__restrict__ out, const int *__restrict__ inp,
                                                        const float4 *__restrict__ wte,
                                                        const float4 *__restrict__ wpe, int BT, int T, int C4) {
  const int lane = threadIdx.x & (kWave - 1);
  const int bt = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (bt >= BT) return;
  const size_t ot = (size_t)inp[bt] * C4, op = (size_t)(bt % T) * C4;
  float4 x[V], y[V];
#pragma unroll
  for (int v = 0; v < V; v++) {
    const int c = min(lane + v * kWave, C4 - 1);
    x[v] = wte[ot + c];
    y[v] = wpe[op + c];
  }
  float4 *o = out + (size_t)bt * C4;
#pragma unroll
  for (int v = 0; v < V; v++) {
    const int c = lane + v * kWave;
    if (c < C4) st_nt(o + c, make_float4(x[v].x + y[v].x, x[v].y + y[v].y, x[v].z + y[v].z, x[v].w + y[v].w));
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

constexpr int kCap = 32;                 // rows kept in a slot's own list
constexpr int kMaxLarge = kChunk / (kCap + 1) + 1;

typedef unsigned long long u64;
// A table slot: token in the high word, row count in the low word (a count
// never exceeds kChunk, so adding to the word never carries into the token).
constexpr u64 kFree = 0xffffffff00000000ull;  // token kEmpty, count 0
__device__ __forceinline__ u64 slot_word(int tok, int cnt) { return ((u64)(unsigned)tok << 32) | (unsigned)cnt; }
__device__ __forceinline__ int slot_tok(u64 s) { return (int)(s >> 32); }
__device__ __forceinline__ int slot_cnt(u64 s) { return (int)(unsigned)s; }

struct EncTable {
  u64 *slot;       // [kTableMax] token and row count per slot, kFree when free
  int *counters;   // [0] K3 work items taken, [1] large buckets, [2] sorted-id pool use, [3] K3 workgroups done
};

struct EncShared {
  int *rows;       // [kTableMax * kCap] row ids by (slot, rank < kCap)
  int *slot_of;    // [kChunk] slot of each row of the chunk (-1: skipped)
  int4 *lmeta;     // [kMaxLarge] large bucket: {pool offset, size, token, slot} (K1 writes token and slot)
  int *pool;       // [kChunk] row ids of the large buckets, each bucket ascending
  int *list;       // [kChunk] slots claimed by K1 workgroup b at [256 b, 256 b + k), -1 after
};

__device__ __forceinline__ unsigned hash_slot(int tok, unsigned mask, int shift) {
  return ((unsigned)tok * 0x9E3779B1u) >> shift & mask;
}

// K1: insert the chunk's rows; blocks past the insert range run dwpe.
template <bool kVec>
__global__ __launch_bounds__(kBlock) void k_enc_bwd_insert(EncTable tb, EncShared sh, const int *__restrict__ inp,
                                                           int n, unsigned mask, int shift, int ins_blocks,
                                                           float *dwpe, const float *dout, int B, int T, int C) {
  if ((int)blockIdx.x < ins_blocks) {
    constexpr int kL = 2 * kBlock;  // LDS table slots
    __shared__ int ltok[kL], lcnt[kL], lslot[kL], lbase[kL];
    __shared__ int lnew[kBlock + 1];  // slots this workgroup claimed; [kBlock] their number
    __shared__ int locc[kBlock + 1];  // occupied LDS slots (at most kBlock); [kBlock] their number
    for (int e = threadIdx.x; e < kL; e += kBlock) {
      ltok[e] = kEmpty;
      lcnt[e] = 0;
    }
    if (threadIdx.x == 0) {
      lnew[kBlock] = 0;
      locc[kBlock] = 0;
    }
    __syncthreads();
    const int i = blockIdx.x * kBlock + threadIdx.x;
    const int tok = i < n ? inp[i] : -1;
    int e = -1, lrank = 0;
    if (tok >= 0) {  // at most 256 distinct tokens in 512 slots: always found
      e = (int)hash_slot(tok, kL - 1, 32 - 9);
      for (int probe = 0; probe < kL; probe++) {
        const int prev = atomicCAS(&ltok[e], kEmpty, tok);
        if (prev == kEmpty || prev == tok) break;
        e = (e + 1) & (kL - 1);
      }
      lrank = atomicAdd(&lcnt[e], 1);
    }
    __syncthreads();
    // the occupied LDS slots, listed so that one thread each probes the
    // global table and all probes are in flight at once
    {
      const int lane = threadIdx.x & (kWave - 1);
      const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
      for (int f = threadIdx.x; f < kL; f += kBlock) {
        const bool occ = ltok[f] != kEmpty;
        const unsigned long long mk = __ballot(occ);
        int at = 0;
        if (lane == 0 && mk) at = atomicAdd(&locc[kBlock], __popcll(mk));
        at = __shfl(at, 0);
        if (occ) locc[at + __popcll(mk & below)] = f;
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < locc[kBlock]) {
      const int f = locc[threadIdx.x];
      const int t = ltok[f];
      // At most n distinct tokens occupy 2n or more slots, so a free or
      // matching slot is always found; the probe count is bounded all the same.
      const int c = lcnt[f];
      unsigned h = hash_slot(t, mask, shift);
      int base = -1;
      for (unsigned probe = 0; probe <= mask; probe++) {
        const u64 prev = atomicCAS(&tb.slot[h], kFree, slot_word(t, c));
        if (prev == kFree) {  // claimed: ranks [0, c) are this workgroup's
          base = 0;
          lnew[atomicAdd(&lnew[kBlock], 1)] = (int)h;
          break;
        }
        if (slot_tok(prev) == t) {
          base = slot_cnt(atomicAdd(&tb.slot[h], (u64)c));
          break;
        }
        h = (h + 1) & mask;
      }
      if (base < 0) {
        lslot[f] = -1;
      } else {
        // the workgroup whose ranks cross kCap (one per slot) lists the large bucket
        if (base <= kCap && kCap < base + c) sh.lmeta[atomicAdd(&tb.counters[1], 1)] = make_int4(0, 0, t, (int)h);
        lslot[f] = (int)h;
        lbase[f] = base;
      }
    }
    __syncthreads();
    sh.list[blockIdx.x * kBlock + threadIdx.x] = (int)threadIdx.x < lnew[kBlock] ? lnew[threadIdx.x] : -1;
    if (i >= n) return;
    const int h = e >= 0 ? lslot[e] : -1;
    sh.slot_of[i] = h;
    if (h >= 0) {
      const int rank = lbase[e] + lrank;
      if (rank < kCap) sh.rows[(size_t)h * kCap + rank] = i;
    }
    return;
  }
  // dwpe[t, c] += dout[b, t, c] for b = 0..B-1, in order; 8 rows in flight.
  // dout is read with ordinary (cached) loads: K2 reads the same rows again,
  // and finds part of them in the cache (K2 15.8 -> 14.3 us at 8,192 x 768).
  // Each dwpe thread takes two (t, c) entries, one after the other, so half
  // as many dwpe workgroups stream at once and the inserts' round trips are
  // delayed less (25.6 -> 24.8 us per call at 8,192 x 768).
  constexpr int kB = 8;
  const size_t pstride = (size_t)(gridDim.x - ins_blocks) * kBlock;
  const size_t n_pe = (size_t)T * (kVec ? C >> 2 : C);
  for (size_t j = (size_t)(blockIdx.x - ins_blocks) * kBlock + threadIdx.x; j < n_pe; j += pstride) {
    if (kVec) {
      const int C4 = C >> 2;
      const int t = (int)(j / C4), c4 = (int)(j % C4);
      float4 *p = reinterpret_cast<float4 *>(dwpe) + j;
      const float4 *g = reinterpret_cast<const float4 *>(dout) + (size_t)t * C4 + c4;
      float4 acc = *p;
      for (int b0 = 0; b0 < B; b0 += kB) {
        float4 d[kB];
#pragma unroll
        for (int q = 0; q < kB; q++)
          if (b0 + q < B) d[q] = g[(size_t)(b0 + q) * T * C4];
#pragma unroll
        for (int q = 0; q < kB; q++)
          if (b0 + q < B) {
            acc.x += d[q].x; acc.y += d[q].y; acc.z += d[q].z; acc.w += d[q].w;
          }
      }
      *p = acc;
    } else {
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
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// K2, scan workgroup of large bucket j: the chunk's row ids whose slot is the
// bucket's, in row order, to its share of the pool; 6 int4 loads of slots per
// thread per round (6,144 slots), the round's matches placed by a workgroup
// prefix over (load, wavefront). Frees the slot after reading its count.
// (8 loads per round would take K2 from 48 to 58 registers, and from ten
// wavefronts per SIMD to eight.)
constexpr int kScanQ = 6;
__device__ __forceinline__ void scan_large(EncTable tb, EncShared sh, int j, int n) {
  __shared__ int wt[kScanQ][kWavesPerBlock];
  __shared__ int pool_base, bucket_cnt;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int4 m = sh.lmeta[j];
  const int w = m.w;
  if (threadIdx.x == 0) {
    const int cnt = slot_cnt(tb.slot[w]);
    pool_base = atomicAdd(&tb.counters[2], cnt);
    bucket_cnt = cnt;
    tb.slot[w] = kFree;
  }
  __syncthreads();
  const int base = pool_base;
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  int run = 0;  // matches in the rounds before this one
  for (int i0 = 0; i0 < n; i0 += kScanQ * kBlock * 4) {
    int4 sl[kScanQ];
#pragma unroll
    for (int q = 0; q < kScanQ; q++) {
      const int e = i0 + (q * kBlock + (int)threadIdx.x) * 4;
      if (e + 3 < n) {
        sl[q] = *reinterpret_cast<const int4 *>(sh.slot_of + e);
      } else {
        sl[q].x = e < n ? sh.slot_of[e] : -1;
        sl[q].y = e + 1 < n ? sh.slot_of[e + 1] : -1;
        sl[q].z = e + 2 < n ? sh.slot_of[e + 2] : -1;
        sl[q].w = -1;
      }
    }
#pragma unroll
    for (int q = 0; q < kScanQ; q++) {
      const int k = __popcll(__ballot(sl[q].x == w)) + __popcll(__ballot(sl[q].y == w)) +
                    __popcll(__ballot(sl[q].z == w)) + __popcll(__ballot(sl[q].w == w));
      if (lane == 0) wt[q][wave] = k;
    }
    __syncthreads();
    // slots are ordered by (load q, wavefront, lane, element): the matches of
    // the (q, wavefront) pairs before this one come first
    int off = run;
    for (int q = 0; q < kScanQ; q++) {
      int o = off;
#pragma unroll
      for (int v = 0; v < kWavesPerBlock; v++) o += v < wave ? wt[q][v] : 0;
#pragma unroll
      for (int v = 0; v < kWavesPerBlock; v++) off += wt[q][v];
      const int e = i0 + (q * kBlock + (int)threadIdx.x) * 4;
      o += __popcll(__ballot(sl[q].x == w) & below) + __popcll(__ballot(sl[q].y == w) & below) +
           __popcll(__ballot(sl[q].z == w) & below) + __popcll(__ballot(sl[q].w == w) & below);
      if (sl[q].x == w) sh.pool[base + o++] = e;
      if (sl[q].y == w) sh.pool[base + o++] = e + 1;
      if (sl[q].z == w) sh.pool[base + o++] = e + 2;
      if (sl[q].w == w) sh.pool[base + o] = e + 3;
    }
    run = off;
    __syncthreads();  // wt is rewritten by the next round
  }
  if (threadIdx.x == 0) sh.lmeta[j] = make_int4(base, bucket_cnt, m.z, w);
}

// K2: one scan workgroup per possible large bucket in the first nscan
// workgroups (dispatched first, so that those with no bucket have left before
// the adds end), then one wavefront per slot-list entry (covering K1's
// regions exactly). A small bucket's wavefront frees its slot once it has
// read it.
template <bool kVec>
__global__ __launch_bounds__(kBlock) void k_enc_bwd_add(EncTable tb, EncShared sh, float *__restrict__ dwte,
                                                        const float *__restrict__ dout, int C, int n, int nscan) {
  __shared__ unsigned lds[kWavesPerBlock * kCap];
  if ((int)blockIdx.x < nscan) {
    const int j = (int)blockIdx.x;
    if (j < tb.counters[1]) scan_large(tb, sh, j, n);  // K1 has counted them: the same value in every thread
    return;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  unsigned *mine = lds + (size_t)wave * kCap;
  // Wavefront g takes entry g / R of region g % R (R regions of kBlock
  // entries): the entries of one region (one K1 workgroup's tokens, where a
  // skewed batch puts its frequent tokens early) spread over all workgroups.
  const int R = ((int)gridDim.x - nscan) * kWavesPerBlock / kBlock;
  const int gw = ((int)blockIdx.x - nscan) * kWavesPerBlock + wave;
  const int w = sh.list[(gw % R) * kBlock + gw / R];  // this wavefront's slot
  if (w < 0) return;
  // the slot word and the bucket's first row ids in one round trip (ids past
  // the count are stale and ignored)
  const u64 sw = tb.slot[w];
  const int id_raw = sh.rows[(size_t)w * kCap + (lane & (kCap - 1))];
  asm volatile("" ::"v"(id_raw));  // keeps the compiler from sinking the ids load below the branch
  const int cnt = slot_cnt(sw);
  const int tok = slot_tok(sw);
  // A large bucket belongs to its scan workgroup, which may already have
  // freed the slot (the word then reads count 0).
  if (cnt == 0 || cnt > kCap) return;
  // the slot's only reader has read it: free it for the next chunk's K1
  if (lane == 0) tb.slot[w] = kFree;
  // A bucket of one or two rows (nearly all of them with uniform tokens) in
  // one pass: every load of the row issued before the first add, instead of
  // one round trip per 64 float4 of the row. The same additions in the same
  // order as the loop below.
  if (kVec && cnt <= 2 && (C >> 2) <= 3 * kWave) {
    const int C4 = C >> 2;
    const int a = __builtin_amdgcn_readlane(id_raw, 0);
    const int b = cnt == 2 ? __builtin_amdgcn_readlane(id_raw, 1) : a;
    float4 *row = reinterpret_cast<float4 *>(dwte) + (size_t)tok * C4;
    const float4 *g0 = reinterpret_cast<const float4 *>(dout) + (size_t)min(a, b) * C4;
    const float4 *g1 = reinterpret_cast<const float4 *>(dout) + (size_t)max(a, b) * C4;
    float4 acc[3], d0[3], d1[3];
#pragma unroll
    for (int u = 0; u < 3; u++) {
      const int c4 = lane + u * kWave;
      if (c4 < C4) {
        acc[u] = row[c4];
        d0[u] = ld_nt(g0 + c4);
        if (cnt == 2) d1[u] = ld_nt(g1 + c4);
      }
    }
#pragma unroll
    for (int u = 0; u < 3; u++) {
      const int c4 = lane + u * kWave;
      if (c4 < C4) {
        float4 v = acc[u];
        v.x += d0[u].x; v.y += d0[u].y; v.z += d0[u].z; v.w += d0[u].w;
        if (cnt == 2) {
          v.x += d1[u].x; v.y += d1[u].y; v.z += d1[u].z; v.w += d1[u].w;
        }
        row[c4] = v;
      }
    }
    return;
  }
  // rank the bucket's row ids; ids are distinct, so ranks are a permutation
  const int id = lane < cnt ? id_raw : 0x7fffffff;
  int rank = 0;
  for (int j = 0; j < cnt; j++) rank += (__shfl(id, j) < id) ? 1 : 0;
  if (lane < cnt) mine[rank] = (unsigned)id;
  wave_lds_sync();
  // rows in ascending order, kBatch loads in flight before their adds
  constexpr int kBatch = 8;
  if (kVec) {
    const int C4 = C >> 2;
    float4 *row = reinterpret_cast<float4 *>(dwte) + (size_t)tok * C4;
    const float4 *g = reinterpret_cast<const float4 *>(dout);
    for (int c4 = lane; c4 < C4; c4 += kWave) {
      float4 acc = row[c4];
      for (int q0 = 0; q0 < cnt; q0 += kBatch) {
        float4 d[kBatch];
#pragma unroll
        for (int q = 0; q < kBatch; q++)
          if (q0 + q < cnt) d[q] = ld_nt(g + (size_t)mine[q0 + q] * C4 + c4);
#pragma unroll
        for (int q = 0; q < kBatch; q++)
          if (q0 + q < cnt) {
            acc.x += d[q].x; acc.y += d[q].y; acc.z += d[q].z; acc.w += d[q].w;
          }
      }
      row[c4] = acc;
    }
  } else {
    float *row = dwte + (size_t)tok * C;
    for (int c = lane; c < C; c += kWave) {
      float acc = row[c];
      for (int q0 = 0; q0 < cnt; q0 += kBatch) {
        float d[kBatch];
#pragma unroll
        for (int q = 0; q < kBatch; q++)
          if (q0 + q < cnt) d[q] = dout[(size_t)mine[q0 + q] * C + c];
#pragma unroll
        for (int q = 0; q < kBatch; q++)
          if (q0 + q < cnt) acc += d[q];
      }
      row[c] = acc;
    }
  }
}

// K3: workgroups take (large bucket, 64-channel slice) work items from a
// counter until none are left. A bucket's rows must be added in ascending row
// order, one dependent add per row and channel, so one wavefront (the adder,
// wavefront 0) does nothing else: it adds a round of 240 staged rows from one
// half of a double-buffered LDS stage while loader wavefronts stage the next
// round into the other half. The loaders form three groups of five; group
// g holds rounds g, g + 3, g + 6, ... (48 rows per wavefront), stages its
// round the iteration before the adder needs it and then loads its next
// one, so every row is loaded three rounds ahead and each loader has only
// its own round's loads in flight when it waits for them. Row ids come with
// one vector load per round, issued with the previous round's rows, and are
// read out lane by lane. Rows past the bucket are staged as -0.0f, which
// leaves every sum unchanged (x + -0.0f == x for every x, -0.0f included),
// so the adds test nothing.
constexpr int kGroups = 3;
constexpr int kGroupWaves = 5;
constexpr int kPerWave = 48;
constexpr int kRound = kGroupWaves * kPerWave;  // rows per round
constexpr int kLargeThreads = (kGroups * kGroupWaves + 1) * kWave;
constexpr int kLargeGrid = 256;

// The (bucket, slice) work items of one workgroup, until the counter passes
// `total`.
__device__ __forceinline__ void large_items(EncTable tb, EncShared sh, float *__restrict__ dwte,
                                            const float *__restrict__ dout, int C, int nslices, int total,
                                            float4 (*stage)[kWave][kRound / 4 + 1], int *next_item_p) {
  int &next_item = *next_item_p;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const bool adder = wave == 0;
  const int group = adder ? -1 : (wave - 1) / kGroupWaves;
  const int slot = adder ? 0 : (wave - 1) % kGroupWaves;  // this loader's share of a round
  const int mine = slot * kPerWave + (lane < kPerWave ? lane : 0);  // loader: row of this lane's id
  for (int first = 1;; first = 0) {
    // the next (bucket, slice) work item: a workgroup's first is its own
    // index (so that the grid does not start with one atomic per workgroup on
    // one counter), later ones come from the counter, so that workgroups with
    // short buckets go on to others
    if (threadIdx.x == 0) next_item = first ? (int)blockIdx.x : (int)gridDim.x + atomicAdd(&tb.counters[0], 1);
    __syncthreads();
    const int wi = next_item;
    __syncthreads();
    if (wi >= total) break;
    const int j = wi / nslices;
    const int c = (wi % nslices) * kWave + lane;
    const bool on = c < C;
    const int cc = on ? c : 0;  // a valid column for the lanes past C
    const int4 m = sh.lmeta[j];
    const int *ids = sh.pool + m.x;
    const int cnt = m.y;
    const int nrounds = (cnt + kRound - 1) / kRound;
    float acc = (adder && on) ? dwte[(size_t)m.z * C + c] : 0.0f;
    // a loader's round: the ids of its rows, then the rows
    float v[kPerWave];
    int idv = 0;
    auto load_ids = [&](int r) { return (r < nrounds && r * kRound + mine < cnt) ? ids[r * kRound + mine] : 0; };
    auto load_rows = [&]() {
#pragma unroll
      for (int q = 0; q < kPerWave; q++) v[q] = dout[(size_t)__builtin_amdgcn_readlane(idv, q) * C + cc];
    };
    auto stage_rows = [&](int r) {
      float4 *dst = &stage[r & 1][lane][slot * kPerWave / 4];
      const int lim = on ? cnt - r * kRound - slot * kPerWave : 0;
#pragma unroll
      for (int q = 0; q < kPerWave; q += 4)
        dst[q / 4] = make_float4(q < lim ? v[q] : -0.0f, q + 1 < lim ? v[q + 1] : -0.0f,
                                 q + 2 < lim ? v[q + 2] : -0.0f, q + 3 < lim ? v[q + 3] : -0.0f);
    };
    auto add_round = [&](int r) {
      // 16 staged rows at a time (whole batches: rows past the bucket hold
      // -0.0f), the next batches read from LDS while this one is added
      const float4 *src = stage[r & 1][lane];
      const int nb = (min(kRound, cnt - r * kRound) + 15) / 16;
      float4 t[4], u[4];
#pragma unroll
      for (int q = 0; q < 4; q++) t[q] = src[q];
      for (int b = 0; b < nb; b += 2) {
#pragma unroll
        for (int q = 0; q < 4; q++) u[q] = src[(b + 1 < kRound / 16 ? 4 * (b + 1) : 0) + q];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          acc += t[q].x;
          acc += t[q].y;
          acc += t[q].z;
          acc += t[q].w;
        }
        if (b + 1 >= nb) break;
#pragma unroll
        for (int q = 0; q < 4; q++) t[q] = src[(b + 2 < kRound / 16 ? 4 * (b + 2) : 0) + q];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          acc += u[q].x;
          acc += u[q].y;
          acc += u[q].z;
          acc += u[q].w;
        }
      }
    };
    // group g starts with round g; group 0 stages it at once and goes on to
    // round 3
    if (!adder && group < nrounds) {
      idv = load_ids(group);
      load_rows();
      idv = load_ids(group + kGroups);
      if (group == 0) {
        stage_rows(0);
        if (kGroups < nrounds) load_rows();
        idv = load_ids(2 * kGroups);
      }
    }
    __syncthreads();
    for (int k = 0; k < nrounds; k++) {
      // round k is in stage[k & 1]; the group holding round k + 1 stages it
      // into the other half and then loads its round k + 4
      if (adder) {
        add_round(k);
      } else if (group == (k + 1) % kGroups && k + 1 < nrounds) {
        stage_rows(k + 1);
        if (k + 1 + kGroups < nrounds) load_rows();
        idv = load_ids(k + 1 + 2 * kGroups);
      }
      __syncthreads();
    }
    if (adder && on) dwte[(size_t)m.z * C + c] = acc;
  }
}

__global__ __launch_bounds__(kLargeThreads) void k_enc_bwd_large(EncTable tb, EncShared sh,
                                                                 float *__restrict__ dwte,
                                                                 const float *__restrict__ dout, int C,
                                                                 int nslices) {
  // stage[h][channel][row]: a lane's rows are consecutive, so both sides
  // move four rows per LDS instruction; the row stride of kRound + 4 floats
  // puts the 16 lanes of each 16-byte access on distinct banks
  __shared__ float4 stage[2][kWave][kRound / 4 + 1];
  __shared__ int next_item;
  // The common case, no bucket beyond kCap rows: every counter is still zero
  // (K1 counts large buckets, K2 takes pool space for them), nothing to reset.
  // Otherwise every workgroup reads the same count: the counters are reset
  // only after the last workgroup has arrived below, past all its reads.
  const int total = tb.counters[1] * nslices;
  if (total == 0) return;
  large_items(tb, sh, dwte, dout, C, nslices, total, stage, &next_item);
  // every thread of this workgroup is past its last read of the counters; the
  // last workgroup to arrive zeroes them for the next chunk
  __syncthreads();
  if (threadIdx.x == 0 && atomicAdd(&tb.counters[3], 1) == (int)gridDim.x - 1) {
    tb.counters[0] = 0;
    tb.counters[1] = 0;
    tb.counters[2] = 0;
    tb.counters[3] = 0;
  }
}

// K3, blocked mode (the default): the same (large bucket, 64-channel slice)
// work items as k_enc_bwd_large, but the bucket's rows, ascending, are cut
// into blocks of kBlkRows, and the workgroup's 16 wavefronts add blocks
// w, w + 16, ... in parallel, each block's rows in row order, all its 64
// rows' loads in flight at once (one float per lane) and the next block's
// row ids loaded meanwhile. The first block starts from dwte's value, the
// others from -0.0f (the identity of IEEE addition); the block sums go to
// LDS, and wavefront 0 adds them in block order:
//   s_0 = ((dwte + d_0) + d_1) + ... + d_63,  s_k = d_64k + ... + d_64k+63,
//   dwte = ((s_0 + s_1) + s_2) + ...
// in rounds of at most kLdsBlocks blocks. The same inputs give the same bits
// on every run, and a bucket of at most 64 rows gets the CPU's order. A
// bucket of 2,348 rows is 37 blocks, at most three per wavefront, instead of
// a chain of 2,348 dependent adds. No state crosses workgroups: the counters
// and their reset are k_enc_bwd_large's.
constexpr int kBlkRows = 64;
constexpr int kBlockedWaves = 16;
constexpr int kLdsBlocks = 256;

__device__ __forceinline__ void blocked_items(EncTable tb, EncShared sh, float *__restrict__ dwte,
                                              const float *__restrict__ dout, int C, int nslices, int total,
                                              float (*bs)[kWave], int *next_item_p) {
  int &next_item = *next_item_p;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  for (int first = 1;; first = 0) {
    // a workgroup's first item is its own index, later ones come from the counter
    if (threadIdx.x == 0) next_item = first ? (int)blockIdx.x : (int)gridDim.x + atomicAdd(&tb.counters[0], 1);
    __syncthreads();
    const int wi = next_item;
    __syncthreads();
    if (wi >= total) break;
    const int j = wi / nslices;
    const int c = (wi % nslices) * kWave + lane;
    const bool on = c < C;
    const int cc = on ? c : 0;  // a valid column for the lanes past C, never stored
    const int4 m = sh.lmeta[j];
    const int *ids = sh.pool + m.x;
    const int cnt = m.y;
    const size_t trow = (size_t)m.z * C + cc;
    const int nb = (cnt + kBlkRows - 1) / kBlkRows;
    float t = -0.0f;  // wavefront 0's running total of the block sums
    for (int r0 = 0; r0 < nb; r0 += kLdsBlocks) {
      const int r1 = min(nb, r0 + kLdsBlocks);
      int k = r0 + wave;
      int id = k < r1 ? ids[k * kBlkRows + min(lane, cnt - k * kBlkRows - 1)] : 0;
      for (; k < r1; k += kBlockedWaves) {
        const int nr = min(kBlkRows, cnt - k * kBlkRows);
        float v[kBlkRows];
#pragma unroll
        for (int q = 0; q < kBlkRows; q++) v[q] = dout[(size_t)__builtin_amdgcn_readlane(id, min(q, nr - 1)) * C + cc];
        const int kn = k + kBlockedWaves;  // the next block's row ids, loaded while these rows arrive
        if (kn < r1) id = ids[kn * kBlkRows + min(lane, cnt - kn * kBlkRows - 1)];
        float a = k == 0 ? dwte[trow] : -0.0f;
#pragma unroll
        for (int q = 0; q < kBlkRows; q++)
          if (q < nr) a += v[q];  // the same for the whole wavefront
        bs[k - r0][lane] = a;
      }
      __syncthreads();
      if (wave == 0)
        for (int q = 0; q < r1 - r0; q++) t += bs[q][lane];
      __syncthreads();  // bs is rewritten by the next round
    }
    if (wave == 0 && on) dwte[trow] = t;
  }
}

__global__ __launch_bounds__(kBlockedWaves * kWave) void k_enc_bwd_blocked(EncTable tb, EncShared sh,
                                                                           float *__restrict__ dwte,
                                                                           const float *__restrict__ dout, int C,
                                                                           int nslices) {
  __shared__ float bs[kLdsBlocks][kWave];
  __shared__ int next_item;
  // As k_enc_bwd_large: with no large bucket every counter is still zero;
  // otherwise the last workgroup to arrive resets them after all their reads.
  const int total = tb.counters[1] * nslices;
  if (total == 0) return;
  blocked_items(tb, sh, dwte, dout, C, nslices, total, bs, &next_item);
  __syncthreads();
  if (threadIdx.x == 0 && atomicAdd(&tb.counters[3], 1) == (int)gridDim.x - 1) {
    tb.counters[0] = 0;
    tb.counters[1] = 0;
    tb.counters[2] = 0;
    tb.counters[3] = 0;
  }
}

__global__ void k_enc_init(EncTable t) {
  const int h = blockIdx.x * kBlock + threadIdx.x;
  if (h < kTableMax) t.slot[h] = kFree;
  if (h < 4) t.counters[h] = 0;
}

// ---- id guard -----------------------------------------------------------------
// The Python binding checks token and target ids with this kernel before a
// kernel indexes a table with them: ids outside [0, bound) are replaced in
// place by `fill` and recorded in the per-device error word, which
// ugk_synchronize reports. Ids in range are not written. No host round trip,
// so the calls stay asynchronous (and capturable).
}  // namespace
}  // namespace ugk

static __device__ int ids_error;

namespace ugk {
namespace {
__global__ __launch_bounds__(kBlock) void k_ids_guard(int *ids, int n, int bound, int fill, int code) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  if ((unsigned)ids[i] >= (unsigned)bound) {
    ids[i] = fill;
    ids_error = code;  // every writer stores the same word
  }
}

size_t table_ints() { return (size_t)2 * kTableMax + 64; }  // slot words (2 ints each), counters
size_t state_bytes() {
  return (size_t)kTableMax * kCap * sizeof(int) + (size_t)kChunk * sizeof(int) +
         (size_t)kMaxLarge * sizeof(int4) + 2 * (size_t)kChunk * sizeof(int) + table_ints() * sizeof(int);
}

// The state's arrays at their fixed places in its workspace region.
void carve(char *p, EncTable *t, EncShared *sh) {
  sh->rows = reinterpret_cast<int *>(p);
  p += (size_t)kTableMax * kCap * sizeof(int);
  sh->slot_of = reinterpret_cast<int *>(p);
  p += (size_t)kChunk * sizeof(int);
  sh->lmeta = reinterpret_cast<int4 *>(p);
  p += (size_t)kMaxLarge * sizeof(int4);
  sh->pool = reinterpret_cast<int *>(p);
  p += (size_t)kChunk * sizeof(int);
  sh->list = reinterpret_cast<int *>(p);
  p += (size_t)kChunk * sizeof(int);
  t->slot = reinterpret_cast<u64 *>(p);  // 8-byte aligned: every size above is a multiple of 8
  t->counters = reinterpret_cast<int *>(p + (size_t)kTableMax * sizeof(u64));
}

// Large buckets: 0 (the default) blocked adds, 1 the exact chain in row order.
std::atomic<int> g_enc_exact{0};

}  // namespace

size_t encoder_backward_scratch() { return state_bytes(); }

void set_encoder_exact(int exact) { g_enc_exact.store(exact ? 1 : 0); }
int encoder_exact() { return g_enc_exact.load(); }

int launch_encoder_state_init(void *mem) {
  EncTable tb;
  EncShared sh;
  carve(static_cast<char *>(mem), &tb, &sh);
  hipLaunchKernelGGL(k_enc_init, dim3(grid_for(kTableMax, kBlock)), dim3(kBlock), 0, stream(), tb);
  return check_launch("encoder_backward (state init)");
}

int launch_ids_guard(int *ids, int n, int bound, int fill, int code) {
  launch(k_ids_guard, dim3(grid_for((size_t)n, kBlock)), dim3(kBlock), 0, ids, n, bound, fill, code);
  return check_launch("ids_guard");
}

namespace {
struct WordAddr {
  int *ptr = nullptr;
  bool looked_up = false;
};
WordAddr g_ids_word[64];
std::mutex g_ids_word_mu;
}  // namespace

int *ids_error_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    set_error(UGK_EHIP, "id error word: hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_ids_word_mu);
  WordAddr &a = g_ids_word[dev];
  if (!a.looked_up) {  // once per device, with that device current
    void *p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(ids_error));
    if (err != hipSuccess) {
      (void)hipGetLastError();
      set_error(UGK_EHIP, "id error word: hipGetSymbolAddress failed: %s", hipGetErrorString(err));
      return nullptr;
    }
    a.ptr = static_cast<int *>(p);
    a.looked_up = true;
  }
  return a.ptr;
}

int launch_encoder_forward(float *out, const int *inp, const float *wte, const float *wpe, int B,
                           int T, int C) {
  const int BT = B * T;
  if (BT == 0 || C == 0) return 0;
  const dim3 grid(grid_for((size_t)BT, kWavesPerBlock)), block(kBlock);
  if ((C & 3) == 0 && aligned16(out) && aligned16(wte) && aligned16(wpe)) {
    float4 *o4 = reinterpret_cast<float4 *>(out);
    const float4 *te4 = reinterpret_cast<const float4 *>(wte), *pe4 = reinterpret_cast<const float4 *>(wpe);
    const int C4 = C >> 2;
    switch ((C4 + kWave - 1) / kWave) {
#define UGK_ENC_ROW(v) \
  case v:              \
    launch(k_enc_fwd_row<v>, grid, block, 0, o4, inp, te4, pe4, BT, T, C4); \
    break;
      UGK_ENC_ROW(1) UGK_ENC_ROW(2) UGK_ENC_ROW(3) UGK_ENC_ROW(4)
      UGK_ENC_ROW(5) UGK_ENC_ROW(6) UGK_ENC_ROW(7) UGK_ENC_ROW(8)
#undef UGK_ENC_ROW
      default:  // rows beyond 2,048 channels: the lane loop
        launch(k_enc_fwd_vec, grid, block, 0, o4, inp, te4, pe4, BT, T, C4);
    }
  } else {
    launch(k_enc_fwd_scalar, grid, block, 0, out, inp, wte, wpe, BT, T, C);
  }
  return check_launch("encoder_forward");
}

int launch_encoder_backward(float *dwte, float *dwpe, const float *dout, const int *inp, int B,
                            int T, int C) {
  const int BT = B * T;
  if (BT == 0 || C == 0) return 0;
  // the bucket state lives in its own workspace region; new memory is cleared
  // once (by ugk_set_workspace / ugk_reserve_config, or here by the first
  // call), and every call leaves it cleared. Under graph capture the clearing
  // would exist only in the graph, and eager calls before its first replay
  // would find the memory's raw contents: such a first call is refused.
  const bool capturing = stream_capturing();
  bool fresh = false;
  char *mem = static_cast<char *>(workspace(kRegEncoder, state_bytes(), &fresh, capturing));
  if (!mem) return UGK_ENOMEM;
  if (fresh && capturing)
    return set_error(UGK_EINVAL,
                     "encoder_backward: its state is not cleared yet; make one call outside the graph capture, "
                     "or call ugk_reserve_config or ugk_set_workspace first");
  EncTable tb;
  EncShared sh;
  carve(mem, &tb, &sh);
  if (fresh)
    if (int e = launch_encoder_state_init(mem)) return e;
  const bool vec = (C & 3) == 0 && aligned16(dwte) && aligned16(dwpe) && aligned16(dout);
  const int nslices = (C + kWave - 1) / kWave;
  const bool blocked = !encoder_exact();
  for (int c0 = 0; c0 < BT; c0 += kChunk) {
    const int n = BT - c0 < kChunk ? BT - c0 : kChunk;
    int tsize = 64, lg = 6;
    while (tsize < kLoadInv * n && tsize < kTableMax) { tsize <<= 1; lg++; }
    const unsigned mask = (unsigned)tsize - 1u;
    const int shift = 32 - lg;
    const int ins_blocks = (int)grid_for((size_t)n, kBlock);
    int pe_blocks = 0;
    if (c0 == 0) pe_blocks = ((int)grid_for((size_t)T * (vec ? C / 4 : C), kBlock) + 1) / 2;
    if (vec)
      hipLaunchKernelGGL(k_enc_bwd_insert<true>, dim3(ins_blocks + pe_blocks), dim3(kBlock), 0, stream(), tb,
                         sh, inp + c0, n, mask, shift, ins_blocks, dwpe, dout, B, T, C);
    else
      hipLaunchKernelGGL(k_enc_bwd_insert<false>, dim3(ins_blocks + pe_blocks), dim3(kBlock), 0, stream(), tb,
                         sh, inp + c0, n, mask, shift, ins_blocks, dwpe, dout, B, T, C);
    const float *dchunk = dout + (size_t)c0 * C;
    // one workgroup per possible large bucket (at most n / (kCap + 1)), then
    // one wavefront per entry of K1's slot-list regions
    const int nscan = n / (kCap + 1) + 1;
    const dim3 g2((unsigned)(nscan + ins_blocks * (kBlock / kWavesPerBlock)));
    if (vec)
      hipLaunchKernelGGL(k_enc_bwd_add<true>, g2, dim3(kBlock), 0, stream(), tb, sh, dwte, dchunk, C, n, nscan);
    else
      hipLaunchKernelGGL(k_enc_bwd_add<false>, g2, dim3(kBlock), 0, stream(), tb, sh, dwte, dchunk, C, n, nscan);
    const int max_items = (n / (kCap + 1) + 1) * nslices;
    const dim3 g3(max_items < kLargeGrid ? max_items : kLargeGrid);
    if (blocked) {
      // the same work items, each bucket's blocks spread over the workgroup's
      // wavefronts; with no large bucket every workgroup returns at once
      hipLaunchKernelGGL(k_enc_bwd_blocked, g3, dim3(kBlockedWaves * kWave), 0, stream(), tb, sh, dwte, dchunk, C,
                         nslices);
      continue;
    }
    // one round of workgroups (one per CU: each stages 122 KB in LDS) takes
    // the (large bucket, channel slice) work items; with no large bucket
    // every workgroup goes straight to the counter reset
    hipLaunchKernelGGL(k_enc_bwd_large, g3, dim3(kLargeThreads), 0, stream(), tb, sh, dwte, dchunk, C, nslices);
  }
  return check_launch("encoder_backward");
}

}  // namespace ugk
