// ugk_map.h - the streaming map shared by the elementwise kernels.
//
// An operator maps kLoads input floats of element i to kStores output floats.
// Each thread owns Op::kUnroll float4 (16-byte) slots strided by the
// workgroup size, so every load and store instruction of a wavefront covers
// one contiguous 1 KiB span, all of a thread's loads are issued before its
// first arithmetic instruction, and every access is non-temporal (each byte
// is touched once). Launch-shape sweeps on MI355X over inputs too large for
// the last-level cache (unroll 1-8, 256-1024 threads, flat or grid-stride,
// with and without nt) put nt loads and stores with unroll 1-2 and 256-512
// threads on top; each operator picks its own (the spread is a few percent).
// Arrays whose pointers are not all 16-byte aligned, and the n % 4 tail, take
// a scalar grid-stride path with identical arithmetic.
//
// An operator is a struct with
//   kLoads, kStores          stream counts;
//   kTable                   stage expf's 2^(i/32) table in LDS (tab != null);
//   kUnroll, kThreads        float4 slots per thread, threads per workgroup;
//   kLdsReserve              bytes of LDS each workgroup reserves without
//                            using them (0: none), which caps the workgroups
//                            resident on a CU (160 KiB of LDS each);
//   Params                   per-launch scalars passed by value;
//   apply(ld, st, tab, i, p) the per-element body; i is the element index;
//   kPre, Pre, pre(i, p)     optionally (kPre true), the part of the body that
//                            reads no stream (a Philox draw): the kernel
//                            computes it for all of a thread's elements while
//                            their loads are in flight and hands it to
//                            apply_pre(ld, st, tab, i, p, pre) instead.
#pragma once

#include "ugk_internal.h"
#include "ugk_libm_dev.h"

namespace ugk {
namespace {

struct MapOp {
  struct Params {};
  static constexpr bool kTable = false;
  static constexpr int kUnroll = 2;
  static constexpr int kThreads = kBlock;
  static constexpr unsigned kLdsReserve = 0;
  static constexpr bool kPre = false;
  struct Pre {};
};

template <class Op>
struct Streams {
  const float *ld[Op::kLoads];
  float *st[Op::kStores];
  typename Op::Params p;
};

template <class Op>
__global__ __launch_bounds__(Op::kThreads) void k_map_vec4(Streams<Op> s, size_t n4) {
  __shared__ uint64_t tab[Op::kTable ? 32 : 1];
  if (Op::kTable) {
    ugk_exp2_stage(tab);
    __syncthreads();
  }
  constexpr int kU = Op::kUnroll, kT = Op::kThreads;
  const size_t base = (size_t)blockIdx.x * (kT * kU) + threadIdx.x;
  float4 v[kU][Op::kLoads];
#pragma unroll
  for (int u = 0; u < kU; u++) {
    const size_t i = base + (size_t)u * kT;
    if (i < n4) {
#pragma unroll
      for (int l = 0; l < Op::kLoads; l++) v[u][l] = ld_nt(reinterpret_cast<const float4 *>(s.ld[l]) + i);
    }
  }
  typename Op::Pre pre[kU][4];
  if constexpr (Op::kPre) {
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const size_t i = base + (size_t)u * kT;
      if (i < n4) {
#pragma unroll
        for (int e = 0; e < 4; e++) pre[u][e] = Op::pre(4 * i + e, s.p);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kU; u++) {
    const size_t i = base + (size_t)u * kT;
    if (i < n4) {
      float in[4][Op::kLoads], out[4][Op::kStores];
#pragma unroll
      for (int l = 0; l < Op::kLoads; l++) {
        in[0][l] = v[u][l].x; in[1][l] = v[u][l].y;
        in[2][l] = v[u][l].z; in[3][l] = v[u][l].w;
      }
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if constexpr (Op::kPre)
          Op::apply_pre(in[e], out[e], tab, 4 * i + e, s.p, pre[u][e]);
        else
          Op::apply(in[e], out[e], tab, 4 * i + e, s.p);
      }
#pragma unroll
      for (int o = 0; o < Op::kStores; o++)
        st_nt(reinterpret_cast<float4 *>(s.st[o]) + i, make_float4(out[0][o], out[1][o], out[2][o], out[3][o]));
    }
  }
}

template <class Op>
__global__ __launch_bounds__(kBlock) void k_map_scalar(Streams<Op> s, size_t begin, size_t n) {
  __shared__ uint64_t tab[Op::kTable ? 32 : 1];
  if (Op::kTable) {
    ugk_exp2_stage(tab);
    __syncthreads();
  }
  for (size_t i = begin + (size_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (size_t)gridDim.x * kBlock) {
    float in[Op::kLoads], out[Op::kStores];
#pragma unroll
    for (int l = 0; l < Op::kLoads; l++) in[l] = s.ld[l][i];
    if constexpr (Op::kPre)
      Op::apply_pre(in, out, tab, i, s.p, Op::pre(i, s.p));
    else
      Op::apply(in, out, tab, i, s.p);
#pragma unroll
    for (int o = 0; o < Op::kStores; o++) s.st[o][i] = out[o];
  }
}

template <class Op>
int run_map(const Streams<Op> &s, size_t n, const char *name) {
  if (n == 0) return 0;
  bool vec = true;
  for (int l = 0; l < Op::kLoads; l++) vec = vec && aligned16(s.ld[l]);
  for (int o = 0; o < Op::kStores; o++) vec = vec && aligned16(s.st[o]);
  size_t done = 0;
  if (vec && n >= 4) {
    const size_t n4 = n / 4;
    launch(k_map_vec4<Op>, dim3(grid_for(n4, (size_t)Op::kThreads * Op::kUnroll)),
                       dim3(Op::kThreads), Op::kLdsReserve, s, n4);
    done = n4 * 4;
  }
  if (done < n) {
    const size_t rest = n - done;
    unsigned g = grid_for(rest, kBlock);
    if (g > 65536u) g = 65536u;
    launch(k_map_scalar<Op>, dim3(g), dim3(kBlock), 0, s, done, n);
  }
  return check_launch(name);
}

}  // namespace
}  // namespace ugk
