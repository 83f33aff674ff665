// A partial sum that a GEMM's epilogue reads, computed by the first workgroups of the same launch
// (mxfp8_gemm_nt_sum): P [rows, r] = bf16(scale · Σ_p part[p, rows, r]), p ascending in fp32, the arithmetic and
// order of mxfp8_sum_parts.  The MLP forward's xS_down (the 96 per-tile partials of the gate|up epilogue) is the
// rank-16 operand of the down GEMM's epilogue (/root/reference/scripts/fused_mlp.py:214, :284).
//
// Ordering.  The summing workgroups are numbered before every tile, so the dispatcher starts them first, and they
// wait for nothing.  Each publishes the launch's id in its flag when its rows are stored (workgroup barrier, then
// a release store at agent scope, as the split-K pieces publish).  A tile reads P only in its epilogue: one
// thread polls the flags of the blocks that cover the tile's rows, then every thread loads its rows of P.  Both
// are relaxed atomic loads at agent scope, which read the coherent level past the XCD's L2 (sc1) and are issued
// after the flag value they depend on has returned.  An acquire would be the same loads plus an invalidation of
// the XCD's whole L2 after each one (buffer_inv sc1): measured, that took the GEMM's cached operands with it and
// made the launch 28 us slower than the two launches it replaces.  The poll is bounded: past `wait_limit` polls
// the tile sums its own rows
// from `part` in the same order, which gives the same bits, so every wave finishes whatever the scheduling.
// The flags hold the id of the last launch that wrote them; ids are unique per process, so flags need no
// clearing between launches.
#pragma once

#include "abi_common.h"
#include "mx_device.h"

namespace mxk {

typedef unsigned long long v2u64 __attribute__((ext_vector_type(2)));

struct PreSum {
  const float* part;          // [n_parts, rows, r] fp32
  uint16_t* out;              // P [rows, r] bf16, row stride r
  unsigned long long* flags;  // one per summing workgroup
  unsigned long long id;      // this launch's id
  int64_t count4;             // rows * r / 4: float4 elements of one partial
  int n_parts;
  int blocks;                 // summing workgroups (a multiple of 8; 0: no sum in this launch)
  int rows_per_block;         // 1024 / r: the rows one summing workgroup covers
  int wait_limit;             // polls before a tile sums its own rows
  float scale;
};

// Summing workgroup b (256 threads, one float4 of P each): eight partials in flight, added in ascending order.
__device__ __forceinline__ void presum_block(const PreSum& a, int b) {
  const int64_t i = (int64_t)b * 256 + threadIdx.x;
  if (i < a.count4) {
    const float4* src = reinterpret_cast<const float4*>(a.part) + i;
    float4 v = src[0];
    int p = 1;
    for (; p + 7 < a.n_parts; p += 8) {
      float4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = src[(int64_t)(p + u) * a.count4];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        v.x += x[u].x; v.y += x[u].y; v.z += x[u].z; v.w += x[u].w;
      }
    }
    for (; p < a.n_parts; ++p) {
      const float4 x = src[(int64_t)p * a.count4];
      v.x += x.x; v.y += x.y; v.z += x.z; v.w += x.w;
    }
    const uint32_t lo = f32_to_bf16_bits(v.x * a.scale) | (f32_to_bf16_bits(v.y * a.scale) << 16);
    const uint32_t hi = f32_to_bf16_bits(v.z * a.scale) | (f32_to_bf16_bits(v.w * a.scale) << 16);
    reinterpret_cast<uint2*>(a.out)[i] = make_uint2(lo, hi);
  }
  __syncthreads();  // every wave's stores have completed (workgroup release)
  if (threadIdx.x == 0) __hip_atomic_store(a.flags + b, a.id, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// A tile about to read rows [r0, r1) of P (r1 > r0): true once the blocks covering them have published this
// launch's id, false when the poll limit ran out first (the tile then sums its rows itself, presum_row8).
// Every thread of the workgroup calls it; `slot` is a workgroup-shared int.  wait_limit 0: no poll at all, every
// tile sums its own rows (how the tests reach that path).
__device__ __forceinline__ bool presum_wait(const PreSum& a, int r0, int r1, int* slot) {
  if (a.wait_limit <= 0) return false;
  if (threadIdx.x == 0) {
    int ok = 1;
    for (int b = r0 / a.rows_per_block; ok && b <= (r1 - 1) / a.rows_per_block; ++b) {
      int n = 0;
      while (__hip_atomic_load(a.flags + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != a.id) {
        if (++n > a.wait_limit) {
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    *slot = ok;
  }
  __syncthreads();
  return *slot != 0;
}

// Eight values of P published in this launch (16-byte aligned), read at the coherent level (see above).
__device__ __forceinline__ v8bf presum_load8(const uint16_t* p) {
  const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
  const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const v2u64 v = {lo, hi};
  return __builtin_bit_cast(v8bf, v);
}

// Eight values of P, row `row`, columns c0 .. c0 + 7 (c0 % 8 == 0), summed from the partials in the summing
// workgroups' order: the same bits as the stored P.
__device__ __forceinline__ v8bf presum_row8(const PreSum& a, int64_t row, int c0, int r) {
  const float4* src = reinterpret_cast<const float4*>(a.part + row * r + c0);
  float4 u = src[0], w = src[1];
  for (int p = 1; p < a.n_parts; ++p) {
    const float4 x = src[(int64_t)p * a.count4], y = src[(int64_t)p * a.count4 + 1];
    u.x += x.x; u.y += x.y; u.z += x.z; u.w += x.w;
    w.x += y.x; w.y += y.y; w.z += y.z; w.w += y.w;
  }
  v8s16 o;
  const float f[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = (short)f32_to_bf16_bits(f[k] * a.scale);
  return __builtin_bit_cast(v8bf, o);
}

}  // namespace mxk
