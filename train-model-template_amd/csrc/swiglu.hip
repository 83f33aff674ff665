// SwiGLU elementwise kernels of the unfused MLP path (/root/reference/scripts/shared_prefix.py:172-197: _SWIGLU, the
// compiled silu(g) * u between the gate/up and down group_linear calls, and its autograd backward).
//   forward   h  = bf16(silu(g) * u)
//   backward  du = bf16(dh * silu(g)),  dg = bf16(dh * u * sig * (g * (1 - sig) + 1)),  sig = sigmoid(g)
// with the sigmoid and the operation order of the fused MLP kernels (csrc/mlp_fused.hip), so that the unfused path's
// h equals the fused path's h; one rounding per output as in a compiled (fused) elementwise kernel.  Eight bf16
// values per thread (16 backward), 16-byte loads and stores: HBM-bound (6 bytes moved per element forward, 10
// backward).
#include <hip/hip_runtime.h>

#include "abi_common.h"
#include "mx_device.h"

using namespace mxk;

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool kNt>
__device__ __forceinline__ void load8(const uint16_t* p, uint32_t* w) {
  u32x4 a;
  if constexpr (kNt) a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else a = *reinterpret_cast<const u32x4*>(p);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
}
template <bool kNt>
__device__ __forceinline__ void store8(uint16_t* p, const uint32_t* w) {
  const u32x4 a = {w[0], w[1], w[2], w[3]};
  if constexpr (kNt) __builtin_nontemporal_store(a, reinterpret_cast<u32x4*>(p));
  else *reinterpret_cast<u32x4*>(p) = a;
}

// Forward: 8 values per thread, h written with streaming (non-temporal) stores.  Backward: 16 values per thread
// (two 16-byte chunks 256 chunks apart, all five loads issued first), g, u, dh read with streaming loads.  Timed
// alone at configuration 3 ([10752, 6144], one box, twice each, bit-identical outputs): forward 68.6 -> 56.3 us
// (5.78 -> 7.03 TB/s), backward 116.1 -> 97.0 us (5.69 -> 6.81 TB/s); 16 values per thread with plain loads, 32
// values, and both hints on both kernels each measured slower than these.
constexpr int kBwdChunks = 2;

__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                         int64_t n8, uint16_t* __restrict__ h) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  uint32_t gw[4], uw[4], hw[4];
  load8<false>(g + i * 8, gw);
  load8<false>(u + i * 8, uw);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float g0 = bf16_lo(gw[k]), g1 = bf16_hi(gw[k]);
    float h0 = (g0 * fast_sigmoid(g0)) * bf16_lo(uw[k]), h1 = (g1 * fast_sigmoid(g1)) * bf16_hi(uw[k]);
    hw[k] = rnd2(h0, h1);
  }
  store8<true>(h + i * 8, hw);
}

__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                         const uint16_t* __restrict__ dh, int64_t n8,
                                                         uint16_t* __restrict__ dg, uint16_t* __restrict__ du) {
  uint32_t gw[kBwdChunks][4], uw[kBwdChunks][4], dw[kBwdChunks][4];
#pragma unroll
  for (int j = 0; j < kBwdChunks; ++j) {
    const int64_t i = ((int64_t)blockIdx.x * kBwdChunks + j) * 256 + threadIdx.x;
    if (i < n8) {
      load8<true>(g + i * 8, gw[j]);
      load8<true>(u + i * 8, uw[j]);
      load8<true>(dh + i * 8, dw[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < kBwdChunks; ++j) {
    const int64_t i = ((int64_t)blockIdx.x * kBwdChunks + j) * 256 + threadIdx.x;
    if (i >= n8) break;
    uint32_t dgw[4], duw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float g0 = bf16_lo(gw[j][k]), g1 = bf16_hi(gw[j][k]);
      const float u0 = bf16_lo(uw[j][k]), u1 = bf16_hi(uw[j][k]);
      const float d0 = bf16_lo(dw[j][k]), d1 = bf16_hi(dw[j][k]);
      const float sg0 = fast_sigmoid(g0), sg1 = fast_sigmoid(g1);
      const float sl0 = g0 * sg0, sl1 = g1 * sg1;
      float du0 = d0 * sl0, du1 = d1 * sl1;
      duw[k] = rnd2(du0, du1);
      float dg0 = ((d0 * u0) * sg0) * (g0 * (1.0f - sg0) + 1.0f);
      float dg1 = ((d1 * u1) * sg1) * (g1 * (1.0f - sg1) + 1.0f);
      dgw[k] = rnd2(dg0, dg1);
    }
    store8<false>(dg + i * 8, dgw);
    store8<false>(du + i * 8, duw);
  }
}

}  // namespace

extern "C" int mxfp8_swiglu(const void* g, const void* u, int64_t n, void* h, void* stream) {
  MX_CHECK_ARG(g && u && h, "mxfp8_swiglu: null pointer");
  MX_CHECK_ARG(n > 0 && n % 8 == 0, "mxfp8_swiglu: need n %% 8 == 0");
  MX_CHECK_ARG(mx_aligned(g, 16) && mx_aligned(u, 16) && mx_aligned(h, 16), "mxfp8_swiglu: misaligned buffer");
  const int64_t n8 = n / 8;
  swiglu_fwd_kernel<<<(unsigned)((n8 + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)g, (const uint16_t*)u, n8, (uint16_t*)h);
  MX_CHECK_LAUNCH("mxfp8_swiglu");
  return MXFP8_OK;
}

extern "C" int mxfp8_swiglu_bwd(const void* g, const void* u, const void* dh, int64_t n, void* dg, void* du,
                                void* stream) {
  MX_CHECK_ARG(g && u && dh && dg && du, "mxfp8_swiglu_bwd: null pointer");
  MX_CHECK_ARG(n > 0 && n % 8 == 0, "mxfp8_swiglu_bwd: need n %% 8 == 0");
  MX_CHECK_ARG(mx_aligned(g, 16) && mx_aligned(u, 16) && mx_aligned(dh, 16) && mx_aligned(dg, 16) &&
                   mx_aligned(du, 16),
               "mxfp8_swiglu_bwd: misaligned buffer");
  const int64_t n8 = n / 8;
  swiglu_bwd_kernel<<<(unsigned)((n8 + 256 * kBwdChunks - 1) / (256 * kBwdChunks)), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)g, (const uint16_t*)u, (const uint16_t*)dh, n8, (uint16_t*)dg, (uint16_t*)du);
  MX_CHECK_LAUNCH("mxfp8_swiglu_bwd");
  return MXFP8_OK;
}
