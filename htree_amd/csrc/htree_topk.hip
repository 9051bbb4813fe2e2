// Row-wise Top-K with the block-wide radix select of the wide forward: the
// micro-benchmark counterpart of /root/reference/topk_test/benchmark.py
// (top 512 of 8192 fp32 per row, int32 payloads 0 / 1 / 8 carried along).
// One block of four waves per row; thread i holds elements 32i .. 32i+31 as
// order-preserving unsigned keys in registers.  The k largest are selected
// (ties to the lower index, as a stable descending sort) and written in
// ascending index order with their payloads.
#include "htree_common.h"

namespace htree {

// float -> unsigned key in the float order (negative values flipped); only
// the all-ones NaN pattern maps to 0, the "no element" key
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int NPAY>
__global__ __launch_bounds__(256) void topk_rows_kernel(const float* __restrict__ x, int n, int k,
                                                        const int32_t* __restrict__ pay,
                                                        float* __restrict__ ov,
                                                        int32_t* __restrict__ oi,
                                                        int32_t* __restrict__ op) {
  constexpr int C = kWideC;
  __shared__ int32_t red[32];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t row = blockIdx.x;
  const float* xr = x + row * n;
  uint32_t key[C];
  // 16-byte loads only where the row starts 16-byte aligned (n % 4 == 0 on
  // an aligned base): rows of other lengths are read element by element
  const bool vec_ok = ((uintptr_t)xr & 15u) == 0u;
  if (vec_ok && tid * C + C <= n) {
#pragma unroll
    for (int i = 0; i < C; i += 4) {
      const float4 f = *(const float4*)(xr + tid * C + i);
      key[i] = order_key(f.x);
      key[i + 1] = order_key(f.y);
      key[i + 2] = order_key(f.z);
      key[i + 3] = order_key(f.w);
    }
  } else {
#pragma unroll
    for (int i = 0; i < C; ++i) key[i] = tid * C + i < n ? order_key(xr[tid * C + i]) : 0u;
  }
  BlockSelect<C> sel{red, lane, wv};
  int o;
  const uint32_t bits = sel.select(key, k, 31, o);
  for (uint32_t bb = bits; bb != 0u; bb &= bb - 1u, ++o) {
    const int pos = tid * C + (__builtin_ffs((int)bb) - 1);
    const int64_t w = row * k + o;
    ov[w] = xr[pos];
    oi[w] = pos;
    if (NPAY == 1) op[w] = pay[row * n + pos];
    if (NPAY == 8) {
      const int4* src = (const int4*)(pay + (row * n + pos) * 8);
      int4* dst = (int4*)(op + w * 8);
      dst[0] = src[0];
      dst[1] = src[1];
    }
  }
}

}  // namespace htree

using namespace htree;

extern "C" int htree_topk_rows(const float* values, int64_t rows, int32_t n, int32_t k,
                               const int32_t* payload, int32_t n_payload, float* out_values,
                               int32_t* out_index, int32_t* out_payload, void* stream) {
  if (!values || !out_values || !out_index) return HTREE_ENULL;
  if (rows < 0 || n <= 0 || k <= 0 || k > n || rows > 0x7fffffff) return HTREE_ESHAPE;
  if (n > kWideMidPos) return HTREE_EUNSUPPORTED;
  if (n_payload != 0 && n_payload != 1 && n_payload != 8) return HTREE_EUNSUPPORTED;
  if (n_payload && (!payload || !out_payload)) return HTREE_ENULL;
  if (rows == 0) return HTREE_OK;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)rows);
  if (n_payload == 0)
    hipLaunchKernelGGL(topk_rows_kernel<0>, grid, dim3(256), 0, st, values, n, k, payload, out_values,
                       out_index, out_payload);
  else if (n_payload == 1)
    hipLaunchKernelGGL(topk_rows_kernel<1>, grid, dim3(256), 0, st, values, n, k, payload, out_values,
                       out_index, out_payload);
  else
    hipLaunchKernelGGL(topk_rows_kernel<8>, grid, dim3(256), 0, st, values, n, k, payload, out_values,
                       out_index, out_payload);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HTREE_OK : (int)e;
}
