// cowsdm_product_key_routes: one wave per route row (routes.h holds the
// selection), kRouteWaves rows per workgroup.

#include "routes.h"

namespace cowsdm_impl {

template <int J, int M>
__global__ __launch_bounds__(kWave * kRouteWaves) void product_key_routes_kernel(
    const float* __restrict__ projected, int64_t rows, int root, int sub, int final_k,
    float* __restrict__ weights, int64_t* __restrict__ indices) {
  __shared__ float stage_val[kRouteWaves][kRouteMaxSelected];
  __shared__ int stage_pos[kRouteWaves][kRouteMaxSelected];
  __shared__ float pool_val[kRouteWaves][kWave];
  __shared__ int pool_pos[kRouteWaves][kWave];
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRouteWaves + wave;
  if (row >= rows) return;
  product_key_route_row<J, M>(projected, row, root, sub, final_k, weights, indices,
                              stage_val[wave], stage_pos[wave], pool_val[wave], pool_pos[wave]);
}

template <int J, int M>
void launch_routes(const float* projected, int64_t rows, int root, int sub, int final_k,
                   float* weights, int64_t* indices, hipStream_t stream) {
  const int64_t blocks = (rows + kRouteWaves - 1) / kRouteWaves;
  hipLaunchKernelGGL((product_key_routes_kernel<J, M>), dim3(static_cast<uint32_t>(blocks)),
                     dim3(kWave * kRouteWaves), 0, stream, projected, rows, root, sub,
                     final_k, weights, indices);
}

template <int J>
void launch_routes_pairs(const float* projected, int64_t rows, int root, int sub,
                         int final_k, float* weights, int64_t* indices,
                         hipStream_t stream) {
  if (route_pair_m(sub, final_k) == 1)
    launch_routes<J, 1>(projected, rows, root, sub, final_k, weights, indices, stream);
  else
    launch_routes<J, 2>(projected, rows, root, sub, final_k, weights, indices, stream);
}

}  // namespace cowsdm_impl

using namespace cowsdm_impl;

extern "C" int32_t cowsdm_product_key_routes(const float* projected, int64_t rows,
                                             int64_t slots, int64_t selected,
                                             float* weights, int64_t* indices,
                                             void* stream) {
  if (rows < 0) return fail(-1, "product_key_routes: rows must be >= 0 (got %lld)",
                            static_cast<long long>(rows));
  int r = 0, k = 0, f = 0;
  if (int32_t e = route_geometry(slots, selected, r, k, f)) return e;
  if (rows > (int64_t{1} << 31) * kRouteWaves - kRouteWaves)
    return fail(-2, "product_key_routes: too many rows (%lld)", static_cast<long long>(rows));
  if (rows == 0) return 0;
  if (!projected || !weights || !indices)
    return fail(-1, "product_key_routes: null pointer argument");
  auto s = static_cast<hipStream_t>(stream);
  if (r <= kWave)
    launch_routes_pairs<1>(projected, rows, r, k, f, weights, indices, s);
  else if (r <= 4 * kWave)
    launch_routes_pairs<4>(projected, rows, r, k, f, weights, indices, s);
  else
    launch_routes_pairs<16>(projected, rows, r, k, f, weights, indices, s);
  return launch_status("product_key_routes");
}
