// The SDM controller's per-token work around the copy-on-write step
// (copy_on_write_sdm/inference.py:459-535): before the step, the input
// LayerNorm, the read / write key, value, forget and input projections and
// the gates; after it, the readings LayerNorm, the sigmoid output gate and
// the output projection.  Routes are selected from the keys by
// cowsdm_product_key_routes (routes.hip), or, for sqrt(N) <= 64, by the
// prepare kernel itself once its tokens' keys are out (one wave per route
// row, routes.h): cowsdm_controller_prepare_routes; with nothing between two
// layers, one layer's finish and the next one's prepare and routes share a
// launch (cowsdm_controller_finish_prepare_routes).
//
// A workgroup takes kCtlTokens tokens.  Each token's normalised input stays
// in LDS, and a wave computes 32 output rows of a projection at a time for
// all of the workgroup's tokens, lanes l and l + 32 the lower and the upper
// half of the inputs of row l: the weights are stored transposed ([width,
// rows]), so a half-wave reads consecutive floats of one input column, and
// each weight is loaded once per workgroup and used for every token.  Each
// half accumulates its products with fused multiply-adds in input order,
// and the row is the lower half's sum plus the upper half's.

#include "common.h"
#include "routes.h"

namespace cowsdm_impl {

constexpr int kCtlTokens = 4;        // tokens per workgroup
constexpr int kCtlThreads = 256;     // finish
// prepare (alone and with its routes): 8 waves, so config 2's 194 rows are
// one pass of 32 rows a wave, and a wave for each of a workgroup's
// 2 x kCtlTokens route rows (one head)
constexpr int kCtlRouteThreads = 2 * kCtlTokens * kWave;
constexpr int kCtlRouteWaves = kCtlRouteThreads / kWave;
constexpr int kCtlMaxWidth = 1024;         // LDS: 3 x 4 tokens x width floats

struct CtlParams {
  cowsdm_controller_t c;
  int64_t batch;
  const float* tokens;        // prepare: [batch, width]
  const float* normalized;    // finish: [batch, width]
  const float* reading;       // finish: [batch * heads, head_width]
  float* out_normalized;      // prepare
  float* read_keys;           // prepare: [batch * heads, key_width]
  float* write_keys;
  float* values;              // prepare: [batch * heads, head_width]
  float* input_gate;          // prepare: [batch * heads]
  float* forget_log_gate;
  float* out;                 // finish: [batch, width]
  const float* residual;      // finish: [batch, width] or null
  float* out_sum;             // finish: residual + out, when residual is set
  int width, heads, head_width, key_width, rows;
};

// The routes the prepare kernel selects itself (sqrt(N) <= 64): every
// token's read and write route rows, one wave per row.
struct CtlRoutes {
  int root, read_sub, read_k, write_sub, write_k;
  float* read_weights;        // [batch * heads, read_k]
  int64_t* read_indices;
  float* write_weights;       // [batch * heads, write_k]
  int64_t* write_indices;
};

__device__ __forceinline__ float wave_sum_f(float v) {
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// LayerNorm of n floats (LDS) by one wave, as torch's layer_norm: the mean,
// the biased variance, then (x - mean) / sqrt(var + eps) * w + b.
__device__ void wave_layer_norm(const float* src, float* dst, int n, const float* w,
                                const float* b, float eps) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  float s = 0.0f;
  for (int i = lane; i < n; i += kWave) s += src[i];
  const float mean = wave_sum_f(s) / static_cast<float>(n);
  float v = 0.0f;
  for (int i = lane; i < n; i += kWave) {
    const float d = src[i] - mean;
    v = __builtin_fmaf(d, d, v);
  }
  const float var = wave_sum_f(v) / static_cast<float>(n);
  const float rstd = 1.0f / sqrtf(var + eps);
  for (int i = lane; i < n; i += kWave) dst[i] = (src[i] - mean) * rstd * w[i] + b[i];
}

// torch.nn.functional.softplus with beta 1 and threshold 20
__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// acc[t] = sum_k x[t][k] * wt[k * rows + j] over the workgroup's tokens,
// row j taken by lanes l and l + 32 of a wave (the inputs below width / 2,
// then the rest); both lanes end with lower + upper.  Every lane of the wave
// calls it (the halves meet through a cross-lane exchange).
__device__ __forceinline__ void project(const float* x, int width, const float* wt, int rows,
                                        int j, float (&acc)[kCtlTokens]) {
  const bool lower = (threadIdx.x & (kWave - 1)) < kWave / 2;
  const int k0 = lower ? 0 : width / 2;
  const int k1 = lower ? width / 2 : width;
#pragma unroll
  for (int t = 0; t < kCtlTokens; ++t) acc[t] = 0.0f;
#pragma unroll 8
  for (int k = k0; k < k1; ++k) {
    const float w = wt[static_cast<int64_t>(k) * rows + j];
#pragma unroll
    for (int t = 0; t < kCtlTokens; ++t) acc[t] = __builtin_fmaf(x[t * width + k], w, acc[t]);
  }
#pragma unroll
  for (int t = 0; t < kCtlTokens; ++t) {
    const float other = __shfl_xor(acc[t], kWave / 2, kWave);
    acc[t] = lower ? acc[t] + other : other + acc[t];
  }
}

// prepare of the workgroup's tokens; with FROM_LDS their inputs are already
// in lds[0 .. kCtlTokens * W) (zeros past the batch), the previous layer's
// finish having put them there
template <int NT, bool FROM_LDS>
__device__ __forceinline__ void controller_prepare_body(const CtlParams& P, float* lds) {
  const int W = P.width, H = P.heads, HW = P.head_width, KW = P.key_width;
  float* const x = lds;                        // [kCtlTokens][W]
  float* const xn = lds + kCtlTokens * W;      // [kCtlTokens][W]
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * kCtlTokens;
  const int T = static_cast<int>(P.batch - b0 < kCtlTokens ? P.batch - b0 : kCtlTokens);
  const int tid = static_cast<int>(threadIdx.x);
  if constexpr (!FROM_LDS) {
    for (int i = tid; i < kCtlTokens * W; i += NT) {
      x[i] = i < T * W ? P.tokens[b0 * W + i] : 0.0f;
    }
  }
  __syncthreads();
  const int wave = tid / kWave;
  for (int t = wave; t < kCtlTokens; t += NT / kWave) {
    if (t < T) {
      wave_layer_norm(x + t * W, xn + t * W, W, P.c.norm_weight, P.c.norm_bias, P.c.norm_eps);
    } else {
      for (int i = tid % kWave; i < W; i += kWave) xn[t * W + i] = 0.0f;
    }
  }
  __syncthreads();
  for (int i = tid; i < T * W; i += NT) P.out_normalized[b0 * W + i] = xn[i];
  // rows: read keys (H x KW), write keys (H x KW), values (W), forget (H), input (H),
  // 32 a wave at a time (lane l and l + 32: row j0 + l)
  for (int j0 = wave * (kWave / 2); j0 < P.rows; j0 += (NT / kWave) * (kWave / 2)) {
    const int j = j0 + (tid & (kWave / 2 - 1));
    const bool on = j < P.rows;
    float acc[kCtlTokens];
    project(xn, W, P.c.proj_weight_t, P.rows, on ? j : P.rows - 1, acc);
    if (!on || (tid & (kWave - 1)) >= kWave / 2) continue;
    const float bias = P.c.proj_bias[j];
    for (int t = 0; t < T; ++t) {
      const int64_t b = b0 + t;
      const float y = acc[t] + bias;
      int r = j;
      if (r < H * KW) {
        const int h = r / KW;
        P.read_keys[(b * H + h) * KW + (r - h * KW)] = y;
      } else if ((r -= H * KW) < H * KW) {
        const int h = r / KW;
        P.write_keys[(b * H + h) * KW + (r - h * KW)] = y;
      } else if ((r -= H * KW) < W) {
        const int h = r / HW;
        P.values[(b * H + h) * HW + (r - h * HW)] = y;
      } else if ((r -= W) < H) {
        P.forget_log_gate[b * H + r] = -expf(P.c.a_log[r]) * softplus(y + P.c.dt_bias[r]);
      } else {
        r -= H;
        P.input_gate[b * H + r] = sigmoid(y);
      }
    }
  }
}

__global__ __launch_bounds__(kCtlRouteThreads) void controller_prepare_kernel(CtlParams P) {
  extern __shared__ float lds[];
  controller_prepare_body<kCtlRouteThreads, false>(P, lds);
}

// The read and write routes of the workgroup's tokens from the keys its
// threads stored (visible to the whole workgroup after a barrier), one wave
// per route row.
struct RouteStage {
  float val[kCtlRouteWaves][kRouteMaxSelected];
  int pos[kCtlRouteWaves][kRouteMaxSelected];
  float pool_val[kCtlRouteWaves][kWave];
  int pool_pos[kCtlRouteWaves][kWave];
};

template <int MR, int MW>
__device__ __forceinline__ void controller_routes_part(const CtlParams& P, const CtlRoutes& R,
                                                       RouteStage& st) {
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * kCtlTokens;
  const int T = static_cast<int>(P.batch - b0 < kCtlTokens ? P.batch - b0 : kCtlTokens);
  const int rows = T * P.heads;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  for (int task = wave; task < 2 * rows; task += kCtlRouteWaves) {
    if (task < rows) {
      product_key_route_row<1, MR>(P.read_keys, b0 * P.heads + task, R.root, R.read_sub,
                                   R.read_k, R.read_weights, R.read_indices, st.val[wave],
                                   st.pos[wave], st.pool_val[wave], st.pool_pos[wave]);
    } else {
      product_key_route_row<1, MW>(P.write_keys, b0 * P.heads + task - rows, R.root,
                                   R.write_sub, R.write_k, R.write_weights, R.write_indices,
                                   st.val[wave], st.pos[wave], st.pool_val[wave],
                                   st.pool_pos[wave]);
    }
  }
}

// prepare, then the routes of the workgroup's tokens
template <int MR, int MW>
__global__ __launch_bounds__(kCtlRouteThreads) void controller_prepare_routes_kernel(
    CtlParams P, CtlRoutes R) {
  extern __shared__ float lds[];
  __shared__ RouteStage stage;
  controller_prepare_body<kCtlRouteThreads, false>(P, lds);
  __syncthreads();
  controller_routes_part<MR, MW>(P, R, stage);
}

// finish of the workgroup's tokens; with TO_LDS the residual sums (the next
// layer's inputs) also go to lds[0 .. kCtlTokens * W), zeros past the batch
// (that region holds the normalised inputs, dead once the gate is applied)
template <int NT, bool TO_LDS>
__device__ __forceinline__ void controller_finish_body(const CtlParams& P, float* lds) {
  constexpr int kWaves = NT / kWave;
  const int W = P.width, HW = P.head_width;
  float* const nrm = lds;                       // normalized inputs
  float* const rd = lds + kCtlTokens * W;       // readings, then gate * normalised readings
  float* const rn = lds + 2 * kCtlTokens * W;   // normalised readings
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * kCtlTokens;
  const int T = static_cast<int>(P.batch - b0 < kCtlTokens ? P.batch - b0 : kCtlTokens);
  const int tid = static_cast<int>(threadIdx.x);
  // a token's readings [heads, head_width] are its `width` contiguous floats
  for (int i = tid; i < kCtlTokens * W; i += NT) {
    nrm[i] = i < T * W ? P.normalized[b0 * W + i] : 0.0f;
    rd[i] = i < T * W ? P.reading[b0 * W + i] : 0.0f;
  }
  __syncthreads();
  const int wave = tid / kWave;
  const int segments = kCtlTokens * P.heads;
  for (int g = wave; g < segments; g += kWaves) {
    wave_layer_norm(rd + g * HW, rn + g * HW, HW, P.c.read_norm_weight, P.c.read_norm_bias,
                    P.c.read_norm_eps);
  }
  __syncthreads();
  const int half_lane = tid & (kWave / 2 - 1);
  const bool writer = (tid & (kWave - 1)) < kWave / 2;
  for (int j0 = wave * (kWave / 2); j0 < W; j0 += kWaves * (kWave / 2)) {
    const int j = j0 + half_lane;
    const bool on = j < W;
    float acc[kCtlTokens];
    project(nrm, W, P.c.gate_weight_t, W, on ? j : W - 1, acc);
    if (!on || !writer) continue;
    const float bias = P.c.gate_bias[j];
#pragma unroll
    for (int t = 0; t < kCtlTokens; ++t) rd[t * W + j] = sigmoid(acc[t] + bias) * rn[t * W + j];
  }
  __syncthreads();
  for (int j0 = wave * (kWave / 2); j0 < W; j0 += kWaves * (kWave / 2)) {
    const int j = j0 + half_lane;
    const bool on = j < W;
    float acc[kCtlTokens];
    project(rd, W, P.c.out_weight_t, W, on ? j : W - 1, acc);
    if (!on || !writer) continue;
    const float bias = P.c.out_bias[j];
    for (int t = 0; t < T; ++t) {
      const int64_t at = (b0 + t) * W + j;
      const float y = acc[t] + bias;
      P.out[at] = y;
      if (P.residual) {
        const float next = P.residual[at] + y;
        P.out_sum[at] = next;
        if constexpr (TO_LDS) nrm[t * W + j] = next;
      }
    }
    if constexpr (TO_LDS) {
      for (int t = T; t < kCtlTokens; ++t) nrm[t * W + j] = 0.0f;
    }
  }
}

__global__ __launch_bounds__(kCtlThreads) void controller_finish_kernel(CtlParams P) {
  extern __shared__ float lds[];
  controller_finish_body<kCtlThreads, false>(P, lds);
}

// one layer's finish with the residual add, then the next layer's prepare
// and routes on the same tokens, whose inputs the finish left in LDS
template <int MR, int MW>
__global__ __launch_bounds__(kCtlRouteThreads) void controller_finish_prepare_routes_kernel(
    CtlParams F, CtlParams P, CtlRoutes R) {
  extern __shared__ float lds[];
  __shared__ RouteStage stage;
  controller_finish_body<kCtlRouteThreads, true>(F, lds);
  __syncthreads();
  controller_prepare_body<kCtlRouteThreads, true>(P, lds);
  __syncthreads();
  controller_routes_part<MR, MW>(P, R, stage);
}

namespace {

int32_t check_controller(const cowsdm_controller_t* c, int64_t batch, CtlParams& P) {
  if (!c) return fail(COWSDM_EARG, "controller: null controller");
  if (batch < 0) return fail(COWSDM_EARG, "controller: negative batch");
  if (c->width <= 0 || c->heads <= 0 || c->width % c->heads != 0) {
    return fail(COWSDM_EARG, "width must be divisible by memory_heads");
  }
  if (c->width > kCtlMaxWidth) {
    return fail(COWSDM_ELIMIT, "controller: width <= %d on the HIP path (got %lld)",
                kCtlMaxWidth, static_cast<long long>(c->width));
  }
  int64_t root = 0;
  while ((root + 1) * (root + 1) <= c->slots) ++root;
  if (c->slots < 1 || root * root != c->slots) {
    return fail(COWSDM_EARG, "faithful SDM slots must be a perfect square");
  }
  P.c = *c;
  P.batch = batch;
  P.width = static_cast<int>(c->width);
  P.heads = static_cast<int>(c->heads);
  P.head_width = static_cast<int>(c->width / c->heads);
  P.key_width = static_cast<int>(2 * root);
  const int64_t rows = 2 * c->heads * 2 * root + c->width + 2 * c->heads;
  if (rows > (int64_t{1} << 24)) return fail(COWSDM_ELIMIT, "controller: too many projection rows");
  P.rows = static_cast<int>(rows);
  return 0;
}

}  // namespace
}  // namespace cowsdm_impl

using namespace cowsdm_impl;

extern "C" int64_t cowsdm_controller_rows(int64_t width, int64_t heads, int64_t slots) {
  int64_t root = 0;
  while ((root + 1) * (root + 1) <= slots) ++root;
  if (width <= 0 || heads <= 0 || slots < 1 || root * root != slots) return -1;
  return 2 * heads * 2 * root + width + 2 * heads;
}

namespace {

int32_t prepare_params(const cowsdm_controller_t* c, const float* tokens, int64_t batch,
                       float* normalized, float* read_keys, float* write_keys, float* values,
                       float* input_gate, float* forget_log_gate, CtlParams& P) {
  if (int32_t e = check_controller(c, batch, P)) return e;
  if (batch == 0) return 0;
  if (!tokens || !normalized || !read_keys || !write_keys || !values || !input_gate ||
      !forget_log_gate || !c->norm_weight || !c->norm_bias || !c->proj_weight_t ||
      !c->proj_bias || !c->a_log || !c->dt_bias) {
    return fail(COWSDM_EARG, "controller prepare: null pointer argument");
  }
  P.tokens = tokens;
  P.out_normalized = normalized;
  P.read_keys = read_keys;
  P.write_keys = write_keys;
  P.values = values;
  P.input_gate = input_gate;
  P.forget_log_gate = forget_log_gate;
  if ((batch + kCtlTokens - 1) / kCtlTokens > (int64_t{1} << 31) - 1) {
    return fail(COWSDM_ELIMIT, "controller: batch too large");
  }
  return 0;
}

template <int MR, int MW>
void launch_prepare_routes(const CtlParams& P, const CtlRoutes& R, hipStream_t s) {
  const int64_t groups = (P.batch + kCtlTokens - 1) / kCtlTokens;
  const size_t lds = sizeof(float) * 2 * kCtlTokens * P.width;
  hipLaunchKernelGGL((controller_prepare_routes_kernel<MR, MW>),
                     dim3(static_cast<unsigned>(groups)), dim3(kCtlRouteThreads), lds, s, P, R);
}

template <int MR, int MW>
void launch_finish_prepare_routes(const CtlParams& F, const CtlParams& P, const CtlRoutes& R,
                                  hipStream_t s) {
  const int64_t groups = (P.batch + kCtlTokens - 1) / kCtlTokens;
  const size_t lds = sizeof(float) * 3 * kCtlTokens * P.width;
  hipLaunchKernelGGL((controller_finish_prepare_routes_kernel<MR, MW>),
                     dim3(static_cast<unsigned>(groups)), dim3(kCtlRouteThreads), lds, s, F, P,
                     R);
}

// The route geometry of `reads` and `writes` selections over c's slots and
// the four output pointers (checked once batch > 0).
int32_t route_params(const cowsdm_controller_t* c, int64_t batch, int64_t reads, int64_t writes,
                     float* read_weights, int64_t* read_indices, float* write_weights,
                     int64_t* write_indices, CtlRoutes& R) {
  if (int32_t e = route_geometry(c->slots, reads, R.root, R.read_sub, R.read_k)) return e;
  if (int32_t e = route_geometry(c->slots, writes, R.root, R.write_sub, R.write_k)) return e;
  if (batch == 0) return 0;
  if (!read_weights || !read_indices || !write_weights || !write_indices) {
    return fail(COWSDM_EARG, "controller prepare: null route pointer");
  }
  R.read_weights = read_weights;
  R.read_indices = read_indices;
  R.write_weights = write_weights;
  R.write_indices = write_indices;
  return 0;
}

int32_t finish_params(const cowsdm_controller_t* c, const float* normalized,
                      const float* reading, int64_t batch, float* out, const float* residual,
                      float* out_sum, CtlParams& P) {
  if (residual && !out_sum) return fail(COWSDM_EARG, "controller finish: null residual sum");
  P.residual = residual;
  P.out_sum = out_sum;
  if (int32_t e = check_controller(c, batch, P)) return e;
  if (batch == 0) return 0;
  if (!normalized || !reading || !out || !c->gate_weight_t || !c->gate_bias ||
      !c->out_weight_t || !c->out_bias || !c->read_norm_weight || !c->read_norm_bias) {
    return fail(COWSDM_EARG, "controller finish: null pointer argument");
  }
  P.normalized = normalized;
  P.reading = reading;
  P.out = out;
  if ((batch + kCtlTokens - 1) / kCtlTokens > (int64_t{1} << 31) - 1) {
    return fail(COWSDM_ELIMIT, "controller: batch too large");
  }
  return 0;
}

}  // namespace

extern "C" int32_t cowsdm_controller_prepare(const cowsdm_controller_t* c, const float* tokens,
                                             int64_t batch, float* normalized, float* read_keys,
                                             float* write_keys, float* values, float* input_gate,
                                             float* forget_log_gate, void* stream) {
  CtlParams P{};
  if (int32_t e = prepare_params(c, tokens, batch, normalized, read_keys, write_keys, values,
                                 input_gate, forget_log_gate, P)) {
    return e;
  }
  if (batch == 0) return 0;
  const int64_t groups = (batch + kCtlTokens - 1) / kCtlTokens;
  const size_t lds = sizeof(float) * 2 * kCtlTokens * P.width;
  hipLaunchKernelGGL(controller_prepare_kernel, dim3(static_cast<unsigned>(groups)),
                     dim3(kCtlRouteThreads), lds, static_cast<hipStream_t>(stream), P);
  return launch_status("controller prepare");
}

extern "C" int32_t cowsdm_product_key_routes(const float* projected, int64_t rows,
                                             int64_t slots, int64_t selected,
                                             float* weights, int64_t* indices, void* stream);

extern "C" int32_t cowsdm_controller_prepare_routes(
    const cowsdm_controller_t* c, const float* tokens, int64_t batch, float* normalized,
    float* read_keys, float* write_keys, float* values, float* input_gate,
    float* forget_log_gate, int64_t reads, int64_t writes, float* read_weights,
    int64_t* read_indices, float* write_weights, int64_t* write_indices, void* stream) {
  CtlParams P{};
  if (int32_t e = prepare_params(c, tokens, batch, normalized, read_keys, write_keys, values,
                                 input_gate, forget_log_gate, P)) {
    return e;
  }
  CtlRoutes R{};
  if (int32_t e = route_params(c, batch, reads, writes, read_weights, read_indices,
                               write_weights, write_indices, R)) {
    return e;
  }
  if (batch == 0) return 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (R.root > kWave) {
    // a shortlist of more than one entry per lane: the separate launches
    if (int32_t e = cowsdm_controller_prepare(c, tokens, batch, normalized, read_keys,
                                              write_keys, values, input_gate, forget_log_gate,
                                              stream)) {
      return e;
    }
    const int64_t rows = batch * c->heads;
    if (int32_t e = cowsdm_product_key_routes(read_keys, rows, c->slots, reads, read_weights,
                                              read_indices, stream)) {
      return e;
    }
    return cowsdm_product_key_routes(write_keys, rows, c->slots, writes, write_weights,
                                     write_indices, stream);
  }
  const int mr = route_pair_m(R.read_sub, R.read_k), mw = route_pair_m(R.write_sub, R.write_k);
  if (mr == 1 && mw == 1) launch_prepare_routes<1, 1>(P, R, s);
  else if (mr == 1) launch_prepare_routes<1, 2>(P, R, s);
  else if (mw == 1) launch_prepare_routes<2, 1>(P, R, s);
  else launch_prepare_routes<2, 2>(P, R, s);
  return launch_status("controller prepare routes");
}

extern "C" int32_t cowsdm_controller_finish_residual(const cowsdm_controller_t* c,
                                                     const float* normalized,
                                                     const float* reading, int64_t batch,
                                                     float* out, const float* residual,
                                                     float* out_sum, void* stream) {
  CtlParams P{};
  if (int32_t e = finish_params(c, normalized, reading, batch, out, residual, out_sum, P)) {
    return e;
  }
  if (batch == 0) return 0;
  const int64_t groups = (batch + kCtlTokens - 1) / kCtlTokens;
  const size_t lds = sizeof(float) * 3 * kCtlTokens * P.width;
  hipLaunchKernelGGL(controller_finish_kernel, dim3(static_cast<unsigned>(groups)),
                     dim3(kCtlThreads), lds, static_cast<hipStream_t>(stream), P);
  return launch_status("controller finish");
}

extern "C" int32_t cowsdm_controller_finish(const cowsdm_controller_t* c,
                                            const float* normalized, const float* reading,
                                            int64_t batch, float* out, void* stream) {
  return cowsdm_controller_finish_residual(c, normalized, reading, batch, out, nullptr, nullptr,
                                           stream);
}

extern "C" int32_t cowsdm_controller_finish_prepare_routes(
    const cowsdm_controller_t* c, const float* normalized, const float* reading, int64_t batch,
    float* out, const float* residual, float* out_sum, const cowsdm_controller_t* next,
    float* next_normalized, float* read_keys, float* write_keys, float* values,
    float* input_gate, float* forget_log_gate, int64_t reads, int64_t writes,
    float* read_weights, int64_t* read_indices, float* write_weights, int64_t* write_indices,
    void* stream) {
  if (!residual || !out_sum) {
    return fail(COWSDM_EARG, "controller finish and prepare: null residual or sum");
  }
  CtlParams F{};
  if (int32_t e = finish_params(c, normalized, reading, batch, out, residual, out_sum, F)) {
    return e;
  }
  CtlParams P{};
  if (int32_t e = prepare_params(next, out_sum, batch, next_normalized, read_keys, write_keys,
                                 values, input_gate, forget_log_gate, P)) {
    return e;
  }
  if (next->width != c->width) {
    return fail(COWSDM_EARG, "controller finish and prepare: the layers' widths differ");
  }
  CtlRoutes R{};
  if (int32_t e = route_params(next, batch, reads, writes, read_weights, read_indices,
                               write_weights, write_indices, R)) {
    return e;
  }
  if (batch == 0) return 0;
  if (R.root > kWave) {
    // the next layer's routes take their own launches: finish, then prepare
    if (int32_t e = cowsdm_controller_finish_residual(c, normalized, reading, batch, out,
                                                      residual, out_sum, stream)) {
      return e;
    }
    return cowsdm_controller_prepare_routes(next, out_sum, batch, next_normalized, read_keys,
                                            write_keys, values, input_gate, forget_log_gate,
                                            reads, writes, read_weights, read_indices,
                                            write_weights, write_indices, stream);
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int mr = route_pair_m(R.read_sub, R.read_k), mw = route_pair_m(R.write_sub, R.write_k);
  if (mr == 1 && mw == 1) launch_finish_prepare_routes<1, 1>(F, P, R, s);
  else if (mr == 1) launch_finish_prepare_routes<1, 2>(F, P, R, s);
  else if (mw == 1) launch_finish_prepare_routes<2, 1>(F, P, R, s);
  else launch_finish_prepare_routes<2, 2>(F, P, R, s);
  return launch_status("controller finish and prepare");
}
