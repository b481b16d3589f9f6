// The elementwise kernels of the attention layer around the operator
// (src/mimir/model/layers.py:169-239): rotary position embedding on the q / k
// splits of the fused gqkv projection and its gradient, and the sigmoid output
// gate's forward for float32 (the bf16 forward applies the gate in the
// attention kernel's store).
//
// RoPE, rotate-half convention (layers.py:24-40): per row and column pair
// (d, d + D/2), x1 = x[d], x2 = x[d + D/2],
//   y1 = x1 * cos[d]       - x2 * sin[d]
//   y2 = x2 * cos[d + D/2] + x1 * sin[d + D/2]
// with fp32 products rounded separately and one rounding of the sum to the
// element type, as (x * cos) + (rotate_half(x) * sin) evaluates it (the bf16 x
// promotes to fp32 against the fp32 cos / sin; .to(x.dtype) at the end).  The
// gradient, g = dL/dy:
//   dx1 = round(round(g1 * cos[d]) + round(g2 * sin[d + D/2]))
//   dx2 = round(round(g2 * cos[d + D/2]) - round(g1 * sin[d]))
// which is how autograd forms it for the reference expression: the backward of
// each promoted product is cast back to x's dtype, and the contributions of
// x * cos and of the two rotate_half slices are summed in that dtype.
// Contraction of the products into FMAs is switched off so that the fp32
// roundings are exactly those of the separate multiplies and adds.
#include "prefixlm_common.h"

namespace mimir {
namespace {

struct RopeArgs {
  const void* x;
  void* y;
  const float* cos;
  const float* sin;
  int64_t x_st, x_sh, y_st, y_sh, cs_st;
  int T, H, D, inverse;
};

template <typename E, int V>  // V elements per 16-byte vector
using Vec = E __attribute__((ext_vector_type(V)));

template <typename E, int V>
__global__ __launch_bounds__(256) void rope_kernel(const RopeArgs a) {
#pragma clang fp contract(off)
  using VE = Vec<E, V>;
  const int half = a.D / 2;
  const int chunks = half / V;  // 16-byte chunks per half row
  const int64_t total = (int64_t)a.T * a.H * chunks;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int c = (int)(i % chunks);
    const int64_t row = i / chunks;
    const int h = (int)(row % a.H);
    const int t = (int)(row / a.H);
    const E* xr = (const E*)a.x + (int64_t)t * a.x_st + (int64_t)h * a.x_sh;
    E* yr = (E*)a.y + (int64_t)t * a.y_st + (int64_t)h * a.y_sh;
    const int d1 = c * V, d2 = d1 + half;
    const VE x1 = *(const VE*)(xr + d1);
    const VE x2 = *(const VE*)(xr + d2);
    const float* cr = a.cos + (int64_t)t * a.cs_st;
    const float* sr = a.sin + (int64_t)t * a.cs_st;
    float c1[V], c2[V], s1[V], s2[V];
#pragma unroll
    for (int j = 0; j < V; j += 4) {
      const f32x4 cc1 = *(const f32x4*)(cr + d1 + j), cc2 = *(const f32x4*)(cr + d2 + j);
      const f32x4 ss1 = *(const f32x4*)(sr + d1 + j), ss2 = *(const f32x4*)(sr + d2 + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c1[j + e] = cc1[e];
        c2[j + e] = cc2[e];
        s1[j + e] = ss1[e];
        s2[j + e] = ss2[e];
      }
    }
    VE y1, y2;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float u = (float)x1[e], w = (float)x2[e];
      float r1, r2;
      if (!a.inverse) {
        r1 = u * c1[e] - w * s1[e];
        r2 = w * c2[e] + u * s2[e];
      } else {
        r1 = round_to(u * c1[e], E()) + round_to(w * s2[e], E());
        r2 = round_to(w * c2[e], E()) - round_to(u * s1[e], E());
      }
      y1[e] = (E)r1;
      y2[e] = (E)r2;
    }
    *(VE*)(yr + d1) = y1;
    *(VE*)(yr + d2) = y2;
  }
}

// gated_out = round(round(sigmoid(gate)) * out) for every row (float32 path).
struct GateArgs {
  const float* o;
  const float* g;
  float* y;
  int64_t o_st, o_sh, g_st, g_sh, y_st, y_sh;
  int T, H, D;
};

__global__ __launch_bounds__(256) void gate_fwd_f32_kernel(const GateArgs a) {
  const int chunks = a.D / 4;
  const int64_t total = (int64_t)a.T * a.H * chunks;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int c = (int)(i % chunks);
    const int64_t row = i / chunks;
    const int h = (int)(row % a.H);
    const int t = (int)(row / a.H);
    const f32x4 o = *(const f32x4*)(a.o + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + 4 * c);
    const f32x4 g = *(const f32x4*)(a.g + (int64_t)t * a.g_st + (int64_t)h * a.g_sh + 4 * c);
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = sigmoid_f32(g[e]) * o[e];
    *(f32x4*)(a.y + (int64_t)t * a.y_st + (int64_t)h * a.y_sh + 4 * c) = y;
  }
}

// float32 gate backward, one thread per (token, head) row: dout_s = dout * s
// (the attention's upstream gradient, contiguous [T, H, D]), delta = rowsum(dout_s * O)
// ([H, T]) and dgate = (dout * O) * (1 - s) * s.
struct GateBwdArgs {
  const float* o;
  const float* dy;
  const float* g;
  float* dgate;
  float* dout_s;
  float* delta;
  int64_t o_st, o_sh, dy_st, dy_sh, g_st, g_sh, dg_st, dg_sh;
  int T, H, D;
};

__global__ __launch_bounds__(256) void gate_bwd_f32_kernel(const GateBwdArgs a) {
#pragma clang fp contract(off)
  const int64_t rows = (int64_t)a.T * a.H;
  for (int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x; row < rows; row += (int64_t)gridDim.x * 256) {
    const int h = (int)(row % a.H);
    const int t = (int)(row / a.H);
    const float* o = a.o + (int64_t)t * a.o_st + (int64_t)h * a.o_sh;
    const float* dy = a.dy + (int64_t)t * a.dy_st + (int64_t)h * a.dy_sh;
    const float* g = a.g + (int64_t)t * a.g_st + (int64_t)h * a.g_sh;
    float* dg = a.dgate + (int64_t)t * a.dg_st + (int64_t)h * a.dg_sh;
    float* ds = a.dout_s + row * a.D;
    float acc = 0.f;
    for (int d = 0; d < a.D; ++d) {
      const float s = sigmoid_f32(g[d]);
      const float dso = dy[d] * s;
      ds[d] = dso;
      dg[d] = (dy[d] * o[d]) * (1.0f - s) * s;
      acc += dso * o[d];
    }
    a.delta[(int64_t)h * a.T + t] = acc;
  }
}

unsigned grid_for(int64_t items) {
  const int64_t b = (items + 255) / 256;
  return (unsigned)(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

}  // namespace

hipError_t launch_rope(const MimirRopeParams& p, hipStream_t stream) {
  RopeArgs a;
  a.x = p.x;
  a.y = p.y;
  a.cos = p.cos;
  a.sin = p.sin;
  a.x_st = p.x_stride_token; a.x_sh = p.x_stride_head;
  a.y_st = p.y_stride_token; a.y_sh = p.y_stride_head;
  a.cs_st = p.cs_stride_token;
  a.T = p.total_tokens;
  a.H = p.num_heads;
  a.D = p.head_dim;
  a.inverse = p.inverse != 0;
  const int v = p.dtype == MIMIR_DTYPE_BFLOAT16 ? 8 : 4;
  const int64_t items = (int64_t)a.T * a.H * (a.D / 2 / v);
  if (items == 0) return hipSuccess;
  if (p.dtype == MIMIR_DTYPE_BFLOAT16)
    hipLaunchKernelGGL((rope_kernel<bf16_t, 8>), dim3(grid_for(items)), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((rope_kernel<float, 4>), dim3(grid_for(items)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_gate_fwd_f32(const MimirPrefixLMFwdParams& p, hipStream_t stream) {
  GateArgs a;
  a.o = (const float*)p.out;
  a.g = (const float*)p.gate;
  a.y = (float*)p.gated_out;
  a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.g_st = p.gate_stride_token; a.g_sh = p.gate_stride_head;
  a.y_st = p.gated_out_stride_token; a.y_sh = p.gated_out_stride_head;
  a.T = p.total_tokens;
  a.H = p.num_q_heads;
  a.D = p.head_dim;
  const int64_t items = (int64_t)a.T * a.H * (a.D / 4);
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL(gate_fwd_f32_kernel, dim3(grid_for(items)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_gate_bwd_f32(const MimirPrefixLMBwdParams& p, float* dout_s, float* delta, hipStream_t stream) {
  GateBwdArgs a;
  a.o = (const float*)p.out;
  a.dy = (const float*)p.dout;
  a.g = (const float*)p.gate;
  a.dgate = (float*)p.dgate;
  a.dout_s = dout_s;
  a.delta = delta;
  a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.dy_st = p.dout_stride_token; a.dy_sh = p.dout_stride_head;
  a.g_st = p.gate_stride_token; a.g_sh = p.gate_stride_head;
  a.dg_st = p.dgate_stride_token; a.dg_sh = p.dgate_stride_head;
  a.T = p.total_tokens;
  a.H = p.num_q_heads;
  a.D = p.head_dim;
  const int64_t rows = (int64_t)a.T * a.H;
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(gate_bwd_f32_kernel, dim3(grid_for(rows)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mimir
