// Scalar device functors for the elementwise registry and the fused
// activations. Formulas and operation order follow the reference registry
// (crates/oxi-tensor/src/ops.rs:55-202) and the reference compositions of
// F.gelu / F.silu (python/oxitorch/nn/functional.py:194-204). The library is
// compiled with -ffp-contract=off so each product and sum rounds on its own,
// as in the reference's one-op-per-pass evaluation.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace oxi {

// ---- unary registry --------------------------------------------------------
template <int OP>
struct Unary {
  __device__ __forceinline__ float operator()(float a) const {
    if constexpr (OP == OXI_UNARY_NEG) return -a;
    else if constexpr (OP == OXI_UNARY_ABS) return fabsf(a);
    else if constexpr (OP == OXI_UNARY_SQRT) return sqrtf(a);
    else if constexpr (OP == OXI_UNARY_RSQRT) return 1.0f / sqrtf(a);
    else if constexpr (OP == OXI_UNARY_EXP) return expf(a);
    else if constexpr (OP == OXI_UNARY_LOG) return logf(a);
    else if constexpr (OP == OXI_UNARY_LOG2) return log2f(a);
    else if constexpr (OP == OXI_UNARY_LOG10) return log10f(a);
    else if constexpr (OP == OXI_UNARY_SIN) return sinf(a);
    else if constexpr (OP == OXI_UNARY_COS) return cosf(a);
    else if constexpr (OP == OXI_UNARY_TANH) return tanhf(a);
    else if constexpr (OP == OXI_UNARY_RELU) return fmaxf(a, 0.0f);  // f32::max: NaN -> 0
    else if constexpr (OP == OXI_UNARY_SIGMOID) return 1.0f / (1.0f + expf(-a));
    else if constexpr (OP == OXI_UNARY_FLOOR) return floorf(a);
    else if constexpr (OP == OXI_UNARY_CEIL) return ceilf(a);
    else if constexpr (OP == OXI_UNARY_ROUND) return roundf(a);  // half away from zero, as f32::round
    else if constexpr (OP == OXI_UNARY_SIGN) return (a != a) ? a : copysignf(1.0f, a);  // f32::signum
    else if constexpr (OP == OXI_UNARY_SQUARE) return a * a;
    else if constexpr (OP == OXI_UNARY_RECIPROCAL) return 1.0f / a;
    else return a;  // identity
  }
};

// ---- binary registry + comparisons ----------------------------------------
template <int OP>
struct Binary {
  __device__ __forceinline__ float operator()(float a, float b) const {
    if constexpr (OP == OXI_BINARY_ADD) return a + b;
    else if constexpr (OP == OXI_BINARY_SUB) return a - b;
    else if constexpr (OP == OXI_BINARY_MUL) return a * b;
    else if constexpr (OP == OXI_BINARY_DIV) return a / b;
    else if constexpr (OP == OXI_BINARY_POW) return powf(a, b);
    else if constexpr (OP == OXI_BINARY_MIN) return fminf(a, b);  // f32::min ignores NaN
    else if constexpr (OP == OXI_BINARY_MAX) return fmaxf(a, b);
    else if constexpr (OP == OXI_CMP_EQ) return a == b ? 1.0f : 0.0f;
    else if constexpr (OP == OXI_CMP_NE) return a != b ? 1.0f : 0.0f;
    else if constexpr (OP == OXI_CMP_LT) return a < b ? 1.0f : 0.0f;
    else if constexpr (OP == OXI_CMP_LE) return a <= b ? 1.0f : 0.0f;
    else if constexpr (OP == OXI_CMP_GT) return a > b ? 1.0f : 0.0f;
    else return a >= b ? 1.0f : 0.0f;
  }
};

// ---- fused activations -----------------------------------------------------
// Constants of F.gelu, rounded to f32 as the reference's Python floats are
// when promoted to tensors (crates/oxi-bindings/src/lib.rs:60-68).
constexpr float GELU_K = 0.044715f;
constexpr float GELU_C = 0.7978845608028654f;  // float(np.sqrt(2/np.pi))
constexpr float SQRT1_2 = 0.7071067811865476f;
constexpr float INV_SQRT_2PI = 0.3989422804014327f;
constexpr float LOG2E_F = 1.44269502f;        // log2(e) rounded to f32
constexpr float LOG2E_LO = 1.925963033e-8f;   // log2(e) - LOG2E_F
constexpr float LN2_F = 0.693147181f;

// y = (x*0.5) * (tanh(((x + (x*(x*x))*K) * C)) + 1)
struct GeluTanhFwd {
  __device__ __forceinline__ float operator()(float x) const {
    const float x32 = x * x;
    const float t1 = x * x32;
    const float t2 = t1 * GELU_K;
    const float t3 = x + t2;
    const float inner = t3 * GELU_C;
    const float th = tanhf(inner);
    const float op = th + 1.0f;
    const float hx = x * 0.5f;
    return hx * op;
  }
};

// The composed VJP of the reference graph, accumulated into x.grad in the
// reference's reverse-topological order (graph.rs:324-438): the 0.5*x branch,
// then x + t2, then x*x32, then both operands of x*x.
struct GeluTanhBwd {
  __device__ __forceinline__ float operator()(float x, float g) const {
    const float x32 = x * x;
    const float t1 = x * x32;
    const float t2 = t1 * GELU_K;
    const float t3 = x + t2;
    const float inner = t3 * GELU_C;
    const float th = tanhf(inner);
    const float op = th + 1.0f;
    const float hx = x * 0.5f;
    const float g_hx = g * op;
    const float g_op = g * hx;
    const float g_inner = g_op * (1.0f - th * th);
    const float g_t3 = g_inner * GELU_C;
    const float g_t1 = g_t3 * GELU_K;
    const float g_x32 = g_t1 * x;
    float dx = g_hx * 0.5f;
    dx = dx + g_t3;
    dx = dx + g_t1 * x32;
    const float c = g_x32 * x;
    dx = dx + c;
    dx = dx + c;
    return dx;
  }
};

// Standard normal CDF Phi(x) and density phi(x) for the exact GELU, through
// erfc(z) = exp(-z*z) * t * Q(t) with z = |x|/sqrt2 and t = 1/(1 + z/2).
// Q is a degree-10 polynomial in t fitted in float64 (weighted least
// squares, relative error) to erfcx(z)/t over t in (0, 1]: 1.1e-8 relative
// before rounding; Q(0) = 1/(2*sqrt(pi)). One exp per element and no branch:
// ROCm's erff evaluates two polynomial ranges and GELU inputs straddle its
// branch point in every wave, which made the forward ALU-bound.
// exp(-x*x/2) carries the rounding error of x*x (fma residual), and |x| is
// clamped at 20 there (exp(-200) is 0 in f32) so that +-inf stay finite.
// In float32 this Phi stays within 6.5e-7 relative of float64, and
// x * Phi(x) within 4e-7 absolute; evaluating Phi as 1 - E/2 for x >= 0 and
// E/2 for x < 0 avoids the cancellation of 0.5 * (1 + erf(x/sqrt2)).
struct NormalCdfPdf {
  float cdf, pdf;
};

__device__ __forceinline__ NormalCdfPdf normal_cdf_pdf(float x) {
  const float ax = fabsf(x);
  const float z = ax * SQRT1_2;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float q = 0.042352393f;
  q = fmaf(q, t, -0.23085676f);
  q = fmaf(q, t, 0.48617718f);
  q = fmaf(q, t, -0.4469757f);
  q = fmaf(q, t, 0.1270884f);
  q = fmaf(q, t, -0.057232074f);
  q = fmaf(q, t, 0.093000494f);
  q = fmaf(q, t, 0.17537685f);
  q = fmaf(q, t, 0.24688059f);
  q = fmaf(q, t, 0.28209385f);
  q = fmaf(q, t, 0.2820948f);
  // exp(-x*x/2) = 2^a * (1 + d): a = p*L rounded, p = -(x*x)/2 rounded; d
  // carries, to first order, the product's rounding (fma residual), the part
  // of log2(e) below L, and the rounding of x*x. 2^a is v_exp_f32.
  const float xe = fminf(ax, 20.0f);
  const float hh = xe * xe;
  const float hl = fmaf(xe, xe, -hh);  // x*x = hh + hl exactly
  const float p = -0.5f * hh;
  const float a = p * LOG2E_F;
  const float r = fmaf(p, LOG2E_LO, fmaf(p, LOG2E_F, -a));
  const float d = fmaf(r, LN2_F, -0.5f * hl);
  const float e0 = __builtin_amdgcn_exp2f(a);
  const float e = fmaf(e0, d, e0);
  const float half = 0.5f * ((t * q) * e);  // erfc(|x|/sqrt2) / 2
  return {x < 0.0f ? half : 1.0f - half, e * INV_SQRT_2PI};
}

// Exact GELU: y = x * Phi(x)  (= 0.5*x*(1 + erf(x/sqrt2))).
struct GeluErfFwd {
  __device__ __forceinline__ float operator()(float x) const { return x * normal_cdf_pdf(x).cdf; }
};

// dy/dx = Phi(x) + x * phi(x)
struct GeluErfBwd {
  __device__ __forceinline__ float operator()(float x, float g) const {
    const NormalCdfPdf p = normal_cdf_pdf(x);
    return g * (p.cdf + x * p.pdf);
  }
};

// y = x * sigmoid(x), sigmoid = 1/(1+exp(-x))   (ops.rs:174-177)
struct SiluFwd {
  __device__ __forceinline__ float operator()(float x) const {
    const float s = 1.0f / (1.0f + expf(-x));
    return x * s;
  }
};

// dx = g*s + (g*x)*(s*(1-s)): the mul VJP then the sigmoid VJP (ops.rs:62-73,236-247)
struct SiluBwd {
  __device__ __forceinline__ float operator()(float x, float g) const {
    const float s = 1.0f / (1.0f + expf(-x));
    const float a = g * s;
    const float b = (g * x) * (s * (1.0f - s));
    return a + b;
  }
};

}  // namespace oxi
