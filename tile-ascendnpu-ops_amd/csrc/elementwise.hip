// Memory-bound elementwise kernels for gfx950:
//   * unary activations / clamp           (tileops_unary_fwd)
//   * float predicates -> bool bytes      (tileops_isfp_fwd)
//   * fused gated GELU (erf and tanh)     (tileops_gated_gelu_fwd)
//
// All three stream HBM with 128-bit non-temporal loads/stores: every lane
// moves whole 16-byte packs, loads are issued before the math, and the math
// is fp32 with a single rounding back to the storage type.
#include "common.h"

namespace tileops {

// ---------------------------------------------------------------------------
// Unary activations.  Comparisons are written so that a NaN input falls
// through every select unchanged (NaN < a and NaN > a are both false), which
// gives torch's NaN propagation without a separate isnan test; fmaxf/fminf
// are avoided because they drop NaN.
// ---------------------------------------------------------------------------
// n / 6 correctly rounded without the IEEE division sequence: q0 = n * RN(1/6)
// is within one ulp, the remainder e = n - 6 q0 is exact under FMA, and
// RN(q0 + e RN(1/6)) is then the correctly rounded quotient (Markstein's
// one-step correction; 6 is not of the form 2^k (2 - 2^-23)).  Exact
// quotients (e == 0, which keeps the sign of zero) and non-finite values
// keep q0.
__device__ __forceinline__ float div6(float n) {
  const float r = 0x1.555556p-3f;  // RN(1/6)
  const float q0 = n * r;
  const float e = fmaf(-q0, 6.0f, n);
  const float q1 = fmaf(e, r, q0);
  return (e == 0.0f || !(__builtin_fabsf(q0) < __builtin_huge_valf())) ? q0 : q1;
}

template <int OP>
__device__ __forceinline__ float unary_op(float x, float lo, float hi, int flags) {
  if constexpr (OP == TILEOPS_HARDSWISH) {
    // x * min(max(x + 3, 0), 6) / 6  (F.hardswish; test_hardswish.py:38-39)
    float t = x + 3.0f;
    t = t < 0.0f ? 0.0f : t;
    t = t > 6.0f ? 6.0f : t;
    return div6(x * t);
  } else if constexpr (OP == TILEOPS_HARDSIGMOID) {
    // min(max(x + 3, 0), 6) / 6  (F.hardsigmoid; test_hardsigmoid.py:38-39)
    float t = x + 3.0f;
    t = t < 0.0f ? 0.0f : t;
    t = t > 6.0f ? 6.0f : t;
    return div6(t);
  } else if constexpr (OP == TILEOPS_MISH) {
    // x * tanh(softplus(x)) (F.mish, test_mish.py:38-39) through
    // tanh(log(1 + u)) = n / (n + 2) with n = u (u + 2), u = e^x: one
    // exponential and one reciprocal instead of exp, log1p and tanh.  Above
    // x = 20 the factor is 1 in fp32 (and n would overflow), so x itself.
    // +inf -> +inf, -inf -> NaN (-inf * 0), NaN -> NaN, as F.mish gives.
    const float u = __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
    const float n = u * (u + 2.0f);
    const float t = n * __builtin_amdgcn_rcpf(n + 2.0f);
    return x * (x > 20.0f ? 1.0f : t);
  } else {
    // torch.clamp(x, min, max) (test_clamp_scalar.py:56-57): NaN input stays
    // NaN; a NaN bound selects the bound itself, i.e. NaN everywhere; with
    // min > max every value ends at max.
    float y = x;
    if (flags & TILEOPS_CLAMP_HAS_MIN) y = (y < lo || lo != lo) ? lo : y;
    if (flags & TILEOPS_CLAMP_HAS_MAX) y = (y > hi || hi != hi) ? hi : y;
    return y;
  }
}

// One-shot grid: thread i owns pack i.  Measured on MI355X, one 16-byte
// non-temporal pack per thread with a grid covering the whole tensor streams
// a read+write workload at ~82% of HBM peak, ahead of grid-stride loops
// (~65%) and of several packs per thread (~75%).
// x and y may be the same buffer (the Ops' in-place path): every thread
// reads its pack before it writes it, so neither pointer is __restrict__.
template <typename T, int OP>
__global__ __launch_bounds__(256) void unary_vec_kernel(const T* x, T* y, int64_t npack,
                                                        float lo, float hi, int flags) {
  constexpr int V = Elem<T>::kVec;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= npack) return;
  const Pack<T> in = load_pack_nt(x + i * V);
  Pack<T> out;
#pragma unroll
  for (int e = 0; e < V; ++e)
    out.v[e] = Elem<T>::from_f32(unary_op<OP>(Elem<T>::to_f32(in.v[e]), lo, hi, flags));
  store_pack_nt(y + i * V, out);
}

// Scalar path: tails after the packed body, and misaligned tensors.
template <typename T, int OP>
__global__ __launch_bounds__(256) void unary_scalar_kernel(const T* x, T* y, int64_t begin,
                                                           int64_t n, float lo, float hi,
                                                           int flags) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = Elem<T>::from_f32(unary_op<OP>(Elem<T>::to_f32(x[i]), lo, hi, flags));
}

template <typename T, int OP>
static int launch_unary(const void* xv, void* yv, int64_t n, float lo, float hi, int flags,
                        hipStream_t s) {
  constexpr int V = Elem<T>::kVec;
  const T* x = static_cast<const T*>(xv);
  T* y = static_cast<T*>(yv);
  int64_t npack = (host_aligned16(x) && host_aligned16(y)) ? n / V : 0;
  if (npack > 0) {
    const int64_t grid = (npack + 255) / 256;
    unary_vec_kernel<T, OP><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, y, npack, lo, hi,
                                                                        flags);
  }
  int64_t done = npack * V;
  if (done < n) {
    int64_t grid = stream_grid(n - done, 256);
    unary_scalar_kernel<T, OP><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, y, done, n, lo, hi,
                                                                          flags);
  }
  return launch_status();
}

template <typename T>
static int dispatch_unary(int op, const void* x, void* y, int64_t n, float lo, float hi,
                          int flags, hipStream_t s) {
  switch (op) {
    case TILEOPS_HARDSWISH: return launch_unary<T, TILEOPS_HARDSWISH>(x, y, n, lo, hi, flags, s);
    case TILEOPS_HARDSIGMOID:
      return launch_unary<T, TILEOPS_HARDSIGMOID>(x, y, n, lo, hi, flags, s);
    case TILEOPS_CLAMP: return launch_unary<T, TILEOPS_CLAMP>(x, y, n, lo, hi, flags, s);
    case TILEOPS_MISH: return launch_unary<T, TILEOPS_MISH>(x, y, n, lo, hi, flags, s);
  }
  return TILEOPS_EINVAL;
}

// ---------------------------------------------------------------------------
// Float predicates.  Pure bit tests on the IEEE encoding, so the result is
// exact for every input including signalling NaNs and subnormals:
//   NaN:    |bits| >  exponent-all-ones
//   inf:    |bits| == exponent-all-ones
//   finite: exponent field != all ones
// ---------------------------------------------------------------------------
template <typename T> struct FpBits;
template <> struct FpBits<float> {
  typedef uint32_t U;
  static constexpr U kAbs = 0x7fffffffu, kExp = 0x7f800000u;
};
template <> struct FpBits<f16> {
  typedef uint16_t U;
  static constexpr U kAbs = 0x7fffu, kExp = 0x7c00u;
};
template <> struct FpBits<bf16> {
  typedef uint16_t U;
  static constexpr U kAbs = 0x7fffu, kExp = 0x7f80u;
};

template <typename T, int PRED>
__device__ __forceinline__ uint32_t pred_bit(typename FpBits<T>::U b) {
  typedef FpBits<T> F;
  const typename F::U a = b & F::kAbs;
  if constexpr (PRED == TILEOPS_ISNAN) return a > F::kExp ? 1u : 0u;
  else if constexpr (PRED == TILEOPS_ISINF) return a == F::kExp ? 1u : 0u;
  else return (b & F::kExp) != F::kExp ? 1u : 0u;
}

// Two input packs per thread, 256 packs apart inside the workgroup's span
// (measured on MI355X: 85% of HBM peak at fp32 8192^2, against 76% with one
// pack per thread); 4 fp32 or 8 half inputs give a 4- or 8-byte store of 0/1
// bytes.
template <typename T> struct PredOut;
template <> struct PredOut<float> { typedef uint32_t W; };
template <> struct PredOut<f16> { typedef uint2 W; };
template <> struct PredOut<bf16> { typedef uint2 W; };
constexpr int kIsfpPacks = 2;

template <typename T, int PRED>
__global__ __launch_bounds__(256) void isfp_vec_kernel(const T* __restrict__ x,
                                                       uint8_t* __restrict__ y, int64_t npack) {
  typedef typename FpBits<T>::U U;
  constexpr int V = Elem<T>::kVec;
  const int64_t base = (int64_t)blockIdx.x * 256 * kIsfpPacks + threadIdx.x;
  u32x4 in[kIsfpPacks];
#pragma unroll
  for (int u = 0; u < kIsfpPacks; ++u) {
    const int64_t i = base + (int64_t)u * 256;
    if (i < npack) in[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + i * V));
  }
#pragma unroll
  for (int u = 0; u < kIsfpPacks; ++u) {
    const int64_t i = base + (int64_t)u * 256;
    if (i < npack) {
      const U* e = reinterpret_cast<const U*>(&in[u]);
      uint32_t words[V / 4];
#pragma unroll
      for (int w = 0; w < V / 4; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) word |= pred_bit<T, PRED>(e[w * 4 + b]) << (8 * b);
        words[w] = word;
      }
      *reinterpret_cast<typename PredOut<T>::W*>(y + i * V) =
          *reinterpret_cast<typename PredOut<T>::W*>(words);
    }
  }
}

template <typename T, int PRED>
__global__ __launch_bounds__(256) void isfp_scalar_kernel(const T* __restrict__ x,
                                                          uint8_t* __restrict__ y, int64_t begin,
                                                          int64_t n) {
  typedef typename FpBits<T>::U U;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (uint8_t)pred_bit<T, PRED>(reinterpret_cast<const U*>(x)[i]);
}

template <typename T, int PRED>
static int launch_isfp(const void* xv, uint8_t* y, int64_t n, hipStream_t s) {
  constexpr int V = Elem<T>::kVec;
  const T* x = static_cast<const T*>(xv);
  const bool aligned = host_aligned16(x) && (reinterpret_cast<uintptr_t>(y) % V) == 0;
  const int64_t npack = aligned ? n / V : 0;
  if (npack > 0) {
    const int64_t grid = (npack + 256 * kIsfpPacks - 1) / (256 * kIsfpPacks);
    isfp_vec_kernel<T, PRED><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, y, npack);
  }
  int64_t done = npack * V;
  if (done < n) {
    int64_t grid = stream_grid(n - done, 256);
    isfp_scalar_kernel<T, PRED><<<dim3((unsigned)grid), dim3(256), 0, s>>>(x, y, done, n);
  }
  return launch_status();
}

template <typename T>
static int dispatch_isfp(int pred, const void* x, uint8_t* y, int64_t n, hipStream_t s) {
  switch (pred) {
    case TILEOPS_ISNAN: return launch_isfp<T, TILEOPS_ISNAN>(x, y, n, s);
    case TILEOPS_ISINF: return launch_isfp<T, TILEOPS_ISINF>(x, y, n, s);
    case TILEOPS_ISFINITE: return launch_isfp<T, TILEOPS_ISFINITE>(x, y, n, s);
  }
  return TILEOPS_EINVAL;
}

// ---------------------------------------------------------------------------
// Gated GELU.
//
// erf form (GeluAndMul): 0.5 * g * (1 + erf(g / sqrt(2))) * v.
//   For half-precision storage the erf comes from Abramowitz & Stegun,
//   Handbook of Mathematical Functions, formula 7.1.26:
//     erf(a) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-a^2),
//     t = 1 / (1 + p a),  a >= 0,  |error| <= 1.5e-7,
//   extended to a < 0 by odd symmetry.  That bound is ~2^-22, far below the
//   2^-8 / 2^-11 spacing of bf16 / fp16 results, and costs one reciprocal and
//   one exp2 instead of the ~35 VALU instructions of the library erff, which
//   keeps the kernel under the HBM roofline.  fp32 storage uses erff.
// tanh form (GeluTanhAndMul): 0.5 g (1 + tanh(u)), u = sqrt(2/pi)(g + 0.044715 g^3),
//   evaluated through the identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float erf_as7126(float x) {
  const float a = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, a, 1.0f));
  float poly = 1.061405429f;
  poly = fmaf(poly, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  poly *= t;
  // exp(-a^2) = exp2(-a^2 * log2(e))
  const float e = __builtin_amdgcn_exp2f(-(a * a) * 1.4426950408889634f);
  const float r = fmaf(-poly, e, 1.0f);
  return copysignf(r, x);
}

template <int APPROX, bool ACCURATE>
__device__ __forceinline__ float gated_gelu(float g, float v) {
  if constexpr (APPROX == 0) {
    const float z = g * 0.7071067811865476f;
    const float erfz = ACCURATE ? erff(z) : erf_as7126(z);
    return 0.5f * g * (1.0f + erfz) * v;
  } else {
    const float u = 0.7978845608028654f * fmaf(0.044715f * g, g * g, g);
    // 1 / (1 + exp(-2u)), exp(-2u) = exp2(-2u * log2(e))
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u * -2.8853900817779268f));
    return g * s * v;
  }
}

// One-shot grid over the flattened [M, N / V] output packs: thread i owns
// output pack i (its row and column from one 32-bit division), loading the
// gate pack and the value pack of that position.  Every thread has a pack,
// where a grid of row chunks leaves the last chunk of each row part idle
// (N = 11008 bf16: 1376 packs per row in chunks of 512); measured ~0.5-1 %
// faster at 16384 x 11008.
template <typename T, int APPROX>
__global__ __launch_bounds__(256) void gated_gelu_vec_kernel(const T* __restrict__ x,
                                                             T* __restrict__ y, uint32_t total,
                                                             uint32_t P) {
  constexpr int V = Elem<T>::kVec;
  constexpr bool ACC = sizeof(T) == 4;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= total) return;
  const uint32_t row = i / P, p = i - row * P;
  const T* gate = x + (int64_t)row * 2 * P * V + (int64_t)p * V;
  const Pack<T> gp = load_pack_nt(gate);
  const Pack<T> vp = load_pack_nt(gate + (int64_t)P * V);
  Pack<T> o;
#pragma unroll
  for (int e = 0; e < V; ++e)
    o.v[e] = Elem<T>::from_f32(
        gated_gelu<APPROX, ACC>(Elem<T>::to_f32(gp.v[e]), Elem<T>::to_f32(vp.v[e])));
  store_pack_nt(y + (int64_t)i * V, o);
}

// Tensors with 2^32 or more output packs: one workgroup per row chunk
// (grid-stride over rows); each thread owns UNROLL packs of the row,
// issuing all gate and value loads before any math.
template <typename T, int APPROX, int UNROLL>
__global__ __launch_bounds__(256) void gated_gelu_rows_kernel(const T* __restrict__ x,
                                                              T* __restrict__ y, int64_t M,
                                                              int64_t N) {
  constexpr int V = Elem<T>::kVec;
  constexpr bool ACC = sizeof(T) == 4;
  const int64_t P = N / V;  // packs per output row
  for (int64_t row = blockIdx.y; row < M; row += gridDim.y) {
    const T* gate = x + row * 2 * N;
    const T* val = gate + N;
    T* out = y + row * N;
    for (int64_t p0 = (int64_t)blockIdx.x * blockDim.x * UNROLL + threadIdx.x; p0 < P;
         p0 += (int64_t)gridDim.x * blockDim.x * UNROLL) {
      Pack<T> gp[UNROLL], vp[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t p = p0 + u * blockDim.x;
        if (p < P) {
          gp[u] = load_pack_nt(gate + p * V);
          vp[u] = load_pack_nt(val + p * V);
        }
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int64_t p = p0 + u * blockDim.x;
        if (p < P) {
          Pack<T> o;
#pragma unroll
          for (int e = 0; e < V; ++e)
            o.v[e] = Elem<T>::from_f32(gated_gelu<APPROX, ACC>(Elem<T>::to_f32(gp[u].v[e]),
                                                               Elem<T>::to_f32(vp[u].v[e])));
          store_pack_nt(out + p * V, o);
        }
      }
    }
  }
}

template <typename T, int APPROX>
__global__ __launch_bounds__(256) void gated_gelu_scalar_kernel(const T* __restrict__ x,
                                                                T* __restrict__ y, int64_t M,
                                                                int64_t N) {
  constexpr bool ACC = sizeof(T) == 4;
  for (int64_t row = blockIdx.y; row < M; row += gridDim.y) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < N;
         j += (int64_t)gridDim.x * blockDim.x) {
      const float g = Elem<T>::to_f32(x[row * 2 * N + j]);
      const float v = Elem<T>::to_f32(x[row * 2 * N + N + j]);
      y[row * N + j] = Elem<T>::from_f32(gated_gelu<APPROX, ACC>(g, v));
    }
  }
}

template <typename T, int APPROX>
static int launch_gated_gelu(const void* xv, void* yv, int64_t M, int64_t N, hipStream_t s) {
  constexpr int V = Elem<T>::kVec;
  const T* x = static_cast<const T*>(xv);
  T* y = static_cast<T*>(yv);
  const unsigned gy = (unsigned)(M < 65535 ? M : 65535);
  const int64_t P = N / V;
  if (N % V == 0 && host_aligned16(x) && host_aligned16(y) && M * P <= (int64_t)UINT32_MAX - 255) {
    const uint32_t total = (uint32_t)(M * P);
    gated_gelu_vec_kernel<T, APPROX><<<dim3((total + 255) / 256), dim3(256), 0, s>>>(
        x, y, total, (uint32_t)P);
  } else if (N % V == 0 && host_aligned16(x) && host_aligned16(y)) {
    constexpr int UNROLL = 2;
    int64_t gx = (P + 256 * UNROLL - 1) / (256 * UNROLL);
    gated_gelu_rows_kernel<T, APPROX, UNROLL><<<dim3((unsigned)gx, gy), dim3(256), 0, s>>>(
        x, y, M, N);
  } else {
    int64_t gx = (N + 255) / 256;
    if (gx > 64) gx = 64;
    gated_gelu_scalar_kernel<T, APPROX><<<dim3((unsigned)gx, gy), dim3(256), 0, s>>>(x, y, M, N);
  }
  return launch_status();
}

template <typename T>
static int dispatch_gated_gelu(int approx, const void* x, void* y, int64_t M, int64_t N,
                               hipStream_t s) {
  if (approx == 0) return launch_gated_gelu<T, 0>(x, y, M, N, s);
  if (approx == 1) return launch_gated_gelu<T, 1>(x, y, M, N, s);
  return TILEOPS_EINVAL;
}

}  // namespace tileops

using namespace tileops;

// ---------------------------------------------------------------------------
// Bitwise NOT (torch.bitwise_not) on the bytes of bool / integer tensors: every
// integer type is its bytes complemented, a bool (one byte, 0 or 1) its byte
// XOR 1.  16-byte non-temporal packs, then single bytes for the tail.
// ---------------------------------------------------------------------------
namespace tileops {

__global__ __launch_bounds__(256) void bitnot_vec_kernel(const u32x4* __restrict__ x,
                                                         u32x4* __restrict__ y, int64_t npack,
                                                         uint32_t mask) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= npack) return;
  u32x4 v = __builtin_nontemporal_load(x + i);
  v ^= u32x4{mask, mask, mask, mask};
  __builtin_nontemporal_store(v, y + i);
}

__global__ __launch_bounds__(256) void bitnot_byte_kernel(const uint8_t* __restrict__ x,
                                                          uint8_t* __restrict__ y, int64_t begin,
                                                          int64_t n, uint32_t mask) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (uint8_t)(x[i] ^ (uint8_t)mask);
}

}  // namespace tileops

namespace tileops {

// ---------------------------------------------------------------------------
// Broadcast element-wise combines of two or three operands, fp32 opmath
// rounded once:
//   BC_ADD          y = a + p * b            (torch.add; torch.sub passes -p, exact)
//   BC_LERP_SCALAR  y = lerp(a, b, p)        (torch.lerp with a scalar weight)
//   BC_LERP_TENSOR  y = lerp(a, b, w)        (torch.lerp with a weight tensor)
// Same-shape contiguous operands stream as 16-byte packs; broadcast operands
// are read through per-dimension strides (0 on a broadcast dimension) of the
// output's multi-index, with no materialised copy.
// ---------------------------------------------------------------------------
constexpr int kMaxDims = 8;
enum { BC_ADD = 0, BC_LERP_SCALAR = 1, BC_LERP_TENSOR = 2 };
struct BcastDesc {
  int ndim;
  int64_t shape[kMaxDims];  // output shape
  int64_t st[3][kMaxDims];  // element strides of a, b, w (0: broadcast)
};

template <int OP> struct BcastArity { static constexpr int n = OP == BC_LERP_TENSOR ? 3 : 2; };

// torch.lerp's two-sided form: start + w (end - start) for |w| < 0.5, else
// end - (1 - w)(end - start), each as one fma: exact at w = 0 and w = 1.
__device__ __forceinline__ float lerp_f32(float s, float e, float w) {
  const float d = e - s;
  return __builtin_fabsf(w) < 0.5f ? fmaf(w, d, s) : fmaf(w - 1.0f, d, e);
}

template <int OP>
__device__ __forceinline__ float bc_apply(float a, float b, float w, float p) {
  if constexpr (OP == BC_ADD) return fmaf(p, b, a);
  else if constexpr (OP == BC_LERP_SCALAR) return lerp_f32(a, b, p);
  else return lerp_f32(a, b, w);
}

template <typename T, int OP>
__global__ __launch_bounds__(256) void bcast_vec_kernel(const T* __restrict__ a,
                                                        const T* __restrict__ b,
                                                        const T* __restrict__ w,
                                                        T* __restrict__ y, int64_t npack,
                                                        float p) {
  constexpr int V = Elem<T>::kVec;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= npack) return;
  const Pack<T> pa = load_pack_nt(a + i * V), pb = load_pack_nt(b + i * V);
  Pack<T> pw;
  if constexpr (BcastArity<OP>::n == 3) pw = load_pack_nt(w + i * V);
  Pack<T> out;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const float we = BcastArity<OP>::n == 3 ? Elem<T>::to_f32(pw.v[e]) : 0.0f;
    out.v[e] = Elem<T>::from_f32(
        bc_apply<OP>(Elem<T>::to_f32(pa.v[e]), Elem<T>::to_f32(pb.v[e]), we, p));
  }
  store_pack_nt(y + i * V, out);
}

template <typename T, int OP>
__global__ __launch_bounds__(256) void bcast_any_kernel(const T* __restrict__ a,
                                                        const T* __restrict__ b,
                                                        const T* __restrict__ w,
                                                        T* __restrict__ y, int64_t begin,
                                                        int64_t n, float p, BcastDesc d) {
  constexpr int NOP = BcastArity<OP>::n;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, off[3] = {0, 0, 0};
    for (int k = d.ndim - 1; k >= 0; --k) {
      const int64_t idx = rem % d.shape[k];
      rem /= d.shape[k];
#pragma unroll
      for (int o = 0; o < NOP; ++o) off[o] += idx * d.st[o][k];
    }
    const float we = NOP == 3 ? Elem<T>::to_f32(w[off[2]]) : 0.0f;
    y[i] = Elem<T>::from_f32(
        bc_apply<OP>(Elem<T>::to_f32(a[off[0]]), Elem<T>::to_f32(b[off[1]]), we, p));
  }
}

// Operands whose innermost dimension is unit-stride or broadcast (bias rows,
// per-channel scales): a thread takes one 16-byte pack of an output row, so
// the outer multi-index is computed once per pack rather than per element,
// in 32-bit arithmetic (I = uint32_t) when every offset fits.  A broadcast
// operand (some stride 0) is re-read across rows and keeps the cached load;
// a streamed one takes the non-temporal load.  Bit o of `vec_mask` marks
// operand o as unit-stride along the row, bit o of `bc_mask` as broadcast
// somewhere.
template <typename T, int OP, typename I>
__global__ __launch_bounds__(256) void bcast_inner_kernel(const T* __restrict__ a,
                                                          const T* __restrict__ b,
                                                          const T* __restrict__ w,
                                                          T* __restrict__ y, I npack,
                                                          I row_packs, float p, BcastDesc d,
                                                          int vec_mask, int bc_mask) {
  constexpr int V = Elem<T>::kVec;
  constexpr int NOP = BcastArity<OP>::n;
  const T* src[3] = {a, b, w};
  const int nd = d.ndim;  // >= 1; dimension nd - 1 is the row
  const I stride = (I)gridDim.x * blockDim.x;
  for (I pk = (I)blockIdx.x * blockDim.x + threadIdx.x; pk < npack; pk += stride) {
    I r = pk / row_packs;
    const I c = (pk - r * row_packs) * V;
    I off[3];
#pragma unroll
    for (int o = 0; o < NOP; ++o) off[o] = ((vec_mask >> o) & 1) ? c : 0;
    for (int k = nd - 2; k >= 0; --k) {
      const I sh = (I)d.shape[k], q = r / sh, idx = r - q * sh;
      r = q;
#pragma unroll
      for (int o = 0; o < NOP; ++o) off[o] += idx * (I)d.st[o][k];
    }
    Pack<T> in[3];
#pragma unroll
    for (int o = 0; o < NOP; ++o) {
      if ((vec_mask >> o) & 1) {
        in[o] = ((bc_mask >> o) & 1) ? load_pack(src[o] + off[o]) : load_pack_nt(src[o] + off[o]);
      } else {
        const T v = src[o][off[o]];
#pragma unroll
        for (int e = 0; e < V; ++e) in[o].v[e] = v;
      }
    }
    Pack<T> out;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float we = NOP == 3 ? Elem<T>::to_f32(in[2].v[e]) : 0.0f;
      out.v[e] = Elem<T>::from_f32(
          bc_apply<OP>(Elem<T>::to_f32(in[0].v[e]), Elem<T>::to_f32(in[1].v[e]), we, p));
    }
    store_pack_nt(y + (int64_t)pk * V, out);
  }
}

// Drops size-1 dimensions and merges a dimension into the one outside it
// where every operand's strides chain (stride[k-1] == stride[k] * shape[k],
// broadcast dimensions included), so the index arithmetic runs over as few
// dimensions as the layout allows.
static void coalesce_dims(BcastDesc& d, int nop) {
  BcastDesc o{};
  int m = 0;
  for (int k = 0; k < d.ndim; ++k) {
    if (d.shape[k] == 1) continue;
    bool chain = m > 0;
    for (int q = 0; q < nop && chain; ++q) chain = o.st[q][m - 1] == d.st[q][k] * d.shape[k];
    if (chain) {
      o.shape[m - 1] *= d.shape[k];
      for (int q = 0; q < nop; ++q) o.st[q][m - 1] = d.st[q][k];
    } else {
      o.shape[m] = d.shape[k];
      for (int q = 0; q < nop; ++q) o.st[q][m] = d.st[q][k];
      ++m;
    }
  }
  o.ndim = m;
  d = o;
}

// The pack kernel applies when the row length is a whole number of packs,
// each operand's row is unit-stride (16-byte aligned base and row offsets) or
// broadcast, and the output is 16-byte aligned.  Returns false otherwise.
template <typename T, int OP>
static bool launch_bcast_inner(const T* const (&src)[3], T* y, const BcastDesc& d, int64_t n,
                               float p, hipStream_t s) {
  constexpr int V = Elem<T>::kVec;
  constexpr int NOP = BcastArity<OP>::n;
  const int nd = d.ndim;
  if (nd < 1 || d.shape[nd - 1] % V != 0 || !host_aligned16(y)) return false;
  int vec_mask = 0, bc_mask = 0;
  bool fits32 = true;
  for (int o = 0; o < NOP; ++o) {
    int64_t omax = 0;
    for (int k = 0; k < nd; ++k) {
      omax += (d.shape[k] - 1) * d.st[o][k];
      if (d.st[o][k] == 0) bc_mask |= 1 << o;
    }
    fits32 &= omax < (int64_t)UINT32_MAX;
    const int64_t in = d.st[o][nd - 1];
    if (in != 0 && in != 1) return false;
    if (in == 1) {
      vec_mask |= 1 << o;
      if (!host_aligned16(src[o])) return false;
      for (int k = 0; k < nd - 1; ++k)
        if (d.st[o][k] % V) return false;
    }
  }
  const int64_t npack = n / V, row_packs = d.shape[nd - 1] / V;
  const unsigned grid = (unsigned)stream_grid(npack, 256);
  if (fits32 && npack < (int64_t)UINT32_MAX - (int64_t)grid * 256)
    bcast_inner_kernel<T, OP, uint32_t><<<dim3(grid), dim3(256), 0, s>>>(
        src[0], src[1], src[2], y, (uint32_t)npack, (uint32_t)row_packs, p, d, vec_mask, bc_mask);
  else
    bcast_inner_kernel<T, OP, int64_t><<<dim3(grid), dim3(256), 0, s>>>(
        src[0], src[1], src[2], y, npack, row_packs, p, d, vec_mask, bc_mask);
  return true;
}

template <typename T, int OP>
static int launch_bcast(const void* av, const void* bv, const void* wv, void* yv, BcastDesc d,
                        int64_t n, float p, hipStream_t s) {
  constexpr int V = Elem<T>::kVec;
  constexpr int NOP = BcastArity<OP>::n;
  const T* const src[3] = {static_cast<const T*>(av), static_cast<const T*>(bv),
                           static_cast<const T*>(wv)};
  T* y = static_cast<T*>(yv);
  coalesce_dims(d, NOP);
  bool flat = true;  // every operand contiguous over the whole output
  bool aligned = host_aligned16(y);
  for (int o = 0; o < NOP; ++o) {
    int64_t expect = 1;
    for (int k = d.ndim - 1; k >= 0; --k) {
      if (d.shape[k] != 1 && d.st[o][k] != expect) flat = false;
      expect *= d.shape[k];
    }
    aligned &= host_aligned16(src[o]);
  }
  if (!flat && launch_bcast_inner<T, OP>(src, y, d, n, p, s)) return launch_status();
  int64_t npack = 0;
  if (flat && aligned) {
    npack = n / V;
    if (npack > 0)
      bcast_vec_kernel<T, OP><<<dim3((unsigned)((npack + 255) / 256)), dim3(256), 0, s>>>(
          src[0], src[1], src[2], y, npack, p);
  }
  const int64_t done = npack * V;
  if (done < n)
    bcast_any_kernel<T, OP><<<dim3((unsigned)stream_grid(n - done, 256)), dim3(256), 0, s>>>(
        src[0], src[1], src[2], y, done, n, p, d);
  return launch_status();
}

// Shared argument checks of the broadcast entry points; fills `d` and `n`.
static int bcast_prepare(int ndim, const int64_t* out_shape, const int64_t* const (&strides)[3],
                         int nop, BcastDesc& d, int64_t& n) {
  if (ndim < 0 || ndim > kMaxDims) return TILEOPS_ESHAPE;
  if (ndim > 0 && !out_shape) return TILEOPS_ENULL;
  for (int o = 0; o < nop; ++o)
    if (ndim > 0 && !strides[o]) return TILEOPS_ENULL;
  d = BcastDesc{};
  d.ndim = ndim;
  n = 1;
  for (int k = 0; k < ndim; ++k) {
    if (out_shape[k] < 0) return TILEOPS_ESHAPE;
    d.shape[k] = out_shape[k];
    for (int o = 0; o < nop; ++o) {
      if (strides[o][k] < 0) return TILEOPS_EINVAL;
      d.st[o][k] = strides[o][k];
    }
    n *= out_shape[k];
  }
  return 0;
}

template <int OP>
static int dispatch_bcast(int dtype, const void* a, const void* b, const void* w, void* y,
                          const BcastDesc& d, int64_t n, float p, hipStream_t s) {
  switch (dtype) {
    case TILEOPS_F32: return launch_bcast<float, OP>(a, b, w, y, d, n, p, s);
    case TILEOPS_F16: return launch_bcast<f16, OP>(a, b, w, y, d, n, p, s);
    default: return launch_bcast<bf16, OP>(a, b, w, y, d, n, p, s);
  }
}

}  // namespace tileops

extern "C" int tileops_add_fwd(const void* a, const void* b, void* y, int ndim,
                               const int64_t* out_shape, const int64_t* a_strides,
                               const int64_t* b_strides, float alpha, int dtype, void* stream) {
  BcastDesc d;
  int64_t n = 0;
  const int64_t* const st[3] = {a_strides, b_strides, nullptr};
  if (int e = bcast_prepare(ndim, out_shape, st, 2, d, n)) return e;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (n == 0) return 0;
  if (!a || !b || !y) return TILEOPS_ENULL;
  return dispatch_bcast<BC_ADD>(dtype, a, b, nullptr, y, d, n, alpha,
                                static_cast<hipStream_t>(stream));
}

extern "C" int tileops_lerp_fwd(const void* a, const void* b, const void* w, void* y, int ndim,
                                const int64_t* out_shape, const int64_t* a_strides,
                                const int64_t* b_strides, const int64_t* w_strides, float weight,
                                int dtype, void* stream) {
  BcastDesc d;
  int64_t n = 0;
  const int64_t* const st[3] = {a_strides, b_strides, w_strides};
  if (int e = bcast_prepare(ndim, out_shape, st, w ? 3 : 2, d, n)) return e;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (n == 0) return 0;
  if (!a || !b || !y) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (w) return dispatch_bcast<BC_LERP_TENSOR>(dtype, a, b, w, y, d, n, 0.0f, s);
  return dispatch_bcast<BC_LERP_SCALAR>(dtype, a, b, nullptr, y, d, n, weight, s);
}

extern "C" int tileops_bitwise_not_fwd(const void* x, void* y, int64_t nbytes, int is_bool,
                                       void* stream) {
  if (nbytes < 0) return TILEOPS_ESHAPE;
  if (nbytes == 0) return 0;
  if (!x || !y) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t mask = is_bool ? 0x01010101u : 0xFFFFFFFFu;
  const int64_t npack = (host_aligned16(x) && host_aligned16(y)) ? nbytes / 16 : 0;
  if (npack > 0)
    bitnot_vec_kernel<<<dim3((unsigned)((npack + 255) / 256)), dim3(256), 0, s>>>(
        static_cast<const u32x4*>(x), static_cast<u32x4*>(y), npack, mask);
  const int64_t done = npack * 16;
  if (done < nbytes)
    bitnot_byte_kernel<<<dim3((unsigned)stream_grid(nbytes - done, 256)), dim3(256), 0, s>>>(
        static_cast<const uint8_t*>(x), static_cast<uint8_t*>(y), done, nbytes, mask);
  return launch_status();
}

extern "C" int tileops_unary_fwd(int op, const void* x, void* y, int64_t n, int dtype, float lo,
                                 float hi, int flags, void* stream) {
  if (n < 0) return TILEOPS_ESHAPE;
  if (op == TILEOPS_CLAMP && (flags & (TILEOPS_CLAMP_HAS_MIN | TILEOPS_CLAMP_HAS_MAX)) == 0)
    return TILEOPS_EINVAL;
  if (op < TILEOPS_HARDSWISH || op > TILEOPS_MISH) return TILEOPS_EINVAL;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (n == 0) return 0;
  if (!x || !y) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TILEOPS_F32: return dispatch_unary<float>(op, x, y, n, lo, hi, flags, s);
    case TILEOPS_F16: return dispatch_unary<f16>(op, x, y, n, lo, hi, flags, s);
    default: return dispatch_unary<bf16>(op, x, y, n, lo, hi, flags, s);
  }
}

extern "C" int tileops_isfp_fwd(int pred, const void* x, uint8_t* y, int64_t n, int dtype,
                                void* stream) {
  if (n < 0) return TILEOPS_ESHAPE;
  if (pred < TILEOPS_ISNAN || pred > TILEOPS_ISFINITE) return TILEOPS_EINVAL;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (n == 0) return 0;
  if (!x || !y) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TILEOPS_F32: return dispatch_isfp<float>(pred, x, y, n, s);
    case TILEOPS_F16: return dispatch_isfp<f16>(pred, x, y, n, s);
    default: return dispatch_isfp<bf16>(pred, x, y, n, s);
  }
}

extern "C" int tileops_gated_gelu_fwd(int approx, const void* x, void* y, int64_t M, int64_t N,
                                      int dtype, void* stream) {
  if (M < 0 || N < 0) return TILEOPS_ESHAPE;
  if (approx != 0 && approx != 1) return TILEOPS_EINVAL;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (M == 0 || N == 0) return 0;
  if (!x || !y) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TILEOPS_F32: return dispatch_gated_gelu<float>(approx, x, y, M, N, s);
    case TILEOPS_F16: return dispatch_gated_gelu<f16>(approx, x, y, M, N, s);
    default: return dispatch_gated_gelu<bf16>(approx, x, y, M, N, s);
  }
}
