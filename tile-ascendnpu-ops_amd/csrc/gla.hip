// Single-token gated linear attention decode for gfx950 (tileops_gla_decode_fwd).
//
// Per (batch b, head h), layout BHD, state [DK][DV]:
//   new_state[dk][dv] = exp(gk[dk]) * state[dk][dv] + k[dk] * v[dv]
//   o[dv]             = scale * sum_dk q[dk] * new_state[dk][dv]
// (golden_gla_decode, tileops/kernels/linear_attention/gla_decode/
// gla_decode_kernel/_gla_decode_kernel.py:211-218): fp32 arithmetic, the
// readout taken from the fp32 new state, both outputs rounded once.
//
// One workgroup per (b, h): the state streams through once (read, update,
// write), so the kernel is bound by HBM traffic on the state.  A thread owns
// VEC consecutive value columns (16 bytes when the row allows it) of rows
// rg, rg + RG, ...; consecutive threads cover a row left to right, so every
// wavefront reads and writes whole contiguous rows.  The readout partial
// sums of the RG row groups meet in LDS.
#include "common.h"

namespace tileops {
namespace gla {

constexpr int kThreads = 256;

template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void gla_decode_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ gk, const T* __restrict__ state, T* __restrict__ o,
    T* __restrict__ new_state, int DK, int DV, float scale) {
  __shared__ float red[kThreads * VEC];  // [RG][CG * VEC] readout partials
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x;
  const int CG = DV / VEC;       // column groups per row (host: CG <= kThreads)
  const int RG = kThreads / CG;  // row groups
  const int cg = tid % CG, rg = tid / CG;
  const bool active = rg < RG;
  const T* S = state + bh * DK * DV;
  T* NS = new_state + bh * DK * DV;
  const T* qh = q + bh * DK;
  const T* kh = k + bh * DK;
  const T* gh = gk + bh * DK;

  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
  if (active) {
    float vv[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) vv[e] = Elem<T>::to_f32(v[bh * DV + cg * VEC + e]);
    // unrolled so that several rows' loads are in flight per thread
#pragma unroll 4
    for (int dk = rg; dk < DK; dk += RG) {
      const float decay = expf(Elem<T>::to_f32(gh[dk]));
      const float kd = Elem<T>::to_f32(kh[dk]), qd = Elem<T>::to_f32(qh[dk]);
      const int64_t off = (int64_t)dk * DV + cg * VEC;
      T in[VEC], out[VEC];
      if constexpr (VEC * sizeof(T) == 16) {
        *reinterpret_cast<u32x4*>(in) = *reinterpret_cast<const u32x4*>(S + off);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) in[e] = S[off + e];
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float ns = fmaf(decay, Elem<T>::to_f32(in[e]), kd * vv[e]);
        acc[e] = fmaf(qd, ns, acc[e]);
        out[e] = Elem<T>::from_f32(ns);
      }
      if constexpr (VEC * sizeof(T) == 16) {
        *reinterpret_cast<u32x4*>(NS + off) = *reinterpret_cast<const u32x4*>(out);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) NS[off + e] = out[e];
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[rg * DV + cg * VEC + e] = acc[e];
  }
  __syncthreads();
  // column c of the readout: thread c sums the RG partials
  for (int c = tid; c < DV; c += kThreads) {
    float sum = 0.0f;
    for (int r = 0; r < RG; ++r) sum += red[r * DV + c];
    o[bh * DV + c] = Elem<T>::from_f32(scale * sum);
  }
}

template <typename T, int VEC>
static void launch(const void* q, const void* k, const void* v, const void* gk, const void* state,
                   void* o, void* ns, int64_t BH, int DK, int DV, float scale, hipStream_t s) {
  gla_decode_kernel<T, VEC><<<dim3((unsigned)BH), dim3(kThreads), 0, s>>>(
      static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
      static_cast<const T*>(gk), static_cast<const T*>(state), static_cast<T*>(o),
      static_cast<T*>(ns), DK, DV, scale);
}

// 16-byte column groups when the rows and both state buffers allow them,
// single elements otherwise
template <typename T>
static int dispatch(const void* q, const void* k, const void* v, const void* gk,
                    const void* state, void* o, void* ns, int64_t BH, int DK, int DV, float scale,
                    hipStream_t s) {
  constexpr int V16 = 16 / sizeof(T);
  if (DV % V16 == 0 && DV / V16 <= kThreads && host_aligned16(state) && host_aligned16(ns))
    launch<T, V16>(q, k, v, gk, state, o, ns, BH, DK, DV, scale, s);
  else if (DV <= kThreads)
    launch<T, 1>(q, k, v, gk, state, o, ns, BH, DK, DV, scale, s);
  else
    return TILEOPS_ESHAPE;
  return launch_status();
}

}  // namespace gla
}  // namespace tileops

using namespace tileops;

extern "C" int tileops_gla_decode_fwd(const void* q, const void* k, const void* v,
                                      const void* gk, const void* state, void* o,
                                      void* new_state, int64_t B, int64_t H, int64_t DK,
                                      int64_t DV, float scale, int dtype, void* stream) {
  if (B <= 0 || H <= 0 || DK <= 0 || DV <= 0) return TILEOPS_ESHAPE;
  if (DK > INT32_MAX / DV || B * H > (int64_t)UINT32_MAX) return TILEOPS_ESHAPE;
  if (!(scale > 0.0f) || !(scale < INFINITY)) return TILEOPS_EINVAL;
  if (!q || !k || !v || !gk || !state || !o || !new_state) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t BH = B * H;
  switch (dtype) {
    case TILEOPS_F32:
      return gla::dispatch<float>(q, k, v, gk, state, o, new_state, BH, (int)DK, (int)DV, scale, s);
    case TILEOPS_F16:
      return gla::dispatch<f16>(q, k, v, gk, state, o, new_state, BH, (int)DK, (int)DV, scale, s);
    case TILEOPS_BF16:
      return gla::dispatch<bf16>(q, k, v, gk, state, o, new_state, BH, (int)DK, (int)DV, scale, s);
  }
  return TILEOPS_EINVAL;
}
