// Single-token gated linear attention decode for gfx950 (tileops_gla_decode_fwd).
//
// Per (batch b, head h), layout BHD, state [DK][DV]:
//   new_state[dk][dv] = exp(gk[dk]) * state[dk][dv] + k[dk] * v[dv]
//   o[dv]             = scale * sum_dk q[dk] * new_state[dk][dv]
// (golden_gla_decode, tileops/kernels/linear_attention/gla_decode/
// gla_decode_kernel/_gla_decode_kernel.py:211-218): fp32 arithmetic, the
// readout taken from the fp32 new state, both outputs rounded once.
//
// The state streams through once (read, update, write), so the kernel is
// bound by HBM traffic on the state.  Two kernels:
// - gla_decode_rows_kernel (16-byte packs, the common shapes): a workgroup
//   takes CG packs of every row of one (b, h) (a whole 256-byte row of a
//   128-wide bf16 head, or 16-pack slices of wider rows); thread (rg, cg)
//   issues the loads of all its RPT rows before anything else, exp(gk), k
//   and q are formed once per row in LDS, the new state goes out by
//   non-temporal stores, and the readout partials meet by lane swaps and
//   LDS.  The state loads are plain up to 128 MiB of state (a state read
//   again soon may then hit in the Infinity Cache; a cold one costs 2-5 %
//   against non-temporal loads) and non-temporal beyond.  Measured against
//   the general kernel below at B8 H64 / B8 H32, bf16 K = V = 128, state
//   cold: 7.13 / 4.73 us against 8.76 / 6.31 (back-to-back launches).
// - gla_decode_kernel (any shape): one workgroup per (b, h); a thread owns
//   VEC consecutive value columns (16 bytes when the row allows it) of rows
//   rg, rg + RG, ...; consecutive threads cover a row left to right, so
//   every wavefront reads and writes whole contiguous rows.  The readout
//   partial sums of the RG row groups meet in LDS.
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

// CG 16-byte packs per row slice, RPT rows per thread (DK = RPT * 256 / CG);
// NTL: non-temporal state loads (a template parameter: the compiler merges a
// runtime choice between the two load forms into plain loads)
template <typename T, int CG, int RPT, bool NTL>
__global__ __launch_bounds__(kThreads) void gla_decode_rows_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ gk, const T* __restrict__ state, T* __restrict__ o,
    T* __restrict__ new_state, int DV, float scale) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int RG = kThreads / CG;  // row groups
  constexpr int DK = RPT * RG;
  constexpr int NW = kThreads / 64;
  static_assert(CG == 4 || CG == 8 || CG == 16, "row slices of 4, 8 or 16 packs");
  __shared__ float dec[DK], ks[DK], qs[DK];
  __shared__ float part[NW][CG][VEC];
  const int wph = DV / (VEC * CG);  // workgroups per head
  const int64_t bh = blockIdx.x / wph;
  const int c0 = (int)(blockIdx.x % wph) * VEC * CG;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = tid % CG, rg = tid / CG;

  const T* S = state + bh * DK * DV + c0 + VEC * cg;
  u32x4 sv[RPT];
  if constexpr (NTL) {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      sv[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(S + (int64_t)(rg + RG * i) * DV));
  } else {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      sv[i] = *reinterpret_cast<const u32x4*>(S + (int64_t)(rg + RG * i) * DV);
  }
  for (int r = tid; r < DK; r += kThreads) {
    dec[r] = expf(Elem<T>::to_f32(gk[bh * DK + r]));
    ks[r] = Elem<T>::to_f32(k[bh * DK + r]);
    qs[r] = Elem<T>::to_f32(q[bh * DK + r]);
  }
  float vv[VEC];
  {
    const Pack<T> vp = load_pack(v + bh * DV + c0 + VEC * cg);
#pragma unroll
    for (int e = 0; e < VEC; ++e) vv[e] = Elem<T>::to_f32(vp.v[e]);
  }
  __syncthreads();  // dec, ks, qs written
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
  T* NS = new_state + bh * DK * DV + c0 + VEC * cg;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = rg + RG * i;
    const float d = dec[r], kd = ks[r], qd = qs[r];
    const Pack<T> in = *reinterpret_cast<const Pack<T>*>(&sv[i]);
    Pack<T> out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float ns = fmaf(d, Elem<T>::to_f32(in.v[e]), kd * vv[e]);
      acc[e] = fmaf(qd, ns, acc[e]);
      out.v[e] = Elem<T>::from_f32(ns);
    }
    store_pack_nt(NS + (int64_t)r * DV, out);
  }
  // the row groups of a wavefront (lanes CG apart), then the wavefronts
  // through LDS
#pragma unroll
  for (int m = CG; m <= 32; m <<= 1) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], m);
  }
  if (lane < CG) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) part[wave][lane][e] = acc[e];
  }
  __syncthreads();
  if (rg == 0) {
    Pack<T> out;
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      out.v[e] = Elem<T>::from_f32(
          scale * ((part[0][cg][e] + part[1][cg][e]) + (part[2][cg][e] + part[3][cg][e])));
    *reinterpret_cast<Pack<T>*>(o + bh * DV + c0 + VEC * cg) = out;
  }
}

template <typename T, int CG, int RPT>
static void launch_rows(const void* q, const void* k, const void* v, const void* gk,
                        const void* state, void* o, void* ns, int64_t nblk, int DV, float scale,
                        bool stream_in, hipStream_t s) {
  const T *qt = static_cast<const T*>(q), *kt = static_cast<const T*>(k);
  const T *vt = static_cast<const T*>(v), *gt = static_cast<const T*>(gk);
  const T* st = static_cast<const T*>(state);
  T *ot = static_cast<T*>(o), *nt = static_cast<T*>(ns);
  if (stream_in)
    gla_decode_rows_kernel<T, CG, RPT, true><<<dim3((unsigned)nblk), dim3(kThreads), 0, s>>>(
        qt, kt, vt, gt, st, ot, nt, DV, scale);
  else
    gla_decode_rows_kernel<T, CG, RPT, false><<<dim3((unsigned)nblk), dim3(kThreads), 0, s>>>(
        qt, kt, vt, gt, st, ot, nt, DV, scale);
}

// The rows kernel where the shape allows it: 16-byte packs, a row slice of
// 4, 8 or 16 packs that tiles the row, K a power-of-two multiple (1 .. 16)
// of the row groups; false otherwise.
template <typename T, int CG>
static bool try_rows(const void* q, const void* k, const void* v, const void* gk,
                     const void* state, void* o, void* ns, int64_t BH, int DK, int DV, float scale,
                     hipStream_t s) {
  constexpr int VEC = 16 / sizeof(T), RG = kThreads / CG;
  if (DK % RG != 0) return false;
  const int64_t nblk = BH * (DV / (VEC * CG));
  if (nblk > INT32_MAX) return false;
  const bool si = BH * DK * DV * (int64_t)sizeof(T) > kCacheFitBytes;
  switch (DK / RG) {
    case 1: launch_rows<T, CG, 1>(q, k, v, gk, state, o, ns, nblk, DV, scale, si, s); return true;
    case 2: launch_rows<T, CG, 2>(q, k, v, gk, state, o, ns, nblk, DV, scale, si, s); return true;
    case 4: launch_rows<T, CG, 4>(q, k, v, gk, state, o, ns, nblk, DV, scale, si, s); return true;
    case 8: launch_rows<T, CG, 8>(q, k, v, gk, state, o, ns, nblk, DV, scale, si, s); return true;
    case 16: launch_rows<T, CG, 16>(q, k, v, gk, state, o, ns, nblk, DV, scale, si, s); return true;
  }
  return false;
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
  const bool packs = DV % V16 == 0 && host_aligned16(state) && host_aligned16(ns) &&
                     host_aligned16(v) && host_aligned16(o);
  if (packs) {
    const int np = DV / V16;  // packs per row
    bool done = false;
    if (np % 16 == 0)
      done = try_rows<T, 16>(q, k, v, gk, state, o, ns, BH, DK, DV, scale, s);
    else if (np == 8)
      done = try_rows<T, 8>(q, k, v, gk, state, o, ns, BH, DK, DV, scale, s);
    else if (np == 4)
      done = try_rows<T, 4>(q, k, v, gk, state, o, ns, BH, DK, DV, scale, s);
    if (done) return launch_status();
  }
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
