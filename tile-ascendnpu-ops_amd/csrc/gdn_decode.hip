// Single-token gated delta-rule (gated DeltaNet) decode step for gfx950
// (tileops_gdn_decode_fwd): the decode step beside the chunked prefill, on
// its state layout.
//
// Per (batch b, head h), state S [DK][DV] fp32:
//   S' = exp(g) S + k e^T,   e = beta (v - exp(g) S^T k)
//   o  = scale q^T S'
// (one token of golden_gdn_sequential, examples/gdn_prefill/probe/
// gdn_prefill_probe.py:60-77).  The readout is formed as
//   o = scale (exp(g) S^T q + (q . k) e)
// so that the state streams through once: every column of S' needs only
// the same column of S and the two column sums S^T k and S^T q, which the
// workgroup forms from the rows it holds in registers before it writes.
//
// A workgroup of 256 threads takes 4 CG value columns of one (b, h): thread
// (rg, cg) holds rows rg, rg + 256 / CG, .. of columns 4 cg .. 4 cg + 3 (one
// 16-byte pack per row), so each wavefront instruction reads or writes
// 64 / CG whole row pieces of 16 CG bytes.  CG is 16 (64 value columns,
// 256-byte row pieces, two workgroups per 128-wide value head) where the
// value width allows it, else 8: measured against whole 512-byte rows
// (CG = 32) it is 2-3 % faster on large batches and 20-27 % faster on
// small ones, whose heads alone do not fill the GPU.  The column sums
// meet by lane swaps inside a wavefront and LDS between the four.  The state
// is read and written once: non-temporal stores, and non-temporal loads when
// the state of the call exceeds what the Infinity Cache could keep (128 MiB;
// a smaller state read again soon may still be there).
// All reads of the state precede the barrier that all its writes follow, and
// each element is read and written by the same thread, so the new state may
// overwrite the old in place.
#include "common.h"

namespace tileops {
namespace gdnd {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxDK = 256;
constexpr int kMaxRPT = 16;  // state rows per thread (4 VGPRs each): DK / 16 at CG = 16

__device__ __forceinline__ f32x4 xor_sum4(f32x4 a, int mask) {
  a.x += __shfl_xor(a.x, mask);
  a.y += __shfl_xor(a.y, mask);
  a.z += __shfl_xor(a.z, mask);
  a.w += __shfl_xor(a.w, mask);
  return a;
}

// CG 16-byte column packs per row slice, RPT rows per thread (DK = RPT * 256 /
// CG); NTL: non-temporal state loads (a template parameter: the compiler
// merges a runtime choice between the two load forms into plain loads)
template <typename T, int CG, int RPT, bool NTL>
__global__ __launch_bounds__(kThreads) void gdn_decode_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta, const float* state, T* o,
    float* new_state, int DV, float scale) {
  constexpr int RG = kThreads / CG;  // row groups
  constexpr int DK = RPT * RG;
  static_assert(CG == 8 || CG == 16, "a row slice is 8 or 16 packs");
  __shared__ float qs[DK], ks[DK];
  __shared__ float qk_part[kWaves];
  __shared__ f32x4 part_u[kWaves][CG], part_w[kWaves][CG];
  const int wph = DV / (4 * CG);  // workgroups per head
  const int64_t bh = blockIdx.x / wph;
  const int c0 = (int)(blockIdx.x % wph) * 4 * CG;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = tid % CG, rg = tid / CG;

  // this thread's rows of its four columns, issued first (non-temporal
  // when the state is too large to stay in the caches)
  const float* S = state + bh * DK * DV + c0 + 4 * cg;
  f32x4 sv[RPT];
  if constexpr (NTL) {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      sv[i] = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4*>(S + (int64_t)(rg + RG * i) * DV));
  } else {
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      sv[i] = *reinterpret_cast<const f32x4*>(S + (int64_t)(rg + RG * i) * DV);
  }
  // q, k as fp32 in LDS, and q . k
  float qk = 0.0f;
  for (int r = tid; r < DK; r += kThreads) {
    const float qv = Elem<T>::to_f32(q[bh * DK + r]);
    const float kv = Elem<T>::to_f32(k[bh * DK + r]);
    qs[r] = qv;
    ks[r] = kv;
    qk = fmaf(qv, kv, qk);
  }
  qk = wave_sum(qk);
  if (lane == 0) qk_part[wave] = qk;
  __syncthreads();  // qs, ks, qk_part written
  f32x4 u = 0.0f, w = 0.0f;  // partial S^T k, S^T q
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = rg + RG * i;
    u += sv[i] * ks[r];
    w += sv[i] * qs[r];
  }
  // the row groups of a wavefront (lanes CG apart), then the wavefronts
  // through LDS
#pragma unroll
  for (int m = CG; m <= 32; m <<= 1) {
    u = xor_sum4(u, m);
    w = xor_sum4(w, m);
  }
  if (lane < CG) {
    part_u[wave][lane] = u;
    part_w[wave][lane] = w;
  }
  __syncthreads();
  u = (part_u[0][cg] + part_u[1][cg]) + (part_u[2][cg] + part_u[3][cg]);
  w = (part_w[0][cg] + part_w[1][cg]) + (part_w[2][cg] + part_w[3][cg]);
  const float qk_all = (qk_part[0] + qk_part[1]) + (qk_part[2] + qk_part[3]);
  const float eg = expf(g[bh]);
  const float bt = beta[bh];
  const T* vp = v + bh * DV + c0 + 4 * cg;
  const f32x4 vv = {Elem<T>::to_f32(vp[0]), Elem<T>::to_f32(vp[1]), Elem<T>::to_f32(vp[2]),
                    Elem<T>::to_f32(vp[3])};
  // e = beta (v - exp(g) S^T k)
  const f32x4 e = bt * (vv - eg * u);
  if (rg == 0) {
    const f32x4 r = scale * (eg * w + qk_all * e);
    T* op = o + bh * DV + c0 + 4 * cg;
    op[0] = Elem<T>::from_f32(r.x);
    op[1] = Elem<T>::from_f32(r.y);
    op[2] = Elem<T>::from_f32(r.z);
    op[3] = Elem<T>::from_f32(r.w);
  }
  // S' = exp(g) S + k e^T
  float* NS = new_state + bh * DK * DV + c0 + 4 * cg;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = rg + RG * i;
    __builtin_nontemporal_store(eg * sv[i] + ks[r] * e,
                                reinterpret_cast<f32x4*>(NS + (int64_t)r * DV));
  }
}

struct Launch {
  const void *q, *k, *v;
  const float *g, *beta, *state;
  void* o;
  float* new_state;
  int64_t BH;
  int DV;
  float scale;
  hipStream_t s;
};

// KB = DK / 32; rows per thread RPT = KB * CG / 8
// (false: no instantiation for these rows per thread; pick_cg never asks for one)
template <typename T, int CG, int KB>
static bool launch(const Launch& L) {
  if constexpr (KB * CG / 8 <= kMaxRPT) {
    const dim3 grid((unsigned)(L.BH * (L.DV / (4 * CG)))), block(kThreads);
    const T* q = static_cast<const T*>(L.q);
    const T* k = static_cast<const T*>(L.k);
    const T* v = static_cast<const T*>(L.v);
    T* o = static_cast<T*>(L.o);
    if (L.BH * (32 * KB) * L.DV * 4 > kCacheFitBytes)
      gdn_decode_kernel<T, CG, KB * CG / 8, true><<<grid, block, 0, L.s>>>(
          q, k, v, L.g, L.beta, L.state, o, L.new_state, L.DV, L.scale);
    else
      gdn_decode_kernel<T, CG, KB * CG / 8, false><<<grid, block, 0, L.s>>>(
          q, k, v, L.g, L.beta, L.state, o, L.new_state, L.DV, L.scale);
    return true;
  } else {
    return false;
  }
}

template <typename T, int CG>
static bool launch_kb(int kb, const Launch& L) {
  switch (kb) {
    case 1: return launch<T, CG, 1>(L);
    case 2: return launch<T, CG, 2>(L);
    case 3: return launch<T, CG, 3>(L);
    case 4: return launch<T, CG, 4>(L);
    case 5: return launch<T, CG, 5>(L);
    case 6: return launch<T, CG, 6>(L);
    case 7: return launch<T, CG, 7>(L);
    case 8: return launch<T, CG, 8>(L);
    default: return false;
  }
}

// 16 packs of 4 columns where they divide DV, else 8 (DV is a multiple of 32)
inline int pick_cg(int DV) { return DV % 64 == 0 ? 16 : 8; }

template <typename T>
static int dispatch(const Launch& L, int DK) {
  const int kb = DK / 32;
  bool ok;
  switch (pick_cg(L.DV)) {
    case 16: ok = launch_kb<T, 16>(kb, L); break;
    default: ok = launch_kb<T, 8>(kb, L); break;
  }
  return ok ? launch_status() : TILEOPS_ESHAPE;
}

}  // namespace gdnd
}  // namespace tileops

using namespace tileops;

extern "C" int tileops_gdn_decode_fwd(const void* q, const void* k, const void* v, const float* g,
                                      const float* beta, const float* state, void* o,
                                      float* new_state, int64_t B, int64_t H, int64_t DK,
                                      int64_t DV, float scale, int dtype, void* stream) {
  if (B <= 0 || H <= 0 || B > INT32_MAX || H > INT32_MAX) return TILEOPS_ESHAPE;
  if (DK <= 0 || DK % 32 != 0 || DK > gdnd::kMaxDK || DV <= 0 || DV % 32 != 0 || DV > 4096)
    return TILEOPS_ESHAPE;
  if (B * H > INT32_MAX / (DV / 32)) return TILEOPS_ESHAPE;  // grid size
  if (!(scale > -INFINITY && scale < INFINITY)) return TILEOPS_EINVAL;  // NaN too
  if (!q || !k || !v || !g || !beta || !state || !o || !new_state) return TILEOPS_ENULL;
  if (!host_aligned16(state) || !host_aligned16(new_state)) return TILEOPS_EINVAL;
  const gdnd::Launch L{q, k, v, g, beta, state, o, new_state, B * H, (int)DV, scale,
                       static_cast<hipStream_t>(stream)};
  switch (dtype) {
    case TILEOPS_BF16:
      return gdnd::dispatch<bf16>(L, (int)DK);
    case TILEOPS_F16:
      return gdnd::dispatch<f16>(L, (int)DK);
    case TILEOPS_F32:
      return gdnd::dispatch<float>(L, (int)DK);
    default:
      return TILEOPS_EINVAL;
  }
}
