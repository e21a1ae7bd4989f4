// Fused residual add + LayerNorm for gfx950 (tileops_fused_add_layernorm_fwd).
//
// Semantics follow FusedAddLayerNormFwdOp's reference program
// (tests/ops/test_fused_add_layer_norm.py:55-72):
//   r_out = round_T(x + residual)                  stored as T
//   y     = round_T((r_out - mean) * rstd * w + b)  mean/var of the *rounded* sum,
//                                                   biased variance, fp32 math
//
// Fast path (N % pack == 0, 16-byte aligned rows, a row fits in 16 packs per
// lane): one wavefront per row, the two row statistics are wavefront
// butterflies, w / b are staged once per workgroup into LDS as fp32 so that
// the HBM stream is only x, residual in and y, r_out out.
// Long rows (up to 32 packs per lane of a wavefront): one 256-lane
// workgroup per row, the row in registers, workgroup reductions.
// Fallback (any N or alignment): grid-stride workgroups, three passes over
// global memory.
#include "common.h"

namespace tileops {

template <typename W>
__device__ __forceinline__ float wload(const W* p, int64_t i) {
  return Elem<W>::to_f32(p[i]);
}

// w / b into LDS as fp32 by the whole workgroup (NT threads).  With 16-byte
// loads (vec: both 16-byte aligned, N a multiple of the pack) the first
// SB * NT packs of each come from one batch of loads issued by stage_fetch
// before the caller's row loads, so that their wait in stage_store does not
// also wait for the row data behind them; longer rows finish in a loop.
template <typename W>
struct ParamBatch {
  static constexpr int SB = 4;
  Pack<W> w[SB], b[SB];
};

template <typename W, int NT>
__device__ __forceinline__ void stage_fetch(ParamBatch<W>& pb, const W* w, const W* b, int N,
                                            bool vec) {
  constexpr int PV = 16 / sizeof(W);
  if (!vec) return;
  const int nv = N / PV;
#pragma unroll
  for (int j = 0; j < ParamBatch<W>::SB; ++j) {
    const int i = min((int)threadIdx.x + j * NT, nv - 1);
    pb.w[j] = *reinterpret_cast<const Pack<W>*>(w + (int64_t)i * PV);
    pb.b[j] = *reinterpret_cast<const Pack<W>*>(b + (int64_t)i * PV);
  }
}

template <typename W>
__device__ __forceinline__ void put_pack(float* dst, const Pack<W>& p) {
  constexpr int PV = 16 / sizeof(W);
#pragma unroll
  for (int e = 0; e < PV; e += 4)
    *reinterpret_cast<float4*>(dst + e) =
        make_float4(Elem<W>::to_f32(p.v[e]), Elem<W>::to_f32(p.v[e + 1]),
                    Elem<W>::to_f32(p.v[e + 2]), Elem<W>::to_f32(p.v[e + 3]));
}

template <typename W, int NT>
__device__ __forceinline__ void stage_store(const ParamBatch<W>& pb, float* sw, float* sb,
                                            const W* w, const W* b, int N, bool vec) {
  constexpr int PV = 16 / sizeof(W);
  constexpr int SB = ParamBatch<W>::SB;
  if (vec) {
    const int nv = N / PV;
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int i = threadIdx.x + j * NT;
      if (i < nv) {
        put_pack<W>(sw + i * PV, pb.w[j]);
        put_pack<W>(sb + i * PV, pb.b[j]);
      }
    }
    for (int i = threadIdx.x + SB * NT; i < nv; i += NT) {
      put_pack<W>(sw + i * PV, *reinterpret_cast<const Pack<W>*>(w + (int64_t)i * PV));
      put_pack<W>(sb + i * PV, *reinterpret_cast<const Pack<W>*>(b + (int64_t)i * PV));
    }
  } else {
    for (int i = threadIdx.x; i < N; i += NT) {
      sw[i] = wload(w, i);
      sb[i] = wload(b, i);
    }
  }
}

// One wavefront per row, WPB rows per workgroup (one-shot grid).  The
// workgroup stages w / b into LDS (fp32), then each lane loads its KP packs
// of x and residual; the rounded sum stays in registers in the storage type
// (exactly representable, so nothing is lost).
template <typename T, typename W, int KP, int WPB>
__global__ __launch_bounds__(WPB * 64) void fused_add_ln_wave_kernel(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    const W* __restrict__ b, T* __restrict__ y, T* __restrict__ rout, int64_t M, int N,
    float eps, bool vec_params) {
  constexpr int V = Elem<T>::kVec;
  extern __shared__ float smem[];  // w[N] then b[N], fp32
  float* sw = smem;
  float* sb = smem + N;
  const int lane = threadIdx.x & 63;
  const int npack = N / V;
  const int64_t row = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6);
  const bool live = row < M;

  // Parameter loads, then the row loads, then the parameters into LDS: the
  // two streams overlap.  Every lane loads all KP packs, past-the-end ones
  // clamped onto the row's last pack, so the loads are one uniform sequence
  // the compiler can wait on one at a time; lanes mask those packs out of
  // the sums and the stores.
  ParamBatch<W> pb;
  stage_fetch<W, WPB * 64>(pb, w, b, N, vec_params);
  Pack<T> xs[KP], rs[KP];
  const int64_t rowc = live ? row : M - 1;  // dead waves load a live row
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const int p = min(k * 64 + lane, npack - 1);
    xs[k] = load_pack_nt(x + rowc * N + (int64_t)p * V);
    rs[k] = load_pack_nt(res + rowc * N + (int64_t)p * V);
  }
  stage_store<W, WPB * 64>(pb, sw, sb, w, b, N, vec_params);
  __syncthreads();
  if (!live) return;

  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const int p = k * 64 + lane;
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const T s = Elem<T>::from_f32(Elem<T>::to_f32(xs[k].v[e]) + Elem<T>::to_f32(rs[k].v[e]));
      xs[k].v[e] = s;
      part += Elem<T>::to_f32(s);
    }
    if (p < npack) {
      sum += part;
      store_pack_nt(rout + row * N + (int64_t)p * V, xs[k]);
    }
  }
  const float inv_n = 1.0f / (float)N;
  const float mean = wave_sum(sum) * inv_n;
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float d = Elem<T>::to_f32(xs[k].v[e]) - mean;
      part = fmaf(d, d, part);
    }
    if (k * 64 + lane < npack) sq += part;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) * inv_n + eps);
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const int p = k * 64 + lane;
    if (p < npack) {
      // N is a multiple of the pack (>= 4 elements) on this path, so both
      // parameter rows and every lane's slice of them are 16-byte aligned
      float wv[V], bv[V];
#pragma unroll
      for (int e = 0; e < V; e += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(sw + p * V + e);
        const float4 b4 = *reinterpret_cast<const float4*>(sb + p * V + e);
        wv[e] = w4.x; wv[e + 1] = w4.y; wv[e + 2] = w4.z; wv[e + 3] = w4.w;
        bv[e] = b4.x; bv[e + 1] = b4.y; bv[e + 2] = b4.z; bv[e + 3] = b4.w;
      }
      Pack<T> o;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float d = Elem<T>::to_f32(xs[k].v[e]) - mean;
        o.v[e] = Elem<T>::from_f32(fmaf(d * rstd, wv[e], bv[e]));
      }
      store_pack_nt(y + row * N + (int64_t)p * V, o);
    }
  }
}

// w[i..i+V) and b[i..i+V) as fp32: 16-byte loads when both are 16-byte
// aligned and N is a multiple of their pack (V is a multiple of it, since W
// is never narrower than T), else element loads.
template <typename T, typename W>
__device__ __forceinline__ void load_params(const W* w, const W* b, int64_t i, bool vec,
                                            float (&wv)[Elem<T>::kVec],
                                            float (&bv)[Elem<T>::kVec]) {
  constexpr int V = Elem<T>::kVec;
  constexpr int PV = 16 / sizeof(W);
  if (vec) {
#pragma unroll
    for (int j = 0; j < V; j += PV) {
      const Pack<W> w4 = *reinterpret_cast<const Pack<W>*>(w + i + j);
      const Pack<W> b4 = *reinterpret_cast<const Pack<W>*>(b + i + j);
#pragma unroll
      for (int e = 0; e < PV; ++e) {
        wv[j + e] = Elem<W>::to_f32(w4.v[e]);
        bv[j + e] = Elem<W>::to_f32(b4.v[e]);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < V; ++e) {
      wv[e] = wload(w, i + e);
      bv[e] = wload(b, i + e);
    }
  }
}

// Sum of v over the 256-lane workgroup (four wavefronts); every lane gets it.
__device__ __forceinline__ float block_sum4(float v, float* part) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  const float t = (part[0] + part[1]) + (part[2] + part[3]);
  __syncthreads();
  return t;
}

// Long rows (1024 < packs <= 2048: fp32 N <= 8192, 16-bit N <= 16384): one
// 256-lane workgroup per row, KP packs per lane held in registers, so the
// rounded sum is never re-read from memory (the three-pass kernel re-reads
// r_out twice, and at thousands of rows in flight those re-reads miss L2).
// w / b come straight from global memory (L2-resident across rows).
template <typename T, typename W, int KP>
__global__ __launch_bounds__(256) void fused_add_ln_block_kernel(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    const W* __restrict__ b, T* __restrict__ y, T* __restrict__ rout, int N, float eps,
    bool vec_params) {
  constexpr int V = Elem<T>::kVec;
  __shared__ float part[4];
  const int npack = N / V;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * N;
  const T* rr = res + row * N;
  // every lane loads all KP packs, past-the-end ones clamped onto the row's
  // last pack (one uniform load sequence); they are masked out below
  Pack<T> xs[KP], rs[KP];
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const int p = min(k * 256 + (int)threadIdx.x, npack - 1);
    xs[k] = load_pack_nt(xr + (int64_t)p * V);
    rs[k] = load_pack_nt(rr + (int64_t)p * V);
  }
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const int p = k * 256 + threadIdx.x;
    float s_part = 0.0f;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const T s = Elem<T>::from_f32(Elem<T>::to_f32(xs[k].v[e]) + Elem<T>::to_f32(rs[k].v[e]));
      xs[k].v[e] = s;
      s_part += Elem<T>::to_f32(s);
    }
    if (p < npack) {
      sum += s_part;
      store_pack_nt(rout + row * N + (int64_t)p * V, xs[k]);
    }
  }
  const float inv_n = 1.0f / (float)N;
  const float mean = block_sum4(sum, part) * inv_n;
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    float q_part = 0.0f;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float d = Elem<T>::to_f32(xs[k].v[e]) - mean;
      q_part = fmaf(d, d, q_part);
    }
    if (k * 256 + (int)threadIdx.x < npack) sq += q_part;
  }
  const float rstd = 1.0f / sqrtf(block_sum4(sq, part) * inv_n + eps);
#pragma unroll
  for (int k = 0; k < KP; ++k) {
    const int p = k * 256 + threadIdx.x;
    if (p < npack) {
      float wv[V], bv[V];
      load_params<T, W>(w, b, (int64_t)p * V, vec_params, wv, bv);
      Pack<T> o;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float d = Elem<T>::to_f32(xs[k].v[e]) - mean;
        o.v[e] = Elem<T>::from_f32(fmaf(d * rstd, wv[e], bv[e]));
      }
      store_pack_nt(y + row * N + (int64_t)p * V, o);
    }
  }
}

// General rows: any N, any alignment.  Pass 1 writes r_out and sums it,
// pass 2 re-reads r_out (L2-resident for one row) for the variance, pass 3
// normalises.
template <typename T, typename W>
__global__ __launch_bounds__(256) void fused_add_ln_generic_kernel(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    const W* __restrict__ b, T* __restrict__ y, T* __restrict__ rout, int64_t M, int64_t N,
    float eps) {
  __shared__ float part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int64_t row = blockIdx.x; row < M; row += gridDim.x) {
    const T* xr = x + row * N;
    const T* rr = res + row * N;
    T* orow = rout + row * N;
    float sum = 0.0f;
    for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
      const T s = Elem<T>::from_f32(Elem<T>::to_f32(xr[j]) + Elem<T>::to_f32(rr[j]));
      orow[j] = s;
      sum += Elem<T>::to_f32(s);
    }
    sum = wave_sum(sum);
    if (lane == 0) part[wave] = sum;
    __syncthreads();
    const float mean = (part[0] + part[1] + part[2] + part[3]) / (float)N;
    __syncthreads();
    float sq = 0.0f;
    for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
      const float d = Elem<T>::to_f32(orow[j]) - mean;
      sq = fmaf(d, d, sq);
    }
    sq = wave_sum(sq);
    if (lane == 0) part[wave] = sq;
    __syncthreads();
    const float var = (part[0] + part[1] + part[2] + part[3]) / (float)N;
    __syncthreads();
    const float rstd = 1.0f / sqrtf(var + eps);
    for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
      const float d = Elem<T>::to_f32(orow[j]) - mean;
      y[row * N + j] = Elem<T>::from_f32(fmaf(d * rstd, wload(w, j), wload(b, j)));
    }
  }
}

// One-shot grid of 4-wavefront workgroups (measured best on MI355X among
// 4 / 8 / 16 wavefronts per workgroup and workgroup-per-row variants).
template <typename T, typename W, int KP>
static void launch_wave(const T* x, const T* r, const W* w, const W* b, T* y, T* ro, int64_t M,
                        int N, float eps, hipStream_t s) {
  constexpr int WPB = 4;
  const size_t lds = (size_t)N * 2 * sizeof(float);
  const int64_t blocks = (M + WPB - 1) / WPB;
  const bool vec = N % (16 / (int)sizeof(W)) == 0 && host_aligned16(w) && host_aligned16(b);
  fused_add_ln_wave_kernel<T, W, KP, WPB><<<dim3((unsigned)blocks), dim3(WPB * 64), lds, s>>>(
      x, r, w, b, y, ro, M, N, eps, vec);
}

template <typename T, typename W>
static int launch_fused_add_ln(const void* xv, const void* rv, const void* wv, const void* bv,
                               void* yv, void* rov, int64_t M, int64_t N, float eps,
                               hipStream_t s) {
  constexpr int V = Elem<T>::kVec;
  const T* x = static_cast<const T*>(xv);
  const T* r = static_cast<const T*>(rv);
  const W* w = static_cast<const W*>(wv);
  const W* b = static_cast<const W*>(bv);
  T* y = static_cast<T*>(yv);
  T* ro = static_cast<T*>(rov);
  const bool packable = N % V == 0 && host_aligned16(x) && host_aligned16(r) &&
                        host_aligned16(y) && host_aligned16(ro);
  const int64_t lane_packs = (N / V + 63) / 64;
  // grid x dimension times block size stays within 32 bits on both fast paths
  if (packable && lane_packs <= 16 && M <= (int64_t)(UINT32_MAX / 64)) {
    const int n = (int)N;
    if (lane_packs <= 1) launch_wave<T, W, 1>(x, r, w, b, y, ro, M, n, eps, s);
    else if (lane_packs <= 2) launch_wave<T, W, 2>(x, r, w, b, y, ro, M, n, eps, s);
    else if (lane_packs <= 4) launch_wave<T, W, 4>(x, r, w, b, y, ro, M, n, eps, s);
    else if (lane_packs <= 8) launch_wave<T, W, 8>(x, r, w, b, y, ro, M, n, eps, s);
    else launch_wave<T, W, 16>(x, r, w, b, y, ro, M, n, eps, s);
  } else if (packable && lane_packs <= 32 && M <= (int64_t)(UINT32_MAX / 256)) {
    // 1024 < N / V <= 2048: KP = ceil(packs / 256) in 5..8
    const int n = (int)N;
    const int kp = (int)((N / V + 255) / 256);
    constexpr int PV = 16 / (int)sizeof(W);
    const bool vec = N % PV == 0 && host_aligned16(w) && host_aligned16(b);
    const dim3 grid((unsigned)M), block(256);
    if (kp <= 5) fused_add_ln_block_kernel<T, W, 5><<<grid, block, 0, s>>>(x, r, w, b, y, ro, n, eps, vec);
    else if (kp == 6) fused_add_ln_block_kernel<T, W, 6><<<grid, block, 0, s>>>(x, r, w, b, y, ro, n, eps, vec);
    else if (kp == 7) fused_add_ln_block_kernel<T, W, 7><<<grid, block, 0, s>>>(x, r, w, b, y, ro, n, eps, vec);
    else fused_add_ln_block_kernel<T, W, 8><<<grid, block, 0, s>>>(x, r, w, b, y, ro, n, eps, vec);
  } else {
    int64_t blocks = M < 256 * 16 ? M : 256 * 16;
    fused_add_ln_generic_kernel<T, W><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(x, r, w, b, y,
                                                                                  ro, M, N, eps);
  }
  return launch_status();
}

template <typename T>
static int dispatch_ln_w(const void* x, const void* r, const void* w, const void* b, void* y,
                         void* ro, int64_t M, int64_t N, float eps, int wdtype, hipStream_t s) {
  if (wdtype == TILEOPS_F32) return launch_fused_add_ln<T, float>(x, r, w, b, y, ro, M, N, eps, s);
  return launch_fused_add_ln<T, T>(x, r, w, b, y, ro, M, N, eps, s);
}

}  // namespace tileops

using namespace tileops;

extern "C" int tileops_fused_add_layernorm_fwd(const void* x, const void* residual, const void* w,
                                               const void* b, void* y, void* r_out, int64_t M,
                                               int64_t N, float eps, int dtype, int wdtype,
                                               void* stream) {
  if (M < 0 || N <= 0 || N > INT32_MAX) return TILEOPS_ESHAPE;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (wdtype != dtype && wdtype != TILEOPS_F32) return TILEOPS_EINVAL;
  if (M == 0) return 0;
  if (!x || !residual || !w || !b || !y || !r_out) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TILEOPS_F32: return launch_fused_add_ln<float, float>(x, residual, w, b, y, r_out, M, N,
                                                              eps, s);
    case TILEOPS_F16: return dispatch_ln_w<f16>(x, residual, w, b, y, r_out, M, N, eps, wdtype, s);
    default: return dispatch_ln_w<bf16>(x, residual, w, b, y, r_out, M, N, eps, wdtype, s);
  }
}
