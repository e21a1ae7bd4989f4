// Row reductions for gfx950: LogSumExp and Argmax / Argmin over the last
// dimension of a row-major [M, N] tensor.
//
// Work split: a wavefront owns a row (WPR = 1, four rows per 256-thread
// workgroup) when there are enough rows to fill the chip; otherwise the four
// wavefronts of a workgroup share one row (WPR = 4) and meet in LDS.  Inside
// a wavefront every lane streams 16-byte packs (64 lanes x one pack = one
// contiguous "chunk" of the row), keeps UNROLL packs in flight, folds them
// into a per-lane partial, and the 64 partials meet in a shuffle butterfly.
#include <float.h>

#include "common.h"

namespace tileops {

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// LogSumExp: online (max, scaled-sum) per lane.
//
// m is the running max of everything folded so far (NaN never wins the
// compare, so m stays in [-inf, +inf]); s = sum exp(x - shift(m)) where
// shift(m) = m for a finite max and 0 for an infinite one, as torch does.
// That reproduces torch.logsumexp's special cases and keeps every finite
// max up to FLT_MAX finite:
//   all -inf    -> shift 0, s = 0, log 0 + 0 = -inf
//   any +inf    -> shift 0, exp(+inf) = +inf in s   (result +inf)
//   any NaN     -> NaN enters s                     (result NaN)
// s == 0 exactly when m == -inf (a finite max contributes exp(0) = 1), and
// such a sum is rescaled to 0 without evaluating a factor that could be
// exp(+huge) = inf (0 * inf would be NaN).
// ---------------------------------------------------------------------------
struct LseState {
  float m;  // running max, -inf while nothing finite or +inf was folded
  float s;  // sum of exp(x - lse_shift(m))
};

__device__ __forceinline__ float lse_shift(float m) {
  return __builtin_fabsf(m) <= FLT_MAX ? m : 0.0f;
}

// s, taken relative to shift `from`, re-expressed relative to shift `to`.
__device__ __forceinline__ float lse_rescale(float s, float from, float to) {
  const float f = __builtin_amdgcn_exp2f((from - to) * kLog2e);
  return s == 0.0f ? 0.0f : s * f;
}

__device__ __forceinline__ LseState lse_merge(LseState a, LseState b) {
  const float m = a.m > b.m ? a.m : b.m;
  const float sh = lse_shift(m);
  return {m, lse_rescale(a.s, lse_shift(a.m), sh) + lse_rescale(b.s, lse_shift(b.m), sh)};
}

template <int CNT>
__device__ __forceinline__ void lse_fold(LseState& st, const float (&v)[CNT]) {
  float bm = v[0];
#pragma unroll
  for (int i = 1; i < CNT; ++i) bm = v[i] > bm ? v[i] : bm;
  const float mn = bm > st.m ? bm : st.m;
  const float sh = lse_shift(mn);
  // exp(x - m) as exp2((x - m) * log2 e): subtracting first keeps the
  // exponent exact for large |m| (an fma(x, log2 e, -m log2 e) would leave
  // the rounding residue of m log2 e, ~1e31 at |m| ~ 1e38).
  float acc = lse_rescale(st.s, lse_shift(st.m), sh);
#pragma unroll
  for (int i = 0; i < CNT; ++i) acc += __builtin_amdgcn_exp2f((v[i] - sh) * kLog2e);
  st.m = mn;
  st.s = acc;
}

__device__ __forceinline__ LseState lse_wave(LseState st) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    LseState other{__shfl_xor(st.m, o, 64), __shfl_xor(st.s, o, 64)};
    st = lse_merge(st, other);
  }
  return st;
}

__device__ __forceinline__ float lse_final(LseState st) {
  // log(s) + shift; s >= 1 whenever the max is finite.
  return logf(st.s) + lse_shift(st.m);
}

// ---------------------------------------------------------------------------
// Arg-reduction (value, index) with torch.argmax semantics: NaN beats every
// number, equal values keep the lowest index.  Index -1 marks "no element".
// ---------------------------------------------------------------------------
struct ArgState {
  float v;
  int i;
};

template <bool IS_MIN>
__device__ __forceinline__ bool arg_better(float a, int ia, float b, int ib) {
  if (ia < 0) return false;
  if (ib < 0) return true;
  const bool an = a != a, bn = b != b;
  if (an || bn) return an && (!bn || ia < ib);
  if (a == b) return ia < ib;
  return IS_MIN ? a < b : a > b;
}

// In-lane update where `i` is known to exceed every index already folded:
// replace unless the current best is NaN, or `a` does not strictly beat it
// (a NaN `a` beats any number).
template <bool IS_MIN>
__device__ __forceinline__ void arg_step(ArgState& st, float a, int i) {
  const bool take = (st.i < 0) | ((st.v == st.v) & (IS_MIN ? !(a >= st.v) : !(a <= st.v)));
  st.v = take ? a : st.v;
  st.i = take ? i : st.i;
}

template <bool IS_MIN>
__device__ __forceinline__ ArgState arg_wave(ArgState st) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ArgState other{__shfl_xor(st.v, o, 64), __shfl_xor(st.i, o, 64)};
    if (arg_better<IS_MIN>(other.v, other.i, st.v, st.i)) st = other;
  }
  return st;
}

// ---------------------------------------------------------------------------
// Shared row driver.  OP 0 = logsumexp, 1 = argmax, 2 = argmin.
// VEC: the row base is 16-byte aligned and N % kVec == 0, so packs are used;
// otherwise every lane reads one element per chunk.
// ---------------------------------------------------------------------------
template <int OP> struct RowState;
template <> struct RowState<0> { typedef LseState S; };
template <> struct RowState<1> { typedef ArgState S; };
template <> struct RowState<2> { typedef ArgState S; };

template <int OP>
__device__ __forceinline__ typename RowState<OP>::S row_init() {
  if constexpr (OP == 0) return LseState{-INFINITY, 0.0f};
  else return ArgState{0.0f, -1};
}

template <int OP>
__device__ __forceinline__ typename RowState<OP>::S row_merge(typename RowState<OP>::S a,
                                                              typename RowState<OP>::S b) {
  if constexpr (OP == 0) return lse_merge(a, b);
  else return arg_better<OP == 2>(b.v, b.i, a.v, a.i) ? b : a;
}

template <int OP>
__device__ __forceinline__ typename RowState<OP>::S row_wave(typename RowState<OP>::S st) {
  if constexpr (OP == 0) return lse_wave(st);
  else return arg_wave<OP == 2>(st);
}

template <typename T, int OP, int WPR, int UNROLL, bool VEC>
__global__ __launch_bounds__(256) void row_reduce_kernel(const T* __restrict__ x,
                                                         void* __restrict__ out, int64_t M,
                                                         int64_t N) {
  typedef typename RowState<OP>::S S;
  constexpr int V = VEC ? Elem<T>::kVec : 1;
  constexpr int ROWS_PER_BLOCK = 4 / WPR;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wave_in_row = wave % WPR;
  const int row_in_block = wave / WPR;
  const int64_t chunk = 64 * V;                 // elements per wave step
  const int64_t nchunk = (N + chunk - 1) / chunk;

  __shared__ S part[4];

  for (int64_t row0 = (int64_t)blockIdx.x * ROWS_PER_BLOCK; row0 < M;
       row0 += (int64_t)gridDim.x * ROWS_PER_BLOCK) {
    const int64_t row = row0 + row_in_block;
    S st = row_init<OP>();
    if (row < M) {
      const T* xr = x + row * N;
      for (int64_t c0 = wave_in_row; c0 < nchunk; c0 += (int64_t)WPR * UNROLL) {
        float vals[UNROLL][V];
        int64_t base[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
          base[u] = (c0 + (int64_t)u * WPR) * chunk + (int64_t)lane * V;
          // Out-of-row slots read as -inf: they add exp(-inf) = 0 to a sum
          // and are skipped by the arg-reduction below.
#pragma unroll
          for (int e = 0; e < V; ++e) vals[u][e] = -INFINITY;
          if constexpr (VEC) {
            if (base[u] < N) {
              Pack<T> p = load_pack_nt(xr + base[u]);
#pragma unroll
              for (int e = 0; e < V; ++e) vals[u][e] = Elem<T>::to_f32(p.v[e]);
            }
          } else {
            if (base[u] < N) vals[u][0] = Elem<T>::to_f32(xr[base[u]]);
          }
        }
        if constexpr (OP == 0) {
          lse_fold<UNROLL * V>(st, reinterpret_cast<const float(&)[UNROLL * V]>(vals));
        } else {
#pragma unroll
          for (int u = 0; u < UNROLL; ++u) {
            if (base[u] < N) {
#pragma unroll
              for (int e = 0; e < V; ++e) arg_step<OP == 2>(st, vals[u][e], (int)(base[u] + e));
            }
          }
        }
      }
    }
    st = row_wave<OP>(st);
    if constexpr (WPR > 1) {
      if (lane == 0) part[wave] = st;
      __syncthreads();
      if (wave == 0) {
        st = part[0];
#pragma unroll
        for (int w = 1; w < WPR; ++w) st = row_merge<OP>(st, part[w]);
      }
      __syncthreads();
    }
    if (lane == 0 && wave_in_row == 0 && row < M) {
      if constexpr (OP == 0) {
        static_cast<T*>(out)[row] = Elem<T>::from_f32(lse_final(st));
      } else {
        static_cast<int64_t*>(out)[row] = st.i < 0 ? 0 : (int64_t)st.i;
      }
    }
  }
}

template <typename T, int OP>
static int launch_row_reduce(const void* xv, void* out, int64_t M, int64_t N, hipStream_t s) {
  const T* x = static_cast<const T*>(xv);
  const bool vec = host_aligned16(x) && (N % Elem<T>::kVec) == 0;
  // Enough rows to give every CU a dozen wavefronts: one row per wavefront.
  const bool wide = M < 256 * 12;
  const int rows_per_block = wide ? 1 : 4;
  int64_t blocks = (M + rows_per_block - 1) / rows_per_block;
  if (blocks > 256 * 32) blocks = 256 * 32;
  dim3 grid((unsigned)blocks), block(256);
  if (vec) {
    if (wide) row_reduce_kernel<T, OP, 4, 4, true><<<grid, block, 0, s>>>(x, out, M, N);
    else row_reduce_kernel<T, OP, 1, 4, true><<<grid, block, 0, s>>>(x, out, M, N);
  } else {
    if (wide) row_reduce_kernel<T, OP, 4, 8, false><<<grid, block, 0, s>>>(x, out, M, N);
    else row_reduce_kernel<T, OP, 1, 8, false><<<grid, block, 0, s>>>(x, out, M, N);
  }
  return launch_status();
}

template <int OP>
static int dispatch_row_reduce(const void* x, void* out, int64_t M, int64_t N, int dtype,
                               hipStream_t s) {
  switch (dtype) {
    case TILEOPS_F32: return launch_row_reduce<float, OP>(x, out, M, N, s);
    case TILEOPS_F16: return launch_row_reduce<f16, OP>(x, out, M, N, s);
    case TILEOPS_BF16: return launch_row_reduce<bf16, OP>(x, out, M, N, s);
  }
  return TILEOPS_EINVAL;
}

}  // namespace tileops

using namespace tileops;

extern "C" int tileops_logsumexp_fwd(const void* x, void* y, int64_t M, int64_t N, int dtype,
                                     void* stream) {
  if (M < 0 || N <= 0 || N > INT32_MAX) return TILEOPS_ESHAPE;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (M == 0) return 0;
  if (!x || !y) return TILEOPS_ENULL;
  return dispatch_row_reduce<0>(x, y, M, N, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int tileops_argreduce_fwd(const void* x, int64_t* y, int64_t M, int64_t N, int dtype,
                                     int is_min, void* stream) {
  if (M < 0 || N <= 0 || N > INT32_MAX) return TILEOPS_ESHAPE;
  if (dtype < TILEOPS_F32 || dtype > TILEOPS_BF16) return TILEOPS_EINVAL;
  if (M == 0) return 0;
  if (!x || !y) return TILEOPS_ENULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return is_min ? dispatch_row_reduce<2>(x, y, M, N, dtype, s)
                : dispatch_row_reduce<1>(x, y, M, N, dtype, s);
}
