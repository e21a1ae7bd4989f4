// Flash-attention forward for gfx950 (tileops_mha_fwd), BSHD layout.
//
// One workgroup = WAVES wavefronts (8 at launch: BM = 256 query rows of one
// (batch, head)); each wavefront owns 32 query rows.  Keys/values stream
// through LDS in tiles of BN = 64 rows, prefetched into registers one tile
// ahead.
//
// Both products run on v_mfma_f32_32x32x16_{bf16,f16} in the *transposed*
// orientation:
//   S^T (kv x q) = K (kv x D) . Q^T (D x q)      A = K from LDS, B = Q in VGPRs
//   O^T (d x q) += V^T (d x kv) . P^T (kv x q)   A = V^T from LDS, B = P in VGPRs
// With 32x32 MFMA results, lane l holds column l % 32, i.e. one query row,
// and 16 key rows of each 32-key block (the other 16 sit in lane l ^ 32).
// The online softmax is therefore lane-local except for one exchange with
// the partner lane, and P feeds the second MFMA straight from registers.
// The summation order over keys inside a 16-key MFMA step is free, so V^T is
// stored in LDS with each 16-key group permuted to match the key rows a lane
// holds: the A operand of every step is then a single 16-byte LDS read.
//
// The softmax runs in the log2 domain (scores scaled by scale * log2 e); the
// per-row LSE written out is m + log2(l), i.e. logsumexp(scale q k^T) / ln 2.
#include <float.h>
#include <stdlib.h>

#include "common.h"

namespace tileops {
namespace mha {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  typedef bf16x8 V8;
  __device__ __forceinline__ static f32x16 run(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<f16> {
  typedef f16x8 V8;
  __device__ __forceinline__ static f32x16 run(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Lazy rescaling: the running max only moves when a tile's max exceeds it by
// more than 2^kLazyLog2 in the exp2 domain, so P <= 2^kLazyLog2 (exact in
// fp32 / bf16) and the O accumulator is rescaled rarely.
constexpr float kLazyLog2 = 8.0f;

// position of key group `group4` (4 keys) inside an LDS row of V^T: within
// each 16-key group the 4-key blocks are stored in the order 0, 2, 1, 3.
__device__ __forceinline__ int vt_pos(int group4) {
  const int j = group4 & 3;
  const int pj = (j == 1) ? 2 : (j == 2 ? 1 : j);
  return (group4 >> 2) * 16 + pj * 4;
}

template <int D, int BN> struct Smem {
  static constexpr int KS = D + 8;   // K row stride (elements): 16 B pad
  static constexpr int VS = BN + 8;  // V^T row stride (elements): 16 B pad
  static constexpr int K_ELEMS = BN * KS;
  static constexpr int V_ELEMS = D * VS;
};

template <typename T, int D, bool CAUSAL, int WAVES, int BN>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void mha_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ o,
    float* __restrict__ lse, int B, int Sq, int Skv, int H, int Hkv, float scale_log2, int nqb) {
  typedef typename Mfma<T>::V8 V8;
  typedef Smem<D, BN> SM;
  constexpr int NKB = BN / 32;           // 32-key blocks per tile
  constexpr int kThreads = WAVES * 64;
  constexpr int BM = WAVES * 32;         // query rows per workgroup
  constexpr int KSTEPS = D / 16;         // MFMA steps over the head dim
  constexpr int DBLK = D / 32;           // 32-row blocks of O^T
  constexpr int KCHUNK = D / 8;          // 16-byte chunks per K row
  constexpr int KLOADS = BN * KCHUNK / kThreads;  // 16-byte K loads per thread
  constexpr int VGROUPS = (BN / 4) * (D / 8);     // (4 keys x 8 dims) units
  static_assert(KLOADS * kThreads == BN * KCHUNK, "K tile must split evenly over threads");
  static_assert(VGROUPS <= kThreads, "one V unit per thread at most");

  __shared__ __attribute__((aligned(16))) T k_lds[SM::K_ELEMS];
  __shared__ __attribute__((aligned(16))) T v_lds[SM::V_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // query row inside the wave's 32
  const int half = lane >> 5;

  // --- XCD-aware block order: workgroups are dealt round-robin to the 8
  // XCDs; regroup so that one XCD works through all query blocks of a head
  // together and that head's K/V stays in the XCD's L2.
  const int total = nqb * H * B;
  int id = blockIdx.x;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  int qb = id % nqb;
  const int hq = (id / nqb) % H;
  const int bb = id / (nqb * H);
  if (CAUSAL) qb = nqb - 1 - qb;  // longest rows first inside a head
  const int hk = hq / (H / Hkv);
  const int q0 = qb * BM;
  const int off = Skv - Sq;  // right-aligned causal offset

  const int64_t q_row = (int64_t)H * D;
  const int64_t kv_row = (int64_t)Hkv * D;
  const T* qbase = q + (int64_t)bb * Sq * q_row + (int64_t)hq * D;
  const T* kbase = k + (int64_t)bb * Skv * kv_row + (int64_t)hk * D;
  const T* vbase = v + (int64_t)bb * Skv * kv_row + (int64_t)hk * D;

  // --- Q^T operand: this lane's query row, 8 dims per MFMA step
  const int qi = q0 + wave * 32 + col;
  V8 qreg[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    if (qi < Sq) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qbase + (int64_t)qi * q_row + ks * 16 + half * 8);
      qreg[ks] = *reinterpret_cast<V8*>(&raw);
    } else {
      qreg[ks] = V8{};
    }
  }

  const int kv_end = CAUSAL ? min(Skv, q0 + BM + off) : Skv;
  const int ntiles = (kv_end + BN - 1) / BN;

  // --- register prefetch of one K / V tile
  u32x4 kpre[KLOADS];
  u32x4 vpre[4];
  constexpr int NG = BN / 4;    // 4-key groups per tile
  const bool v_owner = tid < VGROUPS;
  const int vg = tid % NG;      // 4-key group
  const int vc = tid / NG;      // 8-dim chunk
  auto prefetch = [&](int tile) {
    const int kv0 = tile * BN;
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = tid + i * kThreads;
      const int r = c / KCHUNK, cc = c % KCHUNK;
      const int kv = kv0 + r;
      kpre[i] = kv < Skv ? *reinterpret_cast<const u32x4*>(kbase + (int64_t)kv * kv_row + cc * 8)
                         : u32x4{0, 0, 0, 0};
    }
    if (v_owner) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kv = kv0 + vg * 4 + i;
        vpre[i] = kv < Skv ? *reinterpret_cast<const u32x4*>(vbase + (int64_t)kv * kv_row + vc * 8)
                           : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = tid + i * kThreads;
      const int r = c / KCHUNK, cc = c % KCHUNK;
      *reinterpret_cast<u32x4*>(k_lds + r * SM::KS + cc * 8) = kpre[i];
    }
    if (v_owner) {
      // transpose 4 keys x 8 dims: dim d gets the 4 keys as one 8-byte write
      const int pos = vt_pos(vg);
#pragma unroll
      for (int m = 0; m < 4; ++m) {  // dword m of each row = dims 2m, 2m+1
        const uint32_t a0 = vpre[0][m], a1 = vpre[1][m], a2 = vpre[2][m], a3 = vpre[3][m];
        // low halves -> dim 2m, high halves -> dim 2m + 1
        const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
        const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
        const uint32_t hi01 = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
        const uint32_t hi23 = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
        const int d = vc * 8 + 2 * m;
        *reinterpret_cast<uint2*>(v_lds + d * SM::VS + pos) = make_uint2(lo01, lo23);
        *reinterpret_cast<uint2*>(v_lds + (d + 1) * SM::VS + pos) = make_uint2(hi01, hi23);
      }
    }
  };

  f32x16 acc_o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) acc_o[i] = f32x16{};
  float m_run = -INFINITY;  // running max of raw scores (q . k)
  float l_run = 0.0f;
  const float lazy_raw = kLazyLog2 / scale_log2;

  if (ntiles > 0) prefetch(0);
  for (int t = 0; t < ntiles; ++t) {
    if (t > 0) __syncthreads();  // every wave is done reading the last tile
    commit();
    __syncthreads();
    if (t + 1 < ntiles) prefetch(t + 1);
    const int kv0 = t * BN;

    // S^T = K . Q^T : NKB 32-key blocks, their MFMA chains interleaved
    f32x16 acc_s[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc_s[kb] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const V8 a =
            *reinterpret_cast<const V8*>(k_lds + (kb * 32 + col) * SM::KS + ks * 16 + half * 8);
        acc_s[kb] = Mfma<T>::run(a, qreg[ks], acc_s[kb]);
      }
    }

    // online softmax for query row qi: maxima in raw score units, the scale
    // (times log2 e) folded into one FMA per score inside exp2
    // masking only on the ragged last tile and on causal diagonal tiles
    // (a workgroup-uniform branch, kept out of the common path)
    if ((kv0 + BN > Skv) || (CAUSAL && kv0 + BN - 1 > q0 + off)) {
      const int lim = CAUSAL ? min(Skv - 1, qi + off) : Skv - 1;  // last visible key
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kv = kv0 + kb * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
          acc_s[kb][r] = kv > lim ? -INFINITY : acc_s[kb][r];
        }
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, acc_s[kb][r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const bool grow = tmax > m_run + lazy_raw;
    if (__any(grow)) {
      const float m_new = grow ? tmax : m_run;
      const float alpha = m_run == -INFINITY ? 0.0f
                                             : __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[db][r] *= alpha;
      }
    }
    // rows with no visible key yet keep m = -inf: shift by 0 so exp2 -> 0
    const float neg_mc = m_run == -INFINITY ? 0.0f : -m_run * scale_log2;
    float psum = 0.0f;
    V8 pb[2 * NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        // fp32 probabilities form the row sum (and the LSE); P is rounded to
        // the storage type only as the MFMA operand
        const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[kb][r], scale_log2, neg_mc));
        psum += p;
        pb[kb * 2 + (r >> 3)][r & 7] = (T)p;
      }
    }
    l_run += psum;

    // O^T += V^T . P^T (independent d-blocks interleaved)
#pragma unroll
    for (int ks = 0; ks < BN / 16; ++ks) {
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        const V8 a =
            *reinterpret_cast<const V8*>(v_lds + (db * 32 + col) * SM::VS + ks * 16 + half * 8);
        acc_o[db] = Mfma<T>::run(a, pb[ks], acc_o[db]);
      }
    }
  }

  // --- epilogue: combine the two half-row sums, normalise, store
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < Sq) {
    T* orow = o + ((int64_t)bb * Sq + qi) * q_row + (int64_t)hq * D;
#pragma unroll
    for (int db = 0; db < DBLK; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        T vals[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) vals[e] = (T)(acc_o[db][g * 4 + e] * inv_l);
        const int d = db * 32 + g * 8 + half * 4;
        *reinterpret_cast<uint2*>(orow + d) = *reinterpret_cast<uint2*>(vals);
      }
    }
    if (half == 0)
      lse[((int64_t)bb * H + hq) * Sq + qi] =
          l_tot > 0.0f ? m_run * scale_log2 + __builtin_amdgcn_logf(l_tot) : -INFINITY;
  }
}

template <typename T, int D, int WAVES, int BN>
static int launch(const void* q, const void* k, const void* v, void* o, float* lse, int B, int Sq,
                  int Skv, int H, int Hkv, bool causal, float scale, hipStream_t s) {
  constexpr int BM = WAVES * 32;
  const int nqb = (Sq + BM - 1) / BM;
  const int64_t total = (int64_t)nqb * H * B;
  const float scale_log2 = scale * 1.4426950408889634f;
  dim3 grid((unsigned)total), block(WAVES * 64);
  if (causal)
    mha_fwd_kernel<T, D, true, WAVES, BN><<<grid, block, 0, s>>>(
        static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
        static_cast<T*>(o), lse, B, Sq, Skv, H, Hkv, scale_log2, nqb);
  else
    mha_fwd_kernel<T, D, false, WAVES, BN><<<grid, block, 0, s>>>(
        static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
        static_cast<T*>(o), lse, B, Sq, Skv, H, Hkv, scale_log2, nqb);
  return launch_status();
}

template <typename T, int D>
static int launch_w(const void* q, const void* k, const void* v, void* o, float* lse, int B,
                    int Sq, int Skv, int H, int Hkv, bool causal, float scale, hipStream_t s) {
  // 8 wavefronts x 32 query rows, 64-key tiles: measured best on MI355X
  // among 4 / 8 wavefronts and 64 / 128-key tiles, and among software-
  // pipelined variants with Q in LDS and double-buffered K / V slots.
  return launch<T, D, 8, 64>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, s);
}

template <typename T>
static int dispatch_d(int D, const void* q, const void* k, const void* v, void* o, float* lse,
                      int B, int Sq, int Skv, int H, int Hkv, bool causal, float scale,
                      hipStream_t s) {
  if (D == 128) return launch_w<T, 128>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, s);
  if (D == 64) return launch_w<T, 64>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, s);
  return TILEOPS_ESHAPE;
}

}  // namespace mha
}  // namespace tileops

using namespace tileops;

extern "C" int tileops_mha_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                               int64_t B, int64_t Sq, int64_t Skv, int64_t H, int64_t Hkv,
                               int64_t D, int causal, float scale, int dtype, void* stream) {
  if (B < 0 || Sq < 0 || Skv < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0) return TILEOPS_ESHAPE;
  if (D != 64 && D != 128) return TILEOPS_ESHAPE;
  if (B > INT32_MAX || Sq > INT32_MAX || Skv > INT32_MAX || H > 65535) return TILEOPS_ESHAPE;
  if (causal && Sq > Skv) return TILEOPS_ESHAPE;
  if (dtype != TILEOPS_F16 && dtype != TILEOPS_BF16) return TILEOPS_EINVAL;
  if (B == 0 || Sq == 0) return 0;
  if (Skv == 0) return TILEOPS_ESHAPE;
  if (!q || !k || !v || !o || !lse) return TILEOPS_ENULL;
  if (!host_aligned16(q) || !host_aligned16(k) || !host_aligned16(v) || !host_aligned16(o))
    return TILEOPS_EINVAL;
  if (((Sq + 127) / 128) * H * B > (int64_t)UINT32_MAX) return TILEOPS_ESHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TILEOPS_BF16)
    return mha::dispatch_d<bf16>((int)D, q, k, v, o, lse, (int)B, (int)Sq, (int)Skv, (int)H,
                                 (int)Hkv, causal != 0, scale, s);
  return mha::dispatch_d<f16>((int)D, q, k, v, o, lse, (int)B, (int)Sq, (int)Skv, (int)H,
                              (int)Hkv, causal != 0, scale, s);
}
