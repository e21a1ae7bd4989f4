// Gated delta-rule (gated DeltaNet) chunked prefill for gfx950
// (tileops_gdn_prefill_fwd).
//
// Recurrence per (batch b, head h), token t (state S is K x V, fp32):
//   S_t = exp(g_t) S_{t-1} + beta_t k_t (v_t - exp(g_t) S_{t-1}^T k_t)^T,   o_t = scale q_t^T S_t
//
// Chunked (C = 64 tokens) WY form.  Inside a chunk, with gc the cumulative
// log-decay, G[l,s] = exp(gc_l - gc_s) (l >= s), A = strictly_lower(beta_l
// G[l,s] k_l.k_s) and T = (I + A)^-1:
//   w   = T diag(beta exp(gc)) k                 (C x K)   \  independent of S:
//   u   = T diag(beta) v                         (C x V)    > kernel 1, fully
//   Aqk = scale * lower_incl(G o (q k^T))        (C x C)   /  parallel over chunks
//   W   = u - w S                                             \
//   o   = scale exp(gc) o (q S) + Aqk W                        > kernel 2, sequential
//   S  <- exp(gc_C) S + (exp(gc_C - gc) o k)^T W              /  over chunks
// Only differences gc_l - gc_s <= 0, gc_C - gc_l <= 0 and gc <= 0 are ever
// exponentiated, so nothing overflows however strong the decay.
//
// Kernel 1 (one workgroup per chunk): K K^T and Q K^T on bf16 MFMA, the
// 64x64 unit-lower-triangular inverse by forward substitution in fp32 (one
// lane per column of T), then w and u on MFMA.  Results go to a workspace.
// Kernel 2 (one workgroup per (b, h, 32-wide slice of V), 4 wavefronts):
// the state slice lives in MFMA accumulators (wavefront i owns key rows
// 32i..32i+31), its bf16 copy and W are exchanged through LDS, two
// workgroup barriers per chunk.
#include "common.h"

namespace tileops {
namespace gdn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int C = 64;    // chunk length
constexpr int DK = 128;  // key dim
constexpr int DV = 128;  // value dim
constexpr int VS = 32;   // value columns per kernel-2 workgroup
constexpr int KP = DK + 8;  // LDS row stride of a natural [C][DK] tile (elements)
constexpr int CP = C + 8;   // LDS row stride of a transposed [*][C] tile (elements)
constexpr float kLog2e = 1.4426950408889634f;

// workspace per chunk
constexpr size_t kWOff = 0;                                   // w   [C][DK] bf16
constexpr size_t kUOff = kWOff + (size_t)C * DK * 2;          // u   [C][DV] bf16
constexpr size_t kAqkOff = kUOff + (size_t)C * DV * 2;        // Aqk [C][C]  bf16
constexpr size_t kGcOff = kAqkOff + (size_t)C * C * 2;        // gc  [C]     f32
constexpr size_t kChunkBytes = kGcOff + (size_t)C * 4;

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) {  // 16-byte load (LDS or global)
  return *reinterpret_cast<const bf16x8*>(p);
}

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Store a 4-row x 8-column tile (4 packs of 8 bf16, one per row) transposed
// into an LDS array with row stride `stride`: column d gets the 4 rows as one
// 8-byte write at [d][r0].
__device__ __forceinline__ void store_transposed4x8(bf16* dst, int stride, int d0, int r0,
                                                    const u32x4 (&rows)[4]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t a0 = rows[0][m], a1 = rows[1][m], a2 = rows[2][m], a3 = rows[3][m];
    const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
    const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
    const uint32_t hi01 = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
    const uint32_t hi23 = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
    const int d = d0 + 2 * m;
    *reinterpret_cast<uint2*>(dst + d * stride + r0) = make_uint2(lo01, lo23);
    *reinterpret_cast<uint2*>(dst + (d + 1) * stride + r0) = make_uint2(hi01, hi23);
  }
}

// ---------------------------------------------------------------------------
// kernel 1: per-chunk preparation
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gdn_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta, uint8_t* __restrict__ ws,
    int B, int T, int H, int NC, float scale) {
  __shared__ __attribute__((aligned(16))) bf16 k_s[C * KP];    // k natural [c][d]
  __shared__ __attribute__((aligned(16))) bf16 kT_s[DK * CP];  // k^T [d][c]
  __shared__ __attribute__((aligned(16))) bf16 vT_s[DV * CP];  // v^T [d][c]
  __shared__ __attribute__((aligned(16))) float a_s[C * (C + 4)];  // A (fp32)
  __shared__ __attribute__((aligned(16))) bf16 tw_s[C * CP];   // T diag(beta exp(gc))
  __shared__ __attribute__((aligned(16))) bf16 tu_s[C * CP];   // T diag(beta)
  __shared__ float gc_s[C], beta_s[C];
  constexpr int AS = C + 4;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int chunk = blockIdx.x % NC;
  const int bh = blockIdx.x / NC;
  const int h = bh % H, b = bh / H;
  const int t0 = chunk * C;
  const int n = min(C, T - t0);
  const int64_t tok_stride = (int64_t)H * DK;  // DK == DV
  uint8_t* wsc = ws + (size_t)blockIdx.x * kChunkBytes;
  bf16* w_ws = reinterpret_cast<bf16*>(wsc + kWOff);
  bf16* u_ws = reinterpret_cast<bf16*>(wsc + kUOff);
  bf16* aqk_ws = reinterpret_cast<bf16*>(wsc + kAqkOff);
  float* gc_ws = reinterpret_cast<float*>(wsc + kGcOff);

  // ---- stage k (natural + transposed) and v (transposed); rows past T are 0
  {
    const int vg = tid & 15, vc = tid >> 4;  // rows 4vg..4vg+3, dims 8vc..8vc+7
    u32x4 kr[4], vr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * vg + i;
      const int64_t off = ((int64_t)b * T + t0 + row) * tok_stride + (int64_t)h * DK + vc * 8;
      kr[i] = row < n ? *reinterpret_cast<const u32x4*>(k + off) : u32x4{0, 0, 0, 0};
      vr[i] = row < n ? *reinterpret_cast<const u32x4*>(v + off) : u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(k_s + row * KP + vc * 8) = kr[i];
    }
    store_transposed4x8(kT_s, CP, vc * 8, 4 * vg, kr);
    store_transposed4x8(vT_s, CP, vc * 8, 4 * vg, vr);
  }
  if (wave == 0) {
    const int64_t gi = ((int64_t)b * T + t0 + lane) * H + h;
    float x = lane < n ? g[gi] : 0.0f;
    const float bt = lane < n ? beta[gi] : 0.0f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {  // inclusive prefix sum over the chunk
      const float y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    gc_s[lane] = x;
    beta_s[lane] = bt;
    gc_ws[lane] = x;
  }
  __syncthreads();

  // ---- K K^T -> A (fp32, LDS) and Q K^T -> Aqk (bf16, workspace)
  // 32x32 blocks (row block rb, column block cb); the upper block is zero.
  if (wave < 3) {
    const int rb = wave == 0 ? 0 : 1;
    const int cb = wave == 2 ? 1 : 0;
    const int qrow = rb * 32 + col;
    f32x16 kk = {}, qk = {};
#pragma unroll
    for (int ks = 0; ks < DK / 16; ++ks) {
      const bf16x8 bk = ld8(k_s + (cb * 32 + col) * KP + ks * 16 + half * 8);
      const bf16x8 ak = ld8(k_s + (rb * 32 + col) * KP + ks * 16 + half * 8);
      bf16x8 aq = {};
      if (qrow < n) {
        u32x4 raw = *reinterpret_cast<const u32x4*>(
            q + ((int64_t)b * T + t0 + qrow) * tok_stride + (int64_t)h * DK + ks * 16 + half * 8);
        aq = *reinterpret_cast<bf16x8*>(&raw);
      }
      kk = mfma(ak, bk, kk);
      qk = mfma(aq, bk, qk);
    }
    const int cs = cb * 32 + col;
    const float gcs = gc_s[cs];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int cl = rb * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
      const float gd = cl >= cs ? exp2f_fast((gc_s[cl] - gcs) * kLog2e) : 0.0f;
      a_s[cl * AS + cs] = cl > cs ? beta_s[cl] * gd * kk[r] : 0.0f;
      aqk_ws[cl * C + cs] = (bf16)(scale * gd * qk[r]);
    }
  } else {
    const int cs = 32 + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int cl = (r >> 2) * 8 + half * 4 + (r & 3);
      a_s[cl * AS + cs] = 0.0f;
      aqk_ws[cl * C + cs] = (bf16)0.0f;
    }
  }
  __syncthreads();

  // ---- T = (I + A)^-1 by forward substitution; lane j owns column j:
  //      T[i][j] = [i == j] - sum_{m < i} A[i][m] T[m][j]
  if (wave == 0) {
    float tcol[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
      float s = (i == lane) ? 1.0f : 0.0f;
#pragma unroll
      for (int m4 = 0; m4 < i; m4 += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(a_s + i * AS + m4);
        s = fmaf(-a4.x, tcol[m4], s);
        if (m4 + 1 < i) s = fmaf(-a4.y, tcol[m4 + 1], s);
        if (m4 + 2 < i) s = fmaf(-a4.z, tcol[m4 + 2], s);
        if (m4 + 3 < i) s = fmaf(-a4.w, tcol[m4 + 3], s);
      }
      tcol[i] = s;
    }
    const float bj = beta_s[lane];
    const float bej = bj * exp2f_fast(gc_s[lane] * kLog2e);
#pragma unroll
    for (int i = 0; i < C; ++i) {
      tw_s[i * CP + lane] = (bf16)(tcol[i] * bej);
      tu_s[i * CP + lane] = (bf16)(tcol[i] * bj);
    }
  }
  __syncthreads();

  // ---- w = Tw k (C x DK), u = Tu v (C x DV): wave -> row block rb, column
  // blocks 2 (wave & 1), 2 (wave & 1) + 1 of both products
  {
    const int rb = wave >> 1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int cb = 2 * (wave & 1) + j;
      f32x16 aw = {}, au = {};
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const bf16x8 tw = ld8(tw_s + (rb * 32 + col) * CP + ks * 16 + half * 8);
        const bf16x8 tu = ld8(tu_s + (rb * 32 + col) * CP + ks * 16 + half * 8);
        const bf16x8 bk = ld8(kT_s + (cb * 32 + col) * CP + ks * 16 + half * 8);
        const bf16x8 bv = ld8(vT_s + (cb * 32 + col) * CP + ks * 16 + half * 8);
        aw = mfma(tw, bk, aw);
        au = mfma(tu, bv, au);
      }
      const int d = cb * 32 + col;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int cl = rb * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
        w_ws[cl * DK + d] = (bf16)aw[r];
        u_ws[cl * DV + d] = (bf16)au[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// kernel 2: the sequential recurrence over chunks and the output
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gdn_recur_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const float* __restrict__ h0,
    const uint8_t* __restrict__ ws, bf16* __restrict__ o, float* __restrict__ hT, int B, int T,
    int H, int NC, float scale) {
  constexpr int SP = DK + 8;  // row stride of S^T [v][d]
  __shared__ __attribute__((aligned(16))) bf16 st_s[VS * SP];      // bf16 S^T (slice)
  __shared__ __attribute__((aligned(16))) bf16 wt_s[VS * CP];      // bf16 W^T (slice)
  __shared__ __attribute__((aligned(16))) bf16 kd_s[2][DK * CP];   // (decayed k)^T
  __shared__ float gcb_s[2][C];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  // the VS-slices of one head run on the same XCD (they share q, k, w, Aqk)
  const int total = gridDim.x;
  int id = blockIdx.x;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  const int nvs = DV / VS;
  const int vs = id % nvs;
  const int bh = id / nvs;
  const int h = bh % H, b = bh / H;
  const int v0 = vs * VS;
  const int64_t tok_stride = (int64_t)H * DK;

  // state rows of this wave: d = 32 * wave + (r / 4) * 8 + half * 4 + r % 4
  f32x16 s_acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int d = 32 * wave + (r >> 2) * 8 + half * 4 + (r & 3);
    s_acc[r] = h0 ? h0[(((int64_t)b * H + h) * DK + d) * DV + v0 + col] : 0.0f;
  }
  auto publish_state = [&]() {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      bf16 p[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = (bf16)s_acc[g4 * 4 + e];
      const int d = 32 * wave + g4 * 8 + half * 4;
      *reinterpret_cast<uint2*>(st_s + col * SP + d) = *reinterpret_cast<uint2*>(p);
    }
  };
  publish_state();

  for (int c = 0; c < NC; ++c) {
    const int buf = c & 1;
    const int t0 = c * C;
    const int n = min(C, T - t0);
    const uint8_t* wsc = ws + (((size_t)b * H + h) * NC + c) * kChunkBytes;
    const bf16* w_ws = reinterpret_cast<const bf16*>(wsc + kWOff);
    const bf16* u_ws = reinterpret_cast<const bf16*>(wsc + kUOff);
    const bf16* aqk_ws = reinterpret_cast<const bf16*>(wsc + kAqkOff);
    const float* gc_ws = reinterpret_cast<const float*>(wsc + kGcOff);
    const float gc_last = gc_ws[C - 1];

    // (decayed k)^T for the state update: row l of k scaled by exp(gc_C - gc_l)
    {
      const int vg = tid & 15, vc = tid >> 4;
      u32x4 kr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * vg + i;
        u32x4 raw = row < n ? *reinterpret_cast<const u32x4*>(
                                  k + ((int64_t)b * T + t0 + row) * tok_stride +
                                  (int64_t)h * DK + vc * 8)
                            : u32x4{0, 0, 0, 0};
        const float f = exp2f_fast((gc_last - gc_ws[row]) * kLog2e);
        const bf16* e = reinterpret_cast<const bf16*>(&raw);
        bf16 sc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] = (bf16)((float)e[j] * f);
        kr[i] = *reinterpret_cast<u32x4*>(sc);
      }
      store_transposed4x8(kd_s[buf], CP, vc * 8, 4 * vg, kr);
    }
    if (tid < C) gcb_s[buf][tid] = gc_ws[tid];

    // operands from the workspace / q for this wave's 32 rows of the chunk
    const int rblk = wave & 1;            // chunk rows 32*rblk .. 32*rblk+31
    const int arow = rblk * 32 + col;     // A-operand row of this lane
    bf16x8 areg[DK / 16];
    float uval[16];
    bf16x8 aqk[C / 16];
    if (wave < 2) {
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks) areg[ks] = ld8(w_ws + arow * DK + ks * 16 + half * 8);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int cl = rblk * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
        uval[r] = (float)u_ws[cl * DV + v0 + col];
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks) {
        bf16x8 a = {};
        if (arow < n) {
          u32x4 raw = *reinterpret_cast<const u32x4*>(
              q + ((int64_t)b * T + t0 + arow) * tok_stride + (int64_t)h * DK + ks * 16 + half * 8);
          a = *reinterpret_cast<bf16x8*>(&raw);
        }
        areg[ks] = a;
      }
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) aqk[ks] = ld8(aqk_ws + arow * C + ks * 16 + half * 8);
    }
    __syncthreads();  // (A) S^T, (decayed k)^T, gc of this chunk visible

    // waves 0, 1: W = u - w S ; waves 2, 3: scale exp(gc) (q S)
    f32x16 acc = {};
#pragma unroll
    for (int ks = 0; ks < DK / 16; ++ks)
      acc = mfma(areg[ks], ld8(st_s + col * SP + ks * 16 + half * 8), acc);
    if (wave < 2) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16 p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = (bf16)(uval[g4 * 4 + e] - acc[g4 * 4 + e]);
        const int cl = rblk * 32 + g4 * 8 + half * 4;
        *reinterpret_cast<uint2*>(wt_s + col * CP + cl) = *reinterpret_cast<uint2*>(p);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int cl = rblk * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
        acc[r] *= scale * exp2f_fast(gcb_s[buf][cl] * kLog2e);
      }
    }
    __syncthreads();  // (B) W^T visible

    if (wave >= 2) {  // o = scale exp(gc) (q S) + Aqk W
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks)
        acc = mfma(aqk[ks], ld8(wt_s + col * CP + ks * 16 + half * 8), acc);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int cl = rblk * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
        if (cl < n) o[((int64_t)b * T + t0 + cl) * tok_stride + (int64_t)h * DV + v0 + col] =
            (bf16)acc[r];
      }
    }
    // S <- exp(gc_C) S + (decayed k)^T W   (rows 32 * wave .. of the state)
    const float dec = exp2f_fast(gc_last * kLog2e);
#pragma unroll
    for (int r = 0; r < 16; ++r) s_acc[r] *= dec;
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks)
      s_acc = mfma(ld8(kd_s[buf] + (32 * wave + col) * CP + ks * 16 + half * 8),
                   ld8(wt_s + col * CP + ks * 16 + half * 8), s_acc);
    publish_state();
  }

#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int d = 32 * wave + (r >> 2) * 8 + half * 4 + (r & 3);
    hT[(((int64_t)b * H + h) * DK + d) * DV + v0 + col] = s_acc[r];
  }
}

}  // namespace gdn
}  // namespace tileops

using namespace tileops;

extern "C" size_t tileops_gdn_prefill_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K,
                                                      int64_t V, int64_t chunk) {
  if (B < 0 || T < 0 || H < 0 || K != gdn::DK || V != gdn::DV || chunk != gdn::C) return 0;
  const int64_t nc = (T + gdn::C - 1) / gdn::C;
  return (size_t)(B * H * nc) * gdn::kChunkBytes;
}

extern "C" int tileops_gdn_prefill_fwd(const void* q, const void* k, const void* v, const float* g,
                                       const float* beta, const float* h0, void* o, float* hT,
                                       int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                       int64_t chunk, float scale, int dtype, void* ws,
                                       size_t ws_bytes, void* stream) {
  if (B < 0 || T < 0 || H <= 0) return TILEOPS_ESHAPE;
  if (K != gdn::DK || V != gdn::DV || chunk != gdn::C) return TILEOPS_ESHAPE;
  if (B > 65535 || H > 65535 || T > INT32_MAX / 2) return TILEOPS_ESHAPE;
  if (dtype != TILEOPS_BF16) return TILEOPS_EINVAL;
  if (B == 0) return 0;
  if (!hT) return TILEOPS_ENULL;
  const size_t need = tileops_gdn_prefill_workspace_bytes(B, T, H, K, V, chunk);
  if (T > 0) {
    if (!q || !k || !v || !g || !beta || !o) return TILEOPS_ENULL;
    if (!ws || ws_bytes < need) return TILEOPS_EWORKSPACE;
    if (!host_aligned16(q) || !host_aligned16(k) || !host_aligned16(v) || !host_aligned16(ws))
      return TILEOPS_EINVAL;
  }
  const int nc = (int)((T + gdn::C - 1) / gdn::C);
  const int64_t nblk = B * H * nc;
  if (nblk > (int64_t)UINT32_MAX) return TILEOPS_ESHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bf16* qb = static_cast<const bf16*>(q);
  const bf16* kb = static_cast<const bf16*>(k);
  if (nblk > 0)
    gdn::gdn_prep_kernel<<<dim3((unsigned)nblk), dim3(256), 0, s>>>(
        qb, kb, static_cast<const bf16*>(v), g, beta, static_cast<uint8_t*>(ws), (int)B, (int)T,
        (int)H, nc, scale);
  gdn::gdn_recur_kernel<<<dim3((unsigned)(B * H * (gdn::DV / gdn::VS))), dim3(256), 0, s>>>(
      qb, kb, h0, static_cast<const uint8_t*>(ws), static_cast<bf16*>(o), hT, (int)B, (int)T,
      (int)H, nc, scale);
  return launch_status();
}
