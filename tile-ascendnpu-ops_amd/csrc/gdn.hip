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
//   Tu  = T diag(beta)                           (C x C)    > kernel 1, fully
//   Aqk = scale * lower_incl(G o (q k^T))        (C x C)   /  parallel over chunks
//   W   = Tu v - w S                                          \
//   o   = scale exp(gc) o (q S) + Aqk W                        > kernel 2, sequential
//   S  <- exp(gc_C) S + (exp(gc_C - gc) o k)^T W              /  over chunks
// Only differences gc_l - gc_s <= 0, gc_C - gc_l <= 0 and gc <= 0 are ever
// exponentiated, so nothing overflows however strong the decay.
//
// Kernel 1 (persistent, two workgroups per CU, the next chunk's q / k / g /
// beta loaded while the current one is processed): K K^T and Q K^T on bf16
// MFMA, the 64x64 unit-lower-triangular inverse in fp32 (16x16 diagonal
// blocks by substitution, one wavefront each, the off-diagonal blocks by
// products on fp32 MFMA), then w on bf16 MFMA.  -w, Tu, Aqk, the decayed
// keys (k e^{gc_C - gc})^T and the per-token factors go to a workspace.
// Kernel 2 (one workgroup per (b, h, 32-wide slice of V), 8 wavefronts):
// four compute wavefronts keep the state slice in MFMA accumulators
// (wavefront i owns key rows 32i..32i+31) and exchange its bf16 copy and W
// through LDS; waves 0, 1 form W (rows 0-31, 32-63), waves 2, 3 the output
// rows.  Four loader wavefronts bring the next chunk's operands into LDS
// with direct-to-LDS loads meanwhile.  Two workgroup barriers per chunk.
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
constexpr size_t kWOff = 0;                                   // -w   [C][DK] bf16
constexpr size_t kTuOff = kWOff + (size_t)C * DK * 2;         // Tu   [C][C]  bf16
constexpr size_t kAqkOff = kTuOff + (size_t)C * C * 2;        // Aqk  [C][C]  bf16
constexpr size_t kKdOff = kAqkOff + (size_t)C * C * 2;        // kd^T [DK][C] bf16
constexpr size_t kFacOff = kKdOff + (size_t)DK * C * 2;       // factors, f32 [kFacN]
constexpr int kFacN = 80;  // scale e^{gc_l} (l < C), e^{gc_C} at index C, zero pad
constexpr size_t kChunkBytes = kFacOff + (size_t)kFacN * 4;

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) {  // 16-byte load (LDS or global)
  return *reinterpret_cast<const bf16x8*>(p);
}

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Inclusive prefix sum over the 64 lanes of a wavefront by DPP lane moves,
// with no LDS round trip (a shuffle-based scan waits on the LDS queue, which
// the other workgroup of the CU keeps busy): Hillis-Steele inside each row
// of 16 lanes (row_shr 1, 2, 4, 8; lanes shifted in from outside the row
// read 0), then each row's total carried forward: row_bcast:15 adds lane
// 16 r + 15 to row r + 1 (rows 1 and 3), row_bcast:31 adds lane 31 to rows
// 2 and 3.
__device__ __forceinline__ float dpp_add(float x, int moved) {
  return x + __builtin_bit_cast(float, moved);
}
__device__ __forceinline__ float wave_inclusive_sum(float x) {
#define TILEOPS_DPP(ctrl, rows) \
  __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), ctrl, rows, 0xF, true)
  x = dpp_add(x, TILEOPS_DPP(0x111, 0xF));  // row_shr:1
  x = dpp_add(x, TILEOPS_DPP(0x112, 0xF));  // row_shr:2
  x = dpp_add(x, TILEOPS_DPP(0x114, 0xF));  // row_shr:4
  x = dpp_add(x, TILEOPS_DPP(0x118, 0xF));  // row_shr:8
  x = dpp_add(x, TILEOPS_DPP(0x142, 0xA));  // row_bcast:15 -> rows 1, 3
  x = dpp_add(x, TILEOPS_DPP(0x143, 0xC));  // row_bcast:31 -> rows 2, 3
#undef TILEOPS_DPP
  return x;
}

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

// Workgroup barrier that waits only for this wavefront's LDS accesses
// (lgkmcnt(0); vmcnt and expcnt left at their maxima), so that global loads
// and stores issued before it stay in flight across it (direct-to-LDS loads
// included).  __syncthreads() would also wait for them: its fence drains
// every outstanding memory access.  Only LDS data is exchanged through these
// barriers; register results of global loads are waited for at their use.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// kernel 1: per-chunk preparation
// ---------------------------------------------------------------------------
// LDS plan (two workgroups fit one CU):
//   r0: k natural [C][KP] bf16 (K K^T)            -> T (fp32 [C][AS], inverse)
//   r1: A^T fp32 [C][AS] (A^T[m][i] = A[i][m])    -> Tw, Tu (bf16 [C][CP] each)
//   x_s: A21 T11 (fp32 32 x 32);  kT_s: k^T [d][c] bf16 (w);  aqk_s: Aqk bf16
constexpr int AS = 72;  // fp32 row stride of A^T / T (288 bytes: float4-aligned rows)
constexpr int XS = 36;  // fp32 row stride of X

// Global operands of one chunk for one thread, loaded a chunk ahead: k rows
// 4vg..4vg+3 (dims 8vc..8vc+7), g / beta of token `lane`, and the q row this
// wavefront's Q K^T block needs, in the MFMA A layout.  One uniform sequence
// for every wavefront (wave 3 loads q rows it does not use); rows past T load
// the chunk's last row and are zeroed where they are consumed.
struct PrepLoads {
  u32x4 kr[4];
  bf16x8 aq[DK / 16];
  float g, beta;
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const float* __restrict__ g,
    const float* __restrict__ beta, uint8_t* __restrict__ ws, int B, int T, int H, int NC,
    float scale) {
  __shared__ __attribute__((aligned(16))) float r0[C * AS];
  __shared__ __attribute__((aligned(16))) float r1[C * AS];
  __shared__ __attribute__((aligned(16))) float x_s[32 * XS];
  __shared__ __attribute__((aligned(16))) bf16 kT_s[DK * CP];
  __shared__ __attribute__((aligned(16))) bf16 aqk_s[C * CP];
  __shared__ __attribute__((aligned(16))) float gc_s[C], beta_s[C], be_s[C], dec_s[C];
  static_assert(C * KP * 2 <= C * AS * 4, "k tile must fit the T region");
  static_assert(2 * C * CP * 2 <= C * AS * 4, "Tw and Tu must fit the A region");
  bf16* k_s = reinterpret_cast<bf16*>(r0);
  float* t_s = r0;
  float* at_s = r1;
  bf16* tw_s = reinterpret_cast<bf16*>(r1);
  bf16* tu_s = tw_s + C * CP;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int rb = wave == 0 ? 0 : 1;  // Q K^T / K K^T block of waves 0-2
  const int cb = wave == 2 ? 1 : 0;
  const int qrow = rb * 32 + col;
  const int vg = tid & 15, vc = tid >> 4;
  const int64_t tok_stride = (int64_t)H * DK;  // DK == DV
  const uint64_t nblk = (uint64_t)B * H * NC;

  auto load = [&](uint64_t blk, PrepLoads& L) {
    const int chunk = (int)(blk % NC), bh = (int)(blk / NC);
    const int h = bh % H, b = bh / H;
    const int t0 = chunk * C, n = min(C, T - t0);
    const bf16* kb = k + ((int64_t)b * T + t0) * tok_stride + (int64_t)h * DK + vc * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      L.kr[i] = *reinterpret_cast<const u32x4*>(kb + min(4 * vg + i, n - 1) * tok_stride);
    const int64_t gi = ((int64_t)b * T + t0 + min(lane, n - 1)) * H + h;
    L.g = g[gi];
    L.beta = beta[gi];
    const bf16* qp = q + ((int64_t)b * T + t0 + min(qrow, n - 1)) * tok_stride + (int64_t)h * DK;
#pragma unroll
    for (int ks = 0; ks < DK / 16; ++ks) L.aq[ks] = ld8(qp + ks * 16 + half * 8);
  };

  // Persistent: workgroup i takes chunks i, i + grid, ...; the next chunk's
  // loads are issued as soon as the current one's registers are consumed.
  PrepLoads cur;
  uint64_t blk = blockIdx.x;
  if (blk < nblk) load(blk, cur);
  for (; blk < nblk; blk += gridDim.x) {
    const int chunk = (int)(blk % NC);
    const int t0 = chunk * C;
    const int n = min(C, T - t0);
    uint8_t* wsc = ws + (size_t)blk * kChunkBytes;
    bf16* w_ws = reinterpret_cast<bf16*>(wsc + kWOff);
    bf16* tu_ws = reinterpret_cast<bf16*>(wsc + kTuOff);
    bf16* aqk_ws = reinterpret_cast<bf16*>(wsc + kAqkOff);
    bf16* kd_ws = reinterpret_cast<bf16*>(wsc + kKdOff);
    float* fac_ws = reinterpret_cast<float*>(wsc + kFacOff);
    u32x4 (&kr)[4] = cur.kr;

    // ---- stage k (natural + transposed); rows past T are 0
    {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * vg + i;
        if (row >= n) kr[i] = u32x4{0, 0, 0, 0};
        *reinterpret_cast<u32x4*>(k_s + row * KP + vc * 8) = kr[i];
      }
      store_transposed4x8(kT_s, CP, vc * 8, 4 * vg, kr);
    }
    if (wave == 0) {
      float x = lane < n ? cur.g : 0.0f;
      const float bt = lane < n ? cur.beta : 0.0f;
      x = wave_inclusive_sum(x);  // gc: inclusive prefix sum over the chunk
      gc_s[lane] = x;
      beta_s[lane] = bt;
      be_s[lane] = bt * exp2f_fast(x * kLog2e);
      // factors the recurrence applies: scale e^{gc} per output row, the
      // chunk decay e^{gc_C}, and e^{gc_C - gc} for the decayed keys
      const float gl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), C - 1));
      dec_s[lane] = exp2f_fast((gl - x) * kLog2e);
      fac_ws[lane] = scale * exp2f_fast(x * kLog2e);
      if (lane < kFacN - C) fac_ws[C + lane] = lane == 0 ? exp2f_fast(gl * kLog2e) : 0.0f;
    }
    lds_barrier();

    // ---- K K^T -> A^T (fp32, LDS) and Q K^T -> Aqk (bf16, LDS), in 32x32
    // blocks (row block rb, column block cb).  Only the strictly lower parts of
    // the diagonal blocks and the block A21 of A are ever read back.
    if (wave < 3) {
      // transposed orientation: k rows s of block cb as the A operand, k / q
      // rows l of block rb as B, so that a lane owns one row l (column of the
      // result) and its 16 values run over s: [s][l] = k_s . k_l and k_s . q_l
      f32x16 kk = {}, qk = {};
      const bool qlive = qrow < n;
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks) {
        const bf16x8 bs = ld8(k_s + (cb * 32 + col) * KP + ks * 16 + half * 8);
        const bf16x8 bl = ld8(k_s + (rb * 32 + col) * KP + ks * 16 + half * 8);
        const bf16x8 a = qlive ? cur.aq[ks] : bf16x8{};
        kk = mfma(bs, bl, kk);
        qk = mfma(bs, a, qk);
      }
      const int l = rb * 32 + col;
      const float gl = gc_s[l], bel = beta_s[l];
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int s0 = cb * 32 + g4 * 8 + half * 4;
        const float4 gs4 = *reinterpret_cast<const float4*>(gc_s + s0);
        const float gsv[4] = {gs4.x, gs4.y, gs4.z, gs4.w};
        bf16 q4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = g4 * 4 + e;
          const int sc = s0 + e;
          // branch-free: the decay is evaluated for every element (its
          // argument clamped to <= 0, exact where it is used) and selected
          float gd = exp2f_fast(fminf((gl - gsv[e]) * kLog2e, 0.0f));
          asm volatile("" : "+v"(gd));
          gd = sc <= l ? gd : 0.0f;
          at_s[sc * AS + l] = sc < l ? bel * gd * kk[r] : 0.0f;  // A^T[s][l]
          q4[e] = (bf16)(scale * gd * qk[r]);
        }
        *reinterpret_cast<uint2*>(aqk_s + l * CP + s0) = *reinterpret_cast<uint2*>(q4);
      }
    } else {  // the block l < 32 <= s of Aqk is zero
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *reinterpret_cast<uint2*>(aqk_s + col * CP + 32 + g4 * 8 + half * 4) = make_uint2(0u, 0u);
    }
    if (blk + gridDim.x < nblk) load(blk + gridDim.x, cur);  // operands consumed: next chunk
    lds_barrier();

    // ---- Aqk rows to the workspace (16-byte stores); T = (I + A)^-1, blocked
    // by 16: the four diagonal blocks Tbb by substitution (wave w: block w,
    // lane j: column j; p[i] accumulates sum_m A[i][m] T[m][j]), then on fp32
    // MFMA T10 = -T11 (A10 T00), T32 = -T33 (A32 T22) and, with 32-row
    // blocks, T21 = -T22 (A21 T11).
#pragma unroll
    for (int e = tid; e < C * C / 8; e += 256) {
      const int row = e >> 3, c8 = (e & 7) * 8;
      *reinterpret_cast<u32x4*>(aqk_ws + row * C + c8) =
          *reinterpret_cast<const u32x4*>(aqk_s + row * CP + c8);
    }
    {
      const int base = 16 * wave, jl = lane & 15;
      float p[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) p[i] = 0.0f;
      // av[m & 1][gq] = A[base + 4gq .. 4gq + 3][base + m]; step m + 1's
      // groups are read while step m's FMAs run
      const float4* a4p = reinterpret_cast<const float4*>(at_s + base * AS + base);
      float4 av[2][4];
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) av[0][gq] = a4p[gq];
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        if (m + 1 < 16) {
#pragma unroll
          for (int gq = (m + 2) >> 2; gq < 4; ++gq) av[(m + 1) & 1][gq] = a4p[(m + 1) * (AS / 4) + gq];
        }
        const float t = (m == jl ? 1.0f : 0.0f) - p[m];
        // every lane writes (the four 16-lane groups hold the same columns,
        // so the writes agree): no exec-masked branch in the chain
        t_s[(base + m) * AS + base + jl] = t;
#pragma unroll
        for (int gq = (m + 1) >> 2; gq < 4; ++gq) {
          const float4 a4 = av[m & 1][gq];
          const int i4 = 4 * gq;
          if (i4 + 0 > m) p[i4 + 0] = fmaf(a4.x, t, p[i4 + 0]);
          if (i4 + 1 > m) p[i4 + 1] = fmaf(a4.y, t, p[i4 + 1]);
          if (i4 + 2 > m) p[i4 + 2] = fmaf(a4.z, t, p[i4 + 2]);
          if (i4 + 3 > m) p[i4 + 3] = fmaf(a4.w, t, p[i4 + 3]);
        }
      }
    }
    lds_barrier();
    // v_mfma_f32_16x16x4f32 lanes: A[mi][mk], B[mk][mi], D[4 mk + r][mi]
    const int mi = lane & 15, mk = lane >> 4;
    if (wave < 2) {  // Y = A10 T00 (wave 0) / A32 T22 (wave 1) -> x_s rows 16 wave ..
      const int d0 = 32 * wave;
      f32x4 y = {};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int kx = 4 * kk + mk;
        y = __builtin_amdgcn_mfma_f32_16x16x4f32(at_s[(d0 + kx) * AS + d0 + 16 + mi],
                                                t_s[(d0 + kx) * AS + d0 + mi], y, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) x_s[(16 * wave + 4 * mk + r) * XS + mi] = y[r];
    }
    lds_barrier();
    if (wave < 2) {  // T10 = -T11 Y (wave 0), T32 = -T33 Y (wave 1)
      const int d0 = 32 * wave;
      f32x4 z = {};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int kx = 4 * kk + mk;
        z = __builtin_amdgcn_mfma_f32_16x16x4f32(t_s[(d0 + 16 + mi) * AS + d0 + 16 + kx],
                                                x_s[(16 * wave + kx) * XS + mi], z, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) t_s[(d0 + 16 + 4 * mk + r) * AS + d0 + mi] = -z[r];
    } else {  // the upper blocks T01, T23 are zero
      const int d0 = 32 * (wave - 2);
#pragma unroll
      for (int r = 0; r < 4; ++r) t_s[(d0 + 4 * mk + r) * AS + d0 + 16 + mi] = 0.0f;
    }
    lds_barrier();
    const int qi = wave >> 1, qj = wave & 1;  // 16x16 quadrant of a 32x32 block
    {  // X = A21 T11 -> x_s
      f32x4 x = {};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int kx = 4 * kk + mk;
        x = __builtin_amdgcn_mfma_f32_16x16x4f32(at_s[kx * AS + 32 + 16 * qi + mi],
                                                t_s[kx * AS + 16 * qj + mi], x, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) x_s[(16 * qi + 4 * mk + r) * XS + 16 * qj + mi] = x[r];
    }
    lds_barrier();
    {  // T21 = -T22 X
      f32x4 y = {};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int kx = 4 * kk + mk;
        y = __builtin_amdgcn_mfma_f32_16x16x4f32(t_s[(32 + 16 * qi + mi) * AS + 32 + kx],
                                                x_s[kx * XS + 16 * qj + mi], y, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) t_s[(32 + 16 * qi + 4 * mk + r) * AS + 16 * qj + mi] = -y[r];
    }
    lds_barrier();

    // ---- Tw = T diag(beta exp(gc)), Tu = T diag(beta) in bf16 (T12 is zero)
    // (4 consecutive columns per thread: float4 in, 8-byte bf16 stores out)
#pragma unroll
    for (int e = tid; e < C * C / 4; e += 256) {
      const int i = e >> 4, j = (e & 15) * 4;
      const float4 t = (i < 32 && j >= 32) ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                           : *reinterpret_cast<const float4*>(t_s + i * AS + j);
      const float4 be = *reinterpret_cast<const float4*>(be_s + j);
      const float4 bt = *reinterpret_cast<const float4*>(beta_s + j);
      bf16 pw[4] = {(bf16)(t.x * be.x), (bf16)(t.y * be.y), (bf16)(t.z * be.z), (bf16)(t.w * be.w)};
      bf16 pu[4] = {(bf16)(t.x * bt.x), (bf16)(t.y * bt.y), (bf16)(t.z * bt.z), (bf16)(t.w * bt.w)};
      *reinterpret_cast<uint2*>(tw_s + i * CP + j) = *reinterpret_cast<uint2*>(pw);
      *reinterpret_cast<uint2*>(tu_s + i * CP + j) = *reinterpret_cast<uint2*>(pu);
    }
    lds_barrier();

    // ---- Tu rows to the workspace; -w^T = -(k^T Tw^T): wave -> 32-row block of
    // d; the accumulator holds 4 consecutive d of one token row l (8 bytes),
    // staged in the dead T region as [C][KP] bf16 so that the workspace rows
    // are then written in whole 16-byte chunks (16 lanes per 256-byte row)
#pragma unroll
    for (int e = tid; e < C * C / 8; e += 256) {
      const int row = e >> 3, c8 = (e & 7) * 8;
      *reinterpret_cast<u32x4*>(tu_ws + row * C + c8) =
          *reinterpret_cast<const u32x4*>(tu_s + row * CP + c8);
    }
    bf16* w_s = reinterpret_cast<bf16*>(r0);  // T is dead after the Tw / Tu conversion
    {
      const int db = wave;
#pragma unroll
      for (int lb = 0; lb < 2; ++lb) {
        f32x16 aw = {};
#pragma unroll
        for (int ks = 0; ks < C / 16; ++ks) {
          const bf16x8 ak = ld8(kT_s + (db * 32 + col) * CP + ks * 16 + half * 8);
          const bf16x8 btw = ld8(tw_s + (lb * 32 + col) * CP + ks * 16 + half * 8);
          aw = mfma(ak, btw, aw);
        }
        const int l = lb * 32 + col;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          bf16 pw[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) pw[e] = (bf16)(-aw[g4 * 4 + e]);
          const int d = db * 32 + g4 * 8 + half * 4;
          *reinterpret_cast<uint2*>(w_s + l * KP + d) = *reinterpret_cast<uint2*>(pw);
        }
      }
    }
    // ---- (decayed k)^T = (e^{gc_C - gc} o k)^T to the workspace, [DK][C]
    // rows of 16-byte chunks (k rows past T are zero already)
#pragma unroll
    for (int j = 0; j < DK * C / 8 / 256; ++j) {
      const int idx = tid + 256 * j;
      const int d = idx >> 3, c8 = (idx & 7) * 8;
      const bf16x8 kv = ld8(kT_s + d * CP + c8);
      const float4 f0 = *reinterpret_cast<const float4*>(dec_s + c8);
      const float4 f1 = *reinterpret_cast<const float4*>(dec_s + c8 + 4);
      bf16x8 o8;
      o8[0] = (bf16)((float)kv[0] * f0.x); o8[1] = (bf16)((float)kv[1] * f0.y);
      o8[2] = (bf16)((float)kv[2] * f0.z); o8[3] = (bf16)((float)kv[3] * f0.w);
      o8[4] = (bf16)((float)kv[4] * f1.x); o8[5] = (bf16)((float)kv[5] * f1.y);
      o8[6] = (bf16)((float)kv[6] * f1.z); o8[7] = (bf16)((float)kv[7] * f1.w);
      *reinterpret_cast<bf16x8*>(kd_ws + d * C + c8) = o8;
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < C * DK / 8 / 256; ++j) {  // -w rows, [C][DK]
      const int e = tid + 256 * j;
      const int row = e >> 4, c8 = (e & 15) * 8;
      *reinterpret_cast<u32x4*>(w_ws + row * DK + c8) =
          *reinterpret_cast<const u32x4*>(w_s + row * KP + c8);
    }
    lds_barrier();  // LDS is rewritten by the next chunk
  }
}

// ---------------------------------------------------------------------------
// kernel 2: the sequential recurrence over chunks and the output
// ---------------------------------------------------------------------------
// LDS images of one chunk's operands.  They are filled straight from memory
// by direct-to-LDS loads (global_load_lds_dwordx4: the 16 bytes of lane l
// land at base + 16 l, every lane choosing its own source address), one
// chunk ahead, into two slots.  Rows are stored unpadded with their 16-byte
// chunks XOR-swizzled by row, so that an MFMA operand read (16 consecutive
// rows, one chunk each) touches 16 distinct bank groups.
struct ChunkSlot {
  bf16 w[C * DK];    // -w rows l: chunk p of row l holds chunk p ^ (l & 15)
  bf16 q[C * DK];    // q rows, same swizzle
  bf16 tu[C * C];    // Tu rows: chunk p holds chunk p ^ ((l >> 1) & 7)
  bf16 aqk[C * C];   // Aqk rows, same
  bf16 kd[DK * C];   // (decayed k)^T rows d, same
  float fac[kFacN];  // scale e^{gc_l} (l < C), e^{gc_C} at [C]
};

// element offset of 16-byte chunk `kc` of row `r` in a swizzled image with
// 128-element (16-chunk) or 64-element (8-chunk) rows
__device__ __forceinline__ int swz16(int r, int kc) { return r * DK + ((kc ^ (r & 15)) << 3); }
__device__ __forceinline__ int swz8(int r, int kc) { return r * C + ((kc ^ ((r >> 1) & 7)) << 3); }

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// Fill the swizzled image `dst` (NCH 16-byte chunks, CPR per row) from the
// rows `src + min(r, rmax) * stride` (elements).  Each of the 4 wavefronts
// issues every 4th 1 KB window (64 chunks).
template <int CPR, int NCH>
__device__ __forceinline__ void gather_rows(bf16* dst, const bf16* src, int64_t stride, int rmax,
                                            int wave, int lane) {
  static_assert(NCH % 256 == 0, "whole windows for every wavefront");
#pragma unroll
  for (int i = 0; i < NCH / 256; ++i) {
    const int win = 4 * i + wave;
    const int ch = win * 64 + lane;
    const int r = ch / CPR, p = ch % CPR;
    const int key = CPR == 16 ? (r & 15) : ((r >> 1) & 7);
    const bf16* g = src + (int64_t)min(r, rmax) * stride + ((p ^ key) << 3);
    __builtin_amdgcn_global_load_lds(g, (lds_void_ptr)(dst + win * 512), 16, 0, 0);
  }
}

__global__ __launch_bounds__(512) void gdn_recur_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ v, const float* __restrict__ h0,
    const uint8_t* __restrict__ ws, bf16* __restrict__ o, float* __restrict__ hT, int B, int T,
    int H, int NC) {
  constexpr int SP = DK + 8;  // row stride of S^T [v][d]
  // two separate objects, so that the compiler can tell a slot being read
  // from the one the direct-to-LDS loads are filling
  __shared__ __attribute__((aligned(16))) ChunkSlot slot0;
  __shared__ __attribute__((aligned(16))) ChunkSlot slot1;
  __shared__ __attribute__((aligned(16))) bf16 st_s[VS * SP];      // bf16 S^T (slice)
  __shared__ __attribute__((aligned(16))) bf16 wt_s[VS * CP];      // bf16 W^T (slice)
  __shared__ __attribute__((aligned(16))) bf16 vt_s[2][VS * CP];   // v^T (slice)
  __shared__ __attribute__((aligned(16))) uint32_t touch_s[64];    // landing area of L2 prefetches

  // waves 0-3 compute; waves 4-7 (one per SIMD beside them) only move the
  // next chunk's operands, so that the bounded rate of the CU's load path
  // never holds up a compute wavefront's instruction stream
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool loader = wave >= 4;
  const int lw = wave & 3;     // index among the loaders / among the compute waves
  const int ltid = tid & 255;  // thread index inside its group of four wavefronts
  const int col = lane & 31, half = lane >> 5;
  // the VS-slices of one head run on the same XCD (they share q, w, Aqk, kd)
  const int total = gridDim.x;
  int id = blockIdx.x;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  const int nvs = DV / VS;
  const int vs = id % nvs;
  const int bh = id / nvs;
  const int h = bh % H, b = bh / H;
  const int v0 = vs * VS;
  const int64_t tok_stride = (int64_t)H * DK;
  const int rblk = wave & 1;         // chunk rows 32*rblk .. 32*rblk+31 (A operands)
  const int arow = rblk * 32 + col;  // A-operand row of this lane
  const int vrow = ltid >> 2, vcol = (ltid & 3) * 8;

  // chunk c's operands (loader wavefronts): the LDS images of slot `sl`
  // (direct loads) and this thread's 16 bytes of the v slice (register,
  // transposed into LDS later)
  auto load = [&](int c, ChunkSlot& sl, u32x4& vr) {
    const int t0 = c * C;
    const int last = min(C, T - t0) - 1;  // rows past T read the last row (see below)
    const uint8_t* wsc = ws + (((size_t)b * H + h) * NC + c) * kChunkBytes;
    // Rows past T are clamped onto the chunk's last row rather than zeroed:
    // their q only reaches output rows that are not stored, and their v only
    // meets columns of Tu that are exactly zero (beta = 0).
    vr = *reinterpret_cast<const u32x4*>(
        v + ((int64_t)b * T + t0 + min(vrow, last)) * tok_stride + (int64_t)h * DV + v0 + vcol);
    gather_rows<16, C * DK / 8>(sl.w, reinterpret_cast<const bf16*>(wsc + kWOff), DK, C - 1, lw,
                                lane);
    gather_rows<16, C * DK / 8>(sl.q, q + ((int64_t)b * T + t0) * tok_stride + (int64_t)h * DK,
                                tok_stride, last, lw, lane);
    gather_rows<8, C * C / 8>(sl.tu, reinterpret_cast<const bf16*>(wsc + kTuOff), C, C - 1, lw,
                              lane);
    gather_rows<8, C * C / 8>(sl.aqk, reinterpret_cast<const bf16*>(wsc + kAqkOff), C, C - 1, lw,
                              lane);
    gather_rows<8, DK * C / 8>(sl.kd, reinterpret_cast<const bf16*>(wsc + kKdOff), C, DK - 1, lw,
                               lane);
    if (lw == 0 && lane < kFacN / 4)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const float*>(wsc + kFacOff) + lane * 4,
                                       (lds_void_ptr)sl.fac, 16, 0, 0);
  };
  // L2 prefetch of chunk c (loader wavefronts): one 4-byte load per 128-byte
  // line of its workspace record and q rows (the four V-slices of a head
  // share them, every fourth line each) and of this slice's v rows, landing
  // in a scratch LDS word.  Every thread issues exactly one (spare threads
  // repeat a line), so the wait counts stay exact.
  auto touch = [&](int c) {
    constexpr int kWsLines = (int)((kChunkBytes + 127) / 128);
    constexpr int kShared = kWsLines + 2 * C;  // + q rows, two lines each
    constexpr int kPerSlice = (kShared + 3) / 4;
    const int t0 = c * C;
    const int last = min(C, T - t0) - 1;
    const uint8_t* wsc = ws + (((size_t)b * H + h) * NC + c) * kChunkBytes;
    const void* a;
    const int j = min(ltid, kPerSlice - 1) * 4 + vs;
    if (ltid < kPerSlice && j < kShared) {
      a = j < kWsLines ? static_cast<const void*>(wsc + (size_t)j * 128)
                       : static_cast<const void*>(
                             q + ((int64_t)b * T + t0 + min((j - kWsLines) >> 1, last)) *
                                     tok_stride +
                             (int64_t)h * DK + ((j - kWsLines) & 1) * 64);
    } else {
      const int r = min(max(ltid - kPerSlice, 0), C - 1);
      a = v + ((int64_t)b * T + t0 + min(r, last)) * tok_stride + (int64_t)h * DV + v0;
    }
    __builtin_amdgcn_global_load_lds(a, (lds_void_ptr)touch_s, 4, 0, 0);
  };
  // v^T of a loaded chunk into LDS slot `buf`
  auto stage_v = [&](const u32x4& vr, int buf) {
    const bf16* ve = reinterpret_cast<const bf16*>(&vr);
#pragma unroll
    for (int j = 0; j < 8; ++j) vt_s[buf][(vcol + j) * CP + vrow] = ve[j];
  };

  // state rows of a compute wave: d = 32 * wave + (r / 4) * 8 + half * 4 + r % 4
  f32x16 s_acc = {};
  if (!loader) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * wave + (r >> 2) * 8 + half * 4 + (r & 3);
      s_acc[r] = h0 ? h0[(((int64_t)b * H + h) * DK + d) * DV + v0 + col] : 0.0f;
    }
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

  // one chunk: `cur` holds its operands (and vt_s[c & 1], st_s); the loader
  // wavefronts fill `nxt` and vt_s[(c + 1) & 1] meanwhile
  auto step = [&](int c, const ChunkSlot& cur, ChunkSlot& nxt) {
    const int buf = c & 1;
    const bool more = c + 1 < NC;
    if (loader) {
      // chunk c + 1 into `nxt` (past the end: the last chunk again, never
      // read); after v^T is staged, the L2 prefetch of chunk c + 2.  Both are
      // unconditional so that the wait counts stay exact
      u32x4 vr;
      load(more ? c + 1 : NC - 1, nxt, vr);
      lds_barrier();  // (barrier B)
      if (more) stage_v(vr, buf ^ 1);
      touch(min(c + 2, NC - 1));
      // a wavefront's counters cover only its own loads: each loader waits
      // for its share of the next chunk's images (everything but the one
      // prefetch issued last: vmcnt(1)) before the barrier
      __builtin_amdgcn_s_waitcnt(0x0F71);
      lds_barrier();  // (barrier A)
      return;
    }
    const int t0 = c * C;
    const int n = min(C, T - t0);

    // waves 0, 1: W = Tu v - w S (rows 32 rblk ..); waves 2, 3: the output
    // in the transposed orientation, o^T = S^T q^T (tokens 32 rblk ..), so
    // that a lane owns one token: its row factor is one scalar and its 16
    // values are 4 runs of 4 consecutive v, stored straight to memory
    f32x16 acc = {};
    if (wave < 2) {
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks)
        acc = mfma(ld8(cur.tu + swz8(arow, ks * 2 + half)),
                   ld8(vt_s[buf] + col * CP + ks * 16 + half * 8), acc);
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks)
        acc = mfma(ld8(cur.w + swz16(arow, ks * 2 + half)),
                   ld8(st_s + col * SP + ks * 16 + half * 8), acc);
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16 p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = (bf16)acc[g4 * 4 + e];
        const int cl = rblk * 32 + g4 * 8 + half * 4;
        *reinterpret_cast<uint2*>(wt_s + col * CP + cl) = *reinterpret_cast<uint2*>(p);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks)
        acc = mfma(ld8(st_s + col * SP + ks * 16 + half * 8),
                   ld8(cur.q + swz16(arow, ks * 2 + half)), acc);
      const float f = cur.fac[arow];  // scale e^{gc} of this lane's token
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] *= f;
    }
    lds_barrier();  // (barrier B) W^T visible

    if (wave >= 2) {  // o^T += W^T Aqk^T, then this lane's token row to memory
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks)
        acc = mfma(ld8(wt_s + col * CP + ks * 16 + half * 8),
                   ld8(cur.aqk + swz8(arow, ks * 2 + half)), acc);
      if (arow < n) {
        bf16* orow = o + ((int64_t)b * T + t0 + arow) * tok_stride + (int64_t)h * DV + v0;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          bf16 p[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) p[e] = (bf16)acc[g4 * 4 + e];
          *reinterpret_cast<uint2*>(orow + g4 * 8 + half * 4) = *reinterpret_cast<uint2*>(p);
        }
      }
    }
    // S <- exp(gc_C) S + (decayed k)^T W   (rows 32 * wave .. of the state)
    const float dec = cur.fac[C];
#pragma unroll
    for (int r = 0; r < 16; ++r) s_acc[r] *= dec;
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks)
      s_acc = mfma(ld8(cur.kd + swz8(32 * wave + col, ks * 2 + half)),
                   ld8(wt_s + col * CP + ks * 16 + half * 8), s_acc);
    publish_state();
    lds_barrier();  // (barrier A) next chunk's images, S^T and v^T visible
  };

  if (NC > 0 && loader) {
    u32x4 vr;
    load(0, slot0, vr);
    stage_v(vr, 0);
    touch(min(1, NC - 1));
    __builtin_amdgcn_s_waitcnt(0x0F71);
  }
  if (!loader) publish_state();
  lds_barrier();
  int c = 0;
  for (; c + 1 < NC; c += 2) {
    step(c, slot0, slot1);
    step(c + 1, slot1, slot0);
  }
  if (c < NC) step(c, slot0, slot1);

  if (loader) {
    __builtin_amdgcn_s_waitcnt(0);  // no load may land after the workgroup's LDS is released
    return;
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
    gdn::gdn_prep_kernel<<<dim3((unsigned)std::min<int64_t>(nblk, 2 * device_cu_count())), dim3(256), 0, s>>>(
        qb, kb, g, beta, static_cast<uint8_t*>(ws), (int)B, (int)T, (int)H, nc, scale);
  gdn::gdn_recur_kernel<<<dim3((unsigned)(B * H * (gdn::DV / gdn::VS))), dim3(512), 0, s>>>(
      qb, static_cast<const bf16*>(v), h0, static_cast<const uint8_t*>(ws),
      static_cast<bf16*>(o), hT, (int)B, (int)T, (int)H, nc);
  return launch_status();
}
