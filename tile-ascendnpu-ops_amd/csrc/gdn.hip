// Gated delta-rule (gated DeltaNet) chunked prefill for gfx950
// (tileops_gdn_prefill_fwd).
//
// Recurrence per (batch b, head h), token t (state S is K x V, fp32):
//   S_t = exp(g_t) S_{t-1} + beta_t k_t (v_t - exp(g_t) S_{t-1}^T k_t)^T,   o_t = scale q_t^T S_t
//
// Chunked (C = 64 tokens) WY form.  Inside a chunk, with gc the cumulative
// log-decay, G[l,s] = exp(gc_l - gc_s) (l >= s), A = strictly_lower(beta_l
// G[l,s] k_l.k_s) and T = (I + A)^-1:
//   Tu  = T diag(beta)                                (C x C)   \ independent of S:
//   Aqk = scale * lower_incl(G o (q k^T))             (C x C)   / kernel 1, parallel
//   W   = Tu (v - exp(gc) o (k S))                              \
//   o   = scale exp(gc) o (q S) + Aqk W                          > kernel 2, sequential
//   S  <- exp(gc_C) S + k^T (exp(gc_C - gc) o W)                /  over chunks
// (W = Tu v - w S with w = T diag(beta exp(gc)) k, regrouped so that the
// recurrence multiplies k itself and kernel 1 hands over only two C x C
// matrices and the per-token factors.)  Only differences gc_l - gc_s <= 0,
// gc_C - gc_l <= 0 and gc <= 0 are ever exponentiated, so nothing overflows
// however strong the decay.
//
// Kernel 1 (persistent, two workgroups per CU, the next chunk's q / k / g
// / beta loaded while the current one is processed): K K^T and Q K^T on bf16
// MFMA, the 64x64 unit-lower-triangular inverse in fp32 (16x16 diagonal
// blocks by substitution, one wavefront each, the off-diagonal blocks by
// products on fp32 MFMA), Tu, Aqk and the factors to a 17 KB record per
// chunk.
// Kernel 2 (one workgroup per (b, h, 32-wide slice of V), 8 wavefronts):
// four compute wavefronts keep the state slice in MFMA accumulators
// (wavefront i owns key rows 32i..32i+31) and exchange its bf16 copy, U =
// v - exp(gc) o (k S) and W through LDS; four loader wavefronts bring the
// next chunk's k, q, v slice and record into LDS with direct-to-LDS loads
// meanwhile.  Three workgroup barriers per chunk.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace tileops {
namespace gdn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int C = 64;    // chunk length
constexpr int DK = 128;  // key dim
constexpr int DV = 128;  // value dim
constexpr int VS = 32;   // value columns per kernel-2 workgroup
constexpr int KP = DK + 8;  // LDS row stride of a natural [C][DK] tile (elements)
constexpr int CP = C + 8;   // LDS row stride of a transposed [*][C] tile (elements)
constexpr float kLog2e = 1.4426950408889634f;

// workspace record per chunk
constexpr size_t kTuOff = 0;                                  // Tu   [C][C] bf16
constexpr size_t kAqkOff = kTuOff + (size_t)C * C * 2;        // Aqk  [C][C] bf16
constexpr size_t kFacOff = kAqkOff + (size_t)C * C * 2;       // factors, f32 [kFacN]
constexpr int kFacN = 256;
// factor slots: scale e^{gc_l}, e^{gc_l}, e^{gc_C - gc_l} (l < C), e^{gc_C}
constexpr int kFacOut = 0, kFacG = C, kFacD = 2 * C, kFacChunk = 3 * C;
constexpr size_t kChunkBytes = kFacOff + (size_t)kFacN * 4;  // 17,408

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) {  // 16-byte load (LDS or global)
  return *reinterpret_cast<const bf16x8*>(p);
}

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Inclusive prefix sum over the 64 lanes of a wavefront by DPP lane moves,
// with no LDS round trip (a shuffle-based scan waits on the LDS queue, which
// the other workgroups of the CU keep busy): Hillis-Steele inside each row
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

// Four fp32 values as four bf16 in one 8-byte word.
__device__ __forceinline__ uint2 pack_bf16x4(float a, float b, float c, float d) {
  bf16 p[4] = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
  return *reinterpret_cast<uint2*>(p);
}

// ---------------------------------------------------------------------------
// kernel 1: per-chunk preparation
// ---------------------------------------------------------------------------
// LDS plan (three workgroups would fit one CU; two run per CU, so that the
// kernel keeps every value in registers: at three the compiler spills):
//   r0: k natural [C][KP] bf16 (K K^T)            -> T (fp32 [C][AS], inverse)
//   r1: A^T fp32 [C][AS] (A^T[m][i] = A[i][m])
//   x_s: A10 T00 / A32 T22 / A21 T11 (fp32)
constexpr int AS = 72;  // fp32 row stride of A^T / T (288 bytes: float4-aligned rows)
constexpr int XS = 36;  // fp32 row stride of X

// Global operands of one chunk for one thread, loaded a chunk ahead: 16
// bytes (dims 8 (tid & 15) ..) of k and q rows 16 i + tid / 16 (i < 4), so
// that every load instruction reads four whole 256-byte rows, and g / beta
// of token `lane`.  Rows past T load the chunk's last row and are zeroed
// where they are staged.
struct PrepLoads {
  u32x4 kr[4], qr[4];
  float g, beta;
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const float* __restrict__ g,
    const float* __restrict__ beta, uint8_t* __restrict__ ws, int B, int T, int H, int c0, int NS,
    float scale) {
  __shared__ __attribute__((aligned(16))) float r0[C * AS];
  __shared__ __attribute__((aligned(16))) float r1[C * AS];
  __shared__ __attribute__((aligned(16))) float x_s[32 * XS];
  __shared__ __attribute__((aligned(16))) float gc_s[C], beta_s[C];
  __shared__ __attribute__((aligned(16))) bf16 q_s[C * KP];
  static_assert(C * KP * 2 <= C * AS * 4, "k tile must fit the T region");
  bf16* k_s = reinterpret_cast<bf16*>(r0);
  float* t_s = r0;
  float* at_s = r1;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int rb = wave == 0 ? 0 : 1;  // Q K^T / K K^T block of waves 0-2
  const int cb = wave == 2 ? 1 : 0;
  const int lrow = tid >> 4, lchk = tid & 15;  // row (of 16) and 16-byte chunk of the loads
  const int64_t tok_stride = (int64_t)H * DK;  // DK == DV
  // record blk of the workspace: (b, h) = blk / NS, chunk c0 + blk % NS
  const uint64_t nblk = (uint64_t)B * H * NS;

  auto load = [&](uint64_t blk, PrepLoads& L) {
    const int chunk = c0 + (int)(blk % NS), bh = (int)(blk / NS);
    const int h = bh % H, b = bh / H;
    const int t0 = chunk * C, n = min(C, T - t0);
    const int64_t off0 = ((int64_t)b * T + t0) * tok_stride + (int64_t)h * DK + lchk * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t off = off0 + (int64_t)min(16 * i + lrow, n - 1) * tok_stride;
      L.kr[i] = *reinterpret_cast<const u32x4*>(k + off);
      L.qr[i] = *reinterpret_cast<const u32x4*>(q + off);
    }
    const int64_t gi = ((int64_t)b * T + t0 + min(lane, n - 1)) * H + h;
    L.g = g[gi];
    L.beta = beta[gi];
  };

  // Persistent: workgroup i takes chunks i, i + grid, ...; the next chunk's
  // loads are issued as soon as the current one's registers are consumed.
  PrepLoads cur;
  // (see the settle before the record stores below; here for the first
  // chunk's loads, so that both paths into the loop arrive settled)
  auto settle = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(cur.kr[i]), "+v"(cur.qr[i]));
    asm volatile("" : "+v"(cur.g), "+v"(cur.beta));
  };
  uint64_t blk = blockIdx.x;
  if (blk < nblk) load(blk, cur);
  settle();
  for (; blk < nblk; blk += gridDim.x) {
    const int chunk = c0 + (int)(blk % NS);
    const int t0 = chunk * C;
    const int n = min(C, T - t0);
    uint8_t* wsc = ws + (size_t)blk * kChunkBytes;
    bf16* tu_ws = reinterpret_cast<bf16*>(wsc + kTuOff);
    bf16* aqk_ws = reinterpret_cast<bf16*>(wsc + kAqkOff);
    float* fac_ws = reinterpret_cast<float*>(wsc + kFacOff);

    // ---- stage k and q; rows past T are 0
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * i + lrow;
      if (row >= n) cur.kr[i] = cur.qr[i] = u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(k_s + row * KP + lchk * 8) = cur.kr[i];
      *reinterpret_cast<u32x4*>(q_s + row * KP + lchk * 8) = cur.qr[i];
    }
    if (wave == 3) {
      float x = lane < n ? cur.g : 0.0f;
      const float bt = lane < n ? cur.beta : 0.0f;
      x = wave_inclusive_sum(x);  // gc: inclusive prefix sum over the chunk
      gc_s[lane] = x;
      beta_s[lane] = bt;
      // the factors the recurrence applies: scale e^{gc} per output row,
      // e^{gc} on k S, e^{gc_C - gc} on W for the state update, e^{gc_C}
      const float gl = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), C - 1));
      const float eg = exp2f_fast(x * kLog2e);
      fac_ws[kFacOut + lane] = scale * eg;
      fac_ws[kFacG + lane] = eg;
      fac_ws[kFacD + lane] = exp2f_fast((gl - x) * kLog2e);
      fac_ws[kFacChunk + lane] = lane == 0 ? exp2f_fast(gl * kLog2e) : 0.0f;
    }
    lds_barrier();

    // ---- K K^T -> A^T (fp32, LDS) and Q K^T -> Aqk (bf16, to the record),
    // in 32x32 blocks (row block rb, column block cb).  Only the strictly
    // lower parts of the diagonal blocks and the block A21 of A are ever
    // read back; the block l < 32 <= s of Aqk is zero.
    if (wave < 3) {
      // transposed orientation: k rows s of block cb as the A operand, k / q
      // rows l of block rb as B, so that a lane owns one row l (column of the
      // result) and its 16 values run over s: [s][l] = k_s . k_l and k_s . q_l
      f32x16 kk = {}, qk = {};
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks) {
        const bf16x8 bs = ld8(k_s + (cb * 32 + col) * KP + ks * 16 + half * 8);
        const bf16x8 bl = ld8(k_s + (rb * 32 + col) * KP + ks * 16 + half * 8);
        const bf16x8 a = ld8(q_s + (rb * 32 + col) * KP + ks * 16 + half * 8);
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
        float qv[4];
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
          qv[e] = scale * gd * qk[r];
        }
        *reinterpret_cast<uint2*>(aqk_ws + l * C + s0) = pack_bf16x4(qv[0], qv[1], qv[2], qv[3]);
      }
    } else {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        *reinterpret_cast<uint2*>(aqk_ws + col * C + 32 + g4 * 8 + half * 4) = make_uint2(0u, 0u);
    }
    if (blk + gridDim.x < nblk) load(blk + gridDim.x, cur);  // operands consumed: next chunk
    lds_barrier();

    // ---- T = (I + A)^-1, blocked by 16: the four diagonal blocks Tbb by
    // substitution (wave w: block w, lane j: column j; p[i] accumulates
    // sum_m A[i][m] T[m][j]), then on fp32 MFMA T10 = -T11 (A10 T00),
    // T32 = -T33 (A32 T22) and, with 32-row blocks, T21 = -T22 (A21 T11).
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
    // no barrier: each of waves 0, 1 reads back only its own Y rows, T11 /
    // T33 are settled since the substitution's barrier, and the zero blocks
    // written below are read by no wavefront before the next barrier.  Lanes
    // read Y values other lanes of the same wavefront wrote: the fences keep
    // the compiler from moving those LDS reads above the writes (the LDS
    // operations of one wavefront execute in order, so no s_barrier is needed)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

    // The next chunk's operands (loaded after the products above) pass
    // through an empty asm before the record stores below: the compiler
    // resolves their loads here, while only older stores are in flight.
    // Otherwise its bookkeeping across the loop places those waits at their
    // first use, after these stores, and waits for the stores as well.
    settle();

    // ---- Tu = T diag(beta) in bf16 to the record (T12 is zero); 4
    // consecutive columns per thread: float4 in, one 8-byte store out
#pragma unroll
    for (int e = tid; e < C * C / 4; e += 256) {
      const int i = e >> 4, j = (e & 15) * 4;
      const float4 t = (i < 32 && j >= 32) ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                           : *reinterpret_cast<const float4*>(t_s + i * AS + j);
      const float4 bt = *reinterpret_cast<const float4*>(beta_s + j);
      *reinterpret_cast<uint2*>(tu_ws + i * C + j) =
          pack_bf16x4(t.x * bt.x, t.y * bt.y, t.z * bt.z, t.w * bt.w);
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
  bf16 k[C * DK];    // k rows l: chunk p of row l holds chunk p ^ (l & 15)
  bf16 q[C * DK];    // q rows, same swizzle
  bf16 tu[C * C];    // Tu rows: chunk p holds chunk p ^ ((l >> 1) & 7)
  bf16 aqk[C * C];   // Aqk rows, same
  bf16 v[C * VS];    // v slice rows [token][VS], unswizzled (read transposed)
  float fac[kFacN];  // the record's factors
};

// element offset of 16-byte chunk `kc` of row `r` in a swizzled image with
// 128-element (16-chunk) or 64-element (8-chunk) rows
__device__ __forceinline__ int swz16(int r, int kc) { return r * DK + ((kc ^ (r & 15)) << 3); }
__device__ __forceinline__ int swz8(int r, int kc) { return r * C + ((kc ^ ((r >> 1) & 7)) << 3); }

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void_ptr)p;
}

// Direct-to-LDS loads: lane l reads 16 (4) bytes at `base + off` (base
// uniform, in SGPRs; off a per-lane byte offset) and they land at LDS byte
// address lds + 16 l (4 l).  Issued as inline assembly so that the compiler
// does not track the LDS writes: otherwise it waits for every outstanding
// vector memory operation (the output stores included) before each LDS
// access of the compute wavefronts.  Every wait for these loads is explicit
// (vmcnt) and followed by a workgroup barrier before any wavefront reads
// the data.
// A wavefront-uniform pointer moved into SGPRs: both 32-bit halves are read
// from the first active lane and joined as unsigned words (readfirstlane
// returns int, which must not be sign-extended into the high word).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | (uint64_t)lo);
}

// The compiler's hazard checks do not look into inline assembly, so each
// load starts with the wait states the ISA requires before it: 5 after a
// VALU write (v_readfirstlane) of an SGPR the load reads (its base), 1
// after the SALU write of M0.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(uniform_ptr(base)),
               "{m0}"(lds) : "memory");
}

// Fill the swizzled image `dst` (NCH 16-byte chunks, CPR per row) from the
// rows `src + min(r, rmax) * stride` (elements; `src` uniform).  Each of the
// 4 wavefronts issues every 4th 1 KB window (64 chunks).
template <int CPR, int NCH>
__device__ __forceinline__ void gather_rows(bf16* dst, const bf16* src, int64_t stride, int rmax,
                                            int wave, int lane) {
  static_assert(NCH % 256 == 0, "whole windows for every wavefront");
#pragma unroll
  for (int i = 0; i < NCH / 256; ++i) {
    const int win = 4 * i + wave;
    const int ch = win * 64 + lane;
    const int r = ch / CPR, p = ch % CPR;
    const int key = CPR == 16 ? (r & 15) : CPR == 8 ? ((r >> 1) & 7) : 0;
    const uint32_t off = (uint32_t)(((int64_t)min(r, rmax) * stride + ((p ^ key) << 3)) * 2);
    lds_dma16(src, off, lds_addr(dst + win * 512));
  }
}

// The kernel runs chunks c0 .. c1 - 1 of every head, reading their records
// at (b H + h) NS + (c - c0) of the workspace, starting from state h0 (zero
// when null) and leaving the state in hT.  h0 may be hT itself (a segment
// continuing the previous one): each workgroup reads its own state slice
// before its first chunk and writes it after its last.
__global__ __launch_bounds__(512) void gdn_recur_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* h0, const uint8_t* __restrict__ ws, bf16* __restrict__ o, float* hT, int B,
    int T, int H, int c0, int c1, int NS) {
  constexpr int SP = DK + 8;  // row stride of S^T [v][d]
  // two separate objects, so that the compiler can tell a slot being read
  // from the one the direct-to-LDS loads are filling
  __shared__ __attribute__((aligned(16))) ChunkSlot slot0;
  __shared__ __attribute__((aligned(16))) ChunkSlot slot1;
  __shared__ __attribute__((aligned(16))) bf16 st_s[VS * SP];      // bf16 S^T (slice)
  __shared__ __attribute__((aligned(16))) bf16 ut_s[VS * CP];      // U^T (slice)
  __shared__ __attribute__((aligned(16))) bf16 wt_s[VS * CP];      // W^T (slice)
  __shared__ __attribute__((aligned(16))) bf16 dwt_s[VS * CP];     // (e^{gc_C - gc} o W)^T
  __shared__ __attribute__((aligned(16))) uint32_t touch_s[64];    // landing area of L2 prefetches

  // waves 0-3 compute; waves 4-7 (one per SIMD beside them) only move the
  // next chunk's operands, so that the bounded rate of the CU's load path
  // never holds up a compute wavefront's instruction stream
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool loader = wave >= 4;
  const int lw = wave & 3;     // index among the loaders / among the compute waves
  const int ltid = tid & 255;  // thread index inside its group of four wavefronts
  const int col = lane & 31, half = lane >> 5;
  // the VS-slices of one head run on the same XCD (they share q, k and the
  // chunk records through its L2)
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

  // k^T (A operand of the state update) through transpose reads of the
  // natural k image: in each group of 16 lanes, lane j points at 4 dims
  // (d0 + 4 (j % 4) ..) of token row t0 + j / 4 and receives dim d0 + j of
  // those 4 tokens.  Lane group g covers dims 32 wave + 16 (g & 1) .. and
  // tokens 8 (g >> 1) .. of each 16-token step; the second read takes the
  // next 4 tokens.  The swizzle key (t & 15) does not depend on the step, so
  // the step is a constant 16-row (4 KB) offset.
  int ktoff[2] = {0, 0};
  if (!loader) {
    const int g16 = lane >> 4, j16 = lane & 15;
    const int dd = 32 * wave + 16 * (g16 & 1) + 4 * (j16 & 3);
#pragma unroll
    for (int rd = 0; rd < 2; ++rd) {
      const int t = 8 * (g16 >> 1) + 4 * rd + (j16 >> 2);
      ktoff[rd] = t * DK + (((dd >> 3) ^ (t & 15)) << 3) + (dd & 7);
    }
  }
  // v^T (columns of the natural v image) for the U update: 4 consecutive
  // token rows (32 rblk + 8 g4 + 4 half ..) of v column `col`, by the same
  // transpose read: lane j of a 16-lane group points at 4 columns
  // (16 (g & 1) + 4 (j % 4) ..) of token row 4 (g >> 1) + j / 4 (+ the g4
  // and rblk terms, constants of 8 and 32 rows).
  int vtoff = 0;
  {
    const int g16 = lane >> 4, j16 = lane & 15;
    vtoff = (32 * rblk + 4 * (g16 >> 1) + (j16 >> 2)) * VS + 16 * (g16 & 1) + 4 * (j16 & 3);
  }
  auto read_vt4 = [&](const bf16* vimg, int g4) -> uint2 {
    const uint32_t a = lds_addr(vimg) + (uint32_t)((vtoff + g4 * 8 * VS) * 2);
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(uintptr_t)a));
  };
  auto read_kt = [&](const bf16* kimg, int ks) -> bf16x8 {
    const uint32_t base = lds_addr(kimg) + (uint32_t)(ks * 16 * DK * 2);
    const v4i16 x0 =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(uintptr_t)(base + ktoff[0] * 2));
    const v4i16 x1 =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(uintptr_t)(base + ktoff[1] * 2));
    const u32x2 y0 = __builtin_bit_cast(u32x2, x0), y1 = __builtin_bit_cast(u32x2, x1);
    const u32x4 w4 = {y0.x, y0.y, y1.x, y1.y};
    return __builtin_bit_cast(bf16x8, w4);
  };

  // chunk c's operands (loader wavefronts), all by direct-to-LDS loads into
  // the images of slot `sl`, in two parts so that the CU's load path is busy
  // in two phases of a step rather than one: the q and k rows, then the
  // record and the v slice.
  // Rows past T are clamped onto the chunk's last row rather than zeroed:
  // their k only meets columns of Tu and rows of W that are exactly zero
  // (beta = 0 there), their v only those columns of Tu, and their q only
  // output rows that are not stored.
  auto load_rows = [&](int c, ChunkSlot& sl) {
    const int t0 = c * C;
    const int last = min(C, T - t0) - 1;
    const int64_t row0 = ((int64_t)b * T + t0) * tok_stride + (int64_t)h * DK;
    gather_rows<16, C * DK / 8>(sl.k, k + row0, tok_stride, last, lw, lane);
    gather_rows<16, C * DK / 8>(sl.q, q + row0, tok_stride, last, lw, lane);
  };
  auto load_record = [&](int c, ChunkSlot& sl) {
    const int t0 = c * C;
    const int last = min(C, T - t0) - 1;
    const uint8_t* wsc = ws + (((size_t)b * H + h) * NS + (c - c0)) * kChunkBytes;
    const int64_t row0 = ((int64_t)b * T + t0) * tok_stride + (int64_t)h * DV;
    gather_rows<8, C * C / 8>(sl.tu, reinterpret_cast<const bf16*>(wsc + kTuOff), C, C - 1, lw,
                              lane);
    gather_rows<8, C * C / 8>(sl.aqk, reinterpret_cast<const bf16*>(wsc + kAqkOff), C, C - 1,
                              lw, lane);
    gather_rows<VS / 8, C * VS / 8>(sl.v, v + row0 + v0, tok_stride, last, lw, lane);
    if (lw == 0) lds_dma16(wsc + kFacOff, (uint32_t)lane * 16, lds_addr(sl.fac));
  };
  // L2 prefetch of chunk c (loader wavefronts): one 4-byte load per 128-byte
  // line of its record and of its q and k rows (the four V-slices of a head
  // share them, every fourth line each) and of this slice's v rows, landing
  // in a scratch LDS word.  Every thread issues exactly one (spare threads
  // repeat a line), so the wait counts stay exact.
  auto touch = [&](int c) {
    constexpr int kWsLines = (int)((kChunkBytes + 127) / 128);
    constexpr int kShared = kWsLines + 4 * C;  // + q and k rows, two lines each
    constexpr int kPerSlice = (kShared + 3) / 4;
    static_assert(kPerSlice + C <= 256, "one prefetch per loader thread");
    const int t0 = c * C;
    const int last = min(C, T - t0) - 1;
    const uint8_t* wsc = ws + (((size_t)b * H + h) * NS + (c - c0)) * kChunkBytes;
    const int64_t row0 = ((int64_t)b * T + t0) * tok_stride + (int64_t)h * DK;
    const void* a;
    const int j = min(ltid, kPerSlice - 1) * 4 + vs;
    if (ltid < kPerSlice && j < kShared) {
      if (j < kWsLines) {
        a = wsc + (size_t)j * 128;
      } else {
        const int r = j - kWsLines;  // 4 lines per token row: q then k, two halves each
        a = ((r & 2) ? k : q) + row0 + (int64_t)min(r >> 2, last) * tok_stride + (r & 1) * 64;
      }
    } else {
      const int r = min(max(ltid - kPerSlice, 0), C - 1);
      a = v + row0 + (int64_t)min(r, last) * tok_stride + v0;
    }
    asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, off" : : "v"(a), "{m0}"(lds_addr(touch_s))
                 : "memory");
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
      const int d = 32 * wave + g4 * 8 + half * 4;
      *reinterpret_cast<uint2*>(st_s + col * SP + d) =
          pack_bf16x4(s_acc[g4 * 4 + 0], s_acc[g4 * 4 + 1], s_acc[g4 * 4 + 2], s_acc[g4 * 4 + 3]);
    }
  };
  // a 32-row block of a [token][v] accumulator (rows 32 rblk + ..; lane: v
  // column `col`) as bf16 into the transposed image [v][token], each value
  // scaled by the factor of its token row
  auto put_rows_t = [&](bf16* img, const f32x16& acc, const float* fac) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int cl = rblk * 32 + g4 * 8 + half * 4;
      const float4 f = fac ? *reinterpret_cast<const float4*>(fac + cl)
                           : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
      *reinterpret_cast<uint2*>(img + col * CP + cl) =
          pack_bf16x4(acc[g4 * 4 + 0] * f.x, acc[g4 * 4 + 1] * f.y, acc[g4 * 4 + 2] * f.z,
                      acc[g4 * 4 + 3] * f.w);
    }
  };

  // one chunk: `cur` holds its operands (and st_s); the loader wavefronts
  // fill `nxt` meanwhile
  auto step = [&](int c, const ChunkSlot& cur, ChunkSlot& nxt) {
    if (loader) {
      // chunk c + 1 into `nxt` (past the end: the last chunk again, never
      // read), then the L2 prefetch of chunk c + 2.  Both are unconditional
      // so that the wait counts stay exact
      load_rows(min(c + 1, c1 - 1), nxt);
      lds_barrier();  // (barrier U)
      load_record(min(c + 1, c1 - 1), nxt);
      touch(min(c + 2, c1 - 1));
      lds_barrier();  // (barrier W)
      // a wavefront's counters cover only its own loads: each loader waits
      // for its share of the next chunk's images (everything but the one
      // prefetch issued last: vmcnt(1)) before the barrier
      __builtin_amdgcn_s_waitcnt(0x0F71);
      lds_barrier();  // (barrier A)
      return;
    }
    const int t0 = c * C;
    const int n = min(C, T - t0);

    // waves 0, 1: P = k S (token rows 32 rblk ..), then U = v - e^{gc} o P;
    // waves 2, 3: the output in the transposed orientation, o^T = S^T q^T
    // (tokens 32 rblk ..), so that a lane owns one token: its row factor is
    // one scalar and its 16 values are 4 runs of 4 consecutive v, stored
    // straight to memory
    f32x16 acc = {};
    if (wave < 2) {
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks)
        acc = mfma(ld8(cur.k + swz16(arow, ks * 2 + half)),
                   ld8(st_s + col * SP + ks * 16 + half * 8), acc);
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int cl = rblk * 32 + g4 * 8 + half * 4;
        const float4 eg = *reinterpret_cast<const float4*>(cur.fac + kFacG + cl);
        const uint2 vw = read_vt4(cur.v, g4);  // v[cl .. cl + 3][v0 + col]
        const bf16* vv = reinterpret_cast<const bf16*>(&vw);
        *reinterpret_cast<uint2*>(ut_s + col * CP + cl) =
            pack_bf16x4(fmaf(-eg.x, acc[g4 * 4 + 0], (float)vv[0]),
                        fmaf(-eg.y, acc[g4 * 4 + 1], (float)vv[1]),
                        fmaf(-eg.z, acc[g4 * 4 + 2], (float)vv[2]),
                        fmaf(-eg.w, acc[g4 * 4 + 3], (float)vv[3]));
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks)
        acc = mfma(ld8(st_s + col * SP + ks * 16 + half * 8),
                   ld8(cur.q + swz16(arow, ks * 2 + half)), acc);
      const float f = cur.fac[kFacOut + arow];  // scale e^{gc} of this lane's token
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] *= f;
    }
    lds_barrier();  // (barrier U) U^T visible

    if (wave < 2) {  // W = Tu U; Tu is lower triangular: row block 0 needs tokens < 32 only
      f32x16 wacc = {};
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        if (rblk == 0 && ks >= 2) break;
        wacc = mfma(ld8(cur.tu + swz8(arow, ks * 2 + half)),
                    ld8(ut_s + col * CP + ks * 16 + half * 8), wacc);
      }
      put_rows_t(wt_s, wacc, nullptr);
      put_rows_t(dwt_s, wacc, cur.fac + kFacD);
    }
    lds_barrier();  // (barrier W) W^T and the decayed W^T visible

    if (wave >= 2) {  // o^T += W^T Aqk^T, then this lane's token row to memory
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks)
        acc = mfma(ld8(wt_s + col * CP + ks * 16 + half * 8),
                   ld8(cur.aqk + swz8(arow, ks * 2 + half)), acc);
      if (arow < n) {
        bf16* orow = o + ((int64_t)b * T + t0 + arow) * tok_stride + (int64_t)h * DV + v0;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          *reinterpret_cast<uint2*>(orow + g4 * 8 + half * 4) =
              pack_bf16x4(acc[g4 * 4 + 0], acc[g4 * 4 + 1], acc[g4 * 4 + 2], acc[g4 * 4 + 3]);
      }
    }
    // S <- e^{gc_C} S + k^T (e^{gc_C - gc} o W)   (rows 32 * wave .. of the state)
    const float dec = cur.fac[kFacChunk];
#pragma unroll
    for (int r = 0; r < 16; ++r) s_acc[r] *= dec;
#pragma unroll
    for (int ks = 0; ks < C / 16; ++ks)
      s_acc = mfma(read_kt(cur.k, ks), ld8(dwt_s + col * CP + ks * 16 + half * 8), s_acc);
    publish_state();
    lds_barrier();  // (barrier A) next chunk's images, S^T and v^T visible
  };

  if (c1 > c0 && loader) {
    load_rows(c0, slot0);
    load_record(c0, slot0);
    touch(min(c0 + 1, c1 - 1));
    __builtin_amdgcn_s_waitcnt(0x0F71);
  }
  if (!loader) publish_state();
  lds_barrier();
  int c = c0;
  for (; c + 1 < c1; c += 2) {
    step(c, slot0, slot1);
    step(c + 1, slot1, slot0);
  }
  if (c < c1) step(c, slot0, slot1);

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

namespace tileops {
namespace gdn {

// Workspace bytes for `nchunks` chunks of each of B * H heads.
inline size_t records_bytes(int64_t BH, int64_t nchunks) {
  return (size_t)(BH * nchunks) * kChunkBytes;
}

// Argument checks shared by the entry points (0 when the call may proceed).
static int check_args(const void* q, const void* k, const void* v, const float* g,
                      const float* beta, const void* o, const float* hT, int64_t B, int64_t T,
                      int64_t H, int64_t K, int64_t V, int64_t chunk, int dtype) {
  if (B < 0 || T < 0 || H <= 0) return TILEOPS_ESHAPE;
  if (K != DK || V != DV || chunk != C) return TILEOPS_ESHAPE;
  if (B > 65535 || H > 65535 || T > INT32_MAX / 2) return TILEOPS_ESHAPE;
  if (dtype != TILEOPS_BF16) return TILEOPS_EINVAL;
  if (B == 0) return 0;
  if (!hT) return TILEOPS_ENULL;
  if (T > 0) {
    if (!q || !k || !v || !g || !beta || !o) return TILEOPS_ENULL;
    if (!host_aligned16(q) || !host_aligned16(k) || !host_aligned16(v)) return TILEOPS_EINVAL;
  }
  const int64_t nc = (T + C - 1) / C;
  if (B * H * nc > (int64_t)UINT32_MAX || B * H * (DV / VS) > INT32_MAX) return TILEOPS_ESHAPE;
  return 0;
}

// The whole prefill in segments of `seg` chunks: per segment the parallel
// preparation into `ws` (records of seg chunks per head), then the
// recurrence over the segment, the state carried from one segment to the
// next in hT.  One segment when `ws` holds every chunk's record.
static int run_segments(const bf16* q, const bf16* k, const bf16* v, const float* g,
                        const float* beta, const float* h0, bf16* o, float* hT, int B, int T,
                        int H, float scale, uint8_t* ws, int seg, hipStream_t s) {
  const int nc = (T + C - 1) / C;
  const unsigned rgrid = (unsigned)(B * H * (DV / VS));
  if (nc == 0) {  // no chunk: the state passes through
    gdn_recur_kernel<<<dim3(rgrid), dim3(512), 0, s>>>(q, k, v, h0, ws, o, hT, B, T, H, 0, 0, 1);
    return launch_status();
  }
  for (int c0 = 0; c0 < nc; c0 += seg) {
    const int ns = std::min(seg, nc - c0);
    const int64_t nblk = (int64_t)B * H * ns;
    gdn_prep_kernel<<<dim3((unsigned)std::min<int64_t>(nblk, 2 * device_cu_count())), dim3(256),
                      0, s>>>(q, k, g, beta, ws, B, T, H, c0, ns, scale);
    gdn_recur_kernel<<<dim3(rgrid), dim3(512), 0, s>>>(q, k, v, c0 == 0 ? h0 : hT, ws, o, hT, B,
                                                      T, H, c0, c0 + ns, ns);
    if (int e = launch_status()) return e;
  }
  return 0;
}

// Scratch of the allocation-free entry point: every call on a GPU shares
// that GPU's copy (the last call's records stay in it), so calls that
// overlap on one GPU race.  kScratchBytes bounds the heads per call: one
// chunk record per head must fit, B * H <= 963.
constexpr size_t kScratchBytes = (size_t)16 << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device: in host code the array's name is only a stand-in symbol.
static int scratch_ptr(uint8_t** out) {
  static std::mutex mu;
  static uint8_t* ptrs[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= 64) return TILEOPS_EINVAL;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    ptrs[dev] = static_cast<uint8_t*>(p);
  }
  *out = ptrs[dev];
  return 0;
}

}  // namespace gdn
}  // namespace tileops

extern "C" size_t tileops_gdn_prefill_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K,
                                                      int64_t V, int64_t chunk) {
  if (B < 0 || T < 0 || H < 0 || K != gdn::DK || V != gdn::DV || chunk != gdn::C) return 0;
  return gdn::records_bytes(B * H, (T + gdn::C - 1) / gdn::C);
}

extern "C" int tileops_gdn_prefill_fwd(const void* q, const void* k, const void* v, const float* g,
                                       const float* beta, const float* h0, void* o, float* hT,
                                       int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                       int64_t chunk, float scale, int dtype, void* ws,
                                       size_t ws_bytes, void* stream) {
  if (int e = gdn::check_args(q, k, v, g, beta, o, hT, B, T, H, K, V, chunk, dtype)) return e;
  if (B == 0) return 0;
  const size_t need = tileops_gdn_prefill_workspace_bytes(B, T, H, K, V, chunk);
  if (T > 0 && (!ws || ws_bytes < need || !host_aligned16(ws))) {
    if (ws && !host_aligned16(ws)) return TILEOPS_EINVAL;
    return TILEOPS_EWORKSPACE;
  }
  const int nc = (int)((T + gdn::C - 1) / gdn::C);
  return gdn::run_segments(static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                           static_cast<const bf16*>(v), g, beta, h0, static_cast<bf16*>(o), hT,
                           (int)B, (int)T, (int)H, scale, static_cast<uint8_t*>(ws),
                           nc > 0 ? nc : 1, static_cast<hipStream_t>(stream));
}

extern "C" int tileops_gdn_prefill_fwd_noalloc(const void* q, const void* k, const void* v,
                                               const float* g, const float* beta,
                                               const float* h0, void* o, float* hT, int64_t B,
                                               int64_t T, int64_t H, int64_t K, int64_t V,
                                               int64_t chunk, float scale, int dtype,
                                               void* stream) {
  if (int e = gdn::check_args(q, k, v, g, beta, o, hT, B, T, H, K, V, chunk, dtype)) return e;
  if (B == 0) return 0;
  const int64_t per_chunk = B * H * (int64_t)gdn::kChunkBytes;  // one chunk of every head
  if (T > 0 && per_chunk > (int64_t)gdn::kScratchBytes) return TILEOPS_EWORKSPACE;
  uint8_t* ws = nullptr;
  if (int e = gdn::scratch_ptr(&ws)) return e;
  const int nc = (int)((T + gdn::C - 1) / gdn::C);
  const int seg = (int)std::min<int64_t>(std::max(nc, 1), (int64_t)gdn::kScratchBytes / per_chunk);
  return gdn::run_segments(static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                           static_cast<const bf16*>(v), g, beta, h0, static_cast<bf16*>(o), hT,
                           (int)B, (int)T, (int)H, scale, ws, seg,
                           static_cast<hipStream_t>(stream));
}
