// Gated delta-rule (gated DeltaNet) chunked prefill for gfx950
// (tileops_gdn_prefill_fwd).
//
// Recurrence per (batch b, head h), token t (state S is K x V, fp32):
//   S_t = exp(g_t) S_{t-1} + beta_t k_t (v_t - exp(g_t) S_{t-1}^T k_t)^T,   o_t = scale q_t^T S_t
//
// Chunked (C = 64 tokens) WY form.  Inside a chunk, with gc the cumulative
// log-decay, gamma = gc_C, G[l,s] = exp(gc_l - gc_s) (l >= s),
// A = strictly_lower(beta_l G[l,s] k_l.k_s) and T = (I + A)^-1:
//   Tu  = T diag(beta)                          \ independent of S
//   Aqk = scale * lower_incl(G o (q k^T))        /
//   U   = v - exp(gc) o (k S)
//   W   = Tu U
//   o   = scale exp(gc) o (q S) + Aqk W
//   S  <- exp(gamma) S + k^T (exp(gamma - gc) o W)
// Only differences gc_l - gc_s <= 0, gamma - gc_l <= 0 and gc <= 0 are ever
// exponentiated, so nothing overflows however strong the decay.
//
// Segments.  The chunk map S -> S' is affine, S' = A_c S + B_c, so a run of
// chunks (a segment) maps its start state affinely too: S_end = Phi S_start
// + Bseg, where Phi (K x K) is the segment's end state from start state I
// with values 0, and Bseg (K x V) its end state from start state 0.  The
// nc chunks are cut into N segments:
//   launch 1: segment 0 runs exactly from h0 (outputs, end state), segments
//             1 .. N-2 run from [0 | I] over 256 columns (Bseg | Phi);
//   between:  a small launch composes the start states of segments
//             2 .. N-1 from segment 0's end state through the maps;
//   launch 2: segments 1 .. N-1 run exactly from their start states
//             (outputs; the last segment writes hT).
// The composition uses split-bf16 products (hi*hi + hi*lo + lo*hi): launch 1
// stores each Phi already split, as a bf16 hi image and a bf16 lo image, so
// the composition loads them straight into LDS.  With N = 1 a single launch
// runs every chunk from h0.
//
// Workgroup (one per (head, segment)): NCW chain wavefronts and 4 prep
// wavefronts (launch 1: NCW = 8, three wavefronts per SIMD; launch 2 and
// single-segment runs: NCW = 4, two per SIMD):
//   chain      hold the state in MFMA accumulators, all 128 key rows of
//              their columns (16 or 32 value columns in an exact segment,
//              32 of Bseg or Phi in a map segment), so that the
//              chunk step P = k S -> U -> W = Tu U -> S' runs in registers:
//              an accumulator is fed to the next product as it stands, the
//              rows of each product being chosen so that its accumulator
//              rows land in the order the next product's k-slots expect;
//              in exact segments they also form o and their share of Aqk;
//   prep       prepare the chunks ahead while the chain runs the current
//              one: k k^T products and diagonal blocks of T (blocked
//              substitution, products on fp32 MFMA) for the next chunk, the
//              rest of T and Tu (into LDS) for the current one, the decay
//              scan two chunks ahead, and the direct-to-LDS loads of the
//              chunk operands (the chain wavefronts form Aqk, and L21 when
//              there are four of them).
// Two workgroup barriers per chunk.  Every chunk operand crosses HBM once
// per pass over its segment, and nothing per chunk is written back.
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
constexpr int kMaxSeg = 16;
constexpr int DS = 36;  // fp32 row stride of the diagonal 32x32 blocks of A^T / T
constexpr int XS = 36;  // fp32 row stride of X
constexpr float kLog2e = 1.4426950408889634f;
constexpr size_t kStateFloats = (size_t)DK * DV;

// per-chunk factors (fp32, LDS): scale e^{gc}, e^{gc}, e^{gamma - gc}, gc,
// beta (rows past T zero), e^{gamma}
constexpr int kFacSE = 0, kFacE = 64, kFacD = 128, kFacGC = 192, kFacB = 256, kFacEG = 320;
constexpr int kFacN = 336;

struct Args {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const float* g;
  const float* beta;
  const float* h0;
  bf16* o;
  float* hT;
  float* ws;  // per head: segment 0's end state, then (Phi_j, Bseg_j), j = 1 .. N-2
  int B, T, H;
  float scale;
  int nseg;
  int phase;               // 1 or 2
  int start[kMaxSeg + 1];  // first chunk of each segment; start[nseg] = chunk count
};

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 ld8(const bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
__device__ __forceinline__ bf16x8 pack8(f32x4 a, f32x4 b) {
  bf16x8 r;
  r[0] = (bf16)a[0];
  r[1] = (bf16)a[1];
  r[2] = (bf16)a[2];
  r[3] = (bf16)a[3];
  r[4] = (bf16)b[0];
  r[5] = (bf16)b[1];
  r[6] = (bf16)b[2];
  r[7] = (bf16)b[3];
  return r;
}
// Four fp32 values as four bf16 in one 8-byte word.
__device__ __forceinline__ uint2 pack_bf16x4(float a, float b, float c, float d) {
  bf16 p[4] = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
  return *reinterpret_cast<uint2*>(p);
}
__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Inclusive prefix sum over the 64 lanes of a wavefront by DPP lane moves:
// Hillis-Steele inside each row of 16 lanes (row_shr 1, 2, 4, 8; lanes
// shifted in from outside the row read 0), then each row's total carried
// forward (row_bcast:15 to rows 1 and 3, row_bcast:31 to rows 2 and 3).
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
// and stores issued before it stay in flight across it.  Only LDS data is
// exchanged through these barriers; the direct-to-LDS loads are waited for
// explicitly (vmcnt) by the wavefronts that issued them, before the barrier
// that publishes them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS values written by other lanes of the same wavefront are read back
// after these fences: the LDS operations of one wavefront execute in order,
// and the fences keep the compiler from moving the reads above the writes.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// LDS images.  Rows of 128 (k, q, v) or 64 (Tu, Aqk) bf16 are stored
// unpadded with their 16-byte chunks XOR-swizzled by row, so that the three
// read patterns touch distinct bank groups: 16 consecutive rows at one chunk
// (natural operand rows), the 16 rows 8 (m / 4) + 4 b + m % 4 of a block
// (the rows a chain product reads, lam()), and transpose reads (4
// consecutive rows x 4 8-byte words).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int sw16(int r) {
  return (r & 15) ^ ((r & 3) << 2) ^ (((r >> 4) & 1) << 2);
}
__device__ __forceinline__ int off128(int r, int p) { return r * 128 + ((p ^ sw16(r)) << 3); }
__device__ __forceinline__ int sw8(int r) {
  return ((r >> 1) & 1) | (((r >> 3) & 1) << 1) | ((((r >> 2) ^ (r >> 4)) & 1) << 2);
}
__device__ __forceinline__ int off64(int r, int p) { return r * 64 + ((p ^ sw8(r)) << 3); }
// [32][32] images (4 chunks per row): chunk p ^ ((r / 8) % 4)
__device__ __forceinline__ int off32(int r, int p) { return r * 32 + ((p ^ ((r >> 3) & 3)) << 3); }

// Row read by lane-row m of the A operand for output block blk (16 rows of
// the 32-row group blk / 2).  Then accumulator row 4 g + r of block blk
// (lane group g) holds logical row acc_row(blk, g, r) = 32 (blk / 2) + 8 g +
// 4 (blk % 2) + r, so that blocks 2j and 2j + 1 of an accumulator, taken as
// the 8 k-slots 8 g + e of a 16x16x32 operand (e < 4 from block 2j, e >= 4
// from block 2j + 1), hold rows 32 j + 8 g + e: natural order.
// A lane index the compiler cannot see through: addresses derived from it are
// recomputed where they are used instead of being held in registers across
// the chunk loop (dozens of per-lane swizzled LDS addresses otherwise stay
// live and push the state out to scratch).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Keeps the scheduler from moving instructions across this point: operand
// reads issued before it stay ahead of the products after it, so that the
// LDS latency of one step overlaps the MFMAs of the previous one.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ int lam(int blk, int m) {
  return 32 * (blk >> 1) + 8 * (m >> 2) + 4 * (blk & 1) + (m & 3);
}
__device__ __forceinline__ int acc_row(int blk, int g, int r) {
  return 32 * (blk >> 1) + 8 * g + 4 * (blk & 1) + r;
}

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void_ptr)p;
}
// ds_read_b64_tr_b16: in each group of 16 lanes, lane i receives element
// i % 4 of the 8 bytes addressed by lanes i / 4, 4 + i / 4, 8 + i / 4 and
// 12 + i / 4 (in that order).
__device__ __forceinline__ v4i16 ds_read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(uintptr_t)lds_addr(p));
}

// Direct-to-LDS loads: lane l reads 16 bytes at `base + off` (base uniform,
// in SGPRs) landing at LDS address lds + 16 l, or 4 bytes at a per-lane
// address landing at lds + 4 l.  Inline assembly, so that the compiler does
// not track the LDS writes; every wait for them is explicit.
// A wavefront-uniform pointer moved into SGPRs: both 32-bit halves are read
// from the first active lane and joined as unsigned words.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | (uint64_t)lo);
}
// The compiler's hazard checks do not look into inline assembly, so each
// load starts with the wait states the ISA requires before it: 5 after a
// VALU write (v_readfirstlane) of an SGPR the load reads, 1 after the SALU
// write of M0.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(uniform_ptr(base)),
               "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma4(const void* addr, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, off" : : "v"(addr), "{m0}"(lds) : "memory");
}

// Fill a swizzled [64][128] bf16 image from rows `src + min(r, rmax) *
// stride` (elements, src uniform): 16 windows of 1 KB, loader lw (0, 1)
// issuing every second one.
__device__ __forceinline__ void fill128(bf16* img, const bf16* src, int64_t stride, int rmax,
                                        int lw, int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int win = 2 * i + lw;
    const int ch = win * 64 + lane;
    const int r = ch >> 4;
    const int p = (ch & 15) ^ sw16(r);
    const uint32_t off = (uint32_t)(((int64_t)min(r, rmax) * stride + (p << 3)) * 2);
    lds_dma16(src, off, lds_addr(img + win * 512));
  }
}

struct Smem {
  bf16 k[3][C * DK];     // k of chunks c, c + 1, c + 2 (slot c % 3)
  bf16 q[2][C * DK];     // q of chunks c, c + 1 (slot c % 2)
  bf16 v[C * DV];        // v of chunk c (then c + 1, loaded once U is formed)
  bf16 tu[2][32 * 32];   // Tu11 | Tu22 of chunk c (then c + 1)
  bf16 l21[2][32 * 32];  // L21 of chunks c, c + 1 (slot c % 2)
  bf16 aqk[C * C];       // Aqk of chunk c
  float fac[3][kFacN];   // factors of chunks c .. c + 2 (slot c % 3)
  float gb[4][2 * C];    // raw g | beta of chunks c .. c + 3 (slot c % 4)
  float at[2][C * DS];   // A^T of chunks c, c + 1 (slot c % 2): the diagonal 32x32 blocks
  float t[C * DS];       // T of chunk c + 1 (then c + 2), the diagonal 32x32 blocks
  float x[32 * XS];      // products of the block inverse
};
static_assert(sizeof(Smem) <= 163840, "the LDS of one CU");

// ---------------------------------------------------------------------------
// The preparation of one chunk (prep wavefronts pw = 0 .. 3)
// ---------------------------------------------------------------------------
// The inverse in halves.  With T = (I + A)^-1 = [[T11, 0], [T21, T22]]
// (32-row blocks) and A21 = diag(beta_bot) L21, L21[l - 32][s] = G[l][s]
// k_l.k_s, T21 = -T22 A21 T11, so W = T diag(beta) U is
//   W_top = Tu11 U_top,   W_bot = Tu22 (U_bot - L21 W_top),   Tuii = Tii diag(beta_i):
// the preparation forms only the diagonal blocks Tu11, Tu22 and L21; the
// chain applies the coupling.  A^T and T keep only the two diagonal 32x32
// blocks: element (r, c), with r and c in the same block, at r * DS + c % 32.
//
// PA: the 32x32 block blk of G o (k k^T), blk 0: (l, s) in 00, 1: in 11,
// 2: l in 32-63, s in 0-31 (L21), in the transposed orientation (k rows s
// as the A operand, so that a lane owns one row l and its 16 values run
// over s); blocks 00 and 11 become A^T[s][l] = beta_l G[l][s] k_l.k_s
// (s < l, fp32), block 10 is stored as L21 (bf16).  The operands of BATCH
// key steps are read at a time (8: all in flight; fewer where registers
// are scarce).
template <int BATCH>
__device__ __forceinline__ void prep_products(const bf16* kimg, const float* fc, float* at,
                                              bf16* l21, int blk, int lane) {
  const int col = lane & 31, half = lane >> 5;
  const int rb = blk == 0 ? 0 : 1, cb = blk == 1 ? 1 : 0;
  f32x16 kk = {};
#pragma unroll
  for (int k0 = 0; k0 < DK / 16; k0 += BATCH) {
    bf16x8 bs[BATCH], bl[BATCH];
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
      bs[i] = ld8(kimg + off128(cb * 32 + col, 2 * (k0 + i) + half));
      bl[i] = ld8(kimg + off128(rb * 32 + col, 2 * (k0 + i) + half));
    }
    sched_fence();
#pragma unroll
    for (int i = 0; i < BATCH; ++i) kk = mfma32(bs[i], bl[i], kk);
  }
  const int l = rb * 32 + col;
  const float gl = fc[kFacGC + l], bel = fc[kFacB + l];
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const int s0 = cb * 32 + g4 * 8 + half * 4;
    const float4 gs4 = *reinterpret_cast<const float4*>(fc + kFacGC + s0);
    const float gsv[4] = {gs4.x, gs4.y, gs4.z, gs4.w};
    float val[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // branch-free: the decay is evaluated for every element (argument
      // clamped to <= 0, exact where it is used) and selected
      float gd = exp2f_fast(fminf((gl - gsv[e]) * kLog2e, 0.0f));
      asm volatile("" : "+v"(gd));
      val[e] = gd * kk[g4 * 4 + e];
    }
    if (blk == 2) {  // s < 32 <= l: no mask
      *reinterpret_cast<uint2*>(l21 + off32(l - 32, s0 >> 3) + (s0 & 7)) =
          pack_bf16x4(val[0], val[1], val[2], val[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) at[(s0 + e) * DS + col] = s0 + e < l ? bel * val[e] : 0.0f;
    }
  }
}

// PB (waves pw 0, 1): the diagonal 16x16 blocks 2 pw, 2 pw + 1 of T by
// substitution (lane group (lane / 16) % 2 takes one block, lane j column
// j; p[i] accumulates sum_m A[i][m] T[m][j]; the A columns are read four
// steps ahead).
__device__ __forceinline__ void prep_subst(const float* at, float* t, int pw, int lane) {
  const int base = 16 * (2 * pw + ((lane >> 4) & 1)), jl = lane & 15;
  const int cb = base & 31;  // column of the block inside its 32x32 block
  float p[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = 0.0f;
  // av[m % 4][gq] = A[base + 4gq .. 4gq + 3][base + m], for the groups gq
  // with a row below m
  const float4* a4p = reinterpret_cast<const float4*>(at + base * DS + cb);
  float4 av[4][4];
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int gq = (st + 1) >> 2; gq < 4; ++gq) av[st][gq] = a4p[st * (DS / 4) + gq];
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const float tv = (m == jl ? 1.0f : 0.0f) - p[m];
    // every lane writes (lane groups 0 / 2 and 1 / 3 hold the same
    // columns, so their writes agree): no exec-masked branch in the chain
    t[(base + m) * DS + cb + jl] = tv;
#pragma unroll
    for (int gq = (m + 1) >> 2; gq < 4; ++gq) {
      const float4 a4 = av[m & 3][gq];
      const int i4 = 4 * gq;
      if (i4 + 0 > m) p[i4 + 0] = fmaf(a4.x, tv, p[i4 + 0]);
      if (i4 + 1 > m) p[i4 + 1] = fmaf(a4.y, tv, p[i4 + 1]);
      if (i4 + 2 > m) p[i4 + 2] = fmaf(a4.z, tv, p[i4 + 2]);
      if (i4 + 3 > m) p[i4 + 3] = fmaf(a4.w, tv, p[i4 + 3]);
    }
    if (m + 4 < 16) {
#pragma unroll
      for (int gq = (m + 5) >> 2; gq < 4; ++gq) av[m & 3][gq] = a4p[(m + 4) * (DS / 4) + gq];
    }
  }
}

// PC + PF (waves pw 0, 1): in the diagonal 32x32 block pw of T, the block
// below its diagonal 16x16 blocks, T10 = -T11 (A10 T00) (pw 0) or T32 =
// -T33 (A32 T22) (pw 1), on v_mfma_f32_16x16x4f32 (A[mi][mk], B[mk][mi],
// D[4 mk + r][mi]); then Tu = T diag(beta) of the block in bf16 (its upper
// right 16x16 block is the constant zero block of t).
__device__ __forceinline__ void prep_merge16(const float* at, float* t, float* x, const float* fc,
                                             bf16* tu, int pw, int lane) {
  const int mi = lane & 15, mk = lane >> 4;
  const int d0 = 32 * pw;
  f32x4 y = {};
  float ya[4], yb[4], za[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int kx = 4 * kk + mk;
    ya[kk] = at[(d0 + kx) * DS + 16 + mi];
    yb[kk] = t[(d0 + kx) * DS + mi];
    za[kk] = t[(d0 + 16 + mi) * DS + 16 + kx];
  }
  sched_fence();
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) y = __builtin_amdgcn_mfma_f32_16x16x4f32(ya[kk], yb[kk], y, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) x[(16 * pw + 4 * mk + r) * XS + mi] = y[r];
  wave_lds_fence();
  f32x4 z = {};
  float zb[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) zb[kk] = x[(16 * pw + 4 * kk + mk) * XS + mi];
  sched_fence();
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) z = __builtin_amdgcn_mfma_f32_16x16x4f32(za[kk], zb[kk], z, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) t[(d0 + 16 + 4 * mk + r) * DS + mi] = -z[r];
  wave_lds_fence();
  const int cg = lane & 7;  // the lane's column group in every row it converts
  const float4 bt = *reinterpret_cast<const float4*>(fc + kFacB + d0 + 4 * cg);
  float4 tv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    tv[i] = *reinterpret_cast<const float4*>(t + (d0 + 8 * i + (lane >> 3)) * DS + 4 * cg);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 8 * i + (lane >> 3);
    *reinterpret_cast<uint2*>(tu + off32(row, cg >> 1) + (cg & 1) * 4) =
        pack_bf16x4(tv[i].x * bt.x, tv[i].y * bt.y, tv[i].z * bt.z, tv[i].w * bt.w);
  }
}

// Decay scan of one chunk (one wavefront): factors from the raw g | beta.
__device__ __forceinline__ void prep_scan(const float* gbr, float* fc, int n, float scale,
                                          int lane) {
  float x = lane < n ? gbr[lane] : 0.0f;
  const float bt = lane < n ? gbr[C + lane] : 0.0f;
  x = wave_inclusive_sum(x);  // gc
  const float gl =
      __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), C - 1));
  const float eg = exp2f_fast(x * kLog2e);
  fc[kFacSE + lane] = scale * eg;
  fc[kFacE + lane] = eg;
  fc[kFacD + lane] = exp2f_fast((gl - x) * kLog2e);
  fc[kFacGC + lane] = x;
  fc[kFacB + lane] = bt;
  if (lane == 0) fc[kFacEG] = exp2f_fast(gl * kLog2e);
}

// ---------------------------------------------------------------------------
// The chain wavefronts: NB blocks of 16 state columns each
// ---------------------------------------------------------------------------
// State: s[nb][kb][r] (lane group g, lane ln = lane % 16) holds
// S[acc_row(kb, g, r)][col0 + 16 nb + ln].
template <int NB>
__device__ __forceinline__ void state_load(f32x4 (&s)[NB][8], const float* src, int col0, int g,
                                           int ln) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        s[nb][kb][r] = src ? src[acc_row(kb, g, r) * DV + col0 + 16 * nb + ln] : 0.0f;
}
template <int NB>
__device__ __forceinline__ void state_store(const f32x4 (&s)[NB][8], float* dst, int col0, int g,
                                            int ln) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[acc_row(kb, g, r) * DV + col0 + 16 * nb + ln] = s[nb][kb][r];
}

// x as bf16 hi + lo (x - hi rounded again): a sum of the three products
// hi*hi + hi*lo + lo*hi carries ~16 significant bits.
__device__ __forceinline__ void split8(f32x4 a, f32x4 b, bf16x8& hi, bf16x8& lo) {
  hi = pack8(a, b);
  f32x4 ra, rb;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    ra[e] = a[e] - (float)hi[e];
    rb[e] = b[e] - (float)hi[4 + e];
  }
  lo = pack8(ra, rb);
}

// A map's Phi stored already split: the [128][128] bf16 image of hi, then
// that of lo (the values split8 forms from the fp32 entries).
template <int NB>
__device__ __forceinline__ void phi_store(const f32x4 (&s)[NB][8], float* slot, int col0, int g,
                                          int ln) {
  bf16* hi = reinterpret_cast<bf16*>(slot);
  bf16* lo = hi + DK * DV;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = s[nb][kb][r];
        const bf16 xh = (bf16)x;
        const int idx = acc_row(kb, g, r) * DV + col0 + 16 * nb + ln;
        hi[idx] = xh;
        lo[idx] = (bf16)(x - (float)xh);
      }
}

// k^T as the A operand of S' for key block kb and token step ts: lane-row m
// = ln holds key lam(kb, ln), k-slots 8 g + e tokens 32 ts + 8 g + e.
__device__ __forceinline__ bf16x8 read_kt(const bf16* kimg, int kb, int ts, int g, int ln) {
  const int chunk = 4 * (kb >> 1) + (ln & 3);
  const int within = 4 * (kb & 1);
  const int row = 32 * ts + 8 * g + (ln >> 2);
  const v4i16 x0 = ds_read_tr(kimg + off128(row, chunk) + within);
  const v4i16 x1 = ds_read_tr(kimg + off128(row + 4, chunk) + within);
  const u32x2 y0 = __builtin_bit_cast(u32x2, x0), y1 = __builtin_bit_cast(u32x2, x1);
  const u32x4 w4 = {y0.x, y0.y, y1.x, y1.y};
  return __builtin_bit_cast(bf16x8, w4);
}

// v of tokens t0 .. t0 + 3 at column c0 + ln (c0 a multiple of 16).
__device__ __forceinline__ f32x4 read_v4(const bf16* vimg, int t0, int c0, int ln) {
  const int colw = c0 + 4 * (ln & 3);
  const v4i16 x = ds_read_tr(vimg + off128(t0 + (ln >> 2), colw >> 3) + (colw & 7));
  const bf16* b = reinterpret_cast<const bf16*>(&x);
  return f32x4{(float)b[0], (float)b[1], (float)b[2], (float)b[3]};
}

// Values a chain wavefront carries from the first part of a chunk step to
// the second.
template <int NB>
struct ChainTmp {
  f32x4 u[NB][4];  // U (accumulator rows acc_row)
  f32x4 o[NB][4];  // o^T: rows columns 16 nb + 4 g + r, column token 16 tb + ln
};

// Part 1, from S at the chunk start: P = k S (exact segments also o^T =
// scale e^{gc} o (S^T q^T)), then U = v - e^{gc} o P (v = 0 for Phi
// columns).
template <int NB, bool OUT>
__device__ __forceinline__ void chain_part1(const f32x4 (&s)[NB][8], ChainTmp<NB>& t,
                                            const bf16* kimg, const bf16* vimg, const bf16* qimg,
                                            const float* fc, bool usev, int col0, int g, int ln) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) t.u[nb][tb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (OUT) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) t.o[nb][tb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // P and o^T share the bf16 state operands; the k and q rows of key step
  // ks + 1 are read while the MFMAs of step ks run
  bf16x8 a[2][4], b[2][4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    a[0][tb] = ld8(kimg + off128(lam(tb, ln), g));
    if constexpr (OUT) b[0][tb] = ld8(qimg + off128(16 * tb + ln, g));
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (ks < 3) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        a[(ks + 1) & 1][tb] = ld8(kimg + off128(lam(tb, ln), 4 * (ks + 1) + g));
        if constexpr (OUT)
          b[(ks + 1) & 1][tb] = ld8(qimg + off128(16 * tb + ln, 4 * (ks + 1) + g));
      }
    }
    sched_fence();
    bf16x8 sb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) sb[nb] = pack8(s[nb][2 * ks], s[nb][2 * ks + 1]);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        t.u[nb][tb] = mfma16(a[ks & 1][tb], sb[nb], t.u[nb][tb]);
        if constexpr (OUT) t.o[nb][tb] = mfma16(sb[nb], b[ks & 1][tb], t.o[nb][tb]);
      }
  }
  f32x4 vv[NB][4], ev[4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int t0 = acc_row(tb, g, 0);
    const float4 e4 = *reinterpret_cast<const float4*>(fc + kFacE + t0);
    ev[tb] = f32x4{e4.x, e4.y, e4.z, e4.w};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      vv[nb][tb] = usev ? read_v4(vimg, t0, col0 + 16 * nb, ln) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  sched_fence();
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        t.u[nb][tb][r] = fmaf(-ev[tb][r], t.u[nb][tb][r], vv[nb][tb][r]);
  if constexpr (OUT) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const float f = fc[kFacSE + 16 * tb + ln];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) t.o[nb][tb][r] *= f;
    }
  }
}

// Aqk block bi of the current chunk, in 32x32 blocks (tb, sb) = (0,0)
// (1,0) (1,1): D = k_blk q_blk^T on 32x32x16 MFMA (a lane owns token t = 32
// tb + lane % 32, its 16 values run over s), masked (s <= t), decayed and
// scaled, stored as 4 consecutive s of row t.  The blocks above are constant
// zero.
__device__ __forceinline__ void aqk_block(int bi, const bf16* kimg, const bf16* qimg,
                                          const float* fc, bf16* aqk, float scale, int lane) {
  const int tb = bi == 0 ? 0 : 1, sb = bi == 2 ? 1 : 0;
  const int col = lane & 31, half = lane >> 5;
  f32x16 d = {};
  bf16x8 a[4], b[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ks = 4 * h + i;
      a[i] = ld8(kimg + off128(32 * sb + col, 2 * ks + half));
      b[i] = ld8(qimg + off128(32 * tb + col, 2 * ks + half));
    }
    sched_fence();
#pragma unroll
    for (int i = 0; i < 4; ++i) d = mfma32(a[i], b[i], d);
  }
  const int t = 32 * tb + col;
  const float gt = fc[kFacGC + t];
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const int s0 = 32 * sb + 8 * g4 + 4 * half;
    const float4 gs4 = *reinterpret_cast<const float4*>(fc + kFacGC + s0);
    const float gsv[4] = {gs4.x, gs4.y, gs4.z, gs4.w};
    float val[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float gd = exp2f_fast(fminf((gt - gsv[e]) * kLog2e, 0.0f));
      asm volatile("" : "+v"(gd));
      val[e] = s0 + e <= t ? scale * gd * d[4 * g4 + e] : 0.0f;
    }
    *reinterpret_cast<uint2*>(aqk + off64(t, s0 >> 3) + (s0 & 7)) =
        pack_bf16x4(val[0], val[1], val[2], val[3]);
  }
}

// Part 2: W_top = Tu11 U_top, W_bot = Tu22 (U_bot - L21 W_top); exact
// segments o^T += W^T Aqk^T and store o; then
// S <- e^{gamma} S + k^T (e^{gamma - gc} o W).  DEEP: k^T read two key
// blocks ahead (256-register wavefronts), else one.
template <int NB, bool OUT, bool DEEP>
__device__ __forceinline__ void chain_part2(f32x4 (&s)[NB][8], ChainTmp<NB>& t, const bf16* kimg,
                                            const bf16* tu11, const bf16* tu22, const bf16* l21,
                                            const bf16* aqkimg, const float* fc, bf16* orow0,
                                            int64_t otok, int n, int col0, int g, int ln) {
  bf16x8 wa[2], wl[2], wz[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    wa[j] = ld8(tu11 + off32(lam(j, ln), g));
    wl[j] = ld8(l21 + off32(lam(2 + j, ln) - 32, g));
    wz[j] = ld8(tu22 + off32(lam(2 + j, ln) - 32, g));
  }
  constexpr int KD = DEEP ? 3 : 2;  // k^T ring
  bf16x8 ka[KD][2];
#pragma unroll
  for (int j = 0; j < KD - 1; ++j)
#pragma unroll
    for (int ts = 0; ts < 2; ++ts) ka[j][ts] = read_kt(kimg, j, ts, g, ln);
  bf16x8 b[6];  // Aqk rows: (tb, ss) = (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
  if constexpr (OUT) {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int tb = i < 2 ? i : 2 + ((i - 2) >> 1), ss = i < 2 ? 0 : (i - 2) & 1;
      b[i] = ld8(aqkimg + off64(16 * tb + ln, 4 * ss + g));
    }
  }
  sched_fence();
  f32x4 w[NB][4];
  // W_top = Tu11 U_top (token blocks 0, 1; one 32-token step)
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const bf16x8 ut = pack8(t.u[nb][0], t.u[nb][1]);
#pragma unroll
    for (int j = 0; j < 2; ++j) w[nb][j] = mfma16(wa[j], ut, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
  }
  // W_bot = Tu22 (U_bot - L21 W_top) (token blocks 2, 3)
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const bf16x8 wt = pack8(w[nb][0], w[nb][1]);
    f32x4 r2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) r2[j] = mfma16(wl[j], wt, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
    for (int j = 0; j < 2; ++j) r2[j] = t.u[nb][2 + j] - r2[j];
    const bf16x8 rb = pack8(r2[0], r2[1]);
#pragma unroll
    for (int j = 0; j < 2; ++j) w[nb][2 + j] = mfma16(wz[j], rb, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
  }
  bf16x8 wb[NB][2], dwb[NB][2];
#pragma unroll
  for (int ss = 0; ss < 2; ++ss) {
    const float4 d0 = *reinterpret_cast<const float4*>(fc + kFacD + 32 * ss + 8 * g);
    const float4 d1 = *reinterpret_cast<const float4*>(fc + kFacD + 32 * ss + 8 * g + 4);
    const f32x4 dv0 = {d0.x, d0.y, d0.z, d0.w}, dv1 = {d1.x, d1.y, d1.z, d1.w};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (OUT) wb[nb][ss] = pack8(w[nb][2 * ss], w[nb][2 * ss + 1]);
      dwb[nb][ss] = pack8(w[nb][2 * ss] * dv0, w[nb][2 * ss + 1] * dv1);
    }
  }
  if constexpr (OUT) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
#pragma unroll
      for (int ss = 0; ss <= (tb >> 1); ++ss) {
        const int i = tb < 2 ? tb : 2 + 2 * (tb - 2) + ss;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) t.o[nb][tb] = mfma16(wb[nb][ss], b[i], t.o[nb][tb]);
      }
      const int tok = 16 * tb + ln;
      if (tok < n) {
        bf16* orow = orow0 + (int64_t)tok * otok + col0 + 4 * g;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          *reinterpret_cast<uint2*>(orow + 16 * nb) = pack_bf16x4(
              t.o[nb][tb][0], t.o[nb][tb][1], t.o[nb][tb][2], t.o[nb][tb][3]);
      }
    }
  }
  const float eg = fc[kFacEG];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) s[nb][kb] *= eg;
#pragma unroll
  for (int kb = 0; kb < 8; ++kb) {
    if (kb + KD - 1 < 8) {
#pragma unroll
      for (int ts = 0; ts < 2; ++ts)
        ka[(kb + KD - 1) % KD][ts] = read_kt(kimg, kb + KD - 1, ts, g, ln);
    }
    sched_fence();
#pragma unroll
    for (int ts = 0; ts < 2; ++ts)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s[nb][kb] = mfma16(ka[kb % KD][ts], dwb[nb][ts], s[nb][kb]);
  }
}

// Geometry of one workgroup's segment.
struct Seg {
  int b, h, bh;
  int seg;      // segment index
  bool exact;   // exact segment (outputs) or map segment
  int c0, nch;  // first chunk, chunk count
};

__device__ __forceinline__ float* ws_slot(const Args& A, int bh, int idx) {
  const int nslot = 2 * A.nseg - 3;
  return A.ws + ((size_t)bh * nslot + idx) * kStateFloats;
}

// Chain wavefront program.  Every wavefront of the workgroup passes the same
// barrier sequence: 4 in the prologue, 2 per chunk.
template <int NB, bool OUT, bool DEEP>
__device__ void run_chain(const Args& A, Smem& sm, const Seg& sg, int wave, bool idle, int lane) {
  const int g = lane >> 4, ln = lane & 15;
  const int64_t tok_stride = (int64_t)A.H * DK;
  // columns: exact segments 16 NB wave ..; map segments: waves 0-3 value
  // columns 32 wave .., waves 4-7 Phi columns 32 (wave - 4) ..
  const bool usev = OUT || wave < 4;
  const int col0 = OUT ? 16 * NB * wave : 32 * (wave & 3);
  f32x4 s[NB][8];
  ChainTmp<NB> tmp;
  if (!idle) {
    if (OUT) {
      // segment 0 starts from h0, segment 1 from segment 0's end state, a
      // later segment j from the state gdn_compose_kernel left in the slot of
      // Bseg_{j-1}
      const float* src = sg.seg == 0 ? (A.h0 ? A.h0 + (size_t)sg.bh * kStateFloats : nullptr)
                         : sg.seg == 1 ? ws_slot(A, sg.bh, 0)
                                       : ws_slot(A, sg.bh, 2 + 2 * (sg.seg - 2));
      state_load<NB>(s, src, col0, g, ln);
    } else if (usev) {
      state_load<NB>(s, nullptr, col0, g, ln);
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int kb = 0; kb < 8; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            s[nb][kb][r] = acc_row(kb, g, r) == col0 + 16 * nb + ln ? 1.0f : 0.0f;
    }
  }
  // prologue: loads (P0), scans (P1), chunk 0's products (P2) and
  // diagonal blocks of T (P3)
  for (int i = 0; i < 4; ++i) lds_barrier();

  for (int c = 0; c < sg.nch; ++c) {
    const int cg = sg.c0 + c;
    const int n = min(C, A.T - cg * C);
    const bf16* kimg = sm.k[c % 3];
    const bf16* qimg = sm.q[c & 1];
    const float* fc = sm.fac[c % 3];
    if (!idle) {
      const int l1 = opaque(lane);
      chain_part1<NB, OUT>(s, tmp, kimg, sm.v, qimg, fc, usev, col0, l1 >> 4, l1 & 15);
      if constexpr (OUT) {
        if (wave < 3) aqk_block(wave, kimg, qimg, fc, sm.aqk, A.scale, opaque(lane));
      }
      // with four chain wavefronts, wave 3 (no Aqk block) also forms L21 of
      // the next chunk
      if constexpr (DEEP) {
        if (wave == 3 && c + 1 < sg.nch)
          prep_products<4>(sm.k[(c + 1) % 3], sm.fac[(c + 1) % 3], nullptr, sm.l21[(c + 1) & 1],
                           2, opaque(lane));
      }
    }
    lds_barrier();
    if (!idle) {
      const int l2 = opaque(lane);
      bf16* orow0 =
          A.o + ((int64_t)sg.b * A.T + (int64_t)cg * C) * tok_stride + (int64_t)sg.h * DV;
      chain_part2<NB, OUT, DEEP>(s, tmp, kimg, sm.tu[0], sm.tu[1], sm.l21[c & 1], sm.aqk, fc,
                                 orow0, tok_stride, n, col0, l2 >> 4, l2 & 15);
    }
    lds_barrier();
  }
  if (idle) return;
  float* dst;
  if (OUT) {
    if (sg.seg == A.nseg - 1)
      dst = A.hT + (size_t)sg.bh * kStateFloats;
    else if (sg.seg == 0)
      dst = ws_slot(A, sg.bh, 0);  // segment 0's end state for the composition
    else
      return;  // an inner exact segment: its end state is not needed
  } else if (usev) {
    dst = ws_slot(A, sg.bh, 2 + 2 * (sg.seg - 1));
  } else {
    phi_store<NB>(s, ws_slot(A, sg.bh, 1 + 2 * (sg.seg - 1)), col0, g, ln);
    return;
  }
  state_store<NB>(s, dst, col0, g, ln);
}

// Prep wavefront program (pw = wave - NCW).
template <int NCW>
__device__ void run_prep(const Args& A, Smem& sm, const Seg& sg, int pw, int lane) {
  constexpr bool kDeep = NCW == 4;
  const int64_t tok_stride = (int64_t)A.H * DK;
  const int lw = pw - 2;  // half of the loads that prep waves 2, 3 issue together (v, prologue)
  const bool exact = sg.exact;
  auto rows0 = [&](int c) {  // element offset of the chunk's first token row of head h
    return ((int64_t)sg.b * A.T + (int64_t)(sg.c0 + c) * C) * tok_stride + (int64_t)sg.h * DK;
  };
  auto nrows = [&](int c) { return min(C, A.T - (sg.c0 + c) * C); };
  // loads of one chunk's images, the half h (0, 1) of their 1 KB windows
  auto load_k = [&](int c, int h) {
    if (c < sg.nch) fill128(sm.k[c % 3], A.k + rows0(c), tok_stride, nrows(c) - 1, h, lane);
  };
  auto load_q = [&](int c, int h) {
    if (exact && c < sg.nch)
      fill128(sm.q[c & 1], A.q + rows0(c), tok_stride, nrows(c) - 1, h, lane);
  };
  auto load_v = [&](int c, int h) {
    if (c < sg.nch) fill128(sm.v, A.v + rows0(c), tok_stride, nrows(c) - 1, h, lane);
  };
  auto load_gb = [&](int c, int h) {  // h 0: g, 1: beta
    if (c < sg.nch) {
      const int n = nrows(c);
      const int64_t gi =
          ((int64_t)sg.b * A.T + (int64_t)(sg.c0 + c) * C + min(lane, n - 1)) * A.H + sg.h;
      lds_dma4((h == 0 ? A.g : A.beta) + gi, lds_addr(sm.gb[c & 3] + h * C));
    }
  };
  auto scan = [&](int c) {
    if (c < sg.nch) prep_scan(sm.gb[c & 3], sm.fac[c % 3], nrows(c), A.scale, lane);
  };

  // ---- prologue
  if (pw >= 2) {
    load_k(0, lw);
    load_k(1, lw);
    load_q(0, lw);
    load_v(0, lw);
    load_gb(0, lw);
    load_gb(1, lw);
    load_gb(2, lw);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  } else {
    // constant zeros, in 8-byte groups: the Aqk blocks (tb, sb) with sb > tb
    // (16-row blocks)
    for (int e = 64 * pw + lane; e < 384; e += 128) {
      const int blk = e >> 6, i = e & 63;  // (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
      const int tb = blk < 3 ? 0 : blk < 5 ? 1 : 2;
      const int sb = tb == 0 ? 1 + blk : tb == 1 ? blk - 1 : 3;
      const int arow = 16 * tb + (i >> 2), acg = 4 * sb + (i & 3);
      *reinterpret_cast<uint2*>(sm.aqk + off64(arow, acg >> 1) + (acg & 1) * 4) =
          make_uint2(0u, 0u);
    }
    // T above its diagonal 16x16 blocks inside the 32x32 ones (T01, T23),
    // read as part of Tu11 / Tu22
    for (int e = 64 * pw + lane; e < 512; e += 128) {
      const int blk = e >> 8, i = e & 255;
      sm.t[(32 * blk + (i >> 4)) * DS + 16 + (i & 15)] = 0.0f;
    }
  }
  lds_barrier();  // P0
  if (pw == 3) {
    scan(0);
    scan(1);
  }
  lds_barrier();  // P1
  if (pw < 3) prep_products<kDeep ? 8 : 4>(sm.k[0], sm.fac[0], sm.at[0], sm.l21[0], pw, lane);
  lds_barrier();  // P2
  if (pw < 2) prep_subst(sm.at[0], sm.t, pw, lane);
  lds_barrier();  // P3

  for (int c = 0; c < sg.nch; ++c) {
    const bool more = c + 1 < sg.nch;
    // part 1: waves 0, 1 load half each of k (c + 2), q (c + 1) and g | beta
    // (c + 3), then finish T and Tu of chunk c (their 32x32 halves); waves 2,
    // 3 form the diagonal product blocks of c + 1 (chain wave 3 forms L21)
    if (pw < 2) {
      load_k(c + 2, pw);
      load_q(c + 1, pw);
      load_gb(c + 3, pw);
      prep_merge16(sm.at[c & 1], sm.t, sm.x, sm.fac[c % 3], sm.tu[pw], pw, opaque(lane));
    } else if (more) {
      prep_products<kDeep ? 8 : 4>(sm.k[(c + 1) % 3], sm.fac[(c + 1) % 3], sm.at[(c + 1) & 1],
                                   nullptr, pw - 2, opaque(lane));
      if (!kDeep && pw == 2)  // eight chain wavefronts: L21 here
        prep_products<4>(sm.k[(c + 1) % 3], sm.fac[(c + 1) % 3], nullptr, sm.l21[(c + 1) & 1], 2,
                         opaque(lane));
    }
    lds_barrier();
    // part 2: diagonal blocks of T of c + 1; v of c + 1 (chunk c's U is
    // formed); factors of c + 2
    if (pw < 2 && more) prep_subst(sm.at[(c + 1) & 1], sm.t, pw, opaque(lane));
    if (pw >= 2) load_v(c + 1, lw);
    if (pw == 3) scan(c + 2);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's loads have landed
    lds_barrier();
  }
}

template <int NCW>
__global__ __launch_bounds__(64 * (NCW + 4)) void gdn_fused_kernel(Args A) {
  constexpr int TNB = 8 / NCW;
  __shared__ __attribute__((aligned(16))) Smem sm;
  // wave-uniform in SGPRs: role branches and pointer choices stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int BH = A.B * A.H;
  Seg sg;
  sg.bh = blockIdx.x % BH;
  const int sidx = blockIdx.x / BH;
  sg.seg = A.phase == 1 ? sidx : sidx + 1;
  sg.exact = A.phase == 2 || sg.seg == 0;
  sg.b = sg.bh / A.H;
  sg.h = sg.bh % A.H;
  sg.c0 = A.start[sg.seg];
  sg.nch = A.start[sg.seg + 1] - sg.c0;
  if (wave >= NCW) {
    run_prep<NCW>(A, sm, sg, wave - NCW, lane);
  } else if (sg.exact) {
    run_chain<TNB, true, NCW == 4>(A, sm, sg, wave, false, lane);
  } else if constexpr (NCW == 8) {
    run_chain<2, false, false>(A, sm, sg, wave, false, lane);
  }
}

// Start states of the exact segments 2 .. N-1 (between the two launches):
// S_start(j + 1) = Phi_j S_start(j) + Bseg_j from S_start(1) = segment 0's end
// state.  The composition is independent per state column, so each head's
// 128 columns are split over 8 / NW workgroups of NW wavefronts (the
// workgroups of one head on one XCD, so that its Phi images are read from
// HBM once): wavefront w keeps 16 columns of the state in registers, the
// workgroup loads each Phi_j (as its hi and lo bf16 images) into LDS by
// direct-to-LDS loads while the product with the previous one runs, and
// each composition is written over the columns of Bseg_j it read.  LDS holds an image row r as 16 granules of 16 bytes,
// granule p at position p ^ phi_swz(r): the 16 rows one operand read
// touches then fall in distinct bank groups.
__device__ __forceinline__ int phi_swz(int r) { return (r & 3) | (((r >> 3) & 3) << 2); }

template <int NW>
__global__ __launch_bounds__(64 * NW) void gdn_compose_kernel(Args A) {
  constexpr int WPH = 8 / NW;  // workgroups per head
  __shared__ __attribute__((aligned(16))) bf16 phi_s[2][2 * DK * DK];  // [buf][hi | lo]
  const int BH = A.B * A.H;
  int bh, cq;
  if (BH % 8 == 0) {  // workgroup i runs on XCD i % 8: a head's workgroups share it
    const int i = blockIdx.x, l = i >> 3;
    cq = l % WPH;
    bh = (l / WPH) * 8 + (i & 7);
  } else {
    bh = blockIdx.x / WPH;
    cq = blockIdx.x % WPH;
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, g = lane >> 4, ln = lane & 15;
  const int col0 = 16 * (NW * cq + wave);
  const int nseg = A.nseg;
  float* const ws_head = A.ws + (size_t)bh * (2 * nseg - 3) * kStateFloats;
  auto slot = [&](int idx) { return ws_head + (size_t)idx * kStateFloats; };
  // Phi_j into image buf: 64 windows of 1 KB (four rows each; 0-31 hi,
  // 32-63 lo), wavefront w issuing windows w, w + NW, ..
  auto fetch = [&](int j, int buf) {
    const float* src = slot(1 + 2 * (j - 1));
#pragma unroll
    for (int i = 0; i < 64 / NW; ++i) {
      const int win = NW * i + wave;
      const int r = 4 * (win & 31) + (lane >> 4);
      const int p = (lane & 15) ^ phi_swz(r);
      const uint32_t off = (uint32_t)((win >> 5) * DK * DK * 2 + r * DK * 2 + p * 16);
      lds_dma16(src, off, lds_addr(&phi_s[buf][win * 512]));
    }
  };
  // B_j of the next pass is loaded into registers a pass ahead, and the
  // result of a pass is stored during the next one, so that no global
  // latency sits between two passes
  auto load_b = [&](f32x4 (&dst)[8], int j) {
    const float* src = slot(2 + 2 * (j - 1));
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[kb][r] = src[acc_row(kb, g, r) * DV + col0 + ln];
  };
  auto store_s = [&](const f32x4 (&src)[8], int j) {
    float* dst = slot(2 + 2 * (j - 1));
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[acc_row(kb, g, r) * DV + col0 + ln] = src[kb][r];
  };
  const int last = nseg - 2;  // maps Phi_1 .. Phi_last
  f32x4 s[8], bn[8];
#pragma unroll
  for (int kb = 0; kb < 8; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r) s[kb][r] = slot(0)[acc_row(kb, g, r) * DV + col0 + ln];
  fetch(1, 0);
  load_b(bn, 1);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  for (int j = 1; j <= last; ++j) {
    f32x4 acc[8];
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) acc[kb] = bn[kb];
    if (j + 1 <= last) {
      fetch(j + 1, j & 1);
      load_b(bn, j + 1);
    }
    if (j > 1) store_s(s, j - 1);
    const bf16* phi_hi = phi_s[(j - 1) & 1];
    const bf16* phi_lo = phi_hi + DK * DK;
    bf16x8 bh8[4], bl8[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) split8(s[2 * ks], s[2 * ks + 1], bh8[ks], bl8[ks]);
    // key step outer, key block inner: the eight accumulators' chains
    // interleave
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 8; ++kb) {
        const int row = lam(kb, ln);
        const int at = row * DK + 8 * ((4 * ks + g) ^ phi_swz(row));
        const bf16x8 ah = *reinterpret_cast<const bf16x8*>(phi_hi + at);
        const bf16x8 al = *reinterpret_cast<const bf16x8*>(phi_lo + at);
        acc[kb] = mfma16(ah, bh8[ks], acc[kb]);
        acc[kb] = mfma16(ah, bl8[ks], acc[kb]);
        acc[kb] = mfma16(al, bh8[ks], acc[kb]);
      }
    }
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) s[kb] = acc[kb];
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the next Phi and B have landed
    __syncthreads();
  }
  store_s(s, last);
}

// State pass-through for T = 0: hT = h0 (or 0).
__global__ __launch_bounds__(256) void gdn_copy_state_kernel(const float* h0, float* hT,
                                                             int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) hT[i] = h0 ? h0[i] : 0.0f;
}

// Segment count: enough (head, segment) workgroups for the device's compute
// units in each launch (one workgroup per CU: its LDS images fill one), at
// least 4 chunks per segment, and none when the heads alone fill the device.
static int plan_segments(int64_t BH, int64_t nc, int requested) {
  int ns;
  if (requested > 0) {
    ns = (int)std::min<int64_t>(std::min<int64_t>(requested, kMaxSeg), std::max<int64_t>(nc, 1));
  } else {
    const int cus = device_cu_count();
    if (nc < 8 || 2 * BH > cus) return 1;
    // at most twice the parallelism of one segment: the maps' extra work
    // and the launches' fixed costs only pay off over long sequences
    // (128 heads x 16 chunks: 68 us as one segment, 76 us as three)
    if (cus / BH <= 2 && nc < 32) return 1;
    ns = (int)std::min<int64_t>(std::min<int64_t>(cus / BH + 1, nc / 4), kMaxSeg);
    if (ns < 3) ns = 1;
  }
  return std::max(ns, 1);
}

inline size_t ws_bytes_for(int64_t BH, int nseg) {
  return nseg <= 1 ? 0 : (size_t)BH * (size_t)(2 * nseg - 3) * kStateFloats * sizeof(float);
}

// Argument checks shared by the entry points (0 when the call may proceed).
static int check_args(const void* q, const void* k, const void* v, const float* g,
                      const float* beta, const void* o, const float* hT, int64_t B, int64_t T,
                      int64_t H, int64_t K, int64_t V, int64_t chunk, int dtype) {
  if (B < 0 || T < 0 || H <= 0) return TILEOPS_ESHAPE;
  if (K != DK || V != DV || chunk != C) return TILEOPS_ESHAPE;
  if (B > 65535 || H > 65535 || T > INT32_MAX / 2) return TILEOPS_ESHAPE;
  if (B * H * (int64_t)kMaxSeg > INT32_MAX) return TILEOPS_ESHAPE;
  if (dtype != TILEOPS_BF16) return TILEOPS_EINVAL;
  if (B == 0) return 0;
  if (!hT) return TILEOPS_ENULL;
  if (T > 0) {
    if (!q || !k || !v || !g || !beta || !o) return TILEOPS_ENULL;
    if (!host_aligned16(q) || !host_aligned16(k) || !host_aligned16(v) || !host_aligned16(o))
      return TILEOPS_EINVAL;
  }
  return 0;
}

// The prefill in `nseg` segments (workspace `ws` of ws_bytes_for(BH, nseg)).
static int run(const bf16* q, const bf16* k, const bf16* v, const float* g, const float* beta,
               const float* h0, bf16* o, float* hT, int B, int T, int H, float scale, float* ws,
               int nseg, hipStream_t s) {
  const int64_t BH = (int64_t)B * H;
  if (T == 0) {
    const int64_t n = BH * (int64_t)kStateFloats;
    gdn_copy_state_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(h0, hT, n);
    return launch_status();
  }
  const int nc = (T + C - 1) / C;
  Args a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.g = g;
  a.beta = beta;
  a.h0 = h0;
  a.o = o;
  a.hT = hT;
  a.ws = ws;
  a.B = B;
  a.T = T;
  a.H = H;
  a.scale = scale;
  a.nseg = nseg;
  // Segment 0 gets 4/5 of the others' length: in launch 1 it runs exactly
  // on eight 16-column chains beside the map segments, and per chunk that
  // is the slower of the two (measured at 64 heads x 128 chunks, 5
  // segments: 256 us against 268 us with equal lengths).  Every segment
  // keeps at least one chunk.
  for (int i = 0; i <= kMaxSeg; ++i) a.start[i] = nc;
  a.start[0] = 0;
  {
    const int64_t wsum = 4 + 5 * (int64_t)(nseg - 1);
    for (int i = 1; i < nseg; ++i) {
      const int64_t at = ((int64_t)nc * (4 + 5 * (i - 1)) * 2 + wsum) / (2 * wsum);  // rounded
      a.start[i] = (int)std::min<int64_t>(nc - (nseg - i), std::max<int64_t>(a.start[i - 1] + 1, at));
    }
  }
  const unsigned grid = (unsigned)(BH * std::max(nseg - 1, 1));
  if (nseg == 1) {  // every chunk exact, from h0
    a.phase = 1;
    gdn_fused_kernel<4><<<dim3(grid), dim3(64 * 8), 0, s>>>(a);
    return launch_status();
  }
  a.phase = 1;
  gdn_fused_kernel<8><<<dim3(grid), dim3(64 * 12), 0, s>>>(a);
  if (int e = launch_status()) return e;
  if (nseg > 2) {
    // four workgroups of two wavefronts per head (one per CU at 64 heads)
    gdn_compose_kernel<2><<<dim3((unsigned)(BH * 4)), dim3(128), 0, s>>>(a);
    if (int e = launch_status()) return e;
  }
  a.phase = 2;
  gdn_fused_kernel<4><<<dim3(grid), dim3(64 * 8), 0, s>>>(a);
  return launch_status();
}

// Scratch of the allocation-free entry point: one array per GPU, holding
// the segment maps of the call in flight.  kScratchBytes bounds the
// segments: B * H * (2 N - 3) states of 64 KiB must fit (N = 1 needs none).
constexpr size_t kScratchBytes = (size_t)32 << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

struct DeviceScratch {
  float* ptr = nullptr;
  hipEvent_t last = nullptr;  // completion of the previous call that used the array
  bool recorded = false;
};

// Device address of `scratch` on the current device (looked up once per
// device: in host code the array's name is only a stand-in symbol) and the
// event that orders the calls using it.
static int scratch_of(DeviceScratch** out) {
  static std::mutex mu;
  static DeviceScratch per_dev[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= 64) return TILEOPS_EINVAL;
  std::lock_guard<std::mutex> lock(mu);
  DeviceScratch& d = per_dev[dev];
  if (!d.ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    e = hipEventCreateWithFlags(&d.last, hipEventDisableTiming);
    if (e != hipSuccess) return (int)e;
    d.ptr = static_cast<float*>(p);
  }
  *out = &d;
  return 0;
}

}  // namespace gdn
}  // namespace tileops

using namespace tileops;

extern "C" size_t tileops_gdn_prefill_workspace_bytes_ex(int64_t B, int64_t T, int64_t H,
                                                         int64_t K, int64_t V, int64_t chunk,
                                                         int64_t segments) {
  if (B < 0 || T < 0 || H < 0 || K != gdn::DK || V != gdn::DV || chunk != gdn::C) return 0;
  if (B == 0 || H == 0 || T == 0 || segments < 0 || segments > gdn::kMaxSeg) return 0;
  const int64_t nc = (T + gdn::C - 1) / gdn::C;
  return gdn::ws_bytes_for(B * H, gdn::plan_segments(B * H, nc, (int)segments));
}

extern "C" size_t tileops_gdn_prefill_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K,
                                                      int64_t V, int64_t chunk) {
  return tileops_gdn_prefill_workspace_bytes_ex(B, T, H, K, V, chunk, 0);
}

extern "C" int tileops_gdn_prefill_fwd_ex(const void* q, const void* k, const void* v,
                                          const float* g, const float* beta, const float* h0,
                                          void* o, float* hT, int64_t B, int64_t T, int64_t H,
                                          int64_t K, int64_t V, int64_t chunk, float scale,
                                          int dtype, int64_t segments, void* ws, size_t ws_bytes,
                                          void* stream) {
  if (int e = gdn::check_args(q, k, v, g, beta, o, hT, B, T, H, K, V, chunk, dtype)) return e;
  if (segments < 0 || segments > gdn::kMaxSeg) return TILEOPS_ESHAPE;
  if (B == 0) return 0;
  const int64_t nc = (T + gdn::C - 1) / gdn::C;
  const int nseg = T > 0 ? gdn::plan_segments(B * H, nc, (int)segments) : 1;
  const size_t need = gdn::ws_bytes_for(B * H, nseg);
  if (need > 0) {
    if (ws && !host_aligned16(ws)) return TILEOPS_EINVAL;
    if (!ws || ws_bytes < need) return TILEOPS_EWORKSPACE;
  }
  return gdn::run(static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                  static_cast<const bf16*>(v), g, beta, h0, static_cast<bf16*>(o), hT, (int)B,
                  (int)T, (int)H, scale, static_cast<float*>(ws), nseg,
                  static_cast<hipStream_t>(stream));
}

extern "C" int tileops_gdn_prefill_fwd(const void* q, const void* k, const void* v, const float* g,
                                       const float* beta, const float* h0, void* o, float* hT,
                                       int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                       int64_t chunk, float scale, int dtype, void* ws,
                                       size_t ws_bytes, void* stream) {
  return tileops_gdn_prefill_fwd_ex(q, k, v, g, beta, h0, o, hT, B, T, H, K, V, chunk, scale,
                                    dtype, 0, ws, ws_bytes, stream);
}

extern "C" int tileops_gdn_prefill_fwd_noalloc(const void* q, const void* k, const void* v,
                                               const float* g, const float* beta,
                                               const float* h0, void* o, float* hT, int64_t B,
                                               int64_t T, int64_t H, int64_t K, int64_t V,
                                               int64_t chunk, float scale, int dtype,
                                               void* stream) {
  if (int e = gdn::check_args(q, k, v, g, beta, o, hT, B, T, H, K, V, chunk, dtype)) return e;
  if (B == 0) return 0;
  const int64_t BH = B * H;
  const int64_t nc = (T + gdn::C - 1) / gdn::C;
  int nseg = T > 0 ? gdn::plan_segments(BH, nc, 0) : 1;
  // as many segments as the array holds (fewer segments: a longer chain)
  while (nseg > 1 && gdn::ws_bytes_for(BH, nseg) > gdn::kScratchBytes) --nseg;
  if (nseg == 2) nseg = 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nseg == 1)  // no scratch: nothing to order
    return gdn::run(static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                    static_cast<const bf16*>(v), g, beta, h0, static_cast<bf16*>(o), hT, (int)B,
                    (int)T, (int)H, scale, nullptr, 1, s);
  gdn::DeviceScratch* d = nullptr;
  if (int e = gdn::scratch_of(&d)) return e;
  // Calls that use the array run one after the other on the device: each
  // waits for the previous one's completion event (recorded on whatever
  // stream that call ran on) and records its own.  Under stream capture the
  // graph's own order applies and the event is left alone.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t he = hipStreamIsCapturing(s, &cap);
  if (he != hipSuccess) return (int)he;
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order && d->recorded) {
    he = hipStreamWaitEvent(s, d->last, 0);
    if (he != hipSuccess) return (int)he;
  }
  const int e = gdn::run(static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                         static_cast<const bf16*>(v), g, beta, h0, static_cast<bf16*>(o), hT,
                         (int)B, (int)T, (int)H, scale, d->ptr, nseg, s);
  if (e) return e;
  if (order) {
    he = hipEventRecord(d->last, s);
    if (he != hipSuccess) return (int)he;
    d->recorded = true;
  }
  return 0;
}
