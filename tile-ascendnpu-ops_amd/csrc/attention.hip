// Flash-attention forward for gfx950 (tileops_mha_fwd), BSHD layout.
//
// One workgroup = 8 wavefronts = BM = 256 query rows of one (batch, head);
// each wavefront owns 32 query rows.  Keys/values stream through LDS in
// tiles of BN rows filled by direct-to-LDS loads (no register staging):
// BN = 128 with two LDS slots per operand for D = 128 (128 KB), BN = 64
// with three slots for D = 64.  The longer tile halves the barriers and
// per-tile bookkeeping per key.
//
// Both products run on v_mfma_f32_32x32x16_{bf16,f16} in the *transposed*
// orientation:
//   S^T (kv x q) = K (kv x D) . Q^T (D x q)      A = K from LDS, B = Q in VGPRs
//   O^T (d x q) += V^T (d x kv) . P^T (kv x q)   A = V^T from LDS, B = P in VGPRs
// With 32x32 MFMA results, lane l holds column l % 32, i.e. one query row,
// and 16 key rows of each 32-key block (the other 16 sit in lane l ^ 32).
// The online softmax is therefore lane-local except for one exchange with
// the partner lane, and P feeds the second MFMA straight from registers.
// V stays in LDS as loaded (key rows); its A operand comes from transpose
// reads (ds_read_b64_tr_b16), which deliver one head dim of four
// consecutive keys per lane in the key order P^T has in registers.
//
// The two groups of four wavefronts alternate between MFMA work and the
// softmax (ping-pong), so that every SIMD, which hosts one wavefront of
// each group, has MFMA work while the other wavefront computes exponentials.
//
// The softmax runs in the log2 domain (scores scaled by scale * log2 e); the
// per-row LSE written out is m + log2(l), i.e. logsumexp(scale q k^T) / ln 2.
//
// Head dims that are not powers of two (96, 192) keep the LDS images of the
// next power of two (rows of 128 or 256 elements, the same swizzles): the
// padding chunks are filled with a copy of a real chunk of the row and never
// read, and the MFMA steps cover the real dims only.
#include <float.h>
#include <stdlib.h>

#include <type_traits>

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
constexpr float kLazyBound = 256.0f;  // 2^kLazyLog2

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// K and V tiles live in LDS unpadded, rows of D / 8 16-byte chunks, chunks
// XOR-swizzled by row: K so that an MFMA operand read (16 consecutive key
// rows, one chunk each) hits 16 distinct 16-byte bank groups, V so that the
// transpose reads of a half-wavefront (4 consecutive key rows x 64 bytes)
// cover all 64 banks once.
template <int D> struct Swz {
  static constexpr int CPR = D / 8;  // chunks per row
  __host__ __device__ static constexpr int k_key(int r) { return CPR >= 16 ? (r & 15) : ((r >> 1) & 7); }
  __host__ __device__ static constexpr int v_key(int r) { return CPR == 16 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); }
};

// Workgroup barrier that waits only for this wavefront's LDS accesses, so
// that direct-to-LDS loads issued before it stay in flight across it.  The
// scheduling barriers keep arithmetic on its side as well: s_barrier alone
// orders memory accesses, but MFMA or VALU work could otherwise drift into
// the neighbouring phase, where the ping-pong has the other group's work.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// One 16-byte direct-to-LDS load per lane: lane l reads 16 bytes at
// `base + off` (base uniform, in SGPRs; off a per-lane byte offset) and they
// land at LDS byte address lds + 16 l.  Issued as inline assembly so that the
// compiler does not track the LDS write: every wait for these loads is
// explicit (vmcnt) and followed by a workgroup barrier before any wavefront
// reads the data.  The compiler's hazard checks do not look into inline
// assembly: the load starts with the one wait state the ISA requires after
// the SALU write of M0 that precedes it (its base comes from SALU
// arithmetic, so no VALU-to-SGPR wait is involved).
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "{m0}"(lds)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void_ptr)p;
}

// Combine a value with the one held by the partner lane l ^ 32 (VALU lane
// swap between the two wavefront halves, no LDS round trip): the two
// outputs of v_permlane32_swap on (x, x) are x's low and high halves.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, x), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// Ping-pong schedule.  The 8 wavefronts form two groups, A = waves 0-3 and
// B = waves 4-7, so that each SIMD hosts one wavefront of each.  A tile step
// tau has two phases separated by workgroup barriers; in every phase one
// group runs only MFMA work (O += V^T P^T of tile tau - 1, then S of tile
// tau) while the other runs its softmax.  With three slots (BN = 64) the
// MFMA group also issues the direct-to-LDS loads of a tile two steps ahead
// between its MFMAs:
//   phase 0:  A: O(tau-1), S(tau), V(tau+1) -> slot     B: softmax(tau-1)
//   phase 1:  A: softmax(tau)     B: O(tau-1), S(tau), K(tau+2) -> slot
// (the two-slot schedule of BN = 128 is described at the loops).
// K and V have three LDS slots each (tile t in slot t mod 3).  Numbering the
// phases from 0, K(t) is read in phases 2t (A) and 2t + 1 (B) and issued in
// phase 2t - 3, V(t) is read in phases 2t + 2 (A) and 2t + 3 (B) and issued
// in phase 2t - 2: after the tile three back in the same slot was last read
// (phases 2t - 5 and 2t - 3), and each group ends every MFMA phase waiting
// for everything but the windows it just issued (vmcnt(WPW)), so a tile has
// landed two phases before its first reader.
// tanh(y) = 1 - 2 / (1 + e^{2y}), saturating to +-1 through the
// exponential's overflow / underflow (no branch)
__device__ __forceinline__ float tanh_sat(float y) {
  const float e = __builtin_amdgcn_exp2f(y * (2.0f * 1.4426950408889634f));
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
}

// SOFTCAP: scores are capped, softcap * tanh(scale q.k / softcap) (the
// reference's order: scale, cap, then the causal mask), and carried in log2
// units from the start of the softmax: the caller passes scale_log2 = 1,
// cap_scale = scale / softcap and cap_log2 = softcap * log2 e.
// D: the head dim of q, k and v rows; DV: the v columns (and output columns)
// a workgroup computes, D itself up to 128, half of it for D = 192 and 256
// (two workgroups per query block, each forming the full scores).
template <typename T, int D, int DV, bool CAUSAL, int BN, bool SOFTCAP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void mha_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ o,
    float* __restrict__ lse, int B, int Sq, int Skv, int H, int Hkv, float scale_log2, int nqb,
    float cap_scale, float cap_log2) {
  typedef typename Mfma<T>::V8 V8;
  constexpr int NKB = BN / 32;    // 32-key blocks per tile
  constexpr int BM = 256;         // query rows per workgroup (8 x 32)
  constexpr int KSTEPS = D / 16;  // MFMA steps over the head dim
  constexpr int DBLK = DV / 32;   // 32-row blocks of O^T
  // LDS row widths: the next power of two of D and DV
  constexpr int DP = D <= 64 ? 64 : D <= 128 ? 128 : 256;
  constexpr int DVP = DV <= 64 ? 64 : 128;
  constexpr int TILE_K = BN * DP;  // elements per K tile
  constexpr int TILE_V = BN * DVP; // elements per V tile (this workgroup's columns)
  constexpr int NW_K = TILE_K / 2048, NW_V = TILE_V / 2048;  // 1 KB windows per wavefront
  static_assert(D % 32 == 0 && DV % 32 == 0 && DV <= 128, "head dims");
  static_assert(BN == 64 || (BN == 128 && DP == 128), "tile shapes");
  static_assert(DV == D || (D == 2 * DV && D >= 192), "value split");
  static_assert(NW_V >= 1 && NW_K <= 15, "vmcnt immediate");
  constexpr int NSLOT = BN == 64 ? 3 : 2;  // LDS slots per operand
  // Q through LDS in the prologue (non-causal 128-key tiles; measured
  // 1.5 % faster there and 1.5 % slower on the causal blocks, which keep
  // the register loads)
  constexpr bool QLDS = NSLOT == 2 && !CAUSAL && D == DP;

  // (aligned so that the XOR-formed operand addresses below hold)
  __shared__ __attribute__((aligned(1024))) T k_lds[NSLOT * TILE_K];
  __shared__ __attribute__((aligned(1024))) T v_lds[NSLOT * TILE_V];
  // group A's query rows during the prologue (with QLDS)
  __shared__ __attribute__((aligned(16))) T q_lds[QLDS ? 128 * D : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wavefront-uniform
  const int col = lane & 31;  // query row inside the wave's 32
  const int half = lane >> 5;
  const bool grp_a = wave < 4;
  const int gw = wave & 3;     // wavefront index inside its group

  // --- XCD-aware block order: workgroups are dealt round-robin to the 8
  // XCDs; regroup so that one XCD works through all query blocks of a head
  // together and that head's K/V stays in the XCD's L2.  Causal blocks
  // differ in length: they go longest first over pairs of heads (the query
  // blocks of two heads interleaved), so that the last workgroups an XCD
  // receives are short ones.
  // (the value halves of one query block, D = 192 and 256, are neighbours)
  constexpr int NDV = D / DV;
  const int nblk = (int)gridDim.x;
  int id = blockIdx.x;
  if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);
  const int dv0 = (id % NDV) * DV;
  id /= NDV;
  int qb, head;
  if (CAUSAL) {
    const int pair = id / (2 * nqb), k2 = id - pair * 2 * nqb;
    if (2 * pair + 1 < H * B) {
      // Inside an XCD, consecutive workgroups go to its shader engines in a
      // fixed rotation of four, and dispatch is in order: a shader engine
      // that receives longer blocks holds up the others.  So in each group
      // of four (two lengths, one per head each), the longer pair takes the
      // first two positions in even groups and the last two in odd ones:
      // every position then sums to the same work over two groups.
      const int m = k2 >> 2, s = k2 & 3;
      const int r = 2 * m + 1 >= nqb ? 2 * m : 2 * m + ((s >> 1) ^ (m & 1));
      head = 2 * pair + (s & 1);
      qb = nqb - 1 - r;
    } else {  // an odd last head on its own
      head = 2 * pair;
      qb = nqb - 1 - k2;
    }
  } else {
    qb = id % nqb;
    head = id / nqb;
  }
  const int hq = head % H;
  const int bb = head / H;
  const int hk = hq / (H / Hkv);
  const int q0 = qb * BM;
  const int off = Skv - Sq;  // right-aligned causal offset

  const int64_t q_row = (int64_t)H * D;
  const int64_t kv_row = (int64_t)Hkv * D;
  const T* qbase = q + (int64_t)bb * Sq * q_row + (int64_t)hq * D;
  const T* kbase = k + (int64_t)bb * Skv * kv_row + (int64_t)hk * D;
  const T* vbase = v + (int64_t)bb * Skv * kv_row + (int64_t)hk * D + dv0;

  // --- Q^T operand: this lane's query row, 8 dims per MFMA step (with
  // QLDS it comes through LDS in the prologue instead)
  const int qi = q0 + wave * 32 + col;
  V8 qreg[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    if (QLDS) {
      qreg[ks] = V8{};
    } else if (qi < Sq) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qbase + (int64_t)qi * q_row + ks * 16 + half * 8);
      qreg[ks] = *reinterpret_cast<V8*>(&raw);
    } else {
      qreg[ks] = V8{};
    }
  }

  // last visible key of this lane's query row, less the lane half's key
  // offset inside a 32-key block (4 half): the masks below compare the
  // block-relative key index against it
  const int mask_lim = (CAUSAL ? min(Skv - 1, qi + off) : Skv - 1) - 4 * half;
  const int kv_end = CAUSAL ? min(Skv, q0 + BM + off) : Skv;
  const int ntiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  // Direct-to-LDS tile loads (group B loads K, group A loads V).  Window i
  // (of NW) of tile t: lane l fills LDS chunk (4 i + gw) * 64 + l of the
  // tile's swizzled image, i.e. row r = i * WROWS + rl, position p = l mod
  // CPR (the row's 16-byte chunks), with global chunk p ^ key(r) of key row
  // min(r, rmax): rows past the last key repeat it (their scores are
  // masked).  When WROWS is a multiple of the swizzle key's period (16 rows)
  // the key depends only on rl and the chunk's byte offset is one per-lane
  // constant; with 512-byte rows (D = 192 and 256, WROWS = 8) it is formed per
  // window.  A tile past the last one
  // (the schedule issues its loads regardless) re-reads the last tile into
  // its own slot, which no phase reads, so every load is in bounds and the
  // wait counts never vary.
  const uint32_t row_bytes = (uint32_t)(kv_row * sizeof(T));
  auto loader = [&](auto is_v) __device__ __attribute__((always_inline)) {
    constexpr bool IS_V = decltype(is_v)::value;
    constexpr int DL = IS_V ? DVP : DP, CPR = DL / 8, WROWS = 256 / CPR;
    constexpr int RCPR = (IS_V ? DV : D) / 8;  // chunks of a row in global memory
    constexpr int TL = BN * DL;
    const int rl = gw * (64 / CPR) + lane / CPR;
    auto key = [](int r) { return IS_V ? Swz<DL>::v_key(r) : Swz<DL>::k_key(r); };
    // global chunk of LDS position p of row r; a padding position takes a
    // copy of real chunk c - (CPR - RCPR), never read
    auto gchunk = [](int p, int r) {
      const int c = p ^ (IS_V ? Swz<DL>::v_key(r) : Swz<DL>::k_key(r));
      return c < RCPR ? c : c - (CPR - RCPR);
    };
    (void)key;
    const uint32_t cbyte = (uint32_t)((gchunk(lane % CPR, rl) << 3) * sizeof(T));
    const T* gsrc = IS_V ? vbase : kbase;
    T* gdst = IS_V ? v_lds : k_lds;
    return [=](int t, int i) __device__ __attribute__((always_inline)) {
      const int te = min(t, ntiles - 1);
      const T* src = gsrc + (int64_t)te * BN * kv_row;
      const int rmax = min(BN - 1, Skv - 1 - te * BN);
      const uint32_t lds = lds_addr(gdst + (uint32_t)(t % NSLOT) * TL) + (uint32_t)gw * 1024;
      const int r = i * WROWS + rl;
      const uint32_t cb =
          WROWS % 16 == 0 ? cbyte : (uint32_t)((gchunk(lane % CPR, r) << 3) * sizeof(T));
      lds_dma16(src, (uint32_t)min(r, rmax) * row_bytes + cb, lds + i * 4096);
    };
  };
  const auto load_window_v = loader(std::integral_constant<bool, true>());
  const auto load_window_k = loader(std::integral_constant<bool, false>());
  auto load_tile = [&](int t) __device__ __attribute__((always_inline)) {
    if (grp_a) {
#pragma unroll
      for (int i = 0; i < NW_V; ++i) load_window_v(t, i);
    } else {
#pragma unroll
      for (int i = 0; i < NW_K; ++i) load_window_k(t, i);
    }
  };
  // End of an MFMA phase with NWL windows issued in it: every tile this
  // wavefront loaded earlier has landed; those NWL may stay in flight.
  auto wait_loads = [&](auto nwl) __device__ __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0F70 | decltype(nwl)::value);  // vmcnt(NWL)
  };

  f32x16 acc_o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) acc_o[i] = f32x16{};
  f32x16 acc_s[NKB];
  V8 pb[2 * NKB];
  float m_run = -INFINITY;  // running max of raw scores q . k (capped, log2 units with SOFTCAP)
  float l_run = 0.0f;
  const float lazy_raw = kLazyLog2 / scale_log2;

  // Lane-dependent LDS byte addresses of the operand reads, one register per
  // operand: the per-step terms enter by XOR, the slot and key-block terms
  // as DS immediate offsets.
  // K (S^T A operand): row kb * 32 + col, chunk (2 ks + half) ^ key(col).
  // As 2 ks + half = 2 ks ^ half, the byte offset col 2D + 16 ((2 ks + half)
  // ^ key) equals (col 2D + 16 (half ^ key)) ^ 32 ks: the bits of 32 ks
  // (5 .. log2(2D) - 1) are clear in col 2D and in the LDS base (aligned).
  const uint32_t kbx = lds_addr(k_lds) + (uint32_t)(col * DP * (int)sizeof(T)) +
                       16u * (uint32_t)(half ^ Swz<DP>::k_key(col));
  // V^T (O^T A operand) through transpose reads: in each group of 16 lanes,
  // lane j points at 4 dims (4 (j % 4) ..) of key row j / 4 and receives
  // dim j of those 4 keys.  Key slot 4 rr + e of lane half g is key
  // 16 ks + 8 rr + 4 g + e, the order in which P^T sits in registers; the
  // ks and rr terms are constants (the swizzle key depends on row % 4 only).
  // Dim block db adds 4 db to the chunk index, and the swizzle key is a
  // multiple of 4 below 4 DBLK, so the block enters as XOR with 64 db.
  const int grp16 = lane >> 4, j16 = lane & 15;
  const int vrow = 4 * (grp16 >> 1) + (j16 >> 2);
  uint32_t vbx;
  {
    const int dim = 16 * (grp16 & 1) + 4 * (j16 & 3);
    vbx = lds_addr(v_lds) +
          (uint32_t)((vrow * DVP + ((((dim >> 3) ^ Swz<DVP>::v_key(vrow)) << 3) | (dim & 7))) *
                     (int)sizeof(T));
  }
  static_assert(Swz<DVP>::v_key(0) == 0 && Swz<DVP>::v_key(3) % 4 == 0, "V swizzle key");
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  typedef __attribute__((address_space(3))) V8 lds_v8;
  // A operand of the O^T update: 8 keys (16 ks + 8 rr + ..) of dim block db,
  // two 64-bit transpose reads assembled by whole-register moves
  auto read_vt = [&](uint32_t vb, int ks) __device__ __attribute__((always_inline)) -> V8 {
    const v4i16 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(uintptr_t)(vb + (16 * ks) * DVP * 2));
    const v4i16 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(uintptr_t)(vb + (16 * ks + 8) * DVP * 2));
    const u32x2 y0 = __builtin_bit_cast(u32x2, x0), y1 = __builtin_bit_cast(u32x2, x1);
    const u32x4 w = {y0.x, y0.y, y1.x, y1.y};
    return __builtin_bit_cast(V8, w);
  };
  auto read_k = [&](uint32_t kb, int blk) __device__ __attribute__((always_inline)) -> V8 {
    return *(lds_v8*)(uintptr_t)(kb + blk * 32 * DP * 2);
  };

  // The MFMA phase as one sequence: per 16-key step j, the DBLK O^T blocks
  // of keys 16 j .. 16 j + 15 (when DO_O), then WS of the KSTEPS x NKB S^T
  // products (head-dim step major, key block minor: products WS j .. WS j
  // + WS - 1) (when DO_S), so that up to DBLK + NKB independent accumulators
  // alternate.  Each operand is
  // read from LDS PF MFMAs ahead into a ring of PF + 1 register sets, and
  // the order MFMA, then the reads of the operand PF ahead, is pinned with
  // scheduling groups: left alone, the scheduler issues most reads just
  // before their MFMA and waits out the LDS latency each time.  With LD,
  // the NW windows of tile lt are issued one every N / NW MFMAs.
  auto mfma_phase = [&](auto do_o, auto do_s, auto ld, auto vslot, auto kslot, int lt)
      __device__ __attribute__((always_inline)) {
    constexpr bool DO_O = decltype(do_o)::value, DO_S = decltype(do_s)::value;
    constexpr int LD = decltype(ld)::value;  // 0: no loads, 1: V windows, 2: K windows
    constexpr int NWL = LD == 1 ? NW_V : LD == 2 ? NW_K : 1;
    constexpr int J = BN / 16;                             // 16-key steps per tile
    constexpr int WO = DO_O ? DBLK : 0, WS = DO_S ? KSTEPS * NKB / J : 0;
    constexpr int W = WO + WS;                             // MFMAs per 16-key step
    constexpr int N = J * W;
    // windows issued at MFMAs LDSTEP i + LDPOS, i < NWL
    constexpr int LDSTEP = N / NWL, LDPOS = LDSTEP > 5 ? 5 : LDSTEP - 1;
    static_assert((KSTEPS * NKB) % J == 0, "S products per 16-key step");
    if (DO_S) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) acc_s[kb] = f32x16{};
    }
    // slot offsets: immediate DS offsets when the slot is a compile-time
    // constant (the unrolled loop), one add per address otherwise.  The
    // base registers pass through an empty asm here, so that the per-step
    // XORs are formed inside the phase rather than hoisted into one
    // register each for the whole kernel.
    uint32_t kx = kbx, vx = vbx;
    asm volatile("" : "+v"(kx), "+v"(vx));
    const uint32_t vso = (uint32_t)(int)vslot * TILE_V * (uint32_t)sizeof(T);
    const uint32_t kso = (uint32_t)(int)kslot * TILE_K * (uint32_t)sizeof(T);
    auto vb = [&](int db) __device__ __attribute__((always_inline)) {
      return (vx ^ (64u * (uint32_t)db)) + vso;
    };
    auto kb = [&](int ks) __device__ __attribute__((always_inline)) {
      return (kx ^ (32u * (uint32_t)ks)) + kso;
    };
    auto fetch = [&](int n) __device__ __attribute__((always_inline)) -> V8 {
      const int j = n / W, w = n % W;
      if (w < WO) return read_vt(vb(w), j);
      const int si = WS * j + (w - WO);  // S product: head-dim step si / NKB, key block si % NKB
      return read_k(kb(si / NKB), si % NKB);
    };
    // LDS read instructions of operand n: two transpose reads for V^T, one
    // 16-byte read for K (the scheduling-group sizes must be constants)
    auto group_reads = [&](int n) __device__ __attribute__((always_inline)) {
      if ((n % W) < WO) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    };
    constexpr int PF = 4;  // operand reads in flight ahead of the MFMA using them
    V8 ring[PF + 1];
#pragma unroll
    for (int n = 0; n < PF; ++n) ring[n] = fetch(n);
#pragma unroll
    for (int n = 0; n < PF; ++n) group_reads(n);
#pragma unroll
    for (int n = 0; n < N; ++n) {
      if (n + PF < N) ring[(n + PF) % (PF + 1)] = fetch(n + PF);
      const int j = n / W, w = n % W;
      if (w < WO) {
        acc_o[w] = Mfma<T>::run(ring[n % (PF + 1)], pb[j], acc_o[w]);
      } else {
        const int si = WS * j + (w - WO);
        const int ks = si / NKB, kb = si % NKB;
        acc_s[kb] = Mfma<T>::run(ring[n % (PF + 1)], qreg[ks], acc_s[kb]);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // this MFMA
      if (n + PF < N) group_reads(n + PF);
      if (LD == 1 && n % LDSTEP == LDPOS && n / LDSTEP < NWL) load_window_v(lt, n / LDSTEP);
      if (LD == 2 && n % LDSTEP == LDPOS && n / LDSTEP < NWL) load_window_k(lt, n / LDSTEP);
    }
  };
  typedef std::integral_constant<bool, true> yes;
  typedef std::integral_constant<bool, false> no;
  typedef std::integral_constant<int, 0> ld_none;
  typedef std::integral_constant<int, 1> ld_v;
  typedef std::integral_constant<int, 2> ld_k;
  typedef std::integral_constant<int, NW_V> nw_v;
  typedef std::integral_constant<int, NW_K> nw_k;

  // P = exp2(scale_log2 * s + neg_mc) of the tile in acc_s into pb (the
  // MFMA operand, rounded to the storage type); returns this lane's partial
  // row sum of the fp32 probabilities (the sum and the LSE stay in fp32).
  auto exps = [&](float neg_mc) __device__ __attribute__((always_inline)) -> float {
    float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[kb][r], scale_log2, neg_mc));
        ps[r & 3] += p;
        pb[kb * 2 + (r >> 3)][r & 7] = (T)p;
      }
    }
    return (ps[0] + ps[1]) + (ps[2] + ps[3]);
  };

  // online softmax of tile t for query row qi: maxima in raw score units,
  // the scale (times log2 e) folded into one FMA per score inside exp2
  auto softmax = [&](int t) __device__ __attribute__((always_inline)) {
    if constexpr (SOFTCAP) {  // capped scores in log2 units (monotone: the row max is kept)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_s[kb][r] = cap_log2 * tanh_sat(acc_s[kb][r] * cap_scale);
      }
    }
    const int kv0 = t * BN;
    // masking only on the ragged last tile and on causal diagonal tiles
    // (a workgroup-uniform branch, kept out of the common path)
    if ((kv0 + BN > Skv) || (CAUSAL && kv0 + BN - 1 > q0 + off)) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kv = kv0 + kb * 32 + (r >> 2) * 8 + (r & 3);  // key less 4 half
          acc_s[kb][r] = kv > mask_lim ? -INFINITY : acc_s[kb][r];
        }
      }
    }
    // Exponentials against the running max first: while every P of the
    // tile stays <= 2^kLazyLog2 (certain when this lane's partial sum does,
    // all terms being >= 0) the running max need not move and the tile's
    // max is never formed.  Otherwise (a new row max, a row without a
    // reference max yet, a NaN) the wavefront forms the tile max, rescales
    // and recomputes.  The two lanes of a row see the same max either way.
    float ps = exps(m_run == -INFINITY ? 0.0f : -m_run * scale_log2);
    if (__any(!(ps <= kLazyBound) || m_run == -INFINITY)) {
      float tm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) tm[r & 3] = fmaxf(tm[r & 3], acc_s[kb][r]);
      }
      const float tmax = pair_max(fmaxf(fmaxf(tm[0], tm[1]), fmaxf(tm[2], tm[3])));
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.0f
                                             : __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[db][r] *= alpha;
      }
      // rows with no visible key yet keep m = -inf: shift by 0 so exp2 -> 0
      ps = exps(m_run == -INFINITY ? 0.0f : -m_run * scale_log2);
    }
    l_run += ps;
    // materialise P here: pure arithmetic may otherwise sink past the next
    // barrier into the O update, out of the phase meant to overlap the
    // other group's MFMA work
#pragma unroll
    for (int i = 0; i < 2 * NKB; ++i) asm volatile("" : "+v"(pb[i]));
    asm volatile("" : "+v"(l_run));
  };

  // --- prologue
  if constexpr (QLDS) {
    // Q through LDS: each group's 128 query rows as one swizzled image like
    // a K tile (whole 256-byte rows per load, where register loads in the
    // MFMA layout would touch 32 rows per instruction), group A's in its
    // own region, group B's in V slot 1 (free until V(1) is issued, two
    // barriers later); rows past Sq repeat the last row (never stored).
    // Then V(0) (group A), K(0) and K(1) (group B) into their slots; each
    // group waits for its Q (and group B for K(0)) before the barrier, the
    // rest by the waits of the first phases.
    {
      const int qr0 = min(q0 + (grp_a ? 0 : 128), Sq - 1);
      const int rmax = min(127, Sq - 1 - qr0);
      const T* src = qbase + (int64_t)qr0 * q_row;
      const uint32_t qrow_bytes = (uint32_t)(q_row * sizeof(T));
      const int rl = gw * 4 + lane / 16;
      const uint32_t cb = (uint32_t)((((lane % 16) ^ Swz<D>::k_key(rl)) << 3) * sizeof(T));
      const uint32_t lds = lds_addr(grp_a ? q_lds : v_lds + TILE_V) + (uint32_t)gw * 1024;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        lds_dma16(src, (uint32_t)min(i * 16 + rl, rmax) * qrow_bytes + cb, lds + i * 4096);
    }
    load_tile(0);
    if (grp_a) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | NW_V);  // Q has landed
    } else {
      load_tile(1);
      __builtin_amdgcn_s_waitcnt(0x0F70 | NW_K);  // Q and K(0) have landed
    }
    lds_barrier();
    {
      const uint32_t qb = lds_addr(grp_a ? q_lds : v_lds + TILE_V) + (uint32_t)gw * 32 * D * 2;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
        qreg[ks] = read_k((kbx ^ (32u * (uint32_t)ks)) - lds_addr(k_lds) + qb, 0);
    }
  } else {
    // K(0), K(1) (group B) and V(0) (group A) into their slots
    if (ntiles > 0) {
      load_tile(0);
      if (!grp_a) load_tile(1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // One loop per group, each body a softmax phase then an MFMA phase (group
  // A's steps rotated by half a step so that both loops have that shape);
  // both pass 2 (ntiles + 1) barriers in all.  With phases numbered from 0:
  //   A: phase 0: S(0), V(1);  then per tau: softmax(tau) | O(tau), S(tau+1), V(tau+2)
  //   B: phase 1: S(0), K(2);  then per tau: softmax(tau-1) | O(tau-1), S(tau), K(tau+2)
  // The last step of each loop (O only, no S, no loads) is peeled off, and
  // the loops are unrolled by three so that every slot index is a constant
  // (tile t lives in slot t mod 3).
  typedef std::integral_constant<int, 0> s0;
  typedef std::integral_constant<int, 1> s1;
  typedef std::integral_constant<int, 2> s2;
  if constexpr (NSLOT == 3) {
  // one loop step: softmax phase, then MFMA phase (slots as constants)
  auto step = [&](auto ld, auto nwl, auto vslot, auto kslot, int t_soft, int t_load)
      __device__ __attribute__((always_inline)) {
    softmax(t_soft);
    lds_barrier();
    mfma_phase(yes(), yes(), ld, vslot, kslot, t_load);
    wait_loads(nwl);
    lds_barrier();
  };
  if (grp_a) {
    if (ntiles > 0) {
      mfma_phase(no(), yes(), ld_v(), s0(), s0(), 1);
      wait_loads(nw_v());
    }
    lds_barrier();
    // step tau: softmax(tau) | O(tau) (V slot tau % 3), S(tau + 1) (K slot (tau + 1) % 3)
    int tau = 0;
    for (; tau + 3 < ntiles; tau += 3) {
      step(ld_v(), nw_v(), s0(), s1(), tau, tau + 2);
      step(ld_v(), nw_v(), s1(), s2(), tau + 1, tau + 3);
      step(ld_v(), nw_v(), s2(), s0(), tau + 2, tau + 4);
    }
    if (tau + 1 < ntiles) {
      step(ld_v(), nw_v(), s0(), s1(), tau, tau + 2);
      ++tau;
      if (tau + 1 < ntiles) step(ld_v(), nw_v(), s1(), s2(), tau, tau + 2);
    }
    if (ntiles > 0) {
      const int t = ntiles - 1;
      // a last tile wholly above this wavefront's rows adds nothing (as in
      // the two-slot schedule below)
      const bool live = !CAUSAL || t * BN <= q0 + wave * 32 + 31 + off;
      if (live) softmax(t);
      lds_barrier();
      if (live) mfma_phase(yes(), no(), ld_none(), t % 3, 0, -1);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      lds_barrier();
    }
    lds_barrier();  // softmax phase of step ntiles (nothing left to do)
  } else {
    lds_barrier();  // phase 0: group A computes S(0)
    if (ntiles > 0) {
      mfma_phase(no(), yes(), ld_k(), s0(), s0(), 2);
      wait_loads(nw_k());
    }
    lds_barrier();
    // step tau: softmax(tau - 1) | O(tau - 1) (V slot (tau - 1) % 3), S(tau) (K slot tau % 3)
    int tau = 1;
    for (; tau + 2 < ntiles; tau += 3) {
      step(ld_k(), nw_k(), s0(), s1(), tau - 1, tau + 2);
      step(ld_k(), nw_k(), s1(), s2(), tau, tau + 3);
      step(ld_k(), nw_k(), s2(), s0(), tau + 1, tau + 4);
    }
    if (tau < ntiles) {
      step(ld_k(), nw_k(), s0(), s1(), tau - 1, tau + 2);
      ++tau;
      if (tau < ntiles) step(ld_k(), nw_k(), s1(), s2(), tau - 1, tau + 2);
    }
    if (ntiles > 0) {
      const int t = ntiles;
      softmax(t - 1);
      lds_barrier();
      mfma_phase(yes(), no(), ld_none(), (t - 1) % 3, 0, -1);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      lds_barrier();
    }
  }
  } else {
  // Two slots (128-key tiles).  K(t) is read in phases 2t (A) and 2t + 1
  // (B); group B issues it in its softmax phase 2t - 2 and waits for it at
  // the end of phase 2t - 1.  V(t) is read in phases 2t + 2 (A) and 2t + 3
  // (B); group A issues it between the MFMAs of phase 2t and waits for it
  // at the end of phase 2t + 1.  Either way the slot's previous tile (t - 2)
  // was last read in the phase before the issue.
  if (grp_a) {
    if (ntiles > 0) mfma_phase(no(), yes(), ld_none(), s0(), s0(), -1);  // phase 0: S(0)
    lds_barrier();
    // step tau: softmax(tau) | O(tau) (V slot tau % 2), S(tau + 1), V(tau + 1)
    auto step_a = [&](auto vslot, auto kslot, int tau) __device__ __attribute__((always_inline)) {
      softmax(tau);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): V(tau) has landed
      lds_barrier();
      mfma_phase(yes(), yes(), ld_v(), vslot, kslot, tau + 1);
      lds_barrier();
    };
    int tau = 0;
    for (; tau + 2 < ntiles; tau += 2) {
      step_a(s0(), s1(), tau);
      step_a(s1(), s0(), tau + 1);
    }
    if (tau + 1 < ntiles) {
      step_a(s0(), s1(), tau);
      ++tau;
    }
    if (ntiles > 0) {
      const int t = ntiles - 1;
      // Under a causal mask the last tile can lie wholly above this
      // wavefront's rows (group A's 128 rows against the block's last 128
      // keys): its probabilities are all 0, so its softmax and P V add
      // nothing and are skipped (S(t) was formed, unused; every barrier and
      // wait is kept).
      const bool live = !CAUSAL || t * BN <= q0 + wave * 32 + 31 + off;
      if (live) softmax(t);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      lds_barrier();
      if (live) mfma_phase(yes(), no(), ld_none(), t % 2, 0, -1);
      lds_barrier();
    }
    lds_barrier();  // softmax phase of step ntiles (nothing left to do)
  } else {
    lds_barrier();  // phase 0: group A computes S(0)
    if (ntiles > 0) mfma_phase(no(), yes(), ld_none(), s0(), s0(), -1);  // phase 1: S(0)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K(1), read in phase 2, has landed
    lds_barrier();
    // step tau: softmax(tau - 1), K(tau + 1) | O(tau - 1) (V slot (tau - 1) % 2), S(tau)
    auto step_b = [&](auto vslot, auto kslot, int tau) __device__ __attribute__((always_inline)) {
      load_tile(tau + 1);
      softmax(tau - 1);
      lds_barrier();
      mfma_phase(yes(), yes(), ld_none(), vslot, kslot, -1);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K(tau + 1) has landed
      lds_barrier();
    };
    int tau = 1;
    for (; tau + 1 < ntiles; tau += 2) {
      step_b(s0(), s1(), tau);
      step_b(s1(), s0(), tau + 1);
    }
    if (tau < ntiles) {
      step_b(s0(), s1(), tau);
      ++tau;
    }
    if (ntiles > 0) {
      const int t = ntiles;
      softmax(t - 1);
      lds_barrier();
      mfma_phase(yes(), no(), ld_none(), (t - 1) % 2, 0, -1);
      lds_barrier();
    }
  }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no load may land after the workgroup's LDS is released

  // --- epilogue: combine the two half-row sums, normalise, store.  A lane
  // holds 4-element pieces of its query row spread over the row, so direct
  // stores would touch 32 rows per instruction with 16 bytes each.  Every
  // wavefront instead writes its 32 x DV output block into LDS (rows of
  // 16-byte chunks, swizzled like a K tile) and stores it back as whole
  // rows, 16 bytes per lane.  Every wavefront has passed the last barrier,
  // after its final LDS read of K and V and its last load's wait, so the
  // tile slots are free; each wavefront uses only its own 32 rows.
  const float l_tot = pair_sum(l_run);
  const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  {
    constexpr int OCPR = DVP / 8;                      // 16-byte chunks per staged row
    constexpr int OBLK = 32 * DVP;                     // elements of one wavefront's block
    static_assert((NSLOT * TILE_K) % OBLK == 0 && NSLOT * (TILE_K + TILE_V) >= 8 * OBLK,
                  "output staging blocks fit the tile slots");
    T* ot = wave * OBLK < NSLOT * TILE_K ? k_lds + wave * OBLK
                                         : v_lds + (wave * OBLK - NSLOT * TILE_K);
#pragma unroll
    for (int db = 0; db < DBLK; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        T vals[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) vals[e] = (T)(acc_o[db][g * 4 + e] * inv_l);
        const int ch = (db * 4 + g) ^ Swz<DVP>::k_key(col);  // chunk of d = db * 32 + g * 8
        *reinterpret_cast<uint2*>(ot + col * DVP + ch * 8 + half * 4) =
            *reinterpret_cast<uint2*>(vals);
      }
    }
    constexpr int RPI = 64 / OCPR;  // rows per store instruction
    const int rr = lane / OCPR, cc = lane % OCPR;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = i * RPI + rr;  // row of the wavefront's block
      const u32x4 val =
          *reinterpret_cast<const u32x4*>(ot + r * DVP + ((cc ^ Swz<DVP>::k_key(r)) << 3));
      const int row = q0 + wave * 32 + r;
      if (row < Sq && cc < DV / 8)
        __builtin_nontemporal_store(
            val, reinterpret_cast<u32x4*>(o + ((int64_t)bb * Sq + row) * q_row +
                                          (int64_t)hq * D + dv0 + cc * 8));
    }
  }
  if (qi < Sq && half == 0 && dv0 == 0)
    lse[((int64_t)bb * H + hq) * Sq + qi] =
        l_tot > 0.0f ? m_run * scale_log2 + __builtin_amdgcn_logf(l_tot) : -INFINITY;
}

template <typename T, int D, int DV, int BN, bool SOFTCAP>
static void launch_k(const void* q, const void* k, const void* v, void* o, float* lse, int B,
                     int Sq, int Skv, int H, int Hkv, bool causal, float sl2, float cap_scale,
                     float cap_log2, hipStream_t s) {
  constexpr int BM = 256;
  const int nqb = (Sq + BM - 1) / BM;
  const int64_t total = (int64_t)nqb * H * B * (D / DV);
  dim3 grid((unsigned)total), block(512);
  if (causal)
    mha_fwd_kernel<T, D, DV, true, BN, SOFTCAP><<<grid, block, 0, s>>>(
        static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
        static_cast<T*>(o), lse, B, Sq, Skv, H, Hkv, sl2, nqb, cap_scale, cap_log2);
  else
    mha_fwd_kernel<T, D, DV, false, BN, SOFTCAP><<<grid, block, 0, s>>>(
        static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
        static_cast<T*>(o), lse, B, Sq, Skv, H, Hkv, sl2, nqb, cap_scale, cap_log2);
}

template <typename T, int D>
static int launch_w(const void* q, const void* k, const void* v, void* o, float* lse, int B,
                    int Sq, int Skv, int H, int Hkv, bool causal, float scale, float softcap,
                    hipStream_t s) {
  constexpr float kLog2e = 1.4426950408889634f;
  // D = 96, 128: 128-key tiles, two slots; D = 64: 64-key tiles, three
  // slots; D = 192, 256: two workgroups per query block, each with half the
  // value columns, 64-key tiles
  constexpr int DV = D >= 192 ? D / 2 : D;
  constexpr int BN = D == 128 || D == 96 ? 128 : 64;
  if (softcap > 0.0f)
    launch_k<T, D, DV, BN, true>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, 1.0f,
                                 scale / softcap, softcap * kLog2e, s);
  else
    launch_k<T, D, DV, BN, false>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal,
                                  scale * kLog2e, 0.0f, 0.0f, s);
  return launch_status();
}

template <typename T>
static int dispatch_d(int D, const void* q, const void* k, const void* v, void* o, float* lse,
                      int B, int Sq, int Skv, int H, int Hkv, bool causal, float scale,
                      float softcap, hipStream_t s) {
  if (D == 128)
    return launch_w<T, 128>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, softcap, s);
  if (D == 64)
    return launch_w<T, 64>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, softcap, s);
  if (D == 256)
    return launch_w<T, 256>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, softcap, s);
  if (D == 96)
    return launch_w<T, 96>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, softcap, s);
  if (D == 192)
    return launch_w<T, 192>(q, k, v, o, lse, B, Sq, Skv, H, Hkv, causal, scale, softcap, s);
  return TILEOPS_ESHAPE;
}

}  // namespace mha
}  // namespace tileops

using namespace tileops;

extern "C" int tileops_mha_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                               int64_t B, int64_t Sq, int64_t Skv, int64_t H, int64_t Hkv,
                               int64_t D, int causal, float scale, float softcap, int dtype,
                               void* stream) {
  if (B < 0 || Sq < 0 || Skv < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0) return TILEOPS_ESHAPE;
  if (D != 64 && D != 96 && D != 128 && D != 192 && D != 256) return TILEOPS_ESHAPE;
  if (B > INT32_MAX || Sq > INT32_MAX || Skv > INT32_MAX || H > 65535) return TILEOPS_ESHAPE;
  if (causal && Sq > Skv) return TILEOPS_ESHAPE;
  if (dtype != TILEOPS_F16 && dtype != TILEOPS_BF16) return TILEOPS_EINVAL;
  if (!(softcap >= 0.0f) || !(softcap < INFINITY)) return TILEOPS_EINVAL;  // NaN, < 0, inf
  if (B == 0 || Sq == 0) return 0;
  if (Skv == 0) return TILEOPS_ESHAPE;
  if (!q || !k || !v || !o || !lse) return TILEOPS_ENULL;
  if (!host_aligned16(q) || !host_aligned16(k) || !host_aligned16(v) || !host_aligned16(o))
    return TILEOPS_EINVAL;
  // grid: (Sq / 256) query blocks x H x B (x 2 for D = 192, 256), indexed in int
  if (((Sq + 255) / 256) * H * B * (D >= 192 ? 2 : 1) > (int64_t)INT32_MAX) return TILEOPS_ESHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TILEOPS_BF16)
    return mha::dispatch_d<bf16>((int)D, q, k, v, o, lse, (int)B, (int)Sq, (int)Skv, (int)H,
                                 (int)Hkv, causal != 0, scale, softcap, s);
  return mha::dispatch_d<f16>((int)D, q, k, v, o, lse, (int)B, (int)Sq, (int)Skv, (int)H,
                              (int)Hkv, causal != 0, scale, softcap, s);
}
