// HBM stream ceilings of one MI355X for the traffic mixes of the memory-bound
// operators: R reads + W writes per 16-byte pack, one pack per thread and a
// grid over the whole buffer (the launch shape of unary_vec_kernel,
// add/lerp bcast_vec_kernel, isfp_vec_kernel), non-temporal loads and stores,
// 1 GiB per stream so that the 256 MB Infinity Cache cannot serve it.
//
//   stream_ceiling [--iters N] [--mib M]
//
// M (default 1024) is the size of each stream in MiB; below 1 GiB the
// launches cycle through enough copies of the buffers that the working set
// stays at 4 GiB or more, so that the Infinity Cache cannot serve a repeat.
//
// prints one line per mix: bytes moved per launch, mean kernel time over N
// launches (HIP events), GB/s and the fraction of the 8 TB/s peak.  Two
// block orders are measured: consecutive workgroups on consecutive packs
// (the hardware deals workgroups round-robin to the 8 XCDs), and an
// XCD-contiguous order in which the workgroups one XCD receives cover one
// contiguous eighth of the buffer.  A device-to-device hipMemcpy closes.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int R, int W, bool XCD>
__global__ __launch_bounds__(256) void stream_kernel(const u32x4* __restrict__ s0,
                                                     const u32x4* __restrict__ s1,
                                                     u32x4* __restrict__ d0,
                                                     u32x4* __restrict__ d1, long long npack) {
  long long blk = blockIdx.x;
  if (XCD) {  // the blocks of XCD x = blk % 8 take the x-th eighth, in order
    const long long per = gridDim.x / 8;
    blk = (blk % 8) * per + blk / 8;
  }
  const long long i = blk * 256 + threadIdx.x;
  if (i >= npack) return;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (R >= 1) v = __builtin_nontemporal_load(s0 + i);
  if (R >= 2) v ^= __builtin_nontemporal_load(s1 + i);
  if (R == 0) v = u32x4{(unsigned)i, 1u, 2u, 3u};
  if (W >= 1) __builtin_nontemporal_store(v, d0 + i);
  if (W >= 2) __builtin_nontemporal_store(v + 1u, d1 + i);
  if (W == 0 && v.x == 0x9e3779b9u && v.y == 0u) d0[0] = v;  // keep the loads live
}

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                 \
      return 1;                                                               \
    }                                                                         \
  } while (0)

int main(int argc, char** argv) {
  int iters = 20;
  long long mib = 1024;
  for (int a = 1; a + 1 < argc; ++a) {
    if (!strcmp(argv[a], "--iters")) iters = atoi(argv[a + 1]);
    if (!strcmp(argv[a], "--mib")) mib = atoll(argv[a + 1]);
  }
  if (iters < 1 || mib < 8 || mib > 8192 || (mib & 7)) {
    fprintf(stderr, "--iters >= 1, --mib a multiple of 8 in [8, 8192]\n");
    return 1;
  }
  const long long bytes = mib << 20, npack = bytes / 16;
  const unsigned grid = (unsigned)(npack / 256);  // a multiple of 8
  const int nsets = mib >= 1024 ? 1 : (int)((1024 + mib - 1) / mib);
  constexpr int kMaxSets = 128;
  u32x4 *s0[kMaxSets], *s1[kMaxSets], *d0[kMaxSets], *d1[kMaxSets];
  for (int k = 0; k < nsets; ++k) {
    CHECK(hipMalloc(&s0[k], bytes));
    CHECK(hipMalloc(&s1[k], bytes));
    CHECK(hipMalloc(&d0[k], bytes));
    CHECK(hipMalloc(&d1[k], bytes));
    CHECK(hipMemset(s0[k], 1, bytes));
    CHECK(hipMemset(s1[k], 2, bytes));
  }
  int cur = 0;  // buffer set of the next launch
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  printf("# %lld MiB per stream (%d buffer sets cycled), %d timed launches after 3 warm-up; "
         "peak 8000 GB/s\n", mib, nsets, iters);
  printf("%-28s %12s %10s %10s %7s\n", "mix", "bytes", "us", "GB/s", "peak");
  auto run = [&](const char* name, double moved, auto launch) -> int {
    for (int i = 0; i < 3; ++i) launch();
    CHECK(hipEventRecord(e0));
    for (int i = 0; i < iters; ++i) launch();
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    CHECK(hipGetLastError());
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double us = ms * 1e3 / iters, gbs = moved / (us * 1e-6) / 1e9;
    printf("%-28s %12.0f %10.2f %10.1f %6.1f%%\n", name, moved, us, gbs, gbs / 80.0);
    return 0;
  };
#define MIX(R, W)                                                                              \
  if (run(#R "R/" #W "W", (double)(R + W) * bytes,                                            \
          [&] {                                                                               \
            stream_kernel<R, W, false><<<grid, 256>>>(s0[cur], s1[cur], d0[cur], d1[cur], npack); \
            cur = (cur + 1) % nsets;                                                          \
          }) ||                                                                               \
      run(#R "R/" #W "W xcd-contiguous", (double)(R + W) * bytes,                             \
          [&] {                                                                               \
            stream_kernel<R, W, true><<<grid, 256>>>(s0[cur], s1[cur], d0[cur], d1[cur], npack); \
            cur = (cur + 1) % nsets;                                                          \
          }))                                                                                 \
    return 1;
  MIX(1, 0)
  MIX(0, 1)
  MIX(1, 1)
  MIX(2, 1)
  MIX(1, 2)
  MIX(2, 2)
#undef MIX
  if (run("hipMemcpy device to device", 2.0 * bytes, [&] {
        (void)hipMemcpyAsync(d0[cur], s0[cur], bytes, hipMemcpyDeviceToDevice, 0);
        cur = (cur + 1) % nsets;
      }))
    return 1;
  for (int k = 0; k < nsets; ++k) {
    CHECK(hipFree(s0[k]));
    CHECK(hipFree(s1[k]));
    CHECK(hipFree(d0[k]));
    CHECK(hipFree(d1[k]));
  }
  return 0;
}
