// Measurement kernels behind `bench.py --stream-probe` (not part of the
// decode path's C ABI): a plain streaming read, the ceiling a kernel that only
// reads a decode step's bytes reaches on this GPU, with and without per-wave
// clock stamps. Built with the phase-stamped decode kernels into
// libkvq_probe.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

// Built three times into the library: as is; with KVQ_PROBE_PRELOAD defined
// and -amdgpu-kernarg-preload-count, which has the hardware load the kernels'
// scalar arguments into SGPRs at wave launch (namespace kvq_probe_pl, entry
// points suffixed _preload); and with KVQ_PROBE_NT defined as well, where
// stream_read's loads carry the nontemporal hint (namespace kvq_probe_pl_nt,
// suffix _preload_nt). Preload lets a wave issue its loads without first
// waiting for the argument block to arrive from memory (it helps reads of a
// few MB and more), but costs the smallest launches a little. The hint lets
// the hardware stream lines that one instruction reads whole; it helps large
// reads most. The ceiling takes the best of the three.
#if defined(KVQ_PROBE_PRELOAD) && defined(KVQ_PROBE_NT)
#define KVQ_PROBE_NS kvq_probe_pl_nt
#define KVQ_PROBE_FN(name) name##_preload_nt
#elif defined(KVQ_PROBE_PRELOAD)
#define KVQ_PROBE_NS kvq_probe_pl
#define KVQ_PROBE_FN(name) name##_preload
#else
#define KVQ_PROBE_NS kvq_probe
#define KVQ_PROBE_FN(name) name
#endif

namespace KVQ_PROBE_NS {

// Thread t reads the 16-byte pieces t, t + T, ..., t + (PER - 1) T of the
// buffer (T = threads in the grid; pieces past n16 are skipped), all issued
// before the first is used, and folds them with XOR. Nothing is written
// unless the fold equals a value no test buffer produces, so the kernel's
// traffic is the buffer's bytes.
typedef uint32_t probe_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 read16(const uint4* p) {
#if defined(KVQ_PROBE_NT)
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const probe_u32x4*)p));
#else
  return *p;
#endif
}

template <int PER>
__global__ __launch_bounds__(1024) void stream_read(const uint4* __restrict__ p, uint64_t n16, uint32_t* sink) {
  const uint64_t t = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
  const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
  uint4 v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint64_t j = t + i * T;
    v[i] = j < n16 ? read16(p + j) : make_uint4(0u, 0u, 0u, 0u);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

// The same read with per-wave stamps of the 100 MHz s_memrealtime clock:
// st[(block * 16 + wave) * 4 + k], k = 0 entry, 1 loads issued, 2 first piece
// arrived, 3 every piece arrived. blockDim.x <= 1024.
template <int PER>
__global__ __launch_bounds__(1024) void stream_read_stamped(const uint4* __restrict__ p, uint64_t n16,
                                                            uint32_t* sink, uint64_t* st) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const uint64_t t = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
  const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
  uint4 v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint64_t j = t + i * T;
    v[i] = j < n16 ? p[j] : make_uint4(0u, 0u, 0u, 0u);
  }
  asm volatile("" ::: "memory");
  const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
  asm volatile("" ::"v"(v[0].x));
  const uint64_t t2 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  asm volatile("" ::"v"(acc));
  const uint64_t t3 = __builtin_amdgcn_s_memrealtime();
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
  if ((threadIdx.x & 63) == 0) {
    uint64_t* s = st + ((uint64_t)blockIdx.x * 16 + (threadIdx.x >> 6)) * 4;
    s[0] = t0;
    s[1] = t1;
    s[2] = t2;
    s[3] = t3;
  }
}

// The read of stream_read<10> with N dependent v_add instructions (8 bytes
// each) before its loads (AFTER = false) or after them: what one instruction
// on a wave's path to its first load costs when two waves share a SIMD.
template <int N, bool AFTER>
__global__ __launch_bounds__(512) void stream_read_padded(const uint4* __restrict__ p, uint64_t n16, uint32_t* sink) {
  constexpr int PER = 10;
  const uint64_t t = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
  const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
  uint32_t x = threadIdx.x;
  if (!AFTER) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("v_add_u32 %0, 0x12345, %0" : "+v"(x));
  }
  uint4 v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint64_t j = t + i * T;
    v[i] = j < n16 ? p[j] : make_uint4(0u, 0u, 0u, 0u);
  }
  if (AFTER) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("v_add_u32 %0, 0x12345, %0" : "+v"(x));
  }
  uint32_t acc = x;
#pragma unroll
  for (int i = 0; i < PER; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

typedef void (*read_fn)(const uint4*, uint64_t, uint32_t*);
typedef void (*read_st_fn)(const uint4*, uint64_t, uint32_t*, uint64_t*);

#define KVQ_PROBE_PERS(X) X(1) X(2) X(3) X(4) X(5) X(6) X(8) X(10) X(12) X(16) X(19) X(20) X(24) X(32) X(37) X(40)

static read_fn pick(int per) {
#define KVQ_PROBE_CASE(n) \
  if (per == n) return stream_read<n>;
  KVQ_PROBE_PERS(KVQ_PROBE_CASE)
#undef KVQ_PROBE_CASE
  return nullptr;
}

static read_st_fn pick_stamped(int per) {
#define KVQ_PROBE_CASE(n) \
  if (per == n) return stream_read_stamped<n>;
  KVQ_PROBE_PERS(KVQ_PROBE_CASE)
#undef KVQ_PROBE_CASE
  return nullptr;
}

// Pieces per thread for a grid: the smallest instantiated count that covers
// the buffer, or 0 if none does.
static int pieces_per_thread(uint64_t n16, int grid, int block) {
  const uint64_t T = (uint64_t)grid * block;
  const uint64_t need = (n16 + T - 1) / T;
  static const int pers[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 19, 20, 24, 32, 37, 40};
  for (int p : pers)
    if ((uint64_t)p >= need) return p;
  return 0;
}

}  // namespace KVQ_PROBE_NS

// One streaming read of `bytes` (a multiple of 16) at buf, grid x block
// threads; sink holds >= grid uint32. stamps (may be null): per-wave clock
// stamps, [grid * 16 * 4] uint64, block <= 1024. Returns the pieces per
// thread used, 0 if no instantiation covers the buffer (nothing launched),
// -1 on bad arguments or a launch error.
extern "C" int KVQ_PROBE_FN(kvq_probe_stream_read)(const void* buf, int64_t bytes, int grid, int block, void* sink,
                                     void* stamps, void* stream) {
  if (buf == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 != 0 || grid <= 0 || block <= 0 ||
      block > 1024 || block % 64 != 0)
    return -1;
  const uint64_t n16 = (uint64_t)bytes / 16;
  const int per = KVQ_PROBE_NS::pieces_per_thread(n16, grid, block);
  if (per == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  if (stamps != nullptr)
    hipLaunchKernelGGL(KVQ_PROBE_NS::pick_stamped(per), dim3(grid), dim3(block), 0, st, (const uint4*)buf, n16,
                       (uint32_t*)sink, (uint64_t*)stamps);
  else
    hipLaunchKernelGGL(KVQ_PROBE_NS::pick(per), dim3(grid), dim3(block), 0, st, (const uint4*)buf, n16,
                       (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? per : -1;
}

// stream_read_padded over `bytes` (a multiple of 16, at most 256 * 512 * 10 * 16
// bytes) with grid 256 x 512: pad in {0, 256, 512, 1024, 2048}, after != 0
// places the instructions after the loads. Returns 0, or -1 on bad arguments
// or a launch error.
extern "C" int KVQ_PROBE_FN(kvq_probe_stream_read_padded)(const void* buf, int64_t bytes, int pad, int after, void* sink,
                                            void* stream) {
  using namespace KVQ_PROBE_NS;
  if (buf == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 != 0 || bytes > 256ll * 512 * 10 * 16) return -1;
  read_fn f = nullptr;
#define KVQ_PAD_CASE(n)                                                              \
  if (pad == n) f = after ? stream_read_padded<n, true> : stream_read_padded<n, false>;
  KVQ_PAD_CASE(0) KVQ_PAD_CASE(256) KVQ_PAD_CASE(512) KVQ_PAD_CASE(1024) KVQ_PAD_CASE(2048)
#undef KVQ_PAD_CASE
  if (f == nullptr) return -1;
  hipLaunchKernelGGL(f, dim3(256), dim3(512), 0, (hipStream_t)stream, (const uint4*)buf, (uint64_t)bytes / 16,
                     (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
