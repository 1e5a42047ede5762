// Read-only bandwidth floor of one launch on gfx950: the best time to read
// B bytes (32, 128, 512 MiB) in a single kernel, with no address
// indirection, metadata or merge -- the bound a paged-decode launch of the
// same size is compared against. Two ways of reading, each at several
// in-flight depths (KiB per wave) and work groups per CU:
//   dma:  HBM -> LDS (global_load_lds_dwordx4, non-temporal), a ring of
//         `depth` 1 KiB slots per wave kept full with vmcnt waits;
//   vgpr: HBM -> registers (non-temporal 16-byte loads), `depth` loads in
//         flight, XOR-folded so the loads stay live.
// Successive launches read successive windows of a 2 GiB buffer, so the
// 256 MB MALL cannot serve repeats; 60 launches back to back are timed with
// HIP events. Every address stays inside the buffer: each wave reads a
// contiguous run of whole 1 KiB pieces of its share.
//
// Build and run (one MI355X):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature \
//     -Xclang -packed-fp32-ops read_floor.hip -o read_floor && ./read_floor
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>

template <int N>
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14)); }

template <int DEPTH>
__global__ __launch_bounds__(256) void k_dma(const char* __restrict__ base, int64_t chunk, int* out) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + wave;
  const char* src = base + gw * chunk + lane * 16;
  const uint32_t ring = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)lds) + wave * DEPTH * 1024;
  const int n = (int)(chunk >> 10);
  int i = 0;
  for (; i < DEPTH && i < n; ++i)
    asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(src + (int64_t)i * 1024), "{m0}"(ring + (i % DEPTH) * 1024) : "memory");
  for (; i < n; ++i) {
    wait_vm<DEPTH - 1>();
    asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(src + (int64_t)i * 1024), "{m0}"(ring + (i % DEPTH) * 1024) : "memory");
  }
  wait_vm<0>();
  if (lane == 0 && out) out[gw] = lds[wave * DEPTH * 1024];
}

template <int DEPTH>
__global__ __launch_bounds__(256) void k_vgpr(const char* __restrict__ base, int64_t chunk, int* out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + wave;
  const char* src = base + gw * chunk + lane * 16;
  const int n = (int)(chunk >> 10);
  uint32_t acc = 0;
  for (int i = 0; i + DEPTH <= n; i += DEPTH) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    u32x4 r[DEPTH];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j)
      r[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (int64_t)(i + j) * 1024));
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) acc ^= r[j].x ^ r[j].y ^ r[j].z ^ r[j].w;
  }
  if (out) out[gw * 64 + lane] = acc;
}

__global__ void k_empty(int* out) { if (out && threadIdx.x == 1024) out[0] = 1; }

int main() {
  const int64_t kBuf = int64_t(2) << 30;
  char* buf; int* out;
  if (hipMalloc(&buf, kBuf) != hipSuccess) return 1;
  if (hipMalloc(&out, 256 * 8 * 4 * 64 * sizeof(int)) != hipSuccess) return 1;
  hipMemset(buf, 1, kBuf);
  int cus = 0; hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  const int reps = 60;
  // empty launches
  for (int r = 0; r < 10; ++r) hipLaunchKernelGGL(k_empty, dim3(cus), dim3(256), 0, 0, out);
  hipEventRecord(e0);
  for (int r = 0; r < reps; ++r) hipLaunchKernelGGL(k_empty, dim3(cus), dim3(256), 0, 0, out);
  hipEventRecord(e1); hipEventSynchronize(e1);
  float ms; hipEventElapsedTime(&ms, e0, e1);
  printf("empty kernel back to back: %.2f us\n", ms * 1000 / reps);
  const int64_t sizes[] = {int64_t(32) << 20, int64_t(128) << 20, int64_t(512) << 20};
  for (int64_t B : sizes) {
    for (int mode = 0; mode < 2; ++mode) {
      for (int depth : {4, 8, 16, 32}) {
        for (int gpc : {1, 2, 4}) {
          if (mode == 0 && (4 * depth * 1024 > 64 * 1024 || 4 * depth * 1024 * gpc > 160 * 1024)) continue;
          const int groups = cus * gpc;
          int64_t chunk = B / (groups * 4);
          chunk = chunk / (1024 * depth) * (1024 * depth);
          if (chunk == 0) continue;
          const int64_t bytes = chunk * groups * 4;
          const int64_t span = kBuf - bytes;
          auto launch = [&](int r) {
            const char* p = buf + (int64_t(r) * bytes) % span / 4096 * 4096;
            const size_t lds = 4 * depth * 1024;
            if (mode == 0) {
              switch (depth) {
                case 4: hipLaunchKernelGGL(k_dma<4>, dim3(groups), dim3(256), lds, 0, p, chunk, out); break;
                case 8: hipLaunchKernelGGL(k_dma<8>, dim3(groups), dim3(256), lds, 0, p, chunk, out); break;
                case 16: hipLaunchKernelGGL(k_dma<16>, dim3(groups), dim3(256), lds, 0, p, chunk, out); break;
                default: hipLaunchKernelGGL(k_dma<32>, dim3(groups), dim3(256), lds, 0, p, chunk, out); break;
              }
            } else {
              switch (depth) {
                case 4: hipLaunchKernelGGL(k_vgpr<4>, dim3(groups), dim3(256), 0, 0, p, chunk, out); break;
                case 8: hipLaunchKernelGGL(k_vgpr<8>, dim3(groups), dim3(256), 0, 0, p, chunk, out); break;
                case 16: hipLaunchKernelGGL(k_vgpr<16>, dim3(groups), dim3(256), 0, 0, p, chunk, out); break;
                default: hipLaunchKernelGGL(k_vgpr<32>, dim3(groups), dim3(256), 0, 0, p, chunk, out); break;
              }
            }
          };
          for (int r = 0; r < 5; ++r) launch(r);
          hipEventRecord(e0);
          for (int r = 0; r < reps; ++r) launch(r + 5);
          hipEventRecord(e1);
          if (hipEventSynchronize(e1) != hipSuccess || hipGetLastError() != hipSuccess) { printf("launch or sync failed\n"); return 2; }
          hipEventElapsedTime(&ms, e0, e1);
          const double us = ms * 1000 / reps;
          printf("%s B=%4lld MiB depth %2d KiB/wave groups/CU %d: %8.2f us  %7.1f GB/s\n", mode ? "vgpr" : "dma ",
                 (long long)(bytes >> 20), depth, gpc, us, bytes / us / 1e3);
          fflush(stdout);
        }
      }
    }
  }
  return 0;
}
