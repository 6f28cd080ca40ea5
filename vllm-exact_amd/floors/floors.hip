// Measured ceilings of the memory and matrix paths the exact GEMM and the paged decode
// attention run on (MI355X, gfx950). These kernels compute nothing useful: each exercises one
// path at a chosen depth of requests in flight, so a benchmark can report the achievable rate
// beside the published peak.
//
//   stream   contiguous read of a large buffer, one chunk per workgroup (the weight stream)
//   pages    read of 8 KiB pages in a given (permuted) order (the paged KV stream): a
//            workgroup reads a page at a time, or (wave_pages) each wave reads its own pages
//            in the decode attention kernel's lane pattern
// The stream and page probes take the load's cache policy: nontemporal or the default.
//   l2       16-byte loads of an L2-resident buffer into VGPRs, or straight into LDS with
//            global_load_lds_dwordx4, at Q loads in flight per lane
//   lds      ds_read_b128 of LDS into VGPRs
//   mfma     v_mfma_i32_16x16x64_i8 on 8 independent accumulators per wave
//   mfma_shape  the two INT8 MFMA shapes at equal work per round (16x16x64 on 8 accumulators,
//            32x32x32 on 4), their operands the same in every instruction or drawn at random
//            with a different set in every instruction (as a GEMM's digit fragments are)
//   rowcopy  the packed digitize's grid and traffic with no arithmetic: a workgroup per row,
//            each lane copying 16 bf16 columns into 16-byte pieces of the two digit planes
//   mfma_mix MFMAs and loads (L2-resident, or L2 and HBM) at once, in the large-M exact GEMM's
//            proportion, with the shader clock each workgroup ran at
//
// Every kernel reads inside the buffer it is given (the host checks the sizes; the L2 probe
// masks its offsets with a power of two that the buffer covers) and writes one int per thread
// to `sink`, so no load can be optimised away. Thread 0 of each workgroup b also writes the
// shader cycles (s_memtime) and the 100 MHz ticks (s_memrealtime) of its run, at cycles[b] and
// cycles[blocks + b]: their ratio is the shader clock the probe ran at.

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;

namespace {

// Start stamps of thread 0's run: shader cycles (s_memtime) and 100 MHz ticks (s_memrealtime).
struct Stamp {
  int64_t cycles, ticks;
};
__device__ inline Stamp stamp() { return {(int64_t)clock64(), (int64_t)__builtin_amdgcn_s_memrealtime()}; }

__device__ inline void finish(int* sink, int64_t* cycles, v4i acc, Stamp t0) {
  // An impossible value keeps the loads live without a store per thread in the common case.
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5A5A5A5A) sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = 1;
  if (threadIdx.x == 0) {
    const Stamp t1 = stamp();
    cycles[blockIdx.x] = t1.cycles - t0.cycles;
    cycles[gridDim.x + blockIdx.x] = t1.ticks - t0.ticks;
  }
}

// Workgroup b reads bytes [b * per_wg, (b + 1) * per_wg): Q 16-byte non-temporal loads per lane
// in flight, then the remainder one load per lane at a time. per_wg is a multiple of
// 16 * blockDim.x (host-checked).
template <bool NT>
__device__ inline v4i load16(const v4i* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  return *p;
}

template <int Q, bool NT>
__global__ __launch_bounds__(512) void stream_kernel(const v4i* __restrict__ buf, int64_t per_wg16, int* sink,
                                                     int64_t* cycles) {
  const Stamp t0 = stamp();
  const v4i* p = buf + (int64_t)blockIdx.x * per_wg16;
  const int64_t T = blockDim.x;
  v4i acc = {0, 0, 0, 0};
  int64_t i = threadIdx.x;
  for (; i + (Q - 1) * T < per_wg16; i += T * Q) {
    v4i a[Q];
#pragma unroll
    for (int u = 0; u < Q; ++u) a[u] = load16<NT>(p + i + u * T);
#pragma unroll
    for (int u = 0; u < Q; ++u) acc ^= a[u];
  }
  for (; i < per_wg16; i += T) acc ^= load16<NT>(p + i);
  finish(sink, cycles, acc, t0);
}

// Workgroup b reads pages pages[b * ppw .. (b + 1) * ppw) of 8 KiB each; the 512 lanes of a
// workgroup cover one page per round (one 16-byte load each), Q pages in flight.
template <int Q, bool NT>
__global__ __launch_bounds__(512) void pages_kernel(const v4i* __restrict__ buf, const int32_t* __restrict__ pages,
                                                    int ppw, int* sink, int64_t* cycles) {
  const Stamp t0 = stamp();
  const int32_t* mine = pages + (int64_t)blockIdx.x * ppw;
  v4i acc = {0, 0, 0, 0};
  for (int i = 0; i < ppw; i += Q) {
    v4i a[Q];
#pragma unroll
    for (int u = 0; u < Q; ++u) a[u] = load16<NT>(buf + (int64_t)mine[i + u] * 512 + threadIdx.x);
#pragma unroll
    for (int u = 0; u < Q; ++u) acc ^= a[u];
  }
  finish(sink, cycles, acc, t0);
}

// Wave w of workgroup b reads pages pages[(4b + w) * ppw ..) of 8 KiB, one at a time, as the
// decode attention reads a 16-key page of one KV head (16 rows of 512 bytes: K then V, D = 128):
// four K loads with lane (r, c) on row c, bytes 64i + 16r, then four V loads with lane (r, c)
// on row 4r + j, bytes 256 + 16c. 256 threads; `pad` bytes of dynamic LDS per workgroup cap
// the workgroups per CU the way the attention kernel's registers do.
template <bool NT>
__global__ __launch_bounds__(256) void wave_pages_kernel(const int8_t* __restrict__ buf,
                                                         const int32_t* __restrict__ pages, int ppw, int pad,
                                                         int* sink, int64_t* cycles) {
  extern __shared__ int lds_pad[];
  const Stamp t0 = stamp();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane >> 4, c = lane & 15;
  const int32_t* mine = pages + ((int64_t)blockIdx.x * 4 + wave) * ppw;
  v4i acc = {0, 0, 0, 0};
  for (int i = 0; i < ppw; ++i) {
    const int8_t* pg = buf + (int64_t)mine[i] * 8192;
    v4i a[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = load16<NT>(reinterpret_cast<const v4i*>(pg + c * 512 + 64 * k + 16 * r));
#pragma unroll
    for (int j = 0; j < 4; ++j) a[4 + j] = load16<NT>(reinterpret_cast<const v4i*>(pg + (4 * r + j) * 512 + 256 + 16 * c));
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= a[k];
  }
  if (pad) lds_pad[threadIdx.x] = acc.x;
  finish(sink, cycles, acc, t0);
}

// L2-resident loads: each wave walks a 16 KiB window of the buffer per round (offsets masked
// into [0, n16)), Q 1-KiB wave loads in flight. LDS = 1: global_load_lds_dwordx4 into a ring of
// Q 1-KiB slots per wave (never read: only the arrival is waited for).
template <int Q, bool LDS>
__global__ __launch_bounds__(1024) void l2_kernel(const v4i* __restrict__ buf, int64_t mask16, int rounds, int* sink,
                                                  int64_t* cycles) {
  __shared__ __attribute__((aligned(1024))) int8_t ring[LDS ? 16 * Q * 1024 : 16];
  const Stamp t0 = stamp();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t base = ((int64_t)blockIdx.x * 16 + wave) * 1024;  // in 16-byte units
  v4i acc = {0, 0, 0, 0};
  for (int r = 0; r < rounds; ++r) {
    if constexpr (LDS) {
#pragma unroll
      for (int u = 0; u < Q; ++u) {
        const v4i* src = buf + ((base + (int64_t)(r * Q + u) * 64 + lane) & mask16);
        __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(ring + (wave * Q + u) * 1024), 16, 0, 0);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring is refilled next round
    } else {
      v4i a[Q];
#pragma unroll
      for (int u = 0; u < Q; ++u) a[u] = buf[(base + (int64_t)(r * Q + u) * 64 + lane) & mask16];
#pragma unroll
      for (int u = 0; u < Q; ++u) acc ^= a[u];
    }
  }
  if constexpr (LDS) {
    __syncthreads();
    acc = *reinterpret_cast<const v4i*>(ring + (threadIdx.x % (16 * Q * 64)) * 16);
  }
  finish(sink, cycles, acc, t0);
}

// ds_read_b128: each lane reads 16 bytes per instruction from a 64 KiB LDS tile, 8 reads in
// flight.
__global__ __launch_bounds__(1024) void lds_kernel(int rounds, int* sink, int64_t* cycles) {
  __shared__ __attribute__((aligned(1024))) int8_t tile[64 * 1024];
  for (int i = threadIdx.x; i < 4096; i += blockDim.x) reinterpret_cast<v4i*>(tile)[i] = v4i{i, i + 1, i + 2, i + 3};
  __syncthreads();
  const Stamp t0 = stamp();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v4i acc = {0, 0, 0, 0};
  for (int r = 0; r < rounds; ++r) {
    v4i a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      a[u] = *reinterpret_cast<const v4i*>(tile + (((wave * 8 + u + r) & 63) * 1024) + lane * 16);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= a[u];
  }
  finish(sink, cycles, acc, t0);
}

// v_mfma_i32_16x16x64_i8 on 8 independent accumulators per wave.
__global__ __launch_bounds__(1024) void mfma_kernel(int rounds, int* sink, int64_t* cycles) {
  const Stamp t0 = stamp();
  const v4i a = {(int)threadIdx.x, 3, 5, 7}, b = {11, 13, (int)blockIdx.x, 17};
  v4i c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = v4i{i, 0, 0, 0};
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[i], 0, 0, 0);
  }
  v4i acc = c[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) acc ^= c[i];
  finish(sink, cycles, acc, t0);
}

// 8 waves per workgroup. SHAPE 16: 8 v_mfma_i32_16x16x64_i8 a round on 8 accumulators;
// SHAPE 32: 4 v_mfma_i32_32x32x32_i8 a round on 4 accumulators (the same integer work), rounds
// taken in pairs. RANDOM: eight operand sets drawn from a per-lane linear congruential sequence
// before the loop, instruction i of a round (or of a round pair, for SHAPE 32) using set i, so
// consecutive instructions see different random bits and no operand is rewritten in the loop;
// else every instruction takes the same operands.
template <int SHAPE, bool RANDOM>
__global__ __launch_bounds__(512) void mfma_shape_kernel(int rounds, int* sink, int64_t* cycles) {
  const Stamp t0 = stamp();
  v4i as[8], bs[8];
  uint32_t x = threadIdx.x * 2654435761u + blockIdx.x * 40503u + 1u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (RANDOM || i == 0) {
      uint32_t t[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        x = x * 1664525u + 1013904223u;
        t[j] = x;
      }
      as[i] = v4i{(int)t[0], (int)t[1], (int)t[2], (int)t[3]};
      bs[i] = v4i{(int)t[4], (int)t[5], (int)t[6], (int)t[7]};
    } else {
      as[i] = as[0];
      bs[i] = bs[0];
    }
  }
  v4i acc = {0, 0, 0, 0};
  if constexpr (SHAPE == 16) {
    v4i c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = v4i{i, 0, 0, 0};
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[i], bs[i], c[i], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc ^= c[i];
  } else {
    v16i c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = v16i{};
      c[i][0] = i;
    }
    for (int r = 0; r < rounds; r += 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(as[i], bs[i], c[i], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(as[i + 4], bs[i + 4], c[i], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 16; j += 4) acc ^= v4i{c[i][j], c[i][j + 1], c[i][j + 2], c[i][j + 3]};
  }
  finish(sink, cycles, acc, t0);
}

// One workgroup per row r (rows spread so that the 16 rows of a packed tile run on one XCD, as
// the digitize kernel spreads them), K/16 lanes; lane c reads columns [16c, 16c + 16) of its
// row (32 bytes) and writes 16 bytes into each of the two 1 KiB digit planes of the packed
// fragment-major layout, where the digitize kernel writes that chunk's digits.
__global__ __launch_bounds__(1024) void rowcopy_kernel(const uint16_t* __restrict__ x, int64_t K,
                                                       int8_t* __restrict__ h, int64_t KT) {
  const int64_t lin = blockIdx.x, total = gridDim.x;
  const int64_t xcd = lin % 8, j = lin / 8, base = total / 8, rem = total % 8;
  const int64_t row = xcd * base + (xcd < rem ? xcd : rem) + j;
  const int64_t c = threadIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(x + row * K + c * 16);
  const uint4 a = src[0], b = src[1];
  int8_t* dst = h + ((row >> 4) * KT + (c >> 2)) * 2048 + ((int)(c & 3) * 16 + (int)(row & 15)) * 16;
  *reinterpret_cast<uint4*>(dst) = a;
  *reinterpret_cast<uint4*>(dst + 1024) = b;
}

// MFMAs and loads together, the mix of the large-M exact GEMM: 8 waves per workgroup, one
// workgroup per CU. Each round a wave issues eight 16-byte loads per lane (8 KiB) when
// loads > 0: all from the L2-resident buffer `l2` (offsets masked into it), or with loads == 2
// two of the eight from the workgroup's own chunk of the large buffer `hbm` (read round after
// round, offsets masked into the chunk), then `mfmas` MFMAs over 8 independent chains, then
// consumes the loads. With `vary`, the MFMA operands are redrawn every round (a 32-bit linear
// congruential step per register: random bits, as the GEMM's digits are), else they stay
// constant. Thread 0 records, for its workgroup, the shader cycles (s_memtime) and the
// 100 MHz ticks (s_memrealtime) of the run: their ratio is the shader clock under that load.
__global__ __launch_bounds__(512) void mfma_mix_kernel(const v4i* __restrict__ l2, int64_t mask16,
                                                       const v4i* __restrict__ hbm, int64_t chunk16, int loads,
                                                       int mfmas, int vary, int rounds, int* sink, int64_t* clk) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t base = ((int64_t)blockIdx.x * 8 + wave) * 512;  // 16-byte units
  const v4i* mine = hbm + (int64_t)blockIdx.x * (chunk16 + 1);
  v4i a = {(int)threadIdx.x, 3, 5, 7}, b = {11, 13, (int)blockIdx.x, 17};
  v4i c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = v4i{i, 0, 0, 0};
  v4i acc = {0, 0, 0, 0};
  for (int r = 0; r < rounds; ++r) {
    if (vary) {
      a = a * 1664525 + 1013904223;
      b = b * 22695477 + 1;
    }
    v4i d[8];
    if (loads) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (loads == 2 && u < 2)
          d[u] = mine[((int64_t)(r * 2 + u) * 512 + wave * 64 + lane) & chunk16];
        else
          d[u] = l2[(base + (int64_t)(r * 8 + u) * 64 + lane) & mask16];
      }
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) d[u] = v4i{u, r, 0, 0};
    }
    for (int m = 0; m < mfmas; m += 8) {
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[i], 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= d[u];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) acc ^= c[i];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5A5A5A5A) sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = 1;
  if (threadIdx.x == 0) {
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    clk[2 * blockIdx.x] = (int64_t)(c1 - c0);
    clk[2 * blockIdx.x + 1] = (int64_t)(r1 - r0);
  }
}

}  // namespace

extern "C" {

// Status: 0 ok, 1 bad argument, 4 launch error.
int vxf_stream(const void* buf, int64_t buf_bytes, int64_t per_wg_bytes, int blocks, int threads, int q, int nt,
               int* sink, int64_t* cycles, void* stream) {
  if (!buf || !sink || !cycles || blocks <= 0 || (threads != 256 && threads != 512)) return 1;
  if (q != 4 && q != 8) return 1;
  if (per_wg_bytes <= 0 || per_wg_bytes % (16LL * threads) != 0) return 1;
  if ((int64_t)blocks * per_wg_bytes > buf_bytes) return 1;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t n16 = per_wg_bytes / 16;
  const auto* p = (const v4i*)buf;
#define VXF_STREAM(Q_, NT_) hipLaunchKernelGGL((stream_kernel<Q_, NT_>), dim3(blocks), dim3(threads), 0, st, p, n16, sink, cycles)
  if (q == 4 && nt) VXF_STREAM(4, true);
  else if (q == 8 && nt) VXF_STREAM(8, true);
  else if (q == 4) VXF_STREAM(4, false);
  else VXF_STREAM(8, false);
#undef VXF_STREAM
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// pages: int32 [blocks * ppw] page indices, each in [0, buf_bytes / 8192) (the caller checks).
int vxf_pages(const void* buf, int64_t buf_bytes, const int32_t* pages, int blocks, int ppw, int q, int nt, int* sink,
              int64_t* cycles, void* stream) {
  if (q != 1 && q != 2 && q != 4) return 1;
  if (!buf || !pages || !sink || !cycles || blocks <= 0 || ppw <= 0 || ppw % q != 0 || buf_bytes < 8192) return 1;
  const hipStream_t st = (hipStream_t)stream;
  const auto* p = (const v4i*)buf;
#define VXF_PAGES(Q_, NT_) hipLaunchKernelGGL((pages_kernel<Q_, NT_>), dim3(blocks), dim3(512), 0, st, p, pages, ppw, sink, cycles)
  if (nt) {
    if (q == 1) VXF_PAGES(1, true);
    else if (q == 2) VXF_PAGES(2, true);
    else VXF_PAGES(4, true);
  } else {
    if (q == 1) VXF_PAGES(1, false);
    else if (q == 2) VXF_PAGES(2, false);
    else VXF_PAGES(4, false);
  }
#undef VXF_PAGES
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// wave_pages: pages int32 [blocks * 4 * ppw], each in [0, buf_bytes / 8192) (the caller
// checks); pad_bytes of dynamic LDS per workgroup, 0 or 1024 .. 65536.
int vxf_wave_pages(const void* buf, int64_t buf_bytes, const int32_t* pages, int blocks, int ppw, int nt,
                   int pad_bytes, int* sink, int64_t* cycles, void* stream) {
  if (!buf || !pages || !sink || !cycles || blocks <= 0 || ppw <= 0 || buf_bytes < 8192) return 1;
  if (pad_bytes != 0 && (pad_bytes < 1024 || pad_bytes > 65536)) return 1;
  const hipStream_t st = (hipStream_t)stream;
  const auto* p = (const int8_t*)buf;
  if (nt)
    hipLaunchKernelGGL(wave_pages_kernel<true>, dim3(blocks), dim3(256), pad_bytes, st, p, pages, ppw, pad_bytes, sink,
                       cycles);
  else
    hipLaunchKernelGGL(wave_pages_kernel<false>, dim3(blocks), dim3(256), pad_bytes, st, p, pages, ppw, pad_bytes,
                       sink, cycles);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// l2: buf_bytes a power of two >= 16 KiB; lds = 0 (VGPR loads) or 1 (direct-to-LDS).
int vxf_l2(const void* buf, int64_t buf_bytes, int lds, int q, int waves, int blocks, int rounds, int* sink,
           int64_t* cycles, void* stream) {
  if (!buf || !sink || !cycles || blocks <= 0 || rounds <= 0) return 1;
  if (buf_bytes < 16384 || (buf_bytes & (buf_bytes - 1)) != 0) return 1;
  if (waves != 4 && waves != 8 && waves != 16) return 1;
  const hipStream_t st = (hipStream_t)stream;
  const int64_t mask = buf_bytes / 16 - 1;
  const auto* p = (const v4i*)buf;
  const dim3 g(blocks), b(64 * waves);
#define VXF_L2(Q_)                                                                   \
  if (q == Q_) {                                                                     \
    if (lds) hipLaunchKernelGGL((l2_kernel<Q_, true>), g, b, 0, st, p, mask, rounds, sink, cycles); \
    else hipLaunchKernelGGL((l2_kernel<Q_, false>), g, b, 0, st, p, mask, rounds, sink, cycles);    \
    return hipGetLastError() == hipSuccess ? 0 : 4;                                  \
  }
  VXF_L2(1) VXF_L2(2) VXF_L2(4) VXF_L2(8)
#undef VXF_L2
  return 1;
}

int vxf_lds(int waves, int blocks, int rounds, int* sink, int64_t* cycles, void* stream) {
  if (!sink || !cycles || blocks <= 0 || rounds <= 0 || (waves != 4 && waves != 8 && waves != 16)) return 1;
  hipLaunchKernelGGL(lds_kernel, dim3(blocks), dim3(64 * waves), 0, (hipStream_t)stream, rounds, sink, cycles);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

int vxf_mfma(int waves, int blocks, int rounds, int* sink, int64_t* cycles, void* stream) {
  if (!sink || !cycles || blocks <= 0 || rounds <= 0 || (waves != 4 && waves != 8 && waves != 16)) return 1;
  hipLaunchKernelGGL(mfma_kernel, dim3(blocks), dim3(64 * waves), 0, (hipStream_t)stream, rounds, sink, cycles);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// mfma_shape: shape 16 or 32, random 0 or 1, rounds even and positive; 512 threads a workgroup.
int vxf_mfma_shape(int shape, int random, int blocks, int rounds, int* sink, int64_t* cycles, void* stream) {
  if (!sink || !cycles || blocks <= 0 || rounds <= 0 || rounds % 2 || (shape != 16 && shape != 32) ||
      (random != 0 && random != 1))
    return 1;
  const hipStream_t st = (hipStream_t)stream;
#define VXF_SHAPE(S, R)                                                                                     \
  if (shape == S && random == R)                                                                            \
    hipLaunchKernelGGL((mfma_shape_kernel<S, R != 0>), dim3(blocks), dim3(512), 0, st, rounds, sink, cycles);
  VXF_SHAPE(16, 0) VXF_SHAPE(16, 1) VXF_SHAPE(32, 0) VXF_SHAPE(32, 1)
#undef VXF_SHAPE
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// mfma_mix: l2_bytes a power of two >= 16 KiB; hbm_bytes >= blocks * chunk with chunk =
// hbm_bytes / blocks rounded down to a power of two >= 8 KiB (used only when loads == 2); loads 0,
// 1 or 2; mfmas a multiple of 8 up to 4096, not 0 when loads is 0; vary 0 or 1; clk holds 2 int64
// per workgroup. 512 threads per workgroup.
int vxf_mfma_mix(const void* l2, int64_t l2_bytes, const void* hbm, int64_t hbm_bytes, int loads, int mfmas, int vary,
                 int blocks, int rounds, int* sink, int64_t* clk, void* stream) {
  if (!l2 || !sink || !clk || blocks <= 0 || rounds <= 0) return 1;
  if (l2_bytes < 16384 || (l2_bytes & (l2_bytes - 1)) != 0) return 1;
  if (loads < 0 || loads > 2 || mfmas < 0 || mfmas % 8 != 0 || mfmas > 4096 || (!loads && mfmas == 0)) return 1;
  if (vary != 0 && vary != 1) return 1;
  int64_t chunk = 0;
  if (loads == 2) {
    if (!hbm || hbm_bytes / blocks < 8192) return 1;
    chunk = 8192;
    while (chunk * 2 <= hbm_bytes / blocks) chunk *= 2;
  }
  hipLaunchKernelGGL(mfma_mix_kernel, dim3(blocks), dim3(512), 0, (hipStream_t)stream, (const v4i*)l2,
                     l2_bytes / 16 - 1, (const v4i*)hbm, chunk ? chunk / 16 - 1 : 0, loads, mfmas, vary, rounds, sink,
                     clk);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// rowcopy: rows a positive multiple of 16, K a multiple of 64 with K / 16 lanes in 64 .. 1024,
// x holding rows * K bf16 and h rows * K * 2 bytes.
int vxf_rowcopy(const void* x, int64_t x_bytes, int64_t rows, int64_t k, void* h, int64_t h_bytes, void* stream) {
  if (!x || !h || rows <= 0 || rows % 16 || k % 64 || k / 16 < 64 || k / 16 > 1024 || x_bytes < rows * k * 2 ||
      h_bytes < rows * k * 2 || rows > 0x7FFFFFFFLL)
    return 1;
  hipLaunchKernelGGL(rowcopy_kernel, dim3((unsigned)rows), dim3((unsigned)(k / 16)), 0, (hipStream_t)stream,
                     (const uint16_t*)x, k, (int8_t*)h, k / 64);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

}  // extern "C"
