// Canonical host publication: packs a device tensor into dense row-major big-endian bytes.
//
// Replaces the host-side packing of MetalBackendRuntime.copyToCanonicalHostBytes
// (modules/backend/metal/src/main/java/io/github/pho001/synaptik/backend/metal/
// MetalBackendRuntime.java:304-424): every multi-byte element is byte-reversed into big-endian
// order with its raw bits kept (NaN payloads, signed zeros), a strided / offset view is gathered
// in row-major ordinal order (storageElementIndex, :489-499), and BOOL elements must be 0 or 1
// (:380-385). The reference does this per element in Java after a raw download; here one HBM
// pass on the device writes the canonical bytes into a staging buffer, which is then copied to
// the host as is.
//
// Dense views move 16 bytes per thread per iteration (one uint4 load, in-register byte swaps,
// one uint4 store); transposed matrices go through 64x64 LDS tiles; other strided views gather
// one element per thread.
#include "common.h"
#include "kernels.h"

namespace shk {
namespace {

constexpr int PUB_NT = 256;

// Byte reversal of each W-byte element inside one 16-byte chunk.
template <int W>
__device__ __forceinline__ uint4 swap_chunk(uint4 v) {
  if constexpr (W == 2) {
    auto s = [](uint32_t x) { return ((x & 0x00ff00ffu) << 8) | ((x >> 8) & 0x00ff00ffu); };
    return make_uint4(s(v.x), s(v.y), s(v.z), s(v.w));
  } else if constexpr (W == 4) {
    return make_uint4(__builtin_bswap32(v.x), __builtin_bswap32(v.y), __builtin_bswap32(v.z),
                      __builtin_bswap32(v.w));
  } else if constexpr (W == 8) {
    // two little-endian 64-bit elements: (x, y) and (z, w) as (low, high) words
    return make_uint4(__builtin_bswap32(v.y), __builtin_bswap32(v.x), __builtin_bswap32(v.w),
                      __builtin_bswap32(v.z));
  } else {
    return v;
  }
}

// Flags any byte of the chunk that is neither 0 nor 1.
__device__ __forceinline__ bool bool_chunk_bad(uint4 v) {
  const uint32_t m = 0xfefefefeu;
  return ((v.x | v.y | v.z | v.w) & m) != 0u;
}

// Dense: chunks16 16-byte chunks, then tail_bytes bytes (fewer than 16) done by thread 0 of
// block 0 element by element.
template <int W, bool BOOLV>
__global__ void __launch_bounds__(PUB_NT) pack_dense_kernel(const uint8_t* __restrict__ src,
                                                            uint8_t* __restrict__ dst,
                                                            int64_t chunks16, int64_t tail_bytes,
                                                            uint32_t* status) {
  const uint4* s4 = reinterpret_cast<const uint4*>(src);
  uint4* d4 = reinterpret_cast<uint4*>(dst);
  bool bad = false;
  const int64_t stride = (int64_t)gridDim.x * PUB_NT;
  for (int64_t i = (int64_t)blockIdx.x * PUB_NT + threadIdx.x; i < chunks16; i += stride) {
    const uint4 v = s4[i];
    if (BOOLV) bad |= bool_chunk_bad(v);
    d4[i] = swap_chunk<W>(v);
  }
  if (tail_bytes > 0 && blockIdx.x == 0 && threadIdx.x == 0) {
    const int64_t base = chunks16 * 16;
    for (int64_t e = 0; e < tail_bytes / W; ++e) {
      const uint8_t* a = src + base + e * W;
      uint8_t* b = dst + base + e * W;
#pragma unroll
      for (int k = 0; k < W; ++k) b[k] = a[W - 1 - k];
      if (BOOLV) bad |= a[0] > 1;
    }
  }
  if (BOOLV) {
    const int any = wave_or(bad ? 1 : 0);
    if (any && (threadIdx.x & 63) == 0) atomicOr(status, (uint32_t)DEV_INVALID_BOOL);
  }
}

template <int W>
struct Elem;
template <> struct Elem<1> { using T = uint8_t; __device__ static T swap(T v) { return v; } };
template <> struct Elem<2> { using T = uint16_t; __device__ static T swap(T v) { return __builtin_bswap16(v); } };
template <> struct Elem<4> { using T = uint32_t; __device__ static T swap(T v) { return __builtin_bswap32(v); } };
template <> struct Elem<8> { using T = uint64_t; __device__ static T swap(T v) { return __builtin_bswap64(v); } };

// Strided view: ordinal -> storage element by the row-major mixed-radix decomposition of the
// ordinal over the dimensions (last axis fastest). STORE = false only validates (BOOL).
template <int W, bool BOOLV, bool STORE = true>
__global__ void __launch_bounds__(PUB_NT) pack_strided_kernel(const uint8_t* __restrict__ src,
                                                              uint8_t* __restrict__ dst,
                                                              int64_t elements,
                                                              CanonicalGeometry g,
                                                              uint32_t* status) {
  using T = typename Elem<W>::T;
  const T* s = reinterpret_cast<const T*>(src);
  T* d = reinterpret_cast<T*>(dst);
  bool bad = false;
  const int64_t stride = (int64_t)gridDim.x * PUB_NT;
  for (int64_t o = (int64_t)blockIdx.x * PUB_NT + threadIdx.x; o < elements; o += stride) {
    int64_t rem = o, idx = g.offset;
    for (int a = g.rank - 1; a >= 0; --a) {
      const int64_t dim = g.dims[a];
      const int64_t q = rem / dim;
      idx += (rem - q * dim) * g.strides[a];
      rem = q;
    }
    const T v = s[idx];
    if (BOOLV) bad |= v > 1;
    if (STORE) d[o] = Elem<W>::swap(v);
  }
  if (BOOLV) {
    const int any = wave_or(bad ? 1 : 0);
    if (any && (threadIdx.x & 63) == 0) atomicOr(status, (uint32_t)DEV_INVALID_BOOL);
  }
}

// Transposed rank-2 view: element (a, b) lives at offset + a + b * sb (axis 0 contiguous in
// storage, axis 1 fastest in the output). 64x64 tiles through LDS so that both the storage reads
// (along a) and the canonical writes (along b) are coalesced.
template <int W>
__global__ void __launch_bounds__(PUB_NT) pack_transpose_kernel(const uint8_t* __restrict__ src,
                                                                uint8_t* __restrict__ dst,
                                                                int64_t A, int64_t B, int64_t sb,
                                                                int64_t offset) {
  using T = typename Elem<W>::T;
  __shared__ T tile[64][65];
  const T* s = reinterpret_cast<const T*>(src);
  T* d = reinterpret_cast<T*>(dst);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t a0 = (int64_t)blockIdx.y * 64, b0 = (int64_t)blockIdx.x * 64;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int64_t b = b0 + ty + 4 * j, a = a0 + tx;
    if (a < A && b < B) tile[ty + 4 * j][tx] = s[offset + a + b * sb];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int64_t a = a0 + ty + 4 * j, b = b0 + tx;
    if (a < A && b < B) d[a * B + b] = Elem<W>::swap(tile[tx][ty + 4 * j]);
  }
}

// After dropping unit axes: exactly two axes, the first with stride 1 and the second with a
// stride of at least its extent (a transposed matrix or a column slice of one), each axis small
// enough for the tile grid.
bool transposed2d(const CanonicalGeometry& g) {
  int64_t dims[2], strides[2];
  int k = 0;
  for (int a = 0; a < g.rank; ++a) {
    if (g.dims[a] == 1) continue;
    if (k == 2) return false;
    dims[k] = g.dims[a];
    strides[k] = g.strides[a];
    ++k;
  }
  return k == 2 && strides[0] == 1 && strides[1] >= dims[0] && (dims[0] + 63) / 64 < 65536 &&
         (dims[1] + 63) / 64 < (int64_t)1 << 31;
}

unsigned grid_for(int64_t work) {
  const int64_t blocks = (work + PUB_NT - 1) / PUB_NT;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(blocks, 8192));
}

template <int W, bool BOOLV>
hipError_t launch_w(const void* src, void* dst, int64_t elements, const CanonicalGeometry* g,
                    uint32_t* status, hipStream_t s) {
  const uint8_t* a = static_cast<const uint8_t*>(src);
  uint8_t* b = static_cast<uint8_t*>(dst);
  if (g == nullptr) {
    const int64_t bytes = elements * W;
    const int64_t chunks = bytes / 16;
    hipLaunchKernelGGL((pack_dense_kernel<W, BOOLV>), dim3(grid_for(chunks)), dim3(PUB_NT), 0, s,
                       a, b, chunks, bytes - chunks * 16, status);
  } else if (!BOOLV && transposed2d(*g)) {
    int64_t dims[2], strides[2];
    int k = 0;
    for (int a = 0; a < g->rank; ++a)
      if (g->dims[a] != 1) { dims[k] = g->dims[a]; strides[k] = g->strides[a]; ++k; }
    const dim3 grid((unsigned)((dims[1] + 63) / 64), (unsigned)((dims[0] + 63) / 64));
    hipLaunchKernelGGL((pack_transpose_kernel<W>), grid, dim3(PUB_NT), 0, s, a, b, dims[0],
                       dims[1], strides[1], g->offset);
  } else {
    hipLaunchKernelGGL((pack_strided_kernel<W, BOOLV>), dim3(grid_for(elements)), dim3(PUB_NT),
                       0, s, a, b, elements, *g, status);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_bool_validate(const void* src, int64_t elements, const CanonicalGeometry& g,
                                uint32_t* status, hipStream_t s) {
  if (elements <= 0) return hipSuccess;
  hipLaunchKernelGGL((pack_strided_kernel<1, true, false>), dim3(grid_for(elements)),
                     dim3(PUB_NT), 0, s, static_cast<const uint8_t*>(src), nullptr, elements, g,
                     status);
  return hipGetLastError();
}

hipError_t launch_canonical_pack(const void* src, void* dst, int64_t elements, int width,
                                 int boolean, const CanonicalGeometry* g, uint32_t* status,
                                 hipStream_t s) {
  if (elements <= 0) return hipSuccess;
  if (boolean) return launch_w<1, true>(src, dst, elements, g, status, s);
  switch (width) {
    case 1: return launch_w<1, false>(src, dst, elements, g, status, s);
    case 2: return launch_w<2, false>(src, dst, elements, g, status, s);
    case 4: return launch_w<4, false>(src, dst, elements, g, status, s);
    case 8: return launch_w<8, false>(src, dst, elements, g, status, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace shk
