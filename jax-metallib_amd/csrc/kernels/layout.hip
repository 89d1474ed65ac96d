// Layout ops: one strided copy kernel behind stablehlo.transpose, slice,
// broadcast_in_dim, concatenate (one copy per operand into its place) and
// non-contiguous reshapes, and an iota kernel.  The reference runs these as
// MPSGraph ops (ops/shape_ops.mm: HandleBroadcastInDim :137, HandleTranspose
// :304, HandleSlice :831, HandleConcatenate :1208; iota
// ops/tensor_creation_ops.mm:126).
//
// HBM-bound element moves.  The host merges dimensions that are contiguous
// in both source and destination, so a transpose of [B, T, H, D] is a rank-3
// copy with D-element rows; the kernel walks the destination in order with
// 32-bit index math when every offset fits, and moves 16 bytes per thread
// when the innermost dimension is contiguous on both sides and aligned.
#include "common.h"
#include "../capi_internal.h"

#include <algorithm>

namespace mk {

constexpr int kLayoutMaxRank = 8;

struct LayoutArgs {
  const unsigned char* src;
  unsigned char* dst;
  int rank;
  int64_t n;  // elements (or 16-byte vectors in the vector path)
  int64_t shape[kLayoutMaxRank];
  int64_t ss[kLayoutMaxRank];  // source strides, elements
  int64_t ds[kLayoutMaxRank];  // destination strides, elements
  int64_t so, dof;             // offsets, elements
};

template <typename T, typename I>
__global__ __launch_bounds__(256) void strided_copy_kernel(LayoutArgs a) {
  const T* __restrict__ src = reinterpret_cast<const T*>(a.src);
  T* __restrict__ dst = reinterpret_cast<T*>(a.dst);
  const I n = (I)a.n;
  for (I i = (I)blockIdx.x * 256 + threadIdx.x; i < n; i += (I)gridDim.x * 256) {
    I r = i, s = (I)a.so, d = (I)a.dof;
    for (int k = a.rank - 1; k >= 0; --k) {
      const I sh = (I)a.shape[k];
      const I q = r / sh;
      const I c = r - q * sh;
      s += c * (I)a.ss[k];
      d += c * (I)a.ds[k];
      r = q;
    }
    dst[d] = src[s];
  }
}

template <typename T>
__device__ __forceinline__ T iota_value(int64_t v);
template <> __device__ __forceinline__ uint8_t iota_value<uint8_t>(int64_t v) { return (uint8_t)v; }
template <> __device__ __forceinline__ uint16_t iota_value<uint16_t>(int64_t v) { return (uint16_t)v; }
template <> __device__ __forceinline__ uint32_t iota_value<uint32_t>(int64_t v) { return (uint32_t)v; }
template <> __device__ __forceinline__ uint64_t iota_value<uint64_t>(int64_t v) { return (uint64_t)v; }

// KIND 0: integer of sizeof(T); 1: f32; 2: bf16 (RNE); 3: f64; 4: f16.
template <typename T, int KIND>
__global__ __launch_bounds__(256) void iota_kernel(T* __restrict__ dst, int64_t n, int64_t inner, int64_t len) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t v = (i / inner) % len;
    if constexpr (KIND == 0) {
      dst[i] = iota_value<T>(v);
    } else if constexpr (KIND == 1) {
      const float f = (float)v;
      dst[i] = __float_as_uint(f);
    } else if constexpr (KIND == 2) {
      dst[i] = (T)f32_to_bf16((float)v);
    } else if constexpr (KIND == 3) {
      const double f = (double)v;
      dst[i] = (T)__double_as_longlong(f);
    } else {
      const _Float16 h = (_Float16)(float)v;
      dst[i] = (T)__builtin_bit_cast(uint16_t, h);
    }
  }
}

}  // namespace mk

namespace {

// Merge dimension k-1 into k where both sides are contiguous across them;
// drop size-1 dimensions.  Returns the new rank.
int merge_dims(int rank, int64_t* shape, int64_t* ss, int64_t* ds) {
  int r = 0;
  int64_t sh[mk::kLayoutMaxRank], s1[mk::kLayoutMaxRank], d1[mk::kLayoutMaxRank];
  for (int k = 0; k < rank; ++k) {
    if (shape[k] == 1) continue;
    if (r > 0 && ss[k] * shape[k] == s1[r - 1] && ds[k] * shape[k] == d1[r - 1]) {
      sh[r - 1] *= shape[k];
      s1[r - 1] = ss[k];
      d1[r - 1] = ds[k];
      continue;
    }
    sh[r] = shape[k];
    s1[r] = ss[k];
    d1[r] = ds[k];
    ++r;
  }
  for (int k = 0; k < r; ++k) {
    shape[k] = sh[k];
    ss[k] = s1[k];
    ds[k] = d1[k];
  }
  return r;
}

int launch_blocks(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 256 * 16)); }

}  // namespace

extern "C" int mk_strided_copy(const void* src, void* dst, int elem_bytes, int rank, const int64_t* shape,
                               const int64_t* src_strides, int64_t src_offset, const int64_t* dst_strides,
                               int64_t dst_offset, void* stream) {
  mkc::clear_error();
  const char* fn = "mk_strided_copy";
  if (!src || !dst || (rank > 0 && (!shape || !src_strides || !dst_strides)))
    return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return mkc::fail(MK_EINVAL, "%s: element size %d (1, 2, 4 or 8)", fn, elem_bytes);
  if (rank < 0 || rank > mk::kLayoutMaxRank) return mkc::fail(MK_EINVAL, "%s: rank %d (0..8)", fn, rank);
  mk::LayoutArgs a;
  int64_t n = 1, smax = src_offset, dmax = dst_offset;
  for (int k = 0; k < rank; ++k) {
    if (shape[k] < 0) return mkc::fail(MK_EINVAL, "%s: negative dimension", fn);
    if (src_strides[k] < 0 || dst_strides[k] < 0) return mkc::fail(MK_EINVAL, "%s: negative stride", fn);
    a.shape[k] = shape[k];
    a.ss[k] = src_strides[k];
    a.ds[k] = dst_strides[k];
    n *= shape[k];
  }
  if (src_offset < 0 || dst_offset < 0) return mkc::fail(MK_EINVAL, "%s: negative offset", fn);
  if (n == 0) return MK_OK;
  for (int k = 0; k < rank; ++k) {
    smax += (shape[k] - 1) * src_strides[k];
    dmax += (shape[k] - 1) * dst_strides[k];
  }
  a.rank = merge_dims(rank, a.shape, a.ss, a.ds);
  a.src = static_cast<const unsigned char*>(src);
  a.dst = static_cast<unsigned char*>(dst);
  a.so = src_offset;
  a.dof = dst_offset;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // 16-byte moves when the innermost run is contiguous on both sides and
  // every offset and stride is a whole number of 16-byte vectors.
  const int vec = 16 / elem_bytes;
  bool vok = a.rank > 0 && a.ss[a.rank - 1] == 1 && a.ds[a.rank - 1] == 1 && a.shape[a.rank - 1] % vec == 0 &&
             a.so % vec == 0 && a.dof % vec == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0;
  for (int k = 0; vok && k + 1 < a.rank; ++k) vok = a.ss[k] % vec == 0 && a.ds[k] % vec == 0;
  int eb = elem_bytes;
  if (vok) {
    a.shape[a.rank - 1] /= vec;
    for (int k = 0; k + 1 < a.rank; ++k) {
      a.ss[k] /= vec;
      a.ds[k] /= vec;
    }
    a.so /= vec;
    a.dof /= vec;
    n /= vec;
    smax /= vec;
    dmax /= vec;
    eb = 16;
  }
  a.n = n;
  const bool small = n < (1ll << 31) && smax < (1ll << 31) && dmax < (1ll << 31);
  const int blocks = launch_blocks(n);
#define MK_SC(T)                                                                                   \
  if (small) hipLaunchKernelGGL((mk::strided_copy_kernel<T, uint32_t>), dim3(blocks), dim3(256), 0, st, a); \
  else hipLaunchKernelGGL((mk::strided_copy_kernel<T, int64_t>), dim3(blocks), dim3(256), 0, st, a);
  switch (eb) {
    case 1: MK_SC(uint8_t) break;
    case 2: MK_SC(uint16_t) break;
    case 4: MK_SC(uint32_t) break;
    case 8: MK_SC(uint64_t) break;
    default: MK_SC(mk::u32x4) break;
  }
#undef MK_SC
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}

extern "C" int mk_iota(void* dst, int dtype, int rank, const int64_t* shape, int dim, void* stream) {
  mkc::clear_error();
  const char* fn = "mk_iota";
  if (!dst || (rank > 0 && !shape)) return mkc::fail(MK_EINVAL, "%s: null pointer argument", fn);
  if (rank < 1 || rank > mk::kLayoutMaxRank || dim < 0 || dim >= rank)
    return mkc::fail(MK_EINVAL, "%s: rank %d, dimension %d", fn, rank, dim);
  int64_t n = 1, inner = 1;
  for (int k = 0; k < rank; ++k) {
    if (shape[k] < 0) return mkc::fail(MK_EINVAL, "%s: negative dimension", fn);
    n *= shape[k];
    if (k > dim) inner *= shape[k];
  }
  if (n == 0) return MK_OK;
  const int64_t len = shape[dim];
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int blocks = launch_blocks(n);
  switch (dtype) {
    case MK_IOTA_S8: case MK_IOTA_U8:
      hipLaunchKernelGGL((mk::iota_kernel<uint8_t, 0>), dim3(blocks), dim3(256), 0, st, (uint8_t*)dst, n, inner, len);
      break;
    case MK_IOTA_S16: case MK_IOTA_U16:
      hipLaunchKernelGGL((mk::iota_kernel<uint16_t, 0>), dim3(blocks), dim3(256), 0, st, (uint16_t*)dst, n, inner, len);
      break;
    case MK_IOTA_S32: case MK_IOTA_U32:
      hipLaunchKernelGGL((mk::iota_kernel<uint32_t, 0>), dim3(blocks), dim3(256), 0, st, (uint32_t*)dst, n, inner, len);
      break;
    case MK_IOTA_S64: case MK_IOTA_U64:
      hipLaunchKernelGGL((mk::iota_kernel<uint64_t, 0>), dim3(blocks), dim3(256), 0, st, (uint64_t*)dst, n, inner, len);
      break;
    case MK_IOTA_F32:
      hipLaunchKernelGGL((mk::iota_kernel<uint32_t, 1>), dim3(blocks), dim3(256), 0, st, (uint32_t*)dst, n, inner, len);
      break;
    case MK_IOTA_BF16:
      hipLaunchKernelGGL((mk::iota_kernel<uint16_t, 2>), dim3(blocks), dim3(256), 0, st, (uint16_t*)dst, n, inner, len);
      break;
    case MK_IOTA_F64:
      hipLaunchKernelGGL((mk::iota_kernel<uint64_t, 3>), dim3(blocks), dim3(256), 0, st, (uint64_t*)dst, n, inner, len);
      break;
    case MK_IOTA_F16:
      hipLaunchKernelGGL((mk::iota_kernel<uint16_t, 4>), dim3(blocks), dim3(256), 0, st, (uint16_t*)dst, n, inner, len);
      break;
    default:
      return mkc::fail(MK_EUNSUPPORTED, "%s: element type %d", fn, dtype);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mkc::fail(MK_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return MK_OK;
}
