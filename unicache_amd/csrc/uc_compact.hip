// Keep-mask row compaction of the dense cache (tensor_backend.py:54-77): the
// rows t with keep[t] != 0 move, in order, to the front of the output.
//
// uc_mask_scan: one workgroup of 1024 threads; thread i counts the kept rows
// of its contiguous chunk (16-byte mask loads), an exclusive scan (lane
// shuffles within each wave, then over the 16 wave totals) turns the counts
// into chunk offsets, and every thread writes the destination row of each of
// its kept rows.  Deterministic, one pass over the mask plus one over the
// destination array.
//
// uc_compact_rows: one thread per 16 (or 8, 4, 2, 1) bytes of a row, rows of
// dropped tokens exit at once; the copy of a kept row is fully coalesced.
#include <algorithm>

#include "uc_common.h"

namespace uc {
namespace {

constexpr int kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void mask_scan_kernel(const uint8_t *keep, int64_t n, int64_t chunk,
                                                                 int32_t *dst, int64_t *total) {
  __shared__ int64_t part[2 * kScanThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t b = tid * chunk, e = min(n, b + chunk);
  int64_t cnt = 0;
  if (b < e) {
    int64_t t = b;
    // chunk is a multiple of 16 and keep is 16-byte aligned: whole uint4 runs
    for (; t + 16 <= e; t += 16) {
      const uint4 v = *reinterpret_cast<const uint4 *>(keep + t);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // one per nonzero byte: set bit 0 of each nonzero byte, then count
        const uint32_t nz = ((w[j] | (w[j] >> 1) | (w[j] >> 2) | (w[j] >> 3) | (w[j] >> 4) | (w[j] >> 5) |
                              (w[j] >> 6) | (w[j] >> 7)) & 0x01010101u);
        cnt += __builtin_popcount(nz);
      }
    }
    for (; t < e; ++t) cnt += keep[t] != 0;
  }
  // exclusive scan of the 1024 counts: inclusive within each wave by lane
  // shuffles, then the 16 wave totals (scanned by wave 0) are added
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  int64_t incl = cnt;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int64_t v = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += v;
  }
  if (lane == kWave - 1) part[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int64_t w = lane < kScanThreads / kWave ? part[lane] : 0, wi = w;
#pragma unroll
    for (int o = 1; o < kScanThreads / kWave; o <<= 1) {
      const int64_t v = __shfl_up(wi, o, kWave);
      if (lane >= o) wi += v;
    }
    if (lane < kScanThreads / kWave) part[kScanThreads / kWave + lane] = wi - w;  // exclusive wave offsets
    if (lane == kScanThreads / kWave - 1) *total = wi;
  }
  __syncthreads();
  int64_t pos = part[kScanThreads / kWave + wave] + incl - cnt;
  for (int64_t t = b; t < e; ++t) {
    if (keep[t] != 0) {
      dst[t] = static_cast<int32_t>(pos);
      ++pos;
    } else {
      dst[t] = -1;
    }
  }
}

// Block-wide exclusive scan of one int64 count per thread (1024 threads):
// returns the thread's exclusive prefix and writes the total to *total_out.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t cnt, int64_t *part, int64_t *total_out) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  int64_t incl = cnt;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int64_t v = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += v;
  }
  if (lane == kWave - 1) part[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int64_t w = lane < kScanThreads / kWave ? part[lane] : 0, wi = w;
#pragma unroll
    for (int o = 1; o < kScanThreads / kWave; o <<= 1) {
      const int64_t v = __shfl_up(wi, o, kWave);
      if (lane >= o) wi += v;
    }
    if (lane < kScanThreads / kWave) part[kScanThreads / kWave + lane] = wi - w;
    if (lane == kScanThreads / kWave - 1) part[2 * kScanThreads / kWave] = wi;
  }
  __syncthreads();
  const int64_t pre = part[kScanThreads / kWave + wave] + incl - cnt;
  *total_out = part[2 * kScanThreads / kWave];
  __syncthreads();  // `part` is reused by the next scan
  return pre;
}

// The rows KIVIQuantizationOperator fake-quantizes (operators/builtin.py:
// 394-404): segment tokens, except the last residual_length of them (a token
// whose suffix count of segment tokens, itself included, is at most
// residual_length) and, with preserve, the protected ones; none with bypass.
// One workgroup, a contiguous chunk per thread: a scan of the segment counts
// gives each token's suffix count, a scan of the selected counts its row in
// the compact order (dst, -1 when not selected) and src the inverse.
// counts = (segment tokens, selected tokens, protected segment tokens).
__global__ __launch_bounds__(kScanThreads) void fake_quant_mask_kernel(const uint8_t *segment, const uint8_t *prot,
                                                                      int64_t n, int64_t chunk, int64_t residual,
                                                                      int preserve, int bypass, int32_t *dst,
                                                                      int32_t *src, int64_t *counts) {
  __shared__ int64_t part[2 * kScanThreads / kWave + 1];
  const int tid = threadIdx.x;
  const int64_t b = tid * chunk, e = min(n, b + chunk);
  int64_t seg = 0, pseg = 0;
  for (int64_t t = b; t < e; ++t) {
    const bool sgt = segment[t] != 0;
    seg += sgt;
    pseg += sgt && prot[t] != 0;
  }
  int64_t seg_total = 0, pseg_total = 0;
  int64_t seg_before = block_exclusive_scan(seg, part, &seg_total);
  block_exclusive_scan(pseg, part, &pseg_total);
  // selected count of this chunk
  int64_t sel = 0;
  {
    int64_t sb = seg_before;
    for (int64_t t = b; t < e; ++t) {
      if (segment[t] == 0) continue;
      const int64_t from_end = seg_total - sb;  // segment tokens at t or later
      ++sb;
      const bool q = !bypass && (residual <= 0 || from_end > residual) && !(preserve && prot[t] != 0);
      sel += q;
    }
  }
  int64_t sel_total = 0;
  int64_t pos = block_exclusive_scan(sel, part, &sel_total);
  int64_t sb = seg_before;
  for (int64_t t = b; t < e; ++t) {
    bool q = false;
    if (segment[t] != 0) {
      const int64_t from_end = seg_total - sb;
      ++sb;
      q = !bypass && (residual <= 0 || from_end > residual) && !(preserve && prot[t] != 0);
    }
    if (q) {
      dst[t] = static_cast<int32_t>(pos);
      src[pos] = static_cast<int32_t>(t);
      ++pos;
    } else {
      dst[t] = -1;
    }
  }
  if (tid == 0) {
    counts[0] = seg_total;
    counts[1] = sel_total;
    counts[2] = pseg_total;
  }
}

template <typename V>
__global__ __launch_bounds__(256) void compact_rows_kernel(const char *src, int64_t src_stride, int64_t row_bytes,
                                                           const int32_t *dst_index, int64_t n, char *dst,
                                                           int64_t per_row) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t t = idx / per_row, c = idx % per_row;
  if (t >= n) return;
  const int32_t d = dst_index[t];
  if (d < 0) return;
  const V v = *reinterpret_cast<const V *>(src + t * src_stride + c * int64_t(sizeof(V)));
  *reinterpret_cast<V *>(dst + int64_t(d) * row_bytes + c * int64_t(sizeof(V))) = v;
}

// The inverse copy: compact row dst_index[t] back to row t of a strided array.
template <typename V>
__global__ __launch_bounds__(256) void scatter_rows_kernel(const char *src, int64_t row_bytes,
                                                           const int32_t *dst_index, int64_t n, char *out,
                                                           int64_t out_stride, int64_t per_row) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t t = idx / per_row, c = idx % per_row;
  if (t >= n) return;
  const int32_t d = dst_index[t];
  if (d < 0) return;
  const V v = *reinterpret_cast<const V *>(src + int64_t(d) * row_bytes + c * int64_t(sizeof(V)));
  *reinterpret_cast<V *>(out + t * out_stride + c * int64_t(sizeof(V))) = v;
}

template <typename V>
int launch_scatter(const void *src, int64_t row_bytes, const int32_t *dst_index, int64_t n, void *out,
                   int64_t out_stride, hipStream_t s) {
  const int64_t per_row = row_bytes / int64_t(sizeof(V));
  const int64_t threads = n * per_row;
  hipLaunchKernelGGL(scatter_rows_kernel<V>, dim3(static_cast<unsigned>(ceil_div(threads, int64_t(256)))), dim3(256),
                     0, s, static_cast<const char *>(src), row_bytes, dst_index, n, static_cast<char *>(out),
                     out_stride, per_row);
  return check_launch("uc_scatter_rows");
}

// Several uc_compact_rows copies that share dst_index in one launch:
// blockIdx.y selects the copy, 16-byte chunks.
constexpr int kMaxRowCopies = 4;
struct RowCopies {
  uc_row_copy c[kMaxRowCopies];
  int64_t per_row[kMaxRowCopies];
};

__global__ __launch_bounds__(256) void compact_rows_multi_kernel(RowCopies a, const int32_t *dst_index, int64_t n) {
  const uc_row_copy &c = a.c[blockIdx.y];
  const int64_t per_row = a.per_row[blockIdx.y];
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t t = idx / per_row, k = idx % per_row;
  if (t >= n) return;
  const int32_t d = dst_index[t];
  if (d < 0) return;
  const uint4 v = *reinterpret_cast<const uint4 *>(static_cast<const char *>(c.src) + t * c.src_row_stride_bytes + k * 16);
  *reinterpret_cast<uint4 *>(static_cast<char *>(c.dst) + int64_t(d) * c.row_bytes + k * 16) = v;
}

template <typename V>
int launch_compact(const void *src, int64_t src_stride, int64_t row_bytes, const int32_t *dst_index, int64_t n,
                   void *dst, hipStream_t s) {
  const int64_t per_row = row_bytes / int64_t(sizeof(V));
  const int64_t threads = n * per_row;
  hipLaunchKernelGGL(compact_rows_kernel<V>, dim3(static_cast<unsigned>(ceil_div(threads, int64_t(256)))), dim3(256),
                     0, s, static_cast<const char *>(src), src_stride, row_bytes, dst_index, n,
                     static_cast<char *>(dst), per_row);
  return check_launch("uc_compact_rows");
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int uc_mask_scan(const uint8_t *keep, int64_t n, int32_t *dst_index, int64_t *total,
                            uc_stream_t stream) {
  clear_error();
  UC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "uc_mask_scan: row count %lld out of range", (long long)n);
  UC_REQUIRE(total != nullptr && (n == 0 || (keep != nullptr && dst_index != nullptr)),
             "uc_mask_scan: null pointer");
  UC_REQUIRE((reinterpret_cast<uintptr_t>(keep) & 15) == 0, "uc_mask_scan: keep must be 16-byte aligned");
  const int64_t chunk = ceil_div(ceil_div(n, int64_t(kScanThreads)), int64_t(16)) * 16;
  hipLaunchKernelGGL(mask_scan_kernel, dim3(1), dim3(kScanThreads), 0, as_stream(stream), keep, n,
                     chunk > 0 ? chunk : 16, dst_index, total);
  return check_launch("uc_mask_scan");
}

extern "C" int uc_compact_rows(const void *src, int64_t src_row_stride_bytes, int64_t row_bytes,
                               const int32_t *dst_index, int64_t n, void *dst, uc_stream_t stream) {
  clear_error();
  UC_REQUIRE(n >= 0 && row_bytes >= 0 && src_row_stride_bytes >= row_bytes, "uc_compact_rows: bad shape");
  if (n == 0 || row_bytes == 0) return UC_OK;
  UC_REQUIRE(src != nullptr && dst != nullptr && dst_index != nullptr, "uc_compact_rows: null pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                          static_cast<uintptr_t>(src_row_stride_bytes) | static_cast<uintptr_t>(row_bytes);
  const hipStream_t s = as_stream(stream);
  if ((align & 15) == 0) return launch_compact<uint4>(src, src_row_stride_bytes, row_bytes, dst_index, n, dst, s);
  if ((align & 7) == 0) return launch_compact<uint2>(src, src_row_stride_bytes, row_bytes, dst_index, n, dst, s);
  if ((align & 3) == 0) return launch_compact<uint32_t>(src, src_row_stride_bytes, row_bytes, dst_index, n, dst, s);
  if ((align & 1) == 0) return launch_compact<uint16_t>(src, src_row_stride_bytes, row_bytes, dst_index, n, dst, s);
  return launch_compact<uint8_t>(src, src_row_stride_bytes, row_bytes, dst_index, n, dst, s);
}

extern "C" int uc_scatter_rows(const void *src, int64_t row_bytes, const int32_t *dst_index, int64_t n, void *out,
                               int64_t out_row_stride_bytes, uc_stream_t stream) {
  clear_error();
  UC_REQUIRE(n >= 0 && row_bytes >= 0 && out_row_stride_bytes >= row_bytes, "uc_scatter_rows: bad shape");
  if (n == 0 || row_bytes == 0) return UC_OK;
  UC_REQUIRE(src != nullptr && out != nullptr && dst_index != nullptr, "uc_scatter_rows: null pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(out) |
                          static_cast<uintptr_t>(out_row_stride_bytes) | static_cast<uintptr_t>(row_bytes);
  const hipStream_t s = as_stream(stream);
  if ((align & 15) == 0) return launch_scatter<uint4>(src, row_bytes, dst_index, n, out, out_row_stride_bytes, s);
  if ((align & 7) == 0) return launch_scatter<uint2>(src, row_bytes, dst_index, n, out, out_row_stride_bytes, s);
  if ((align & 3) == 0) return launch_scatter<uint32_t>(src, row_bytes, dst_index, n, out, out_row_stride_bytes, s);
  if ((align & 1) == 0) return launch_scatter<uint16_t>(src, row_bytes, dst_index, n, out, out_row_stride_bytes, s);
  return launch_scatter<uint8_t>(src, row_bytes, dst_index, n, out, out_row_stride_bytes, s);
}

namespace uc {
namespace {

constexpr int kMaxSpans = 8;
struct CopySpans {
  const uint8_t *src[kMaxSpans];
  uint8_t *dst[kMaxSpans];
  int64_t bytes[kMaxSpans];
  int vec[kMaxSpans];  // 1: 16-byte units (addresses and size 16-aligned), 0: bytes
};

// Span blockIdx.y; thread i of the span's grid copies unit i (and i + grid
// stride): 16 bytes when the span allows, else one byte.
__global__ __launch_bounds__(256) void copy_spans_kernel(CopySpans c) {
  const int s = blockIdx.y;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c.vec[s]) {
    const int64_t n = c.bytes[s] / 16;
    for (; i < n; i += stride)
      reinterpret_cast<uint4 *>(c.dst[s])[i] = reinterpret_cast<const uint4 *>(c.src[s])[i];
  } else {
    for (; i < c.bytes[s]; i += stride) c.dst[s][i] = c.src[s][i];
  }
}

}  // namespace
}  // namespace uc

extern "C" int uc_copy_spans(const uc_copy_span *spans_host, int n, uc_stream_t stream) {
  clear_error();
  UC_REQUIRE(n >= 0 && n <= kMaxSpans, "uc_copy_spans: 0..%d spans per call (got %d)", kMaxSpans, n);
  UC_REQUIRE(n == 0 || spans_host != nullptr, "uc_copy_spans: spans is NULL");
  CopySpans c{};
  int64_t most = 0;
  for (int i = 0; i < n; ++i) {
    const uc_copy_span &sp = spans_host[i];
    UC_REQUIRE(sp.bytes >= 0, "uc_copy_spans: negative size");
    UC_REQUIRE(sp.bytes == 0 || (sp.src != nullptr && sp.dst != nullptr), "uc_copy_spans: null pointer");
    c.src[i] = static_cast<const uint8_t *>(sp.src);
    c.dst[i] = static_cast<uint8_t *>(sp.dst);
    c.bytes[i] = sp.bytes;
    c.vec[i] = ((reinterpret_cast<uintptr_t>(sp.src) | reinterpret_cast<uintptr_t>(sp.dst) |
                 static_cast<uintptr_t>(sp.bytes)) & 15) == 0;
    most = std::max(most, c.vec[i] ? sp.bytes / 16 : sp.bytes);
  }
  if (most == 0) return UC_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(most, int64_t(256)), 1024);
  hipLaunchKernelGGL(copy_spans_kernel, dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(n)), dim3(256), 0,
                     as_stream(stream), c);
  return check_launch("uc_copy_spans");
}

extern "C" int uc_compact_rows_multi(const uc_row_copy *copies, int n_copies, const int32_t *dst_index, int64_t n,
                                     uc_stream_t stream) {
  clear_error();
  UC_REQUIRE(n_copies >= 0 && (n_copies == 0 || copies != nullptr) && n >= 0, "uc_compact_rows_multi: bad arguments");
  if (n == 0 || n_copies == 0) return UC_OK;
  UC_REQUIRE(dst_index != nullptr, "uc_compact_rows_multi: null pointer");
  RowCopies a{};
  int m = 0;
  int64_t most = 0;
  for (int i = 0; i < n_copies; ++i) {
    const uc_row_copy &c = copies[i];
    UC_REQUIRE(c.row_bytes >= 0 && c.src_row_stride_bytes >= c.row_bytes, "uc_compact_rows_multi: bad shape");
    if (c.row_bytes == 0) continue;
    UC_REQUIRE(c.src != nullptr && c.dst != nullptr, "uc_compact_rows_multi: null pointer");
    const uintptr_t align = reinterpret_cast<uintptr_t>(c.src) | reinterpret_cast<uintptr_t>(c.dst) |
                            static_cast<uintptr_t>(c.src_row_stride_bytes) | static_cast<uintptr_t>(c.row_bytes);
    if ((align & 15) != 0 || m == kMaxRowCopies) {  // its own launch, the widest access its alignment allows
      const int rc = uc_compact_rows(c.src, c.src_row_stride_bytes, c.row_bytes, dst_index, n, c.dst, stream);
      if (rc != UC_OK) return rc;
      continue;
    }
    a.c[m] = c;
    a.per_row[m] = c.row_bytes / 16;
    most = a.per_row[m] > most ? a.per_row[m] : most;
    ++m;
  }
  if (m == 0) return UC_OK;
  const dim3 grid(static_cast<unsigned>(ceil_div(n * most, int64_t(256))), static_cast<unsigned>(m));
  hipLaunchKernelGGL(compact_rows_multi_kernel, grid, dim3(256), 0, as_stream(stream), a, dst_index, n);
  return check_launch("uc_compact_rows_multi");
}

extern "C" int uc_fake_quant_mask(const uint8_t *segment, const uint8_t *protected_mask, int64_t n,
                                  int64_t residual_length, int preserve_protected, int bypass, int32_t *dst_index,
                                  int32_t *src_index, int64_t *counts, uc_stream_t stream) {
  clear_error();
  UC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "uc_fake_quant_mask: row count %lld out of range", (long long)n);
  UC_REQUIRE(counts != nullptr && (n == 0 || (segment != nullptr && protected_mask != nullptr &&
                                              dst_index != nullptr && src_index != nullptr)),
             "uc_fake_quant_mask: null pointer");
  const int64_t chunk = ceil_div(n, int64_t(kScanThreads));
  hipLaunchKernelGGL(fake_quant_mask_kernel, dim3(1), dim3(kScanThreads), 0, as_stream(stream), segment,
                     protected_mask, n, chunk > 0 ? chunk : 1, residual_length, preserve_protected, bypass, dst_index,
                     src_index, counts);
  return check_launch("uc_fake_quant_mask");
}
