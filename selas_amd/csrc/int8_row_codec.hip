// int8_row codec on gfx950: decode (bit-exact with the reference decode) and encode.
//
// Format (selas/codecs.py:86-96): a weight [rows, ...] is stored as q, int8 of
// the same shape, and one fp32 scale per row: scale = absmax(row) / 127 (1 for
// an all-zero row), q = clamp(round_half_even(w / scale), -127, 127).
// Decode (selas/codecs.py:273-277) computes q.to(dt) * scale.to(dt) in the
// output type dt: q converts exactly, the scale is rounded to dt, and their
// product (exact in fp32 for bf16 and fp16) is rounded once to dt.
#include "common.h"

namespace selas {
namespace {

constexpr int kThreads = 256;

// The row scale as the reference's decode sees it: rounded to the output type.
template <int DT>
__device__ __forceinline__ float scale_as(float s) {
  if constexpr (DT == SELAS_F32) return s;
  else if constexpr (DT == SELAS_F16) return f16_bits_to_f32(f16_bits_rne(s));
  else return bf16_bits_to_f32(bf16_bits_rne(s));
}

// --------------------------------------------------------------------------- decode

// Vector path (cols % 16 == 0, 16-byte aligned): each thread decodes 16 values
// of one row.
template <int DT>
__global__ __launch_bounds__(kThreads) void int8_row_dequant_vec16(const uint4 *__restrict__ q,
                                                                   const float *__restrict__ scale, int64_t n16,
                                                                   int64_t chunks_per_row, void *__restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n16) return;
  const uint4 w = q[i];
  const float s = scale_as<DT>(scale[i / chunks_per_row]);
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  float v[16];
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[4 * d + j] = static_cast<float>(static_cast<int8_t>((words[d] >> (8 * j)) & 0xffu)) * s;
  if constexpr (DT == SELAS_F32) {
    float4 *o = reinterpret_cast<float4 *>(out) + i * 4;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = make_float4(v[4 * d], v[4 * d + 1], v[4 * d + 2], v[4 * d + 3]);
  } else {
    uint32_t pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (DT == SELAS_BF16)
        pr[j] = bf16_bits_rne(v[2 * j]) | (static_cast<uint32_t>(bf16_bits_rne(v[2 * j + 1])) << 16);
      else
        pr[j] = f16_bits_rne(v[2 * j]) | (static_cast<uint32_t>(f16_bits_rne(v[2 * j + 1])) << 16);
    }
    uint4 *o = reinterpret_cast<uint4 *>(out) + i * 2;
    o[0] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    o[1] = make_uint4(pr[4], pr[5], pr[6], pr[7]);
  }
}

// Generic path: one value per thread.
template <int DT>
__global__ __launch_bounds__(kThreads) void int8_row_dequant_elems(const int8_t *__restrict__ q,
                                                                   const float *__restrict__ scale, int64_t n,
                                                                   int64_t cols, void *__restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  store_f<DT>(out, i, static_cast<float>(q[i]) * scale_as<DT>(scale[i / cols]));
}

template <int DT>
int dequant_typed(const int8_t *q, const float *scale, int64_t rows, int64_t cols, void *out, hipStream_t stream) {
  const int64_t n = rows * cols;
  if (cols % 16 == 0 && aligned(q, 16) && aligned(out, 16)) {
    const int64_t n16 = n / 16;
    int8_row_dequant_vec16<DT><<<dim3(static_cast<uint32_t>(cdiv(n16, kThreads))), dim3(kThreads), 0, stream>>>(
        reinterpret_cast<const uint4 *>(q), scale, n16, cols / 16, out);
  } else {
    int8_row_dequant_elems<DT><<<dim3(static_cast<uint32_t>(cdiv(n, kThreads))), dim3(kThreads), 0, stream>>>(
        q, scale, n, cols, out);
  }
  return check_launch("int8_row_dequant");
}

// --------------------------------------------------------------------------- encode

// NaN-propagating max, as torch.amax.
__device__ __forceinline__ float max_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

// One workgroup per row (grid-stride): |w| max over the row, scale = max / 127
// (1 when the max is not positive, as torch.where(absmax > 0, ...) picks), then
// q = clamp(rint(w / scale), -127, 127) with IEEE division and round half to even
// (torch.round).
__global__ __launch_bounds__(kThreads) void int8_row_encode_rows(const float *__restrict__ w, int64_t rows,
                                                                 int64_t cols, int8_t *__restrict__ q,
                                                                 float *__restrict__ scale) {
  __shared__ float part[kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const float *src = w + r * cols;
    float m = 0.0f;
    for (int64_t j = tid; j < cols; j += kThreads) m = max_nan(m, fabsf(src[j]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max_nan(m, __shfl_xor(m, o, 64));
    if (lane == 0) part[wave] = m;
    __syncthreads();
    m = max_nan(max_nan(part[0], part[1]), max_nan(part[2], part[3]));
    __syncthreads();  // part is rewritten by the next row
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    for (int64_t j = tid; j < cols; j += kThreads) {
      const float v = fminf(fmaxf(rintf(src[j] / sc), -127.0f), 127.0f);
      q[r * cols + j] = static_cast<int8_t>(static_cast<int>(v));
    }
    if (tid == 0) scale[r] = sc;
  }
}

}  // namespace
}  // namespace selas

using namespace selas;

extern "C" int selas_int8_row_dequant(const int8_t *q, const float *scale, int64_t rows, int64_t cols, void *out,
                                      int out_dtype, void *stream) {
  if (rows < 0 || cols < 0)
    return set_error(SELAS_EINVAL, "int8_row_dequant: bad shape %lld x %lld", (long long)rows, (long long)cols);
  if (!valid_dtype(out_dtype)) return set_error(SELAS_EINVAL, "int8_row_dequant: bad output dtype %d", out_dtype);
  if (rows == 0 || cols == 0) return ok();
  if (!q || !scale || !out) return set_error(SELAS_EINVAL, "int8_row_dequant: null pointer");
  if (rows * cols / kThreads >= (1ll << 31))
    return set_error(SELAS_EUNSUPPORTED, "int8_row_dequant: %lld elements exceed one launch", (long long)(rows * cols));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case SELAS_F32: return dequant_typed<SELAS_F32>(q, scale, rows, cols, out, s);
    case SELAS_F16: return dequant_typed<SELAS_F16>(q, scale, rows, cols, out, s);
    default: return dequant_typed<SELAS_BF16>(q, scale, rows, cols, out, s);
  }
}

extern "C" int selas_int8_row_encode(const float *w, int64_t rows, int64_t cols, int8_t *q, float *scale,
                                     void *stream) {
  if (rows < 0 || cols < 0)
    return set_error(SELAS_EINVAL, "int8_row_encode: bad shape %lld x %lld", (long long)rows, (long long)cols);
  if (rows == 0) return ok();
  if (!w || !q || !scale) return set_error(SELAS_EINVAL, "int8_row_encode: null pointer");
  int64_t grid = rows < 65536 ? rows : 65536;
  int8_row_encode_rows<<<dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, static_cast<hipStream_t>(stream)>>>(
      w, rows, cols, q, scale);
  return check_launch("int8_row_encode");
}
