// NF4 codec on gfx950: decode (bit-exact with the reference decode) and encode.
//
// Decode restates selas/codecs.py:178-199 (nf4_dequant_torch) and :207-228
// (the Triton kernel): value = code[nibble] * absmax[block] in fp32, rounded
// once to the output type. Encode restates selas/codecs.py:99-119.
#include "common.h"

namespace selas {
namespace {

constexpr int kThreads = 256;

// --------------------------------------------------------------------------- decode

// Vector path: each thread decodes 16 packed bytes (32 values) that lie in one
// absmax block (blocksize % 32 == 0), reading 16 B and writing 64 B (bf16/fp16)
// or 128 B (fp32) with 16-byte accesses.
template <int DT>
__global__ __launch_bounds__(kThreads) void nf4_dequant_vec16(const uint4 *__restrict__ packed,
                                                              const float *__restrict__ absmax, int64_t n16,
                                                              int64_t chunks_per_block, Code16 code,
                                                              void *__restrict__ out) {
  __shared__ float s_code[16];
  if (threadIdx.x < 16) s_code[threadIdx.x] = code.v[threadIdx.x];
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n16) return;
  const uint4 w = packed[i];
  const float a = absmax[i / chunks_per_block];
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  if constexpr (DT == SELAS_F32) {
    float4 *o = reinterpret_cast<float4 *>(out) + i * 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t d = words[q];
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t byte = (d >> (8 * j)) & 0xffu;
        v[2 * j] = s_code[byte >> 4] * a;
        v[2 * j + 1] = s_code[byte & 15u] * a;
      }
      o[2 * q] = make_float4(v[0], v[1], v[2], v[3]);
      o[2 * q + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  } else {
    uint4 *o = reinterpret_cast<uint4 *>(out) + i * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t d = words[q];
      uint32_t pr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t byte = (d >> (8 * j)) & 0xffu;
        const float hi = s_code[byte >> 4] * a;
        const float lo = s_code[byte & 15u] * a;
        if constexpr (DT == SELAS_BF16) pr[j] = bf16_bits_rne(hi) | (static_cast<uint32_t>(bf16_bits_rne(lo)) << 16);
        else pr[j] = f16_bits_rne(hi) | (static_cast<uint32_t>(f16_bits_rne(lo)) << 16);
      }
      o[q] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    }
  }
}

// Generic path: one byte per thread, any even blocksize and any alignment.
template <int DT>
__global__ __launch_bounds__(kThreads) void nf4_dequant_bytes(const uint8_t *__restrict__ packed,
                                                              const float *__restrict__ absmax, int64_t begin,
                                                              int64_t n_bytes, int64_t bytes_per_block, Code16 code,
                                                              void *__restrict__ out) {
  __shared__ float s_code[16];
  if (threadIdx.x < 16) s_code[threadIdx.x] = code.v[threadIdx.x];
  __syncthreads();
  const int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n_bytes) return;
  const uint32_t byte = packed[i];
  const float a = absmax[i / bytes_per_block];
  store_f<DT>(out, 2 * i, s_code[byte >> 4] * a);
  store_f<DT>(out, 2 * i + 1, s_code[byte & 15u] * a);
}

template <int DT>
int dequant_typed(const uint8_t *packed, const float *absmax, int64_t n_bytes, int64_t bpb, const Code16 &code,
                  void *out, hipStream_t stream) {
  int64_t done = 0;
  if (bpb % 16 == 0 && aligned(packed, 16) && aligned(out, 16) && n_bytes >= 16) {
    const int64_t n16 = n_bytes / 16;
    const int64_t grid = cdiv(n16, kThreads);
    nf4_dequant_vec16<DT><<<dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream>>>(
        reinterpret_cast<const uint4 *>(packed), absmax, n16, bpb / 16, code, out);
    done = n16 * 16;
  }
  if (done < n_bytes) {
    const int64_t grid = cdiv(n_bytes - done, kThreads);
    nf4_dequant_bytes<DT><<<dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream>>>(
        packed, absmax, done, n_bytes, bpb, code, out);
  }
  return check_launch("nf4_dequant");
}

// --------------------------------------------------------------------------- encode

struct Mids15 {
  float v[15];
};

// NaN-propagating max, as torch.amax.
__device__ __forceinline__ float max_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

// One wavefront per block: |w| max across the block, then each element's code
// index = number of midpoints m with !(m >= w / absmax) (torch.bucketize with
// right=False counts exactly these), packed two per byte, first element high.
__global__ __launch_bounds__(kThreads) void nf4_encode_waves(const float *__restrict__ w, int64_t nblocks,
                                                             int blocksize, Mids15 mids, uint8_t *__restrict__ packed,
                                                             float *__restrict__ absmax) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 6;
  const int64_t nwaves = (static_cast<int64_t>(gridDim.x) * kThreads) >> 6;
  for (int64_t b = wave; b < nblocks; b += nwaves) {
    const float *src = w + b * blocksize;
    float m = 0.0f;
    for (int j = lane; j < blocksize; j += 64) m = max_nan(m, fabsf(src[j]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max_nan(m, __shfl_xor(m, o, 64));
    const float safe = m > 0.0f ? m : 1.0f;
    for (int j0 = 0; j0 < blocksize; j0 += 64) {
      const int j = j0 + lane;
      uint32_t idx = 0;
      if (j < blocksize) {
        const float x = src[j] / safe;
#pragma unroll
        for (int t = 0; t < 15; ++t) idx += !(mids.v[t] >= x) ? 1u : 0u;
      }
      const uint32_t next = __shfl_down(idx, 1, 64);
      if (j < blocksize && (lane & 1) == 0) packed[(b * blocksize + j) >> 1] = static_cast<uint8_t>((idx << 4) | next);
    }
    if (lane == 0) absmax[b] = m;
  }
}

}  // namespace
}  // namespace selas

using namespace selas;

extern "C" int selas_nf4_dequant(const uint8_t *packed, const float *absmax, int64_t n_bytes, int64_t blocksize,
                                 const float code[16], void *out, int out_dtype, void *stream) {
  if (n_bytes < 0) return set_error(SELAS_EINVAL, "nf4_dequant: negative byte count %lld", (long long)n_bytes);
  if (blocksize <= 0 || blocksize % 2)
    return set_error(SELAS_EINVAL, "nf4_dequant: blocksize must be positive and even, got %lld", (long long)blocksize);
  if (!valid_dtype(out_dtype)) return set_error(SELAS_EINVAL, "nf4_dequant: bad output dtype %d", out_dtype);
  if (n_bytes == 0) return ok();
  if (!packed || !absmax || !out || !code) return set_error(SELAS_EINVAL, "nf4_dequant: null pointer");
  Code16 c;
  for (int i = 0; i < 16; ++i) c.v[i] = code[i];
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t bpb = blocksize / 2;
  switch (out_dtype) {
    case SELAS_F32: return dequant_typed<SELAS_F32>(packed, absmax, n_bytes, bpb, c, out, s);
    case SELAS_F16: return dequant_typed<SELAS_F16>(packed, absmax, n_bytes, bpb, c, out, s);
    default: return dequant_typed<SELAS_BF16>(packed, absmax, n_bytes, bpb, c, out, s);
  }
}

extern "C" int selas_nf4_encode(const float *w, int64_t n, int64_t blocksize, const float code[16], uint8_t *packed,
                                float *absmax, void *stream) {
  if (blocksize <= 0 || blocksize % 2 || blocksize > (1 << 20))
    return set_error(SELAS_EINVAL, "nf4_encode: blocksize must be positive and even, got %lld", (long long)blocksize);
  if (n < 0 || n % blocksize)
    return set_error(SELAS_EINVAL, "nf4 needs numel divisible by blocksize (%lld %% %lld)", (long long)n,
                     (long long)blocksize);
  if (n == 0) return ok();
  if (!w || !packed || !absmax || !code) return set_error(SELAS_EINVAL, "nf4_encode: null pointer");
  Mids15 mids;
  // Midpoints in fp32 exactly as (code[1:] + code[:-1]) / 2 evaluates them.
  for (int i = 0; i < 15; ++i) mids.v[i] = (code[i + 1] + code[i]) / 2.0f;
  const int64_t nblocks = n / blocksize;
  const int64_t waves_per_wg = kThreads / 64;
  int64_t grid = cdiv(nblocks, waves_per_wg);
  if (grid > 65536) grid = 65536;
  nf4_encode_waves<<<dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, static_cast<hipStream_t>(stream)>>>(
      w, nblocks, static_cast<int>(blocksize), mids, packed, absmax);
  return check_launch("nf4_encode");
}
