// The memory-bound "segments" between the FLUX block linears, on gfx950.
//
// Restates the eager segments of selas/models/flux.py:164-200 (with the
// primitives _res 141-143, _ln 146-147, qk_rms 124-126, apply_rope 117-121,
// _heads 129-132): same fp32 math, one kernel per segment, every tensor read
// and written once.
//
// Row kernels (LayerNorm-based) use one 256-thread workgroup per token row:
// the row stays in registers between the mean pass, the variance pass and the
// output pass (two-pass statistics in fp32), and the cross-wave sums are
// combined in a fixed order. Attention prep gives each thread 8 consecutive
// channels of q, k and v (16-byte accesses); the Dh/8 threads of a head are
// adjacent lanes, so the RMS sum is a short cross-lane reduction and the
// interleaved RoPE pairs stay in-thread (other head sizes and alignments: one
// wavefront per (token, head), lane i owning the pair (2i, 2i+1)).
#include "common.h"

namespace selas {
namespace {

constexpr int kRowThreads = 256;
constexpr int kMaxVec = 4;  // float4 groups per thread: D <= 256 * 4 * 4 = 4096
constexpr float kFp16Max = 65504.0f;
constexpr float kLnEps = 1e-6f;
constexpr float kRmsEps = 1e-6f;

// Sum over the 256 threads of a workgroup, combined in wave order. Each call
// site passes its own 4-float slot, so one barrier suffices.
__device__ __forceinline__ float block_sum(float v, float *slot) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((slot[0] + slot[1]) + slot[2]) + slot[3];
}

__device__ __forceinline__ float clamp_guard(float v) {
  return v < -kFp16Max ? -kFp16Max : (v > kFp16Max ? kFp16Max : v);  // NaN passes through
}

// Loads 4 consecutive elements (d multiple of 4) of a 16/32-bit float row.
template <int DT>
__device__ __forceinline__ float4 load4(const void *p, int64_t i) {
  if constexpr (DT == SELAS_F32) return *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
  const uint2 u = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(p) + i);
  if constexpr (DT == SELAS_BF16)
    return make_float4(bf16_bits_to_f32(u.x & 0xffffu), bf16_bits_to_f32(u.x >> 16), bf16_bits_to_f32(u.y & 0xffffu),
                       bf16_bits_to_f32(u.y >> 16));
  return make_float4(f16_bits_to_f32(u.x & 0xffffu), f16_bits_to_f32(u.x >> 16), f16_bits_to_f32(u.y & 0xffffu),
                     f16_bits_to_f32(u.y >> 16));
}

template <int DT>
__device__ __forceinline__ void store4(void *p, int64_t i, float4 v) {
  if constexpr (DT == SELAS_F32) {
    *reinterpret_cast<float4 *>(static_cast<float *>(p) + i) = v;
  } else {
    uint2 u;
    if constexpr (DT == SELAS_BF16) {
      u.x = bf16_bits_rne(v.x) | (static_cast<uint32_t>(bf16_bits_rne(v.y)) << 16);
      u.y = bf16_bits_rne(v.z) | (static_cast<uint32_t>(bf16_bits_rne(v.w)) << 16);
    } else {
      u.x = f16_bits_rne(v.x) | (static_cast<uint32_t>(f16_bits_rne(v.y)) << 16);
      u.y = f16_bits_rne(v.z) | (static_cast<uint32_t>(f16_bits_rne(v.w)) << 16);
    }
    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p) + i) = u;
  }
}

// LayerNorm (no affine, eps 1e-6) of a row held as float4 groups v[0..n) at
// columns 4*(tid + 256*j), then (. * (1 + scale) + shift) stored as OUT.
// CNV > 0: the row is exactly CNV groups per thread (D = 1024 * CNV), known at
// compile time (the same sums in the same order, without the bounds tests).
template <int OUT, int CNV>
__device__ __forceinline__ void ln_modulate_store(float4 (&v)[kMaxVec], int nvec, int D, const float *shift,
                                                  const float *scale, void *out, int64_t out_row, float *scratch) {
  const int tid = threadIdx.x;
  if constexpr (CNV > 0) {
    nvec = CNV;
    D = 4 * kRowThreads * CNV;
  }
  auto in_row = [&](int j) { return CNV > 0 ? j < CNV : (j < nvec && 4 * (tid + kRowThreads * j) < D); };
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j)
    if (in_row(j)) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float mean = block_sum(s, scratch) / static_cast<float>(D);
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j)
    if (in_row(j)) {
      const float a = v[j].x - mean, b = v[j].y - mean, c = v[j].z - mean, d = v[j].w - mean;
      q += (a * a + b * b) + (c * c + d * d);
    }
  const float var = block_sum(q, scratch + 4) / static_cast<float>(D);
  const float rstd = 1.0f / sqrtf(var + kLnEps);
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int d = 4 * (tid + kRowThreads * j);
    if (in_row(j)) {
      const float4 sc = *reinterpret_cast<const float4 *>(scale + d);
      const float4 sh = *reinterpret_cast<const float4 *>(shift + d);
      float4 o;
      o.x = ((v[j].x - mean) * rstd) * (1.0f + sc.x) + sh.x;
      o.y = ((v[j].y - mean) * rstd) * (1.0f + sc.y) + sh.y;
      o.z = ((v[j].z - mean) * rstd) * (1.0f + sc.z) + sh.z;
      o.w = ((v[j].w - mean) * rstd) * (1.0f + sc.w) + sh.w;
      store4<OUT>(out, out_row + d, o);
    }
  }
}

// ------------------------------------------------------------------ mod_in

template <int OUT, int CNV>
__global__ __launch_bounds__(kRowThreads) void mod_in_kernel(const float *__restrict__ x, int L, int D, int64_t x_sb,
                                                             int64_t x_sl, const float *__restrict__ shift,
                                                             const float *__restrict__ scale, int64_t mod_sb,
                                                             void *__restrict__ out) {
  __shared__ float scratch[8];  // two block sums
  const int row = blockIdx.x;
  const int b = row / L, l = row - b * L;
  const float *xr = x + b * x_sb + l * x_sl;
  const int nvec = CNV > 0 ? CNV : (D + 4 * kRowThreads - 1) / (4 * kRowThreads);
  float4 v[kMaxVec];
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int d = 4 * (threadIdx.x + kRowThreads * j);
    v[j] = (CNV > 0 ? j < CNV : (j < nvec && d < D)) ? *reinterpret_cast<const float4 *>(xr + d) : make_float4(0, 0, 0, 0);
  }
  ln_modulate_store<OUT, CNV>(v, nvec, D, shift + b * mod_sb, scale + b * mod_sb, out, static_cast<int64_t>(row) * D,
                         scratch);
}

// ------------------------------------------------------------------ gated_add (+ mod_in)

template <int YT, bool MOD, int OUT, int CNV>
__global__ __launch_bounds__(kRowThreads) void gated_add_kernel(
    const float *__restrict__ x, int L, int D, int64_t x_sb, int64_t x_sl, const float *__restrict__ g, int64_t g_sb,
    const void *__restrict__ y, int64_t y_sb, int64_t y_sl, int guard, const float *__restrict__ shift,
    const float *__restrict__ scale, int64_t mod_sb, float *__restrict__ x_out, void *__restrict__ h) {
  __shared__ float scratch[8];  // two block sums
  const int row = blockIdx.x;
  const int b = row / L, l = row - b * L;
  const float *xr = x + b * x_sb + l * x_sl;
  const float *gr = g + b * g_sb;
  const int64_t yoff = b * y_sb + l * y_sl;
  const int nvec = CNV > 0 ? CNV : (D + 4 * kRowThreads - 1) / (4 * kRowThreads);
  if constexpr (CNV > 0) D = 4 * kRowThreads * CNV;
  float4 v[kMaxVec];
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int d = 4 * (threadIdx.x + kRowThreads * j);
    if (CNV > 0 ? j < CNV : (j < nvec && d < D)) {
      const float4 xv = *reinterpret_cast<const float4 *>(xr + d);
      const float4 gv = *reinterpret_cast<const float4 *>(gr + d);
      float4 yv = load4<YT>(y, yoff + d);
      if (guard) {
        yv.x = clamp_guard(yv.x); yv.y = clamp_guard(yv.y);
        yv.z = clamp_guard(yv.z); yv.w = clamp_guard(yv.w);
      }
      v[j] = make_float4(xv.x + gv.x * yv.x, xv.y + gv.y * yv.y, xv.z + gv.z * yv.z, xv.w + gv.w * yv.w);
      *reinterpret_cast<float4 *>(x_out + static_cast<int64_t>(row) * D + d) = v[j];
    } else {
      v[j] = make_float4(0, 0, 0, 0);
    }
  }
  if constexpr (MOD)
    ln_modulate_store<OUT, CNV>(v, nvec, D, shift + b * mod_sb, scale + b * mod_sb, h, static_cast<int64_t>(row) * D,
                           scratch);
}

// ------------------------------------------------------------------ attention prep

struct HeadSrc {
  const uint16_t *qkv;  // 16-bit elements (bf16 or fp16)
  int64_t sb, sl;
  int L;
  const float *qs, *ks;
};

template <int DT>
__device__ __forceinline__ float2 load_pair(const uint16_t *p) {
  const uint32_t u = *reinterpret_cast<const uint32_t *>(p);
  if constexpr (DT == SELAS_BF16) return make_float2(bf16_bits_to_f32(u & 0xffffu), bf16_bits_to_f32(u >> 16));
  return make_float2(f16_bits_to_f32(u & 0xffffu), f16_bits_to_f32(u >> 16));
}

template <int DT>
__device__ __forceinline__ uint32_t pack_pair(float a, float b) {
  if constexpr (DT == SELAS_BF16) return bf16_bits_rne(a) | (static_cast<uint32_t>(bf16_bits_rne(b)) << 16);
  return f16_bits_rne(a) | (static_cast<uint32_t>(f16_bits_rne(b)) << 16);
}

// RMSNorm over the head (sum across the wave), learned scale, RoPE on the pair.
__device__ __forceinline__ float2 rms_rope(float2 x, bool active, int Dh, float s0, float s1, float cs, float sn) {
  const float ss = wave_sum(active ? x.x * x.x + x.y * x.y : 0.0f);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(Dh) + kRmsEps);
  const float a = (x.x * r) * s0, b = (x.y * r) * s1;
  return make_float2(a * cs - b * sn, a * sn + b * cs);
}

// One wave per (batch, joint row, head). Joint rows [0, L0) come from src0 and
// [L0, L0+L1) from src1 (text then image, as torch.cat((txt, img), dim=2)).
template <int DT>
__global__ __launch_bounds__(256) void qkv_prep_kernel(HeadSrc s0, HeadSrc s1, int B, int H, int Dh,
                                                       const float *__restrict__ cos, const float *__restrict__ sin,
                                                       uint16_t *__restrict__ q, uint16_t *__restrict__ k,
                                                       uint16_t *__restrict__ v) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int Lj = s0.L + s1.L;
  if (item >= static_cast<int64_t>(B) * Lj * H) return;
  const int hh = static_cast<int>(item % H);
  const int64_t bl = item / H;
  const int l = static_cast<int>(bl % Lj), b = static_cast<int>(bl / Lj);
  const bool first = l < s0.L;
  const HeadSrc &s = first ? s0 : s1;
  const int ls = first ? l : l - s0.L;
  const int HD = H * Dh;
  const uint16_t *base = s.qkv + b * s.sb + ls * s.sl + hh * Dh + 2 * lane;
  const bool active = 2 * lane < Dh;
  const int half = Dh >> 1;
  float2 xq = make_float2(0, 0), xk = make_float2(0, 0), xv = make_float2(0, 0);
  float cs = 1.0f, sn = 0.0f, q0 = 0, q1 = 0, k0 = 0, k1 = 0;
  if (active) {
    xq = load_pair<DT>(base);
    xk = load_pair<DT>(base + HD);
    xv = load_pair<DT>(base + 2 * HD);
    cs = cos[static_cast<int64_t>(l) * half + lane];
    sn = sin[static_cast<int64_t>(l) * half + lane];
    q0 = s.qs[2 * lane]; q1 = s.qs[2 * lane + 1];
    k0 = s.ks[2 * lane]; k1 = s.ks[2 * lane + 1];
  }
  const float2 oq = rms_rope(xq, active, Dh, q0, q1, cs, sn);
  const float2 ok = rms_rope(xk, active, Dh, k0, k1, cs, sn);
  if (active) {
    const int64_t o = ((static_cast<int64_t>(b) * H + hh) * Lj + l) * Dh + 2 * lane;
    *reinterpret_cast<uint32_t *>(q + o) = pack_pair<DT>(oq.x, oq.y);
    *reinterpret_cast<uint32_t *>(k + o) = pack_pair<DT>(ok.x, ok.y);
    *reinterpret_cast<uint32_t *>(v + o) = *reinterpret_cast<const uint32_t *>(base + 2 * HD);
  }
  (void)xv;
}

// Attention prep, 8 channels per thread. Thread t of a (batch, joint row)
// takes channels [8*(t % LPH), +8) of head t / LPH (LPH = Dh / 8 adjacent
// lanes per head, so a head never straddles a wave); rows follow each other
// in thread order, so every access is a 16-byte vector.
template <int DT, int LPH>
__global__ __launch_bounds__(256) void qkv_prep_vec_kernel(HeadSrc s0, HeadSrc s1, int B, int H,
                                                           const float *__restrict__ cos,
                                                           const float *__restrict__ sin, uint16_t *__restrict__ q,
                                                           uint16_t *__restrict__ k, uint16_t *__restrict__ v) {
  constexpr int Dh = 8 * LPH, half = Dh / 2;
  const int Lj = s0.L + s1.L, per_row = H * LPH, HD = H * Dh;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const bool live = item < static_cast<int64_t>(B) * Lj * per_row;
  const int64_t bl = live ? item / per_row : 0;
  const int t = static_cast<int>(item - bl * per_row);
  const int hh = live ? t / LPH : 0, part = t % LPH;
  const int l = static_cast<int>(bl % Lj), b = static_cast<int>(bl / Lj);
  const bool first = l < s0.L;
  const HeadSrc &s = first ? s0 : s1;
  const int ls = first ? l : l - s0.L;
  const int d0 = 8 * part;
  float xq[8] = {}, xk[8] = {}, cs[4] = {1, 1, 1, 1}, sn[4] = {}, qs[8] = {}, ks[8] = {};
  uint4 vv = make_uint4(0, 0, 0, 0);
  if (live) {
    const uint16_t *base = s.qkv + b * s.sb + ls * s.sl + hh * Dh + d0;
    const uint4 uq = *reinterpret_cast<const uint4 *>(base), uk = *reinterpret_cast<const uint4 *>(base + HD);
    vv = *reinterpret_cast<const uint4 *>(base + 2 * HD);
    const uint32_t wq[4] = {uq.x, uq.y, uq.z, uq.w}, wk[4] = {uk.x, uk.y, uk.z, uk.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 a = load_pair<DT>(reinterpret_cast<const uint16_t *>(&wq[i]));
      const float2 c = load_pair<DT>(reinterpret_cast<const uint16_t *>(&wk[i]));
      xq[2 * i] = a.x; xq[2 * i + 1] = a.y; xk[2 * i] = c.x; xk[2 * i + 1] = c.y;
    }
    const float4 c4 = *reinterpret_cast<const float4 *>(cos + static_cast<int64_t>(l) * half + 4 * part);
    const float4 s4 = *reinterpret_cast<const float4 *>(sin + static_cast<int64_t>(l) * half + 4 * part);
    cs[0] = c4.x; cs[1] = c4.y; cs[2] = c4.z; cs[3] = c4.w;
    sn[0] = s4.x; sn[1] = s4.y; sn[2] = s4.z; sn[3] = s4.w;
    const float4 q0 = *reinterpret_cast<const float4 *>(s.qs + d0), q1 = *reinterpret_cast<const float4 *>(s.qs + d0 + 4);
    const float4 k0 = *reinterpret_cast<const float4 *>(s.ks + d0), k1 = *reinterpret_cast<const float4 *>(s.ks + d0 + 4);
    qs[0] = q0.x; qs[1] = q0.y; qs[2] = q0.z; qs[3] = q0.w; qs[4] = q1.x; qs[5] = q1.y; qs[6] = q1.z; qs[7] = q1.w;
    ks[0] = k0.x; ks[1] = k0.y; ks[2] = k0.z; ks[3] = k0.w; ks[4] = k1.x; ks[5] = k1.y; ks[6] = k1.z; ks[7] = k1.w;
  }
  // RMS over the head: this thread's 8 squares, then the LPH adjacent lanes (every lane takes part).
  float sq = 0.0f, sk = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    sq += xq[i] * xq[i];
    sk += xk[i] * xk[i];
  }
#pragma unroll
  for (int o = 1; o < LPH; o <<= 1) {
    sq += __shfl_xor(sq, o, 64);
    sk += __shfl_xor(sk, o, 64);
  }
  if (!live) return;
  const float rq = 1.0f / sqrtf(sq / static_cast<float>(Dh) + kRmsEps);
  const float rk = 1.0f / sqrtf(sk / static_cast<float>(Dh) + kRmsEps);
  uint32_t oq[4], ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = (xq[2 * i] * rq) * qs[2 * i], bq = (xq[2 * i + 1] * rq) * qs[2 * i + 1];
    oq[i] = pack_pair<DT>(a * cs[i] - bq * sn[i], a * sn[i] + bq * cs[i]);
    const float c = (xk[2 * i] * rk) * ks[2 * i], bk = (xk[2 * i + 1] * rk) * ks[2 * i + 1];
    ok[i] = pack_pair<DT>(c * cs[i] - bk * sn[i], c * sn[i] + bk * cs[i]);
  }
  const int64_t o = ((static_cast<int64_t>(b) * H + hh) * Lj + l) * Dh + d0;
  *reinterpret_cast<uint4 *>(q + o) = make_uint4(oq[0], oq[1], oq[2], oq[3]);
  *reinterpret_cast<uint4 *>(k + o) = make_uint4(ok[0], ok[1], ok[2], ok[3]);
  *reinterpret_cast<uint4 *>(v + o) = vv;
}

// ------------------------------------------------------------------ GELU / concat

__device__ __forceinline__ float gelu_tanh(float x) {
  const float kBeta = 0.7978845608028654f;  // sqrt(2 / pi)
  const float kKappa = 0.044715f;
  const float inner = kBeta * (x + kKappa * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}


// out[r, 0:Da] = a[r, :] and out[r, Da:Da+Dm] = gelu(m[r, :]); Da may be 0.
// Eight 16-bit elements per thread when every row is 16-byte aligned.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void concat_gelu_kernel(const uint16_t *__restrict__ a, int64_t lda, int Da,
                                                          const uint16_t *__restrict__ m, int64_t ldm, int Dm,
                                                          int64_t rows, uint16_t *__restrict__ out) {
  const int W = Da + Dm;
  constexpr int E = VEC ? 8 : 1;
  const int per_row = W / E;
  const int64_t total = rows * per_row;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / per_row;
    const int col = static_cast<int>(i - r * per_row) * E;
    uint16_t *dst = out + r * W + col;
    if (col < Da) {
      if constexpr (VEC) *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(a + r * lda + col);
      else *dst = a[r * lda + col];
    } else {
      const uint16_t *src = m + r * ldm + (col - Da);
      if constexpr (VEC) {
        const uint4 u = *reinterpret_cast<const uint4 *>(src);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        uint32_t o[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float lo, hi;
          if constexpr (DT == SELAS_BF16) { lo = bf16_bits_to_f32(w[t] & 0xffffu); hi = bf16_bits_to_f32(w[t] >> 16); }
          else { lo = f16_bits_to_f32(w[t] & 0xffffu); hi = f16_bits_to_f32(w[t] >> 16); }
          if constexpr (DT == SELAS_BF16) o[t] = gelu_bf16x2(lo, hi);
          else o[t] = pack_pair<DT>(gelu_tanh_fast(lo), gelu_tanh_fast(hi));
        }
        *reinterpret_cast<uint4 *>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
        float xv;
        if constexpr (DT == SELAS_BF16) xv = bf16_bits_to_f32(*src);
        else xv = f16_bits_to_f32(*src);
        if constexpr (DT == SELAS_BF16) *dst = static_cast<uint16_t>(gelu_bf16x2(xv, 0.0f) & 0xffffu);
        else *dst = f16_bits_rne(gelu_tanh_fast(xv));
      }
    }
  }
}

// fp32 GELU (the reference also applies the segment in fp32 compute dtype).
__global__ __launch_bounds__(256) void gelu_f32_kernel(const float *__restrict__ m, int64_t ldm, int Dm, int64_t rows,
                                                       float *__restrict__ out) {
  const int64_t total = rows * Dm;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / Dm;
    const int col = static_cast<int>(i - r * Dm);
    out[i] = gelu_tanh(m[r * ldm + col]);
  }
}

// ------------------------------------------------------------------ host helpers

bool row_ok(int64_t D, const void *p, int64_t sb, int64_t sl) {
  return D % 4 == 0 && aligned(p, 16) && sb % 4 == 0 && sl % 4 == 0;
}

int check_rows(const char *what, int64_t B, int64_t L, int64_t D) {
  if (B < 0 || L < 0 || D <= 0) return set_error(SELAS_EINVAL, "%s: bad shape B=%lld L=%lld D=%lld", what,
                                                 (long long)B, (long long)L, (long long)D);
  if (D > 4 * kRowThreads * kMaxVec || D % 4)
    return set_error(SELAS_EUNSUPPORTED, "%s: row kernels take D %% 4 == 0 and D <= %d (D=%lld)", what,
                     4 * kRowThreads * kMaxVec, (long long)D);
  if (B * L >= (1ll << 31)) return set_error(SELAS_EUNSUPPORTED, "%s: too many rows", what);
  return SELAS_OK;
}

uint32_t grid_for(int64_t work, int64_t per_block) {
  int64_t g = cdiv(work, per_block);
  if (g > (1 << 20)) g = 1 << 20;
  if (g < 1) g = 1;
  return static_cast<uint32_t>(g);
}

}  // namespace
}  // namespace selas

using namespace selas;

extern "C" int selas_mod_in(const float *x, int64_t B, int64_t L, int64_t D, int64_t x_sb, int64_t x_sl,
                            const float *shift, const float *scale, int64_t mod_sb, void *out, int out_dtype,
                            void *stream) {
  if (int e = check_rows("mod_in", B, L, D)) return e;
  if (!valid_dtype(out_dtype)) return set_error(SELAS_EINVAL, "mod_in: bad dtype %d", out_dtype);
  if (B * L == 0) return ok();
  if (!x || !shift || !scale || !out) return set_error(SELAS_EINVAL, "mod_in: null pointer");
  if (!row_ok(D, x, x_sb, x_sl) || !row_ok(D, shift, mod_sb, 0) || !row_ok(D, scale, mod_sb, 0) || !aligned(out, 8))
    return set_error(SELAS_EUNSUPPORTED, "mod_in: rows must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(B * L)), blk(kRowThreads);
  const int Li = static_cast<int>(L), Di = static_cast<int>(D);
  // The FLUX width (3072) has its own instantiation: three groups of 4 per thread, no bounds tests.
#define SELAS_MI(OT, CNV) mod_in_kernel<OT, CNV><<<grid, blk, 0, s>>>(x, Li, Di, x_sb, x_sl, shift, scale, mod_sb, out)
  if (D == 3072) {
    switch (out_dtype) {
      case SELAS_F32: SELAS_MI(SELAS_F32, 3); break;
      case SELAS_F16: SELAS_MI(SELAS_F16, 3); break;
      default: SELAS_MI(SELAS_BF16, 3);
    }
  } else {
    switch (out_dtype) {
      case SELAS_F32: SELAS_MI(SELAS_F32, 0); break;
      case SELAS_F16: SELAS_MI(SELAS_F16, 0); break;
      default: SELAS_MI(SELAS_BF16, 0);
    }
  }
#undef SELAS_MI
  return check_launch("mod_in");
}

namespace {
template <bool MOD>
int gated_add_impl(const char *what, const float *x, int64_t B, int64_t L, int64_t D, int64_t x_sb, int64_t x_sl,
                   const float *g, int64_t g_sb, const void *y, int y_dtype, int64_t y_sb, int64_t y_sl, int guard,
                   const float *shift, const float *scale, int64_t mod_sb, float *x_out, void *h, int h_dtype,
                   hipStream_t s) {
  if (int e = check_rows(what, B, L, D)) return e;
  if (!valid_dtype(y_dtype) || (MOD && !valid_dtype(h_dtype))) return set_error(SELAS_EINVAL, "%s: bad dtype", what);
  if (B * L == 0) return ok();
  if (!x || !g || !y || !x_out || (MOD && (!shift || !scale || !h))) return set_error(SELAS_EINVAL, "%s: null pointer", what);
  const int64_t ya = y_dtype == SELAS_F32 ? 16 : 8;
  if (!row_ok(D, x, x_sb, x_sl) || !row_ok(D, g, g_sb, 0) || !aligned(y, ya) || y_sb % 4 || y_sl % 4 ||
      !aligned(x_out, 16) || (MOD && (!row_ok(D, shift, mod_sb, 0) || !row_ok(D, scale, mod_sb, 0) || !aligned(h, 8))))
    return set_error(SELAS_EUNSUPPORTED, "%s: rows must be 16-byte aligned", what);
  const dim3 grid(static_cast<uint32_t>(B * L)), blk(kRowThreads);
  const int Li = static_cast<int>(L), Di = static_cast<int>(D);
#define SELAS_GA(YT, OT)                                                                                              \
  if (D == 3072)                                                                                                      \
    gated_add_kernel<YT, MOD, OT, 3><<<grid, blk, 0, s>>>(x, Li, Di, x_sb, x_sl, g, g_sb, y, y_sb, y_sl, guard, shift, \
                                                         scale, mod_sb, x_out, h);                                     \
  else                                                                                                                \
    gated_add_kernel<YT, MOD, OT, 0><<<grid, blk, 0, s>>>(x, Li, Di, x_sb, x_sl, g, g_sb, y, y_sb, y_sl, guard, shift, \
                                                         scale, mod_sb, x_out, h)
#define SELAS_GA_Y(YT)                                  \
  switch (MOD ? h_dtype : SELAS_F32) {                  \
    case SELAS_F32: SELAS_GA(YT, SELAS_F32); break;     \
    case SELAS_F16: SELAS_GA(YT, SELAS_F16); break;     \
    default: SELAS_GA(YT, SELAS_BF16);                  \
  }
  switch (y_dtype) {
    case SELAS_F32: SELAS_GA_Y(SELAS_F32); break;
    case SELAS_F16: SELAS_GA_Y(SELAS_F16); break;
    default: SELAS_GA_Y(SELAS_BF16);
  }
#undef SELAS_GA_Y
#undef SELAS_GA
  return check_launch(what);
}
}  // namespace

extern "C" int selas_gated_add(const float *x, int64_t B, int64_t L, int64_t D, int64_t x_sb, int64_t x_sl,
                               const float *g, int64_t g_sb, const void *y, int y_dtype, int64_t y_sb, int64_t y_sl,
                               int guard, float *out, void *stream) {
  return gated_add_impl<false>("gated_add", x, B, L, D, x_sb, x_sl, g, g_sb, y, y_dtype, y_sb, y_sl, guard, nullptr,
                               nullptr, 0, out, nullptr, SELAS_F32, static_cast<hipStream_t>(stream));
}

extern "C" int selas_gated_add_mod(const float *x, int64_t B, int64_t L, int64_t D, int64_t x_sb, int64_t x_sl,
                                   const float *g, int64_t g_sb, const void *y, int y_dtype, int64_t y_sb,
                                   int64_t y_sl, int guard, const float *shift, const float *scale, int64_t mod_sb,
                                   float *x_out, void *h, int h_dtype, void *stream) {
  return gated_add_impl<true>("gated_add_mod", x, B, L, D, x_sb, x_sl, g, g_sb, y, y_dtype, y_sb, y_sl, guard, shift,
                              scale, mod_sb, x_out, h, h_dtype, static_cast<hipStream_t>(stream));
}

namespace {
int qkv_launch(const char *what, HeadSrc s0, HeadSrc s1, int64_t B, int64_t H, int64_t Dh, const float *cos,
               const float *sin, void *q, void *k, void *v, int dtype, hipStream_t st) {
  if (B < 0 || H <= 0 || Dh <= 0 || s0.L < 0 || s1.L < 0) return set_error(SELAS_EINVAL, "%s: bad shape", what);
  if (dtype != SELAS_BF16 && dtype != SELAS_F16)
    return set_error(SELAS_EUNSUPPORTED, "%s: takes bf16 or fp16 qkv, got %s", what, dtype_name(dtype));
  if (Dh % 2 || Dh > 128) return set_error(SELAS_EUNSUPPORTED, "%s: head_dim must be even and <= 128 (%lld)", what,
                                           (long long)Dh);
  const int64_t items = B * (s0.L + s1.L) * H;
  if (items == 0) return ok();
  if (!q || !k || !v || !cos || !sin) return set_error(SELAS_EINVAL, "%s: null pointer", what);
  for (const HeadSrc *s : {&s0, &s1})
    if (s->L > 0 && (!s->qkv || !s->qs || !s->ks || !aligned(s->qkv, 4) || s->sb % 2 || s->sl % 2))
      return set_error(SELAS_EUNSUPPORTED, "%s: qkv rows must be 4-byte aligned", what);
  if (!aligned(q, 4) || !aligned(k, 4) || !aligned(v, 4)) return set_error(SELAS_EUNSUPPORTED, "%s: misaligned output", what);
  if (items / 4 >= (1ll << 31)) return set_error(SELAS_EUNSUPPORTED, "%s: too many rows", what);
  uint16_t *qo = static_cast<uint16_t *>(q), *ko = static_cast<uint16_t *>(k), *vo = static_cast<uint16_t *>(v);
  // 16-byte path: Dh in {16, 32, 64, 128}, every row and output 16-byte aligned.
  bool vec = (Dh == 16 || Dh == 32 || Dh == 64 || Dh == 128) && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) &&
             aligned(cos, 16) && aligned(sin, 16) && (H * Dh) % 8 == 0 && items * (Dh / 8) < (1ll << 31);
  for (const HeadSrc *s : {&s0, &s1})
    if (s->L > 0) vec = vec && aligned(s->qkv, 16) && s->sb % 8 == 0 && s->sl % 8 == 0 && aligned(s->qs, 16) &&
                        aligned(s->ks, 16);
  if (vec) {
    const dim3 vgrid(static_cast<uint32_t>(cdiv(items * (Dh / 8), 256))), vblk(256);
#define SELAS_QV(DT, LPH) \
  qkv_prep_vec_kernel<DT, LPH><<<vgrid, vblk, 0, st>>>(s0, s1, (int)B, (int)H, cos, sin, qo, ko, vo)
#define SELAS_QV_DT(DT)                   \
  switch (Dh) {                           \
    case 16: SELAS_QV(DT, 2); break;      \
    case 32: SELAS_QV(DT, 4); break;      \
    case 64: SELAS_QV(DT, 8); break;      \
    default: SELAS_QV(DT, 16);            \
  }
    if (dtype == SELAS_BF16) { SELAS_QV_DT(SELAS_BF16) } else { SELAS_QV_DT(SELAS_F16) }
#undef SELAS_QV_DT
#undef SELAS_QV
    return check_launch(what);
  }
  const dim3 grid(static_cast<uint32_t>(cdiv(items, 4))), blk(256);
  if (dtype == SELAS_BF16)
    qkv_prep_kernel<SELAS_BF16><<<grid, blk, 0, st>>>(s0, s1, (int)B, (int)H, (int)Dh, cos, sin, qo, ko, vo);
  else
    qkv_prep_kernel<SELAS_F16><<<grid, blk, 0, st>>>(s0, s1, (int)B, (int)H, (int)Dh, cos, sin, qo, ko, vo);
  return check_launch(what);
}
}  // namespace

extern "C" int selas_qkv_single(const void *qkv, int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t qkv_sb,
                                int64_t qkv_sl, const float *q_scale, const float *k_scale, const float *cos,
                                const float *sin, void *q, void *k, void *v, int dtype, void *stream) {
  if (L < 0 || L >= (1ll << 30)) return set_error(SELAS_EINVAL, "qkv_single: bad L");
  HeadSrc s0{static_cast<const uint16_t *>(qkv), qkv_sb, qkv_sl, static_cast<int>(L), q_scale, k_scale};
  HeadSrc s1{nullptr, 0, 0, 0, nullptr, nullptr};
  return qkv_launch("qkv_single", s0, s1, B, H, Dh, cos, sin, q, k, v, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int selas_qkv_double(const void *tqkv, int64_t t_sb, int64_t t_sl, int64_t Lt, const void *iqkv,
                                int64_t i_sb, int64_t i_sl, int64_t Li, int64_t B, int64_t H, int64_t Dh,
                                const float *tq_scale, const float *tk_scale, const float *iq_scale,
                                const float *ik_scale, const float *cos, const float *sin, void *q, void *k, void *v,
                                int dtype, void *stream) {
  if (Lt < 0 || Li < 0 || Lt + Li >= (1ll << 30)) return set_error(SELAS_EINVAL, "qkv_double: bad L");
  HeadSrc s0{static_cast<const uint16_t *>(tqkv), t_sb, t_sl, static_cast<int>(Lt), tq_scale, tk_scale};
  HeadSrc s1{static_cast<const uint16_t *>(iqkv), i_sb, i_sl, static_cast<int>(Li), iq_scale, ik_scale};
  return qkv_launch("qkv_double", s0, s1, B, H, Dh, cos, sin, q, k, v, dtype, static_cast<hipStream_t>(stream));
}

namespace {
int concat_gelu(const char *what, const void *a, int64_t lda, int64_t Da, const void *m, int64_t ldm, int64_t Dm,
                int64_t rows, void *out, int dtype, hipStream_t st) {
  if (rows < 0 || Da < 0 || Dm < 0 || lda < Da || ldm < Dm) return set_error(SELAS_EINVAL, "%s: bad shape", what);
  if (!valid_dtype(dtype)) return set_error(SELAS_EINVAL, "%s: bad dtype %d", what, dtype);
  if (rows == 0 || Da + Dm == 0) return ok();
  if (!out || (Da && !a) || (Dm && !m)) return set_error(SELAS_EINVAL, "%s: null pointer", what);
  if (Da + Dm >= (1ll << 31)) return set_error(SELAS_EUNSUPPORTED, "%s: rows too wide", what);
  if (dtype == SELAS_F32) {
    if (Da) return set_error(SELAS_EUNSUPPORTED, "%s: concat takes 16-bit tensors", what);
    gelu_f32_kernel<<<dim3(grid_for(rows * Dm, 256 * 8)), dim3(256), 0, st>>>(
        static_cast<const float *>(m), ldm, static_cast<int>(Dm), rows, static_cast<float *>(out));
    return check_launch(what);
  }
  const bool vec = Da % 8 == 0 && Dm % 8 == 0 && lda % 8 == 0 && ldm % 8 == 0 && (!Da || aligned(a, 16)) &&
                   (!Dm || aligned(m, 16)) && aligned(out, 16);
  const uint16_t *ap = static_cast<const uint16_t *>(a), *mp = static_cast<const uint16_t *>(m);
  uint16_t *op = static_cast<uint16_t *>(out);
  const int64_t per = (Da + Dm) / (vec ? 8 : 1);
  const dim3 grid(grid_for(rows * per, 256 * 4)), blk(256);
  const int da = static_cast<int>(Da), dm = static_cast<int>(Dm);
  if (dtype == SELAS_BF16) {
    if (vec) concat_gelu_kernel<SELAS_BF16, true><<<grid, blk, 0, st>>>(ap, lda, da, mp, ldm, dm, rows, op);
    else concat_gelu_kernel<SELAS_BF16, false><<<grid, blk, 0, st>>>(ap, lda, da, mp, ldm, dm, rows, op);
  } else {
    if (vec) concat_gelu_kernel<SELAS_F16, true><<<grid, blk, 0, st>>>(ap, lda, da, mp, ldm, dm, rows, op);
    else concat_gelu_kernel<SELAS_F16, false><<<grid, blk, 0, st>>>(ap, lda, da, mp, ldm, dm, rows, op);
  }
  return check_launch(what);
}
}  // namespace

extern "C" int selas_gelu(const void *h, int64_t rows, int64_t cols, int64_t ld, void *out, int dtype, void *stream) {
  return concat_gelu("gelu", nullptr, 0, 0, h, ld, cols, rows, out, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int selas_attn_mlp(const void *attn, int64_t rows, int64_t Da, int64_t lda, const void *mlp, int64_t Dm,
                              int64_t ldm, void *out, int dtype, void *stream) {
  if (dtype == SELAS_F32) return set_error(SELAS_EUNSUPPORTED, "attn_mlp: takes 16-bit tensors");
  return concat_gelu("attn_mlp", attn, lda, Da, mlp, ldm, Dm, rows, out, dtype, static_cast<hipStream_t>(stream));
}
