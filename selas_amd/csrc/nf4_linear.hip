// Quantized linear y = x W^T + b with W stored as NF4 (blocksize 64), on gfx950.
//
// Replaces UnitView.linear for NF4 weights (selas/store.py:289-293), which
// decodes the whole weight to a bf16 temporary (selas/codecs.py:269-280) and
// calls F.linear. Here the weight never exists in bf16 outside registers.
//
// Two kernels, chosen from M alone:
//   * M <= 32  (hoisted adaLN modulation linears, M = number of steps):
//     nf4_gemv_kernel, HBM-bound. Weight codes are looked up as bf16(code)
//     pairs from a bank-replicated LDS table (one LDS read per byte, no bank
//     conflicts), multiplied with x on MFMA per 64-element block, and the
//     block's fp32 absmax is applied to the fp32 block partial sum.
//   * M > 32 (block linears, M = tokens): nf4_gemm_kernel, MFMA-bound.
//     256x256 output tile per workgroup, 4 waves, each wave owns 64 output
//     columns for all 256 rows. x tiles are staged through LDS (double
//     buffered, XOR-swizzled 16-byte chunks); weight codes go straight from
//     HBM to registers and are decoded to the bit-exact reference operand
//     bf16(code[nibble] * absmax) with a per-block 16-entry product table and
//     v_perm_b32 byte lookups, then fed to v_mfma_f32_32x32x16_bf16.
//
// MFMA operand layout (32x32x16, wave64): lane l holds, for A, row l%32 and
// 8 k-values of half h = l/32; for B, column l%32 and the same 8 k-values of
// half h. Any assignment of actual k indices to (h, element) works as long as
// both operands use the same one: here half h of a 64-block covers k in
// [32h, 32h+32) and sub-step s covers k in [32h+8s, 32h+8s+8), so one 16-byte
// load of packed codes feeds a lane for a whole 64-block. The 32x32 fp32
// result has, in lane l, column l%32 and rows 8*(r/4) + 4*h + r%4, r = 0..15.
#include "common.h"

namespace selas {
namespace {

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// Raw buffer resource over `bytes` bytes (gfx9 descriptor word 3: 0x00020000).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}
__device__ __forceinline__ uint4 load_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float load_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// =========================================================================== GEMV (M <= 32)

constexpr int kGemvThreads = 256;
constexpr int kGemvGroups = 2;     // 32-column groups per workgroup
constexpr int kGemvRepl = 64;      // LDS table replicas (one per lane: conflict-free)

// Workgroup: 64 output columns, all M (<= 32) rows. The four waves split the
// K blocks round-robin (wave w takes blocks w, w+4, ...) and their fp32
// partial results are summed in LDS in wave order, so the result does not
// depend on scheduling.
__global__ __launch_bounds__(kGemvThreads) void nf4_gemv_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, int M, int K, const uint8_t *__restrict__ packed,
    const float *__restrict__ absmax, Code16 code, int N, const uint16_t *__restrict__ bias,
    uint16_t *__restrict__ y, int64_t ldy) {
  extern __shared__ uint32_t lds[];  // [256 byte values][kGemvRepl] bf16 pairs; later the reduction buffer
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;

  {  // byte b -> (bf16(code[b >> 4]) low, bf16(code[b & 15]) high), replicated per lane
    uint32_t cb[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) cb[i] = bf16_bits_rne(code.v[i]);
    for (int e = tid; e < 256 * kGemvRepl; e += kGemvThreads) {
      const int b = e / kGemvRepl;
      uint32_t hi = 0, lo = 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        hi = (b >> 4) == i ? cb[i] : hi;
        lo = (b & 15) == i ? cb[i] : lo;
      }
      lds[e] = hi | (lo << 16);
    }
  }
  __syncthreads();

  const int kblocks = K >> 6;
  const int n_base = blockIdx.x * (32 * kGemvGroups);
  const uint16_t *xr = x + static_cast<int64_t>(min(c, M - 1)) * ldx + 32 * h;
  const uint8_t *wr[kGemvGroups];
  const float *ar[kGemvGroups];
#pragma unroll
  for (int g = 0; g < kGemvGroups; ++g) {
    const int64_t n = min(n_base + 32 * g + c, N - 1);
    wr[g] = packed + n * (K >> 1) + 16 * h;
    ar[g] = absmax + n * kblocks;
  }
  const uint32_t lane_off = static_cast<uint32_t>(lane);

  f32x16 acc[kGemvGroups];
#pragma unroll
  for (int g = 0; g < kGemvGroups; ++g) acc[g] = f32x16{};

  for (int kb = wave; kb < kblocks; kb += 4) {
    uint4 wq[kGemvGroups];
    float a[kGemvGroups];
#pragma unroll
    for (int g = 0; g < kGemvGroups; ++g) {
      wq[g] = *reinterpret_cast<const uint4 *>(wr[g] + kb * 32);
      a[g] = ar[g][kb];
    }
    bf16x8 xf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) xf[s] = *reinterpret_cast<const bf16x8 *>(xr + kb * 64 + 8 * s);
#pragma unroll
    for (int g = 0; g < kGemvGroups; ++g) {
      const uint32_t words[4] = {wq[g].x, wq[g].y, wq[g].z, wq[g].w};
      f32x16 p = f32x16{};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t P = words[s];
        uint4 t;
        t.x = lds[((P & 0xffu) * kGemvRepl) + lane_off];
        t.y = lds[(((P >> 8) & 0xffu) * kGemvRepl) + lane_off];
        t.z = lds[(((P >> 16) & 0xffu) * kGemvRepl) + lane_off];
        t.w = lds[((P >> 24) * kGemvRepl) + lane_off];
        p = mfma32(xf[s], __builtin_bit_cast(bf16x8, t), p);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][r] += p[r] * a[g];
    }
  }

  __syncthreads();  // every wave is done with the table: reuse LDS for the reduction
  float *red = reinterpret_cast<float *>(lds);
  constexpr int kOut = kGemvGroups * 16 * 64;  // per wave: [g][r][lane]
#pragma unroll
  for (int g = 0; g < kGemvGroups; ++g)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave * kOut + (g * 16 + r) * 64 + lane] = acc[g][r];
  __syncthreads();
  for (int e = tid; e < kOut; e += kGemvThreads) {
    const float v = ((red[e] + red[kOut + e]) + red[2 * kOut + e]) + red[3 * kOut + e];
    const int l = e & 63, gr = e >> 6;
    const int g = gr >> 4, r = gr & 15;
    const int m = 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const int n = n_base + 32 * g + (l & 31);
    if (m < M && n < N) {
      const float b = bias ? bf16_bits_to_f32(bias[n]) : 0.0f;
      y[static_cast<int64_t>(m) * ldy + n] = bf16_bits_rne(v + b);
    }
  }
}

// =========================================================================== GEMM (M > 32)

constexpr int kBM = 256, kBN = 256;
constexpr int kGemmThreads = 256;
constexpr int kATileBytes = kBM * 128;  // 256 rows x 64 bf16

// 16 bf16(code[i] * a) values as four byte planes (TL = low bytes, TH = high
// bytes), entries 4j..4j+3 in plane register j. Lanes l and l+32 serve the
// same (row, block); each computes eight products and the halves are
// exchanged with v_permlane32_swap.
struct Tables {
  uint32_t lo[4], hi[4];
};

__device__ __forceinline__ Tables make_tables(const float (&cl)[8], float a) {
  uint32_t e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = pack_bf16x2(cl[2 * j] * a, cl[2 * j + 1] * a);
  const uint32_t la = perm(e[1], e[0], 0x06040200u), lb = perm(e[3], e[2], 0x06040200u);
  const uint32_t ha = perm(e[1], e[0], 0x07050301u), hb = perm(e[3], e[2], 0x07050301u);
  Tables t;
  // After the swap the first result holds lanes 0-31's value everywhere and the
  // second lanes 32-63's: entries 0-7 and 8-15 respectively.
  auto sla = __builtin_amdgcn_permlane32_swap(la, la, false, false);
  auto slb = __builtin_amdgcn_permlane32_swap(lb, lb, false, false);
  auto sha = __builtin_amdgcn_permlane32_swap(ha, ha, false, false);
  auto shb = __builtin_amdgcn_permlane32_swap(hb, hb, false, false);
  t.lo[0] = sla[0]; t.lo[2] = sla[1];
  t.lo[1] = slb[0]; t.lo[3] = slb[1];
  t.hi[0] = sha[0]; t.hi[2] = sha[1];
  t.hi[1] = shb[0]; t.hi[3] = shb[1];
  return t;
}

// Looks up 4 entries: `s7` holds the low three bits of four indices (one per
// byte), `m` is 0xFF in the bytes whose index is >= 8. Returns the bf16 pairs
// (index0, index1) and (index2, index3).
__device__ __forceinline__ void lookup4(const Tables &t, uint32_t s7, uint32_t m, uint32_t &p01, uint32_t &p23) {
  const uint32_t l0 = perm(t.lo[1], t.lo[0], s7), l1 = perm(t.lo[3], t.lo[2], s7);
  const uint32_t h0 = perm(t.hi[1], t.hi[0], s7), h1 = perm(t.hi[3], t.hi[2], s7);
  const uint32_t lo = (m & l1) | (~m & l0);
  const uint32_t hi = (m & h1) | (~m & h0);
  p01 = perm(hi, lo, 0x05010400u);
  p23 = perm(hi, lo, 0x07030602u);
}

// Eight codes of one packed dword (bytes B0..B3, element 2i = high nibble of
// Bi) -> bf16x8 operand in k order.
__device__ __forceinline__ bf16x8 dequant8(const Tables &t, uint32_t P) {
  const uint32_t H7 = (P >> 4) & 0x07070707u, L7 = P & 0x07070707u;
  const uint32_t sx = perm(H7, L7, 0x02060004u);  // elements 0,1,4,5
  const uint32_t sy = perm(H7, L7, 0x03070105u);  // elements 2,3,6,7
  // Bit 3 of each index sits at bit 7 of a byte of P or P<<4; v_perm selectors
  // 8..11 replicate bit 7 of bytes 1,3,5,7 of {S0,S1}.
  const uint32_t mx = perm(P << 12, P << 8, 0x0B090A08u);
  const uint32_t my = perm(P << 4, P, 0x0B090A08u);
  uint4 r;
  lookup4(t, sx, mx, r.x, r.z);
  lookup4(t, sy, my, r.y, r.w);
  return __builtin_bit_cast(bf16x8, r);
}

__global__ __launch_bounds__(kGemmThreads, 1) void nf4_gemm_kernel(
    const uint16_t *__restrict__ X, int64_t ldx, int M, int K, const uint8_t *__restrict__ packed,
    const float *__restrict__ absmax, Code16 code, int N, const uint16_t *__restrict__ bias,
    uint16_t *__restrict__ Y, int64_t ldy, int tiles_m) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kATileBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;
  const int tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int kblocks = K >> 6;
  const uint32_t ldx_b = static_cast<uint32_t>(ldx) * 2u;

  // Buffer resources: loads past the end of a tensor return zeros, so rows
  // beyond M or N need no clamping (their results are never stored).
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(X, static_cast<uint32_t>(M) * ldx_b);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(packed, static_cast<uint32_t>(N) * static_cast<uint32_t>(K >> 1));
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(absmax, static_cast<uint32_t>(N) * static_cast<uint32_t>(kblocks) * 4u);

  // x tile loader: thread handles rows (tid>>3) + 32j of the tile, 16-byte chunk tid&7,
  // stored XOR-swizzled so that the fragment reads below are bank-conflict free.
  // The hardware range check covers the per-lane offset only, so the row term
  // lives there: rows >= M are out of range and read as zeros.
  const int a_row0 = tid >> 3, a_chunk = tid & 7;
  const uint32_t a_voff = static_cast<uint32_t>(m0 + a_row0) * ldx_b + a_chunk * 16u;
  const uint32_t a_wr = a_row0 * 128 + ((a_chunk ^ (a_row0 & 7)) << 4);
  const uint32_t a_jstride = 32u * ldx_b;
  // Weight rows of this wave: n0 + 64*wave + 32*cb + c.
  uint32_t b_voff[2], s_voff[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const uint32_t n = static_cast<uint32_t>(n0 + 64 * wave + 32 * cb + c);
    b_voff[cb] = n * static_cast<uint32_t>(K >> 1) + 16u * h;
    s_voff[cb] = n * static_cast<uint32_t>(kblocks) * 4u;
  }
  float cl[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cl[i] = h ? code.v[8 + i] : code.v[i];
  // LDS offset of the x fragment for sub-step s (row c of each 32-row slab mb,
  // slab mb adds mb*4096).
  uint32_t a_rd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) a_rd[s] = c * 128 + (((4 * h + s) ^ (c & 7)) << 4);

  f32x16 acc[8][2];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) acc[mb][cb] = f32x16{};

  uint4 areg[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) areg[j] = load_b128(xr, a_voff + j * a_jstride, 0);
#pragma unroll
  for (int j = 0; j < 8; ++j) *reinterpret_cast<uint4 *>(smem + a_wr + j * 4096) = areg[j];
  uint4 bq[2];
  float bs[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    bq[cb] = load_b128(wr, b_voff[cb], 0);
    bs[cb] = load_f32(sr, s_voff[cb], 0);
  }
  __syncthreads();

  for (int kb = 0; kb < kblocks; ++kb) {
    const uint32_t buf = (kb & 1) * kATileBytes;
    const bool more = kb + 1 < kblocks;
    uint4 bq_next[2];
    float bs_next[2];
    if (more) {
      const uint32_t ka = (kb + 1) * 128u;
#pragma unroll
      for (int j = 0; j < 8; ++j) areg[j] = load_b128(xr, a_voff + j * a_jstride, ka);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        bq_next[cb] = load_b128(wr, b_voff[cb], (kb + 1) * 32u);
        bs_next[cb] = load_f32(sr, s_voff[cb], (kb + 1) * 4u);
      }
    }
    Tables tab[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) tab[cb] = make_tables(cl, bs[cb]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 wf[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const uint32_t P = s == 0 ? bq[cb].x : s == 1 ? bq[cb].y : s == 2 ? bq[cb].z : bq[cb].w;
        wf[cb] = dequant8(tab[cb], P);
      }
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const bf16x8 xf = *reinterpret_cast<const bf16x8 *>(smem + buf + a_rd[s] + mb * 4096);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[mb][cb] = mfma32(wf[cb], xf, acc[mb][cb]);
      }
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < 8; ++j) *reinterpret_cast<uint4 *>(smem + (kATileBytes - buf) + a_wr + j * 4096) = areg[j];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        bq[cb] = bq_next[cb];
        bs[cb] = bs_next[cb];
      }
    }
    __syncthreads();
  }

  // Epilogue: acc[mb][cb] holds D[n][m] for n = n0 + 64*wave + 32*cb + 8*(r/4) + 4*h + r%4
  // and m = m0 + 32*mb + c; four consecutive n per r/4 are stored as one 8-byte write.
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + 64 * wave + 32 * cb + 8 * q + 4 * h;
      float bv[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) bv[t] = (bias && n + t < N) ? bf16_bits_to_f32(bias[n + t]) : 0.0f;
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const int m = m0 + 32 * mb + c;
        if (m >= M) continue;
        uint16_t *dst = Y + static_cast<int64_t>(m) * ldy + n;
        const float v0 = acc[mb][cb][4 * q] + bv[0], v1 = acc[mb][cb][4 * q + 1] + bv[1];
        const float v2 = acc[mb][cb][4 * q + 2] + bv[2], v3 = acc[mb][cb][4 * q + 3] + bv[3];
        if (n + 3 < N) {
          *reinterpret_cast<uint2 *>(dst) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
        } else {
          const float v[4] = {v0, v1, v2, v3};
          for (int t = 0; t < 4 && n + t < N; ++t) dst[t] = bf16_bits_rne(v[t]);
        }
      }
    }
  }
}

}  // namespace
}  // namespace selas

using namespace selas;

extern "C" int selas_nf4_linear(const void *x, int64_t M, int64_t K, int64_t ldx, const uint8_t *packed,
                                const float *absmax, int64_t blocksize, const float code[16], int64_t N,
                                const void *bias, void *y, int64_t ldy, int dtype, void *stream) {
  if (M < 0 || K <= 0 || N <= 0) return set_error(SELAS_EINVAL, "nf4_linear: bad shape M=%lld K=%lld N=%lld",
                                                   (long long)M, (long long)K, (long long)N);
  if (!valid_dtype(dtype)) return set_error(SELAS_EINVAL, "nf4_linear: bad dtype %d", dtype);
  if (ldx < K || ldy < N) return set_error(SELAS_EINVAL, "nf4_linear: row strides ldx=%lld ldy=%lld below K, N",
                                           (long long)ldx, (long long)ldy);
  if (M == 0) return ok();
  if (!x || !packed || !absmax || !y || !code) return set_error(SELAS_EINVAL, "nf4_linear: null pointer");
  if (dtype != SELAS_BF16) return set_error(SELAS_EUNSUPPORTED, "nf4_linear: fused kernels take bf16, got %s",
                                            dtype_name(dtype));
  if (blocksize != 64 || K % 64) return set_error(SELAS_EUNSUPPORTED,
                                                  "nf4_linear: fused kernels need blocksize 64 and K %% 64 == 0 "
                                                  "(blocksize %lld, K %lld)", (long long)blocksize, (long long)K);
  if (!aligned(x, 16) || ldx % 8 || !aligned(packed, 16) || !aligned(absmax, 4) || !aligned(y, 8) || ldy % 4 ||
      (bias && !aligned(bias, 2)))
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear: fused kernels need 16-byte aligned x rows and codes, "
                                         "8-byte aligned y rows");
  // Buffer offsets are 32-bit: every operand (plus one tile of overhang) must span < 4 GiB.
  const int64_t lim = (1ll << 32) - 1;
  if ((M + 256) * ldx * 2 > lim || (N + 256) * (K / 2) > lim || (N + 256) * (K / 64) * 4 > lim)
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear: operand above 4 GiB");
  Code16 c;
  for (int i = 0; i < 16; ++i) c.v[i] = code[i];
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t *xb = static_cast<const uint16_t *>(x);
  const uint16_t *bb = static_cast<const uint16_t *>(bias);
  uint16_t *yb = static_cast<uint16_t *>(y);
  if (M <= 32) {
    const int64_t grid = cdiv(N, 32 * kGemvGroups);
    const size_t lds = 256 * kGemvRepl * sizeof(uint32_t);
    nf4_gemv_kernel<<<dim3(static_cast<uint32_t>(grid)), dim3(kGemvThreads), lds, s>>>(
        xb, ldx, static_cast<int>(M), static_cast<int>(K), packed, absmax, c, static_cast<int>(N), bb, yb, ldy);
    return check_launch("nf4_linear (gemv)");
  }
  const int64_t tiles_m = cdiv(M, kBM), tiles_n = cdiv(N, kBN);
  nf4_gemm_kernel<<<dim3(static_cast<uint32_t>(tiles_m * tiles_n)), dim3(kGemmThreads), 0, s>>>(
      xb, ldx, static_cast<int>(M), static_cast<int>(K), packed, absmax, c, static_cast<int>(N), bb, yb, ldy,
      static_cast<int>(tiles_m));
  return check_launch("nf4_linear (gemm)");
}
