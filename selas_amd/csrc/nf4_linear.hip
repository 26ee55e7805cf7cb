// Quantized linear y = x W^T + b with W stored as NF4 (blocksize 64), on gfx950.
//
// Replaces UnitView.linear for NF4 weights (selas/store.py:289-293), which
// decodes the whole weight to a bf16 temporary (selas/codecs.py:269-280) and
// calls F.linear. Here the weight never exists in bf16 outside registers.
//
// Kernels, chosen from M and K:
//   * M <= 32 (hoisted adaLN modulation linears, M = number of steps), HBM-bound:
//     nf4_gemv_stream for K = 1024, 2048, 3072 (one launch can cover many
//     weights), nf4_gemv_kernel for other K. Both multiply x by the codes on
//     MFMA and apply the block's fp32 absmax to the fp32 block partial sums;
//     codes come from bank-replicated LDS tables indexed by the packed byte.
//   * M > 32 (block linears, M = tokens), MFMA-bound: nf4_gemm_kernel.
//     256x256 output tile per workgroup, 4 waves, each wave owns 64 output
//     columns for all 256 rows. x tiles are staged through LDS (XOR-swizzled
//     16-byte chunks, three stages in flight); weight codes go straight from
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
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"

namespace selas {
namespace {

// =========================================================================== GEMV (M <= 32)

// The skinny kernels multiply x by codes and apply the block absmax to the
// fp32 block sums. A code c is fed to the MFMA as two bf16 terms hi + lo with
// hi = bf16(c) and lo = bf16(c - hi) (|c - hi - lo| <= 2^-17 |c|): with hi
// alone, the fixed rounding error of each code would add up coherently over K
// for inputs with a nonzero mean. Two LDS tables map a packed byte to the bf16
// pair (code of the high nibble, code of the low nibble): hi terms in the
// first, lo terms in the second, each with kSplitRepl replicas so that the
// lanes of a ds_read_b32 spread over the banks.
constexpr int kSplitRepl = 32;
constexpr int kSplitTableWords = 2 * 256 * kSplitRepl;

// Builds both tables with nthreads threads (a multiple of 256); each lane
// writes its replicas in a rotated order so that a store touches distinct banks.
__device__ __forceinline__ void build_split_table(uint32_t *table, const Code16 &code, uint32_t *scratch32,
                                                  int tid, int nthreads) {
  if (tid < 16) {
    const float c = code.v[tid];
    const uint32_t hi = bf16_bits_rne(c);
    scratch32[tid] = hi | (static_cast<uint32_t>(bf16_bits_rne(c - bf16_bits_to_f32(hi))) << 16);
  }
  __syncthreads();
  const int b = tid & 255, part = tid >> 8, parts = nthreads >> 8;
  const uint32_t chi = scratch32[b >> 4], clo = scratch32[b & 15];
  const uint32_t vhi = (chi & 0xffffu) | (clo << 16), vlo = (chi >> 16) | (clo & 0xffff0000u);
  const int per = kSplitRepl / parts, lane = tid & 63;
  for (int j = 0; j < per; ++j) {
    const int r = (per * part + j + lane) & (kSplitRepl - 1);
    table[b * kSplitRepl + r] = vhi;
    table[256 * kSplitRepl + b * kSplitRepl + r] = vlo;
  }
}

// hi and lo bf16 operand fragments for the eight codes of packed dword P.
// lane_hi = lane % 32; lane_lo = lane % 32 + (offset of the lo table), made
// opaque once so that the compiler keeps the hi and lo reads separate (merged
// into one two-address read they would land interleaved and need moves).
struct CodeFrags {
  uint4 hi, lo;
};
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ CodeFrags lookup_codes(const uint32_t *table, uint32_t P, uint32_t lane_hi,
                                                  uint32_t lane_lo) {
  const uint32_t b0 = (P & 0xffu) * kSplitRepl, b1 = ((P >> 8) & 0xffu) * kSplitRepl;
  const uint32_t b2 = ((P >> 16) & 0xffu) * kSplitRepl, b3 = (P >> 24) * kSplitRepl;
  CodeFrags f;
  f.hi = make_uint4(table[b0 + lane_hi], table[b1 + lane_hi], table[b2 + lane_hi], table[b3 + lane_hi]);
  f.lo = make_uint4(table[b0 + lane_lo], table[b1 + lane_lo], table[b2 + lane_lo], table[b3 + lane_lo]);
  return f;
}
__device__ __forceinline__ f32x16 mfma_codes(const CodeFrags &f, bf16x8 xf, f32x16 p) {
  p = mfma32(xf, __builtin_bit_cast(bf16x8, f.hi), p);
  return mfma32(xf, __builtin_bit_cast(bf16x8, f.lo), p);
}

constexpr int kGemvThreads = 256;
constexpr int kGemvGroups = 2;  // 32-column groups per workgroup

// Workgroup: 64 output columns, all M (<= 32) rows. The four waves split the
// K blocks round-robin (wave w takes blocks w, w+4, ...) and their fp32
// partial results are summed in LDS in wave order, so the result does not
// depend on scheduling.
__global__ __launch_bounds__(kGemvThreads) void nf4_gemv_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, int M, int K, const uint8_t *__restrict__ packed,
    const float *__restrict__ absmax, Code16 code, int N, const uint16_t *__restrict__ bias,
    uint16_t *__restrict__ y, int64_t ldy) {
  extern __shared__ uint32_t lds[];  // split code table; later the reduction buffer
  __shared__ uint32_t codes[16];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;
  build_split_table(lds, code, codes, tid, kGemvThreads);
  __syncthreads();
  const uint32_t lane_lo = opaque_u32(static_cast<uint32_t>(c) + 256 * kSplitRepl);

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
      CodeFrags f[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) f[s] = lookup_codes(lds, words[s], c, lane_lo);
      f32x16 p = f32x16{};
#pragma unroll
      for (int s = 0; s < 4; ++s) p = mfma_codes(f[s], xf[s], p);
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

// ------------------------------------------------------------- int8_row skinny GEMM
//
// For M <= 32 with int8_row weights (q [N, K] int8, one fp32 scale per row):
// y[m, n] = bf16(s_n * sum_k x[m, k] q[n, k] + b_n), s_n = bf16(scale_n). The
// row scale is applied to the fp32 sums instead of to every weight: the sums
// are those of the exact quantized weight q * s_n, where the reference's
// operand bf16(q * s_n) carries one bf16 rounding per element (relative
// 2^-9 at most). The MFMA operand is the biased byte u = q + 128, exact in
// bf16 (integers up to 256 are), and sum_k x u - 128 sum_k x = sum_k x q, the
// second sum coming from one more MFMA against ones.
//
// This kernel serves K other than 1024, 2048, 3072 (those take int8_gemv_stream).
// Workgroup: 32 output columns, all M rows; the eight waves take the K blocks
// round-robin, three blocks in flight each, and their partial results are
// summed in LDS in wave order (deterministic). Its 16-byte loads each touch 32
// rows, 32 bytes of a 128-byte line per row, which holds it near 1.8 TB/s
// (31 us for an 18432 x 3072 weight at M = 28) whatever the number of columns
// per workgroup, loads in flight or waves per SIMD.
constexpr int kI8GemvWaves = 8;
constexpr int kI8GemvThreads = 64 * kI8GemvWaves;
constexpr int kI8G = 1;  // 32-column groups per workgroup
constexpr int kI8B = 3;  // K blocks per wave in flight

__device__ __forceinline__ bf16x8 biased_i8_to_bf16(uint32_t d0, uint32_t d1) {
  const uint32_t u0 = d0 ^ 0x80808080u, u1 = d1 ^ 0x80808080u;
  auto f = [](uint32_t u, int j) { return static_cast<float>((u >> (8 * j)) & 0xffu); };
  uint4 r;
  r.x = pack_bf16x2(f(u0, 0), f(u0, 1));
  r.y = pack_bf16x2(f(u0, 2), f(u0, 3));
  r.z = pack_bf16x2(f(u1, 0), f(u1, 1));
  r.w = pack_bf16x2(f(u1, 2), f(u1, 3));
  return __builtin_bit_cast(bf16x8, r);
}

__global__ __launch_bounds__(kI8GemvThreads, 4) void int8_row_gemv_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, int M, int K, const int8_t *__restrict__ q,
    const float *__restrict__ scale, int N, const uint16_t *__restrict__ bias, uint16_t *__restrict__ y,
    int64_t ldy) {
  constexpr int G = kI8G, NW = kI8GemvWaves, B = kI8B;
  __shared__ float red[NW][G * 16][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;
  const int kblocks = K >> 6;
  const int n_base = blockIdx.x * (32 * G);
  const uint16_t *xr = x + static_cast<int64_t>(min(c, M - 1)) * ldx + 32 * h;
  const int8_t *wr[G];
#pragma unroll
  for (int g = 0; g < G; ++g) wr[g] = q + static_cast<int64_t>(min(n_base + 32 * g + c, N - 1)) * K + 32 * h;
  const uint32_t one2 = 0x3F803F80u;  // two bf16 ones
  const bf16x8 ones = __builtin_bit_cast(bf16x8, make_uint4(one2, one2, one2, one2));

  f32x16 acc[G], accx = f32x16{};
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = f32x16{};
  auto load = [&](int kb, uint4 (&wq)[G][2], bf16x8 (&xf)[4]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      wq[g][0] = *reinterpret_cast<const uint4 *>(wr[g] + kb * 64);
      wq[g][1] = *reinterpret_cast<const uint4 *>(wr[g] + kb * 64 + 16);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) xf[s] = *reinterpret_cast<const bf16x8 *>(xr + kb * 64 + 8 * s);
  };
  auto mul = [&](const uint4 (&wq)[G][2], const bf16x8 (&xf)[4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      accx = mfma32(xf[s], ones, accx);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint4 &w = wq[g][s >> 1];
        acc[g] = mfma32(xf[s], biased_i8_to_bf16((s & 1) ? w.z : w.x, (s & 1) ? w.w : w.y), acc[g]);
      }
    }
  };
  // This wave's blocks kb = wave, wave + NW, ...: B per pass, all loaded before the MFMAs.
  for (int kb0 = wave; kb0 < kblocks; kb0 += B * NW) {
    uint4 wq[B][G][2];
    bf16x8 xf[B][4];
#pragma unroll
    for (int b = 0; b < B; ++b) load(min(kb0 + b * NW, kblocks - 1), wq[b], xf[b]);
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (kb0 + b * NW < kblocks) mul(wq[b], xf[b]);
  }
  // Per wave: its partial sum_k x q, in the MFMA layout (row m of lane l, register r:
  // 8*(r/4) + 4*(l/32) + r%4; column l%32).
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][g * 16 + r][lane] = acc[g][r] - 128.0f * accx[r];
  __syncthreads();
  for (int e = tid; e < G * 16 * 64; e += kI8GemvThreads) {
    const int l = e & 63, gr = e >> 6;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[w][gr][l];
    const int g = gr >> 4, r = gr & 15;
    const int m = 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const int n = n_base + 32 * g + (l & 31);
    if (m < M && n < N) {
      const float sb = bf16_bits_to_f32(bf16_bits_rne(scale[n]));
      const float b = bias ? bf16_bits_to_f32(bias[n]) : 0.0f;
      y[static_cast<int64_t>(m) * ldy + n] = bf16_bits_rne(sb * v + b);
    }
  }
}

// ------------------------------------------------------------- streaming skinny GEMM
//
// For M <= 32 and K = 1024, 2048, 3072 (the hoisted modulation linears have
// K = hidden = 3072). One workgroup of NW waves per CU streams 32-row slabs
// ("units") of one or many weights; the units are dealt out round-robin
// (workgroup b takes units b, b + G, b + 2G, ... for a grid of G), so that at
// any time the CUs read one contiguous window of the weights.
//
//   * Wave w owns the K slice of blocks [w*BPW, (w+1)*BPW) (K = 64*NW*BPW) and
//     keeps x for that slice in registers for the whole launch, as fp16 MFMA
//     A fragments (rows past M repeat row M-1).
//   * Each wave copies its slice of the unit's codes (32 rows x BPW*32 bytes)
//     from HBM into its own LDS stage with buffer-load-to-LDS DMA; the unit's
//     scales (32 rows x K/64 floats, one contiguous block) are copied by the
//     waves together into a shared double buffer. Consecutive lanes fetch
//     consecutive 16-byte chunks, so every request covers whole cache lines;
//     the chunk order inside a code row, and inside a row of scales, is
//     XOR-swizzled so that the MFMA-order reads (lane (c, h) reads row c) are
//     free of bank conflicts.
//   * Once its codes are in registers a wave issues the next unit's DMA and
//     multiplies: each code byte is looked up in a 64-way replicated LDS table
//     of fp16 code pairs (one v_perm for the address, one ds_read_b32), four
//     lookups make the B operand of one v_mfma_f32_32x32x16_f16, and the fp32
//     block sums are scaled by absmax.
//   * The NW partial results of a unit are summed in LDS in wave order
//     (deterministic). Every wave drains its DMAs before the barrier that
//     follows the partial-sum stores, so after it the next unit's codes and
//     scales are in LDS for everyone. With 4 waves the partial sums are double
//     buffered and a unit needs that one barrier; with 8 a second barrier
//     guards the single buffer. The sum and the bf16 stores of unit u run
//     during unit u+1, before its DMA is issued.

constexpr int kSgRows = 32;
constexpr int kSgTableBytes = 256 * 64 * 4;  // [byte][lane] -> fp16 code pair
constexpr int kSgMaxDescs = 1023;
constexpr int kSgAhead = 1;  // sub-steps of table lookups in flight
constexpr int kSgWaves = 8;  // waves per workgroup (8: two per SIMD; 4 measured 25 % slower)

template <int NW, int BPW>
struct SgLayout {
  static constexpr int kThreads = 64 * NW;
  // A wave's slice of a code row is kChunks 16-byte chunks; the 32 rows of a unit
  // are kCodeInstrs DMA instructions of 64 chunks.
  static constexpr int kChunks = 2 * BPW;
  static constexpr int kCodeInstrs = BPW;
  static constexpr int kCodeBytes = kSgRows * kChunks * 16;
  static constexpr int kBlocks = NW * BPW;                         // K / 64
  static constexpr int kScaleBytes = kSgRows * kBlocks * 4;        // a unit's scales
  static constexpr int kScaleInstrs = kScaleBytes / 1024;          // DMA instructions of 1 KiB
  static constexpr int kRedBufs = NW == 4 ? 2 : 1;
  static constexpr int kRedBytes = kRedBufs * NW * 16 * 64 * 4;   // [buf][wave][r][lane] partial sums
  static constexpr int kStage = kSgTableBytes;                     // byte offsets in dynamic LDS
  static constexpr int kScales = kStage + NW * kCodeBytes;         // two buffers
  static constexpr int kRed = kScales + 2 * kScaleBytes;
  static constexpr int kPrefix = kRed + kRedBytes;
  static constexpr int kMaxBytes = kPrefix + (kSgMaxDescs + 1) * 4;
  static constexpr int kOuts = 1024 / kThreads;                    // outputs of a 32x32 unit tile per thread
  static_assert(kScaleBytes % 1024 == 0 && kChunks % 4 == 0, "layout");
  static_assert(kMaxBytes <= 160 * 1024, "LDS");
};

struct GemvDesc {
  const uint8_t *packed;
  const float *absmax;
  const uint16_t *bias;
  uint16_t *y;
  int64_t n;
  int64_t ldy;
};

// A descriptor held in scalar registers (every field wave-uniform; n and ldy fit 32 bits).
struct SDesc {
  const uint8_t *packed;
  const float *absmax;
  const uint16_t *bias;
  uint16_t *y;
  int n, ldy;
};
template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32)));
  return reinterpret_cast<T *>(lo | (hi << 32));
}
__device__ __forceinline__ SDesc uniform_desc(const GemvDesc &d) {
  return SDesc{uniform_ptr(d.packed), uniform_ptr(d.absmax), uniform_ptr(d.bias), uniform_ptr(d.y),
               __builtin_amdgcn_readfirstlane(static_cast<int>(d.n)),
               __builtin_amdgcn_readfirstlane(static_cast<int>(d.ldy))};
}

// 16 bytes per lane from a buffer straight into LDS: lane i writes lds + 16*i.
__device__ __forceinline__ void load_lds16_at(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voff, 0, 0, 0);
}

// XOR applied to the chunk index of row r inside a wave's code stage: chosen
// so that 16 consecutive rows, read at one chunk, hit 16 distinct 16-byte bank
// groups (a row is kChunks*16 bytes; 64 banks of 4 bytes).
template <int kChunks>
__device__ __forceinline__ int sg_swz(int r) {
  if constexpr (kChunks % 16 == 0) return r & 15;
  else if constexpr (kChunks % 8 == 0) return (r >> 1) & 7;
  else return (r >> 2) & 3;
}

// A wave's slice of x for the streaming skinny kernels, in MFMA order: out[b][s] holds, for lane (c, h),
// the 8 elements k = 64*(kb0+b) + 32h + 8s .. +8 of row c (rows past M repeat row M-1).
// Lane (c, h) needs row c, so loads straight into registers in that order touch 32 rows, 32 cache
// lines, per instruction, and measured slower by 2.2 us per launch. The slice goes through LDS
// instead: one 64-wide block (32 rows x 128 bytes) per round of 4 DMA instructions, each covering 8
// whole rows, two rounds in flight in the wave's two 4 KiB buffers at LDS [8192 wave, +8192). Chunk p
// of row r sits at physical chunk p ^ swz(r), so that the MFMA-order reads are free of bank conflicts.
// The caller owns LDS [0, 65536) until a barrier after this returns (its code table or stages are
// built there afterwards), and has no vector memory operation of this wave in flight.
template <int BPW>
__device__ __forceinline__ void load_x_slice(const uint16_t *x, int64_t ldx, int M, int K, int kb0, int wave,
                                             int lane, uint4 (&out)[BPW][4]) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int h = lane >> 5, c = lane & 31;
  uint32_t off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q = 64 * j + lane, r = q >> 3, p = (q & 7) ^ sg_swz<8>(r);
    off[j] = (static_cast<uint32_t>(min(r, M - 1)) * static_cast<uint32_t>(ldx) + static_cast<uint32_t>(64 * kb0)) *
                 2u + 16u * static_cast<uint32_t>(p);
  }
  // The make_rsrc descriptor as four words for the asm operand.
  const uint64_t xp = reinterpret_cast<uint64_t>(x);
  const u32x4 desc = {static_cast<uint32_t>(xp), static_cast<uint32_t>(xp >> 32) & 0xffffu,
                      static_cast<uint32_t>(((M - 1) * ldx + K) * 2), 0x00020000u};
  const uint32_t base = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(wave)) * 8192u;
  // The DMAs are issued by inline asm, uncounted by the compiler: for a counted LDS DMA it waits for all
  // of them (the next round's included) before every LDS read. The explicit waits order the reads
  // instead; any wait of the compiler's own is only made longer by the uncounted ones. M0 (the DMA's
  // LDS address) is saved and restored around each, since the compiler keeps M0 out of clobber lists;
  // an SALU write of M0 needs one wait state before an LDS DMA reads it.
  auto issue = [&](int b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
          "s_nop 0\n\ts_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(base + static_cast<uint32_t>((b & 1) * 4096 + 1024 * j)), "v"(off[j]), "s"(desc), "s"(128u * b)
          : "memory");
    }
  };
  // Reads by LDS address (this file's skinny kernels declare no static LDS, so dynamic LDS starts at 0).
  const uint32_t rd = base + static_cast<uint32_t>(c * 128);
  const int sw = sg_swz<8>(c);
  issue(0);
  if constexpr (BPW > 1) issue(1);
#pragma unroll
  for (int b = 0; b < BPW; ++b) {
    if (b + 1 < BPW) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // round b landed, round b+1 may not
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t a = rd + static_cast<uint32_t>((b & 1) * 4096 + 16 * ((4 * h + s) ^ sw));
      out[b][s] = __builtin_bit_cast(
          uint4, *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(static_cast<uintptr_t>(a)));
    }
    if (b + 2 < BPW) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the buffer's reads are done before it is refilled
      issue(b + 2);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

template <int NW, int BPW>
__global__ __launch_bounds__(64 * NW, 1) void nf4_gemv_stream(
    const uint16_t *__restrict__ x, int64_t ldx, int M, const GemvDesc *__restrict__ descs, int count,
    GemvDesc one, Code16 code) {
  using L = SgLayout<NW, BPW>;
  constexpr int kblocks = L::kBlocks, K = 64 * kblocks, row_bytes = K / 2, kThreads = L::kThreads;
  extern __shared__ __align__(16) uint32_t lds_words[];
  uint8_t *lds = reinterpret_cast<uint8_t *>(lds_words);
  int *prefix = reinterpret_cast<int *>(lds + L::kPrefix);
  float *red = reinterpret_cast<float *>(lds + L::kRed);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;

  // fp16 codebook, staged in the reduction area until the table is built.
  uint32_t *code16 = reinterpret_cast<uint32_t *>(red);
  if (tid < 16) code16[tid] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(code.v[tid]));
  if (wave == 0) {
    // prefix[g] = units (32-row slabs) before weight g: a wave-wide scan, 64 weights at a time.
    int carry = 0;
    for (int base = 0; base < count; base += 64) {
      const int g = base + lane;
      int v = 0;
      if (g < count) v = static_cast<int>(((descs ? descs[g].n : one.n) + kSgRows - 1) / kSgRows);
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(v, off);
        if (lane >= off) v += t;
      }
      if (g < count) prefix[g + 1] = carry + v;
      carry += __shfl(v, 63);
    }
    if (lane == 0) prefix[0] = 0;
  }
  // This wave's slice of x (block b, sub-step s: k = 64*(kb0+b) + 32h + 8s .. +8 of row c), staged
  // through the table area before the table is built.
  const int kb0 = wave * BPW;
  uint4 xraw[BPW][4];
  static_assert(8 * 8192 <= kSgTableBytes, "x staging fits the table area");
  load_x_slice<BPW>(x, ldx, M, K, kb0, wave, lane, xraw);
  __syncthreads();  // prefix and fp16 codebook ready

  uint8_t *stage = lds + L::kStage + wave * L::kCodeBytes;
  // MFMA-order reads: lane (c, h) takes chunk 2b + h of row c.
  const int rd_base = c * L::kChunks * 16, rd_swz = sg_swz<L::kChunks>(c);
  const int sc_swz = sg_swz<kblocks / 4>(c);
  // v_perm source for table addresses: byte 0 = 4 * lane, byte 1 <- code byte.
  const uint32_t tsel = static_cast<uint32_t>(lane) * 4u;

  const int units_total = prefix[count];
  // Units are dealt out round-robin: workgroup b takes units b, b + G, b + 2G, ... (G = grid size), so
  // that at any time the CUs stream one contiguous window of the weights.
  const int G = gridDim.x;
  const int u_begin = blockIdx.x;
  const int u_end = units_total;
  if (u_begin >= u_end) return;  // uniform over the workgroup

  auto locate = [&](int u, int g) {
    while (prefix[g + 1] <= u) ++g;
    return __builtin_amdgcn_readfirstlane(g);
  };
  // Descriptors are uniform: kept in scalar registers and reloaded only when the weight changes.
  auto desc = [&](int g) { return uniform_desc(descs ? descs[g] : one); };
  // Scale buffer of the workgroup's it-th unit (double buffered).
  auto scales = [&](int it) { return reinterpret_cast<float *>(lds + L::kScales + (it & 1) * L::kScaleBytes); };
  // Code instruction j fetches chunk (p ^ swz(r)) of row r into stage slot
  // 64j + lane = r*kChunks + p; scale instructions j = wave, wave + NW, ... fetch
  // 1 KiB each. The buffers start at the unit's first row, so rows past the
  // weight's end fall outside their ranges and read as 0.
  auto issue = [&](int it, const SDesc &d, int row0) {
    const auto rc = make_rsrc(d.packed + static_cast<int64_t>(row0) * row_bytes,
                              static_cast<uint32_t>(max(d.n - row0, 0)) * row_bytes);
#pragma unroll
    for (int j = 0; j < L::kCodeInstrs; ++j) {
      const uint32_t q = 64u * j + lane, r = q / L::kChunks, p = q - r * L::kChunks;
      load_lds16_at(rc, stage + 1024 * j, r * row_bytes + 32 * kb0 + 16 * (p ^ sg_swz<L::kChunks>(r)));
    }
    const auto ra = make_rsrc(d.absmax + static_cast<int64_t>(row0) * kblocks,
                              static_cast<uint32_t>(max(d.n - row0, 0)) * (kblocks * 4));
#pragma unroll
    for (int jj = 0; jj < (L::kScaleInstrs + NW - 1) / NW; ++jj) {
      const int j = wave + NW * jj;
      if (j < L::kScaleInstrs) {
        // slot s holds chunk (q ^ swz(r)) of row r, so that the 32 rows' reads of one scale spread over
        // the banks (row r's scales at a fixed stride alone would share 4 banks)
        const uint32_t s = 64u * j + lane, r = s / (kblocks / 4), q = s - r * (kblocks / 4);
        load_lds16_at(ra, reinterpret_cast<uint8_t *>(scales(it)) + 1024 * j,
                      (r * (kblocks / 4) + (q ^ sg_swz<kblocks / 4>(r))) * 16u);
      }
    }
  };
  // The first unit's codes and scales: their latency overlaps the table build and the x conversion.
  int g_cur = locate(u_begin, 0);
  SDesc d_cur = desc(g_cur);
  int row_cur = (u_begin - prefix[g_cur]) * kSgRows;
  issue(0, d_cur, row_cur);

  {
    // Entry (b, j) at b*256 + 4*j: fp16 pair (code[b >> 4], code[b & 15]), one replica per lane j.
    constexpr int kParts = kThreads / 256, kPer = 64 / kParts;
    const int b = tid & 255, part = tid >> 8;
    const uint32_t e = code16[b >> 4] | (code16[b & 15] << 16);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int r = kPer * part + ((j + lane) & (kPer - 1));
      *reinterpret_cast<uint32_t *>(lds + b * 256 + r * 4) = e;
    }
  }

  // The skinny kernel multiplies in fp16: each row of this wave's slice of x is
  // scaled by a power of two that brings the slice's largest magnitude into
  // [2^14, 2^15), which makes the bf16 -> fp16 conversion exact (8 significant
  // bits into 11; values below 2^-38 of that maximum fall into fp16 subnormals
  // or to zero), and the products with the fp16 codebook accumulate in fp32.
  // Each wave scales its fp32 partial sums back (exactly: a power of two) before
  // the waves' partials are added, so no row maximum over all of K is needed.
  // Rows whose slice maximum is 0, Inf or NaN keep scale 1.
  f16x8 xf[BPW][4];
  float inv[16];  // inverse scale of the row each partial-sum register holds
  {
    // |x| as bf16 magnitude bits, ordered like the values (NaN above Inf): a running maximum per 16-bit
    // half (one mask and one packed max per word), the two halves combined at the end.
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 mx2 = {0, 0};
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t w[4] = {xraw[b][s].x, xraw[b][s].y, xraw[b][s].z, xraw[b][s].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(u16x2, w[i] & 0x7fff7fffu));
      }
    uint32_t mx = max(static_cast<uint32_t>(mx2.x), static_cast<uint32_t>(mx2.y));
    mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), 32)));  // both halves of row c's slice
    const unsigned e = (mx >> 7) & 0xffu;  // bf16 exponent field of the slice maximum
    const int k = (e == 0u || e == 0xffu) ? 0 : 14 - (static_cast<int>(e) - 127);  // scale = 2^k
    const float sc = __uint_as_float(static_cast<uint32_t>(max(-126, min(127, k)) + 127) << 23);
    const float isc = __uint_as_float(static_cast<uint32_t>(max(-126, min(127, -k)) + 127) << 23);
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t w[4] = {xraw[b][s].x, xraw[b][s].y, xraw[b][s].z, xraw[b][s].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xf[b][s][2 * i] = static_cast<_Float16>(__uint_as_float(w[i] << 16) * sc);
          xf[b][s][2 * i + 1] = static_cast<_Float16>(__uint_as_float(w[i] & 0xffff0000u) * sc);
        }
      }
    // Register r of a 32x32 result holds row 8*(r/4) + 4h + r%4, whose scale lane (that row) computed.
#pragma unroll
    for (int r = 0; r < 16; ++r) inv[r] = __shfl(isc, 8 * (r >> 2) + 4 * h + (r & 3));
  }
  // Bias and outputs go through buffer resources, not generic pointers: a
  // flat access might touch LDS and would make every later LDS read wait for
  // all outstanding memory operations, the stage DMA included.
  // Bias bits of the output column this thread stores (loaded one unit ahead).
  auto load_bias = [&](const SDesc &d, int row0) -> uint32_t {
    if (!d.bias) return 0u;
    const int n = min(row0 + c, d.n - 1);
    const auto rb = make_rsrc(d.bias, static_cast<uint32_t>(d.n * 2));
    return __builtin_amdgcn_raw_buffer_load_b16(rb, static_cast<uint32_t>(n) * 2u, 0, 0);
  };
  // The outputs this thread owns of the unit whose partials are in buffer `buf`:
  // the NW partials (each already scaled back) summed in wave order, bias
  // added, rounded to bf16.
  auto finish = [&](int buf, const SDesc &d, int row0, uint32_t bias_bits) {
    const int N = d.n;
    const float bv = bf16_bits_to_f32(static_cast<uint16_t>(bias_bits));
    const auto ry = make_rsrc(d.y, static_cast<uint32_t>(((M - 1) * d.ldy + N) * 2));
    const float *rb = red + buf * NW * 1024;
    // All partials first (one batch of LDS reads), then the sums in wave order.
    float part[L::kOuts][NW];
#pragma unroll
    for (int i = 0; i < L::kOuts; ++i)
#pragma unroll
      for (int w = 0; w < NW; ++w) part[i][w] = rb[w * 1024 + tid + kThreads * i];
#pragma unroll
    for (int i = 0; i < L::kOuts; ++i) {
      const int e = tid + kThreads * i;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += part[i][w];
      const int r = e >> 6;
      const int m = 8 * (r >> 2) + 4 * h + (r & 3);
      const int n = row0 + c;
      if (m < M && n < N)
        __builtin_amdgcn_raw_buffer_store_b16(bf16_bits_rne(v + bv), ry,
                                              static_cast<uint32_t>(m * d.ldy + n) * 2u, 0, 0);
    }
  };
  // This wave's codes and scales of unit u, from LDS into registers.
  uint4 cw[BPW];
  float a[BPW];
  auto read_stage = [&](int it) {
    const float *sc = scales(it) + c * kblocks;
#pragma unroll
    for (int b = 0; b < BPW; ++b)
      cw[b] = *reinterpret_cast<const uint4 *>(stage + rd_base + 16 * ((2 * b + h) ^ rd_swz));
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
      const int f = kb0 + b;
      a[b] = sc[4 * ((f >> 2) ^ sc_swz) + (f & 3)];
    }
  };

  wait_vmcnt<0>();
  __syncthreads();  // the first unit's codes and scales, and the table, are in LDS
  read_stage(0);
  SDesc d_prev = d_cur;
  int row_prev = row_cur;
  uint32_t bias_prev = 0;
  int it = 0;
  for (int u = u_begin; u < u_end; u += G, ++it) {
    const int buf = it & (L::kRedBufs - 1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage read before the next DMA overwrites it
    const uint32_t bias_cur = load_bias(d_cur, row_cur);
    int g_nxt = g_cur, row_nxt = row_cur;
    SDesc d_nxt = d_cur;
    const bool more = u + G < u_end;
    if (more) {
      g_nxt = locate(u + G, g_cur);
      if (g_nxt != g_cur) d_nxt = desc(g_nxt);
      row_nxt = (u + G - prefix[g_nxt]) * kSgRows;
    }
    if (u > u_begin) finish(buf ^ (L::kRedBufs - 1), d_prev, row_prev, bias_prev);  // unit u-1
    if (more) issue(it + 1, d_nxt, row_nxt);

    // Table lookups run kSgAhead sub-steps ahead of the MFMAs that use them.
    auto word = [&](int t) {
      const uint4 &q = cw[t >> 2];
      return (t & 3) == 0 ? q.x : (t & 3) == 1 ? q.y : (t & 3) == 2 ? q.z : q.w;
    };
    auto lookup = [&](uint32_t P, uint32_t (&e)[4]) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t addr = perm(P, tsel, 0x0C0C0400u | ((4u + i) << 8));
        // The table starts at LDS address 0: this kernel declares no static LDS.
        e[i] = *reinterpret_cast<const __attribute__((address_space(3))) uint32_t *>(static_cast<uintptr_t>(addr));
      }
    };
    uint32_t ebuf[kSgAhead + 1][4];
#pragma unroll
    for (int t = 0; t < kSgAhead; ++t) lookup(word(t), ebuf[t]);
    // Block b's sums go to p[b & 1]; they are scaled into acc after block b+1's second MFMA,
    // when the MFMA results are ready, so the wave does not wait for them.
    f32x16 acc = f32x16{};
    f32x16 p[2];
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
      p[b & 1] = f32x16{};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int t = 4 * b + s;
        if (t + kSgAhead < 4 * BPW) lookup(word(t + kSgAhead), ebuf[(t + kSgAhead) % (kSgAhead + 1)]);
        // Keep those reads ahead of this sub-step's MFMAs (the scheduler would sink them to their use).
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t(&e)[4] = ebuf[t % (kSgAhead + 1)];
        p[b & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            xf[b][s], __builtin_bit_cast(f16x8, make_uint4(e[0], e[1], e[2], e[3])), p[b & 1], 0, 0, 0);
        if (s == 1 && b > 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] += p[(b - 1) & 1][r] * a[b - 1];
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] += p[(BPW - 1) & 1][r] * a[BPW - 1];
    wait_vmcnt<0>();  // this wave's DMAs of unit u+1 have landed
    float *rw = red + buf * NW * 1024;
    if constexpr (L::kRedBufs == 1) {
      __syncthreads();  // every wave has summed unit u-1 from the single buffer
#pragma unroll
      for (int r = 0; r < 16; ++r) rw[(wave * 16 + r) * 64 + lane] = acc[r] * inv[r];
      if (more) read_stage(it + 1);  // its latency overlaps the barrier
      __syncthreads();
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) rw[(wave * 16 + r) * 64 + lane] = acc[r] * inv[r];
      __syncthreads();  // partials of unit u complete; every wave's DMAs of unit u+1 landed
      if (more) read_stage(it + 1);
    }
    d_prev = d_cur;
    row_prev = row_cur;
    bias_prev = bias_cur;
    g_cur = g_nxt;
    d_cur = d_nxt;
    row_cur = row_nxt;
  }
  finish((it - 1) & (L::kRedBufs - 1), d_prev, row_prev, bias_prev);
}

// ------------------------------------------------------- int8_row streaming skinny GEMM
//
// For M <= 32, K = 1024, 2048, 3072 and int8_row weights: the structure of
// nf4_gemv_stream (persistent workgroups of NW waves over 32-row units of one
// or many weights, wave w owning the K blocks [w*BPW, (w+1)*BPW), each wave's
// slice of a unit's rows copied HBM -> LDS by whole-line DMA, XOR-swizzled so
// that the MFMA-order reads are conflict-free, partial sums added in LDS in
// wave order) with the operand of int8_row_gemv_kernel: x stays bf16 in
// registers for the whole launch, the biased byte u = q + 128 converts exactly
// to bf16, sum_k x q = sum_k x u - 128 sum_k x (the second sum computed once,
// per wave, against ones), and the fp32 row sums are scaled by bf16(scale).
template <int NW, int BPW>
struct I8Layout {
  static constexpr int kThreads = 64 * NW;
  static constexpr int kChunks = 4 * BPW;        // 16-byte chunks of a row's slice (64 * BPW bytes)
  static constexpr int kCodeInstrs = 2 * BPW;    // 32 rows x kChunks chunks / 64 lanes
  static constexpr int kCodeBytes = kSgRows * kChunks * 16;
  static constexpr int kRedBufs = NW == 4 ? 2 : 1;
  static constexpr int kRedBytes = kRedBufs * NW * 16 * 64 * 4;
  static constexpr int kRed = NW * kCodeBytes;   // byte offsets in dynamic LDS; the stages start at 0
  static constexpr int kPrefix = kRed + kRedBytes;
  static constexpr int kMaxBytes = kPrefix + (kSgMaxDescs + 1) * 4;
  static constexpr int kOuts = 1024 / kThreads;
  static_assert(kChunks % 8 == 0, "the swizzle permutes chunks within aligned groups of 8");
  static_assert(kMaxBytes <= 160 * 1024, "LDS");
};

template <int NW, int BPW>
__global__ __launch_bounds__(64 * NW, 1) void int8_gemv_stream(
    const uint16_t *__restrict__ x, int64_t ldx, int M, const GemvDesc *__restrict__ descs, int count,
    GemvDesc one) {
  using L = I8Layout<NW, BPW>;
  constexpr int kblocks = L::kThreads / 64 * BPW, row_bytes = 64 * kblocks, kThreads = L::kThreads;
  extern __shared__ __align__(16) uint32_t lds_words[];
  uint8_t *lds = reinterpret_cast<uint8_t *>(lds_words);
  int *prefix = reinterpret_cast<int *>(lds + L::kPrefix);
  float *red = reinterpret_cast<float *>(lds + L::kRed);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;

  if (wave == 0) {
    // prefix[g] = units (32-row slabs) before weight g: a wave-wide scan, 64 weights at a time.
    int carry = 0;
    for (int base = 0; base < count; base += 64) {
      const int g = base + lane;
      int v = 0;
      if (g < count) v = static_cast<int>(((descs ? descs[g].n : one.n) + kSgRows - 1) / kSgRows);
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(v, off);
        if (lane >= off) v += t;
      }
      if (g < count) prefix[g + 1] = carry + v;
      carry += __shfl(v, 63);
    }
    if (lane == 0) prefix[0] = 0;
  }

  // x fragments of this wave's slice (block b, sub-step s: k = 64*(kb0+b) + 32h + 8s .. +8; rows
  // past M repeat row M-1), staged through the stage and reduction areas before the first unit's DMA,
  // and the slice's sum_k x per row, against ones.
  const int kb0 = wave * BPW;
  static_assert(8 * 8192 <= L::kPrefix, "x staging fits below the prefix area");
  bf16x8 xf[BPW][4];
  {
    uint4 xraw[BPW][4];
    load_x_slice<BPW>(x, ldx, M, 64 * kblocks, kb0, wave, lane, xraw);
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
      for (int s = 0; s < 4; ++s) xf[b][s] = __builtin_bit_cast(bf16x8, xraw[b][s]);
  }
  const uint32_t one2 = 0x3F803F80u;
  const bf16x8 ones = __builtin_bit_cast(bf16x8, make_uint4(one2, one2, one2, one2));
  f32x16 accx = f32x16{};
#pragma unroll
  for (int b = 0; b < BPW; ++b)
#pragma unroll
    for (int s = 0; s < 4; ++s) accx = mfma32(xf[b][s], ones, accx);

  uint8_t *stage = lds + wave * L::kCodeBytes;
  // MFMA-order reads: lane (c, h) takes chunks 4b + 2h and 4b + 2h + 1 of row c.
  const int rd_base = c * L::kChunks * 16, rd_swz = sg_swz<L::kChunks>(c);
  __syncthreads();  // prefix ready

  const int units_total = prefix[count];
  const int units_per_wg = (units_total + gridDim.x - 1) / gridDim.x;
  const int u_begin = blockIdx.x * units_per_wg;
  const int u_end = min(u_begin + units_per_wg, units_total);
  if (u_begin >= u_end) return;  // uniform over the workgroup

  auto locate = [&](int u, int g) {
    while (prefix[g + 1] <= u) ++g;
    return __builtin_amdgcn_readfirstlane(g);
  };
  auto desc = [&](int g) { return uniform_desc(descs ? descs[g] : one); };
  // Code instruction j fetches chunk (p ^ swz(r)) of row r into stage slot 64j + lane = r*kChunks + p.
  // The buffer starts at the unit's first row, so rows past the weight's end read as 0.
  auto issue = [&](const SDesc &d, int row0) {
    const auto rc = make_rsrc(d.packed + static_cast<int64_t>(row0) * row_bytes,
                              static_cast<uint32_t>(max(d.n - row0, 0)) * row_bytes);
#pragma unroll
    for (int j = 0; j < L::kCodeInstrs; ++j) {
      const uint32_t q = 64u * j + lane, r = q / L::kChunks, p = q - r * L::kChunks;
      load_lds16_at(rc, stage + 1024 * j, r * row_bytes + 64 * kb0 + 16 * (p ^ sg_swz<L::kChunks>(r)));
    }
  };
  // Bias bits and row scale of the output column this thread stores (loaded one unit ahead,
  // through buffer resources: a flat access could make LDS reads wait for the stage DMA).
  auto load_col = [&](const SDesc &d, int row0, uint32_t &bias_bits, float &scale) {
    const int n = min(row0 + c, d.n - 1);
    bias_bits = 0u;
    if (d.bias)
      bias_bits = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(d.bias, static_cast<uint32_t>(d.n * 2)),
                                                       static_cast<uint32_t>(n) * 2u, 0, 0);
    scale = load_f32(make_rsrc(d.absmax, static_cast<uint32_t>(d.n * 4)), static_cast<uint32_t>(n) * 4u, 0);
  };
  auto finish = [&](int buf, const SDesc &d, int row0, uint32_t bias_bits, float scale) {
    const int N = d.n;
    const float bv = bf16_bits_to_f32(static_cast<uint16_t>(bias_bits));
    const float sb = bf16_bits_to_f32(bf16_bits_rne(scale));
    const auto ry = make_rsrc(d.y, static_cast<uint32_t>(((M - 1) * d.ldy + N) * 2));
    const float *rb = red + buf * NW * 1024;
#pragma unroll
    for (int i = 0; i < L::kOuts; ++i) {
      const int e = tid + kThreads * i;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += rb[w * 1024 + e];
      const int r = e >> 6;
      const int m = 8 * (r >> 2) + 4 * h + (r & 3);
      const int n = row0 + c;
      if (m < M && n < N)
        __builtin_amdgcn_raw_buffer_store_b16(bf16_bits_rne(sb * v + bv), ry,
                                              static_cast<uint32_t>(m * d.ldy + n) * 2u, 0, 0);
    }
  };
  uint4 cw[BPW][2];
  auto read_stage = [&]() {
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        cw[b][t] = *reinterpret_cast<const uint4 *>(stage + rd_base + 16 * ((4 * b + 2 * h + t) ^ rd_swz));
  };

  int g_cur = locate(u_begin, 0);
  SDesc d_cur = desc(g_cur);
  int row_cur = (u_begin - prefix[g_cur]) * kSgRows;
  issue(d_cur, row_cur);
  wait_vmcnt<0>();
  __syncthreads();  // the first unit's rows are in LDS
  read_stage();
  SDesc d_prev = d_cur;
  int row_prev = row_cur;
  uint32_t bias_prev = 0;
  float scale_prev = 0.0f;
  for (int u = u_begin; u < u_end; ++u) {
    const int buf = (u - u_begin) & (L::kRedBufs - 1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage read before the next DMA overwrites it
    uint32_t bias_cur;
    float scale_cur;
    load_col(d_cur, row_cur, bias_cur, scale_cur);
    int g_nxt = g_cur, row_nxt = row_cur + kSgRows;
    SDesc d_nxt = d_cur;
    const bool more = u + 1 < u_end;
    if (more && row_nxt >= d_cur.n) {
      g_nxt = locate(u + 1, g_cur);
      d_nxt = desc(g_nxt);
      row_nxt = (u + 1 - prefix[g_nxt]) * kSgRows;
    }
    if (u > u_begin) finish(buf ^ (L::kRedBufs - 1), d_prev, row_prev, bias_prev, scale_prev);  // unit u-1
    if (more) issue(d_nxt, row_nxt);

    f32x16 acc = f32x16{};
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 &w = cw[b][s >> 1];
        acc = mfma32(xf[b][s], biased_i8_to_bf16((s & 1) ? w.z : w.x, (s & 1) ? w.w : w.y), acc);
      }
    wait_vmcnt<0>();  // this wave's DMAs of unit u+1 have landed
    float *rw = red + buf * NW * 1024;
    if constexpr (L::kRedBufs == 1) {
      __syncthreads();  // every wave has summed unit u-1 from the single buffer
#pragma unroll
      for (int r = 0; r < 16; ++r) rw[(wave * 16 + r) * 64 + lane] = acc[r] - 128.0f * accx[r];
      if (more) read_stage();  // its latency overlaps the barrier
      __syncthreads();
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) rw[(wave * 16 + r) * 64 + lane] = acc[r] - 128.0f * accx[r];
      __syncthreads();  // partials of unit u complete; every wave's DMAs of unit u+1 landed
      if (more) read_stage();
    }
    d_prev = d_cur;
    row_prev = row_cur;
    bias_prev = bias_cur;
    scale_prev = scale_cur;
    g_cur = g_nxt;
    d_cur = d_nxt;
    row_cur = row_nxt;
  }
  finish((u_end - 1 - u_begin) & (L::kRedBufs - 1), d_prev, row_prev, bias_prev, scale_prev);
}

// The current device's CU count (queried once per device).
int cu_count() {
  constexpr int kDevices = 64;
  static std::atomic<int> counts[kDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    dev = 0;
  }
  const int slot = dev >= 0 && dev < kDevices ? dev : 0;
  int v = counts[slot].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) {
    (void)hipGetLastError();
    v = 256;
  }
  counts[slot].store(v, std::memory_order_relaxed);
  return v;
}

// True when the streaming kernel covers K.
bool stream_k(int64_t K) { return K == 1024 || K == 2048 || K == 3072; }

template <int NW, int BPW>
int launch_stream(const uint16_t *x, int64_t ldx, int64_t M, const GemvDesc *descs, int count, const GemvDesc &one,
                  int64_t total_n, const Code16 &c, hipStream_t s) {
  using L = SgLayout<NW, BPW>;
  const int64_t units = cdiv(total_n, kSgRows) + count;
  const int64_t grid = min(units, static_cast<int64_t>(cu_count()));
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&nf4_gemv_stream<NW, BPW>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, L::kMaxBytes);
  if (attr != hipSuccess)
    return set_error(SELAS_EHIP, "nf4_linear: cannot reserve %d bytes of LDS: %s", L::kMaxBytes,
                     hipGetErrorString(attr));
  const size_t lds = L::kPrefix + (count + 1) * sizeof(int);
  nf4_gemv_stream<NW, BPW><<<dim3(static_cast<uint32_t>(grid)), dim3(L::kThreads), lds, s>>>(
      x, ldx, static_cast<int>(M), descs, count, one, c);
  return check_launch("nf4_linear (streaming skinny gemm)");
}

// total_n: sum of the weights' row counts (an upper bound on the work, for the grid size).
int launch_gemv_stream(const uint16_t *x, int64_t ldx, int64_t M, int64_t K, const GemvDesc *descs, int count,
                       const GemvDesc &one, int64_t total_n, const Code16 &c, hipStream_t s) {
  constexpr int NW = kSgWaves;
  switch (K) {
    case 1024: return launch_stream<NW, 1024 / 64 / NW>(x, ldx, M, descs, count, one, total_n, c, s);
    case 2048: return launch_stream<NW, 2048 / 64 / NW>(x, ldx, M, descs, count, one, total_n, c, s);
    case 3072: return launch_stream<NW, 3072 / 64 / NW>(x, ldx, M, descs, count, one, total_n, c, s);
    default: return set_error(SELAS_EUNSUPPORTED, "nf4_linear: streaming skinny kernel takes K = 1024, 2048, 3072");
  }
}

template <int NW, int BPW>
int launch_i8_stream(const uint16_t *x, int64_t ldx, int64_t M, const GemvDesc *descs, int count,
                     const GemvDesc &one, int64_t total_n, hipStream_t s) {
  using L = I8Layout<NW, BPW>;
  const int64_t units = cdiv(total_n, kSgRows) + count;
  const int64_t grid = min(units, static_cast<int64_t>(cu_count()));
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&int8_gemv_stream<NW, BPW>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, L::kMaxBytes);
  if (attr != hipSuccess)
    return set_error(SELAS_EHIP, "int8_row_linear: cannot reserve %d bytes of LDS: %s", L::kMaxBytes,
                     hipGetErrorString(attr));
  const size_t lds = L::kPrefix + (count + 1) * sizeof(int);
  int8_gemv_stream<NW, BPW><<<dim3(static_cast<uint32_t>(grid)), dim3(L::kThreads), lds, s>>>(
      x, ldx, static_cast<int>(M), descs, count, one);
  return check_launch("int8_row_linear (streaming skinny gemm)");
}

int launch_i8_gemv_stream(const uint16_t *x, int64_t ldx, int64_t M, int64_t K, const GemvDesc *descs, int count,
                          const GemvDesc &one, int64_t total_n, hipStream_t s) {
  constexpr int NW = 8;
  switch (K) {
    case 1024: return launch_i8_stream<NW, 1024 / 64 / NW>(x, ldx, M, descs, count, one, total_n, s);
    case 2048: return launch_i8_stream<NW, 2048 / 64 / NW>(x, ldx, M, descs, count, one, total_n, s);
    case 3072: return launch_i8_stream<NW, 3072 / 64 / NW>(x, ldx, M, descs, count, one, total_n, s);
    default:
      return set_error(SELAS_EUNSUPPORTED, "int8_row_linear: streaming skinny kernel takes K = 1024, 2048, 3072");
  }
}

// =========================================================================== GEMM (M > 32)

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


// LDS reads done, then a workgroup barrier; a compiler fence for LDS accesses.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }


// A compile-time bool for generic lambdas (decltype(tag)::value).
template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

// Interleaving of one sub-step: after each of the N MFMAs, V VALU
// instructions, and one LDS read after every R-th MFMA.
template <int N, int R, int V>
__device__ __forceinline__ void interleave_substep() {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                // MFMA
    if (i % R == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x002, V, 0);                // VALU
  }
}

// Fused-dequant GEMM. A workgroup is NW waves side by side along N; a wave
// owns MB*32 rows x CB*32 columns of the output (MB*CB tiles of 32x32, 16
// accumulator registers each):
//   MB=8, CB=2, NW=4: 256 x 256 tile, 256 accumulators, one wave per SIMD;
//                     each decoded weight fragment serves 8 MFMAs.
//   MB=4, CB=2, NW=8: 128 x 512 tile, 128 accumulators, two waves per SIMD
//                     (one wave's waits overlap the other's MFMAs); each
//                     decoded fragment serves 4 MFMAs.
// Either way the workgroup reads 128 KiB of x fragments from LDS per K block.
//
// Grid: workgroup b runs on XCD b % 8; tile t = (b % 8) * per_xcd + b / 8
// gives each XCD a contiguous range of tiles. Within a problem the tiles go in
// groups of 4 row slabs, row fastest, so that the workgroups an XCD runs at
// once share 4 row slabs of x and 8 weight strips in its L2.
//
// Pipeline per 64-wide K block kb (LDS stage kb % STAGES):
//   * the x tile of block kb+STAGES-1 is loaded by buffer->LDS DMA and its
//     packed codes / absmax into registers, STAGES-1 blocks ahead;
//   * sub-step s runs the MFMAs for k-slice s; after each MFMA the register
//     that held its x fragment is refilled with the next sub-step's fragment,
//     and the next sub-step's weight fragments are decoded in between;
//   * before sub-step 3 the block kb+1 loads are waited for and the
//     workgroup synchronises; sub-step 3 then overlaps with building the
//     product tables and first fragments of block kb+1.
// Weight codecs of the tiled GEMM. kNF4: `packed` holds two 4-bit codes per
// byte, `absmax` one fp32 scale per 64-block. kInt8Row: `packed` holds int8
// values q [N, K], `absmax` one fp32 scale s per row; the operand is
// bf16(q * bf16(s)) (selas/codecs.py:273-277 decodes with q.to(bf16) *
// s.to(bf16)).
enum class WCodec { kNF4, kInt8Row };

// The per-block weight registers of one wave: CB column groups, one 64-wide K
// block. NF4: 16 code bytes and the block scale per lane; int8: 32 bytes.
template <WCodec WC, int CB>
struct WRegs {
  uint4 q[CB];
  float s[CB];
};
template <int CB>
struct WRegs<WCodec::kInt8Row, CB> {
  uint4 q[CB][2];
};

// Eight int8 values (dwords d0, d1, element j in byte j % 4 of d(j / 4)) ->
// bf16(q * sb) in k order, sb = bf16(scale) as fp32 and nb = -128 * sb. The
// biased byte u = q + 128 converts exactly to fp32 and fma(u, sb, nb) is the
// exact product q * sb (at most 16 significant bits), rounded once to bf16.
__device__ __forceinline__ bf16x8 dequant8_i8(uint32_t d0, uint32_t d1, float sb, float nb) {
  const uint32_t u0 = d0 ^ 0x80808080u, u1 = d1 ^ 0x80808080u;
  auto f = [&](uint32_t u, int j) { return __builtin_fmaf(static_cast<float>((u >> (8 * j)) & 0xffu), sb, nb); };
  uint4 r;
  r.x = pack_bf16x2(f(u0, 0), f(u0, 1));
  r.y = pack_bf16x2(f(u0, 2), f(u0, 3));
  r.z = pack_bf16x2(f(u1, 0), f(u1, 1));
  r.w = pack_bf16x2(f(u1, 2), f(u1, 3));
  return __builtin_bit_cast(bf16x8, r);
}

// One problem of a batched launch; its tiles are global tiles [tile0, tile0 + tiles_m * tiles_n).
// Output columns [n_split, N) are written as bf16(gelu_tanh(bf16(acc + bias)))
// to Y2 at column n - n_split (row stride ldy2); n_split is N (no such columns)
// or a multiple of the 256-column tile, so that a tile lies on one side.
struct GemmProblem {
  const uint16_t *X;
  const uint8_t *packed;
  const float *absmax;
  const uint16_t *bias;
  uint16_t *Y, *Y2;
  int64_t ldx, ldy, ldy2;
  int M, K, N, n_split, tiles_n, tile0;
};
constexpr int kGemmMaxProblems = 4;
// Tiles [0, tiles - tail) run whole, one workgroup each: workgroup b < dp_blocks
// takes tile (b % 8) * per_xcd + b / 8. The last `tail` tiles (a last round that
// would leave most CUs idle) run as `split` K ranges each, one workgroup per
// (range r, tile): item j = r * tail + q, taken by workgroup dp_blocks + b' with
// j = (b' % 8) * tail_per_xcd + b' / 8, so each XCD runs one K range of
// consecutive tiles. A split item leaves its fp32 partial tile in part[j] and
// gemm_tail_sum adds the ranges in K order.
struct GemmBatch {
  GemmProblem p[kGemmMaxProblems];
  int count, tiles, per_xcd;
  int tail, split, dp_blocks, tail_per_xcd;
  float *part;
};

// Origin (m0, n0) of tile t of problem P (t in [P.tile0, P.tile0 + tiles)). The
// tiles go in groups of kGroupM row slabs, the row index fastest inside a
// group: the 32 tiles an XCD runs at once then cover 4 row slabs x 8 weight
// strips instead of 1 x 32, so fewer distinct x and weight blocks miss its L2
// per K step (linear1 558 us instead of 563 us).
template <int TM, int TN>
__device__ __forceinline__ void tile_origin(const GemmProblem &P, int t, int &m0, int &n0) {
  constexpr int kGroupM = 4;
  const int lt = t - P.tile0, tiles_m = (P.M + TM - 1) / TM, tiles_n = P.tiles_n;
  const int group = lt / (kGroupM * tiles_n), first_m = group * kGroupM;
  const int gm = min(kGroupM, tiles_m - first_m), in = lt - group * kGroupM * tiles_n;
  m0 = (first_m + in % gm) * TM;
  n0 = (in / gm) * TN;
}

// The problem a tile belongs to (uniform: scalar selects over the kernel arguments).
__device__ __forceinline__ GemmProblem tile_problem(const GemmBatch &batch, int t) {
  GemmProblem P = batch.p[0];
#pragma unroll
  for (int i = 1; i < kGemmMaxProblems; ++i)
    if (i < batch.count && t >= batch.p[i].tile0) P = batch.p[i];
  return P;
}

// SPLIT: the launch has split items (a kernel of its own, since the partial-tile
// stores make the compiler spill registers in the epilogue of every tile).
template <WCodec WC, int MB, int CB, int STAGES, int NW, bool SPLIT = false>
__device__ __forceinline__ void qgemm_body(GemmBatch batch, const Code16 &code) {
  constexpr bool kI8 = WC == WCodec::kInt8Row;
  using WR = WRegs<WC, CB>;
  constexpr int TM = 32 * MB, WN = 32 * CB, TN = NW * WN;
  constexpr int SB = TM * 128;      // bytes of one x stage: TM rows x 64 bf16
  constexpr int LOOK = STAGES - 1;
  constexpr int XL = 4 * MB / NW;   // x DMAs (8 rows each) per K block and wave
  constexpr int LPB = 2 * CB + XL;  // vector-memory loads issued per K block and wave
  static_assert(MB * CB * NW <= 64 && 4 * MB % NW == 0 && (STAGES == 2 || STAGES == 3), "tile shape");
  // The x stages, then 1 KiB per wave for its bias columns.
  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * SB + NW * 1024];
  // Work item: a whole tile t, or split item j (K range j / tail of tile t).
  int t, j = -1;
  if (!SPLIT || static_cast<int>(blockIdx.x) < batch.dp_blocks) {
    t = (blockIdx.x & 7) * batch.per_xcd + (blockIdx.x >> 3);
    if (t >= batch.tiles - (SPLIT ? batch.tail : 0)) return;
  } else {
    const int bt = static_cast<int>(blockIdx.x) - batch.dp_blocks;
    j = (bt & 7) * batch.tail_per_xcd + (bt >> 3);
    if (j >= batch.tail * batch.split) return;
    t = batch.tiles - batch.tail + j % batch.tail;
  }
  const GemmProblem P = tile_problem(batch, t);
  const int64_t ldx = P.ldx, ldy = P.ldy;
  const int M = P.M, K = P.K, N = P.N;
  const int kblocks = K >> 6;
  // K blocks [kb_lo, kb_lo + nblk) of the tile: all of them, or range j / tail of `split` near-equal ranges.
  int kb_lo = 0, nblk = kblocks;
  if (SPLIT && j >= 0) {
    const int r = j / batch.tail;
    kb_lo = r * kblocks / batch.split;
    nblk = (r + 1) * kblocks / batch.split - kb_lo;
  }
  // The operands start at block kb_lo; the loop below indexes blocks from 0.
  const uint16_t *__restrict__ X = P.X + 64 * kb_lo;
  const uint8_t *__restrict__ packed = P.packed + (kI8 ? 64 : 32) * kb_lo;
  const float *__restrict__ absmax = P.absmax + (kI8 ? 0 : kb_lo);
  const uint16_t *__restrict__ bias = P.bias;
  uint16_t *__restrict__ Y = P.Y;
  const int tid = threadIdx.x;
  // The wave index as a scalar: the LDS addresses of the x DMA (taken from M0) are then scalar arithmetic.
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, c = lane & 31;
  int m0, n0;
  tile_origin<TM, TN>(P, t, m0, n0);
  const uint32_t ldx_b = static_cast<uint32_t>(ldx) * 2u;

  // Buffer resources; the range check covers the per-lane offset, which holds
  // the row term, so rows past M or N read as zeros (never stored). With the
  // bases moved to block kb_lo the ranges shrink by the same amount, so the
  // last row's blocks stay inside and the rows past the end stay outside.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(X, static_cast<uint32_t>(M) * ldx_b - 128u * kb_lo);
  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(packed, static_cast<uint32_t>(N) * static_cast<uint32_t>(kI8 ? K : (K >> 1)) - (kI8 ? 64u : 32u) * kb_lo);
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(absmax, static_cast<uint32_t>(N) * static_cast<uint32_t>(kI8 ? 1 : kblocks) * 4u - (kI8 ? 0u : 4u) * kb_lo);

  // x tile DMA: wave w fills tile rows [8*XL*w, 8*XL*(w+1)) with XL loads of 8
  // rows; lane i of load j lands at row r = 8*XL*w + 8j + i/8, physical
  // 16-byte chunk i%8, and so fetches logical chunk (i%8) ^ ((r/2)%8). With
  // that swizzle the 16 lanes one LDS cycle serves in a fragment read (16
  // consecutive rows, one logical chunk) hit 16 distinct 4-bank groups of the
  // 64 banks. (r/2)%8 = (4(XL*w + j) + i/16) % 8 depends on w and j only
  // through the parity of XL*w + j.
  uint32_t a_voff[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    a_voff[par] = static_cast<uint32_t>(m0 + 8 * XL * wave + (lane >> 3)) * ldx_b +
                  (static_cast<uint32_t>((lane & 7) ^ ((4 * (par ^ ((XL * wave) & 1)) + (lane >> 4)) & 7)) << 4);
  const uint32_t a_vstep = 8u * ldx_b;
  uint8_t *const a_dst = smem + wave * XL * 1024;
  // Weight rows of this wave: n0 + WN*wave + 32*cb + c.
  uint32_t b_voff[CB], s_voff[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const uint32_t n = static_cast<uint32_t>(n0 + WN * wave + 32 * cb + c);
    if constexpr (kI8) {
      b_voff[cb] = n * static_cast<uint32_t>(K) + 32u * h;
      s_voff[cb] = n * 4u;
    } else {
      b_voff[cb] = n * static_cast<uint32_t>(K >> 1) + 16u * h;
      s_voff[cb] = n * static_cast<uint32_t>(kblocks) * 4u;
    }
  }
  // int8: the row scale, bf16-rounded as the reference's decode rounds it, and -128 times it.
  float sb[CB], nb[CB];
  if constexpr (kI8) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      sb[cb] = bf16_bits_to_f32(bf16_bits_rne(load_f32(sr, s_voff[cb], 0)));
      nb[cb] = -128.0f * sb[cb];
    }
  }
  float cl[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cl[i] = h ? code.v[8 + i] : code.v[i];
  // LDS offset of this lane's x fragment for sub-step s (row slab mb adds mb*4096).
  uint32_t a_rd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) a_rd[s] = c * 128 + (((4 * h + s) ^ ((c >> 1) & 7)) << 4);

  // Loads block `blk` into LDS stage `stage` and the registers bq/bs; the
  // register loads go first so that later uses of them do not wait for the DMA.
  auto load_w = [&](uint32_t kb, WR &w) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      if constexpr (kI8) {
        w.q[cb][0] = load_b128(wr, b_voff[cb], kb * 64u);
        w.q[cb][1] = load_b128(wr, b_voff[cb], kb * 64u + 16u);
      } else {
        w.q[cb] = load_b128(wr, b_voff[cb], kb * 32u);
        w.s[cb] = load_f32(sr, s_voff[cb], kb * 4u);
      }
    }
  };
  auto issue = [&](int stage, int blk, WR &w) {
    const uint32_t kb = static_cast<uint32_t>(blk);
    load_w(kb, w);
    uint8_t *dst = a_dst + stage * SB;
#pragma unroll
    for (int j = 0; j < XL; ++j) load_lds16(xr, dst + j * 1024, a_voff[j & 1] + j * a_vstep, kb * 128u);
  };
  // The same loads in four parts, one per sub-step, so that a wave never
  // queues a whole block's loads at once (issue would stall on the address
  // unit instead of overlapping the MFMAs): part 0 the codes, scales and the
  // first x loads, parts 1-3 the rest of the x tile (x load j in part 4j/XL).
  constexpr int P3 = XL - (3 * XL + 3) / 4;  // x loads in part 3
  auto issue_part = [&](int stage, int blk, int part, WR &w) {
    const uint32_t kb = static_cast<uint32_t>(blk);
    if (part == 0) load_w(kb, w);
    uint8_t *dst = a_dst + stage * SB;
#pragma unroll
    for (int j = (part * XL + 3) / 4; j < ((part + 1) * XL + 3) / 4; ++j)
      load_lds16(xr, dst + j * 1024, a_voff[j & 1] + j * a_vstep, kb * 128u);
  };
  auto frag = [&](int kb, int s, int mb) {
    return *reinterpret_cast<const bf16x8 *>(smem + (kb % STAGES) * SB + a_rd[s] + mb * 4096);
  };
  auto word = [](const uint4 &q, int s) { return s == 0 ? q.x : s == 1 ? q.y : s == 2 ? q.z : q.w; };
  // Weight fragment of column group cb for sub-step s (k in [32h + 8s, 32h + 8s + 8) of the block).
  auto wfrag = [&](const WR &w, int cb, int s, const Tables &t) -> bf16x8 {
    if constexpr (kI8) {
      const uint4 &q = w.q[cb][s >> 1];
      return dequant8_i8((s & 1) ? q.z : q.x, (s & 1) ? q.w : q.y, sb[cb], nb[cb]);
    } else {
      return dequant8(t, word(w.q[cb], s));
    }
  };

  f32x16 acc[MB][CB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[mb][cb] = f32x16{};

  // The wave's 64 bias values (128 bytes) into its LDS bias area by DMA, ahead of
  // the first block's loads (the first wait below covers it); the staged
  // epilogue reads them there instead of waiting for loads issued after the K
  // loop. Lanes 8-63 read past the range and write zeros.
  uint8_t *const bias_lds = smem + STAGES * SB + wave * 1024;
  const bool bias_dma = (!SPLIT || j < 0) && bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 15) == 0;
  if (bias_dma)
    load_lds16(make_rsrc(bias, static_cast<uint32_t>(N) * 2u), bias_lds,
               lane < 8 ? static_cast<uint32_t>(n0 + WN * wave + 8 * lane) * 2u : 0xfffffff0u, 0);
  // Every iteration issues the loads of block kb+LOOK; past the last block the
  // last block is loaded again (valid addresses, into the stage that is free)
  // so that the loop body has no branches and schedules as one region.
  WR w0, w1, w2;
  issue(0, 0, w0);
  if constexpr (STAGES == 3) {
    issue(1, min(1, nblk - 1), w1);
    wait_vmcnt<LPB>();
  } else {
    wait_vmcnt<0>();
  }
  lds_barrier();

  bf16x8 af[MB], wf[2][CB];
  Tables tab[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    if constexpr (!kI8) tab[cb] = make_tables(cl, w0.s[cb]);
    wf[0][cb] = wfrag(w0, cb, 0, tab[cb]);
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) af[mb] = frag(0, 0, mb);

  // One K block. cw holds block kb's weights, nw block kb+1's, fw receives
  // block kb+LOOK's (with one block of lookahead that is nw itself). The loop
  // below is unrolled STAGES times so that the register sets rotate by name,
  // never by copying registers that a load in flight still targets.
  //
  // The blocks after the unrolled loop (K/64 not a multiple of STAGES) issue no
  // loads and wait for all outstanding ones before their barrier: all their
  // look-ahead would be past the end of K, and the compiler deletes register
  // loads whose values are never used, so a count of younger loads (as the
  // loop's wait uses) would be short there and let the next block's last x
  // loads still be in flight at the barrier (measured: wrong outputs for
  // K = 2048 when another kernel ran on the GPU at the same time).
  auto block = [&](int kb, const WR &cw, const WR &nw, WR &fw, auto tail_tag) __attribute__((always_inline)) {
    constexpr bool kTail = decltype(tail_tag)::value;
    const int fstage = (kb + LOOK) % STAGES, fblk = min(kb + LOOK, nblk - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s < 3) {
        if constexpr (kTail) {
        } else if constexpr (LOOK >= 2) {
          issue_part(fstage, fblk, s, fw);
        } else if (s == 0) {
#pragma unroll
          for (int part = 0; part < 4; ++part) issue_part(fstage, fblk, part, fw);
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) wf[nxt][cb] = wfrag(cw, cb, s + 1, tab[cb]);
      } else {
        if constexpr (kTail) {
          wait_vmcnt<0>();
          lds_barrier();
        } else if constexpr (LOOK >= 2) {
          // Block kb+1's loads are older than parts 0-2 of block kb+LOOK's.
          wait_vmcnt<(LOOK - 1) * LPB - P3>();
          lds_barrier();
          issue_part(fstage, fblk, 3, fw);
        } else {
          wait_vmcnt<0>();
          lds_barrier();
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          if constexpr (!kI8) tab[cb] = make_tables(cl, nw.s[cb]);
          wf[nxt][cb] = wfrag(nw, cb, 0, tab[cb]);
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[mb][cb] = mfma32(wf[cur][cb], af[mb], acc[mb][cb]);
        af[mb] = s < 3 ? frag(kb, s + 1, mb) : frag(kb + 1, 0, mb);
      }
      constexpr int F = MB * CB;  // MFMAs per sub-step
      // VALU per column group and sub-step: NF4 26 (50 with the product tables), int8 22.
      constexpr int VS = kI8 ? 22 : 26, VL = kI8 ? 22 : 50;
      if (s < 3) interleave_substep<F, CB, (VS * CB + F - 1) / F + 1>();
      else interleave_substep<F, CB, (VL * CB + F - 1) / F + 1>();
    }
    // One scheduling region per K block. Without this fence the slot matching
    // of the interleave shifts by one sub-step after the first block's barrier
    // and two thirds of the x-fragment reads land 3-5 MFMAs before their use;
    // with it most land 9-13 MFMAs ahead (NF4 block linears +1.3 %). The int8 operand's
    // reads stay about 3 MFMAs ahead with or without it.
    if constexpr (!kI8) __builtin_amdgcn_sched_barrier(0);
  };

  // In the split kernel, wait here for everything read through the scalar cache
  // (the workspace pointer is a kernel argument that only the epilogue uses):
  // with a scalar load still pending at the loop, the first LDS wait of every
  // iteration would have to be lgkmcnt(0), since scalar loads complete out of
  // order (measured on linear1: 4 % slower).
  if constexpr (SPLIT) __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt and expcnt unconstrained
  int kb = 0;
  if constexpr (STAGES == 3) {
    for (; kb + 3 <= nblk; kb += 3) {
      block(kb, w0, w1, w2, BoolTag<false>{});
      block(kb + 1, w1, w2, w0, BoolTag<false>{});
      block(kb + 2, w2, w0, w1, BoolTag<false>{});
    }
    if (kb < nblk) block(kb, w0, w1, w2, BoolTag<true>{});
    if (kb + 1 < nblk) block(kb + 1, w1, w2, w0, BoolTag<true>{});
  } else {
    for (; kb + 2 <= nblk; kb += 2) {
      block(kb, w0, w1, w1, BoolTag<false>{});
      block(kb + 1, w1, w0, w0, BoolTag<false>{});
    }
    if (kb < nblk) block(kb, w0, w1, w1, BoolTag<true>{});
  }
  (void)w2;

  if constexpr (SPLIT) {
    if (j >= 0) {
      // A split item leaves its fp32 partial tile in part[j], fragment-major:
      // each store instruction writes 1 KiB (64 lanes x 16 bytes). Its wave's
      // DMAs land before it ends, so none can reach the LDS of a later workgroup.
      const __amdgpu_buffer_rsrc_t pr = make_rsrc(batch.part + static_cast<int64_t>(j) * (TM * TN), TM * TN * 4);
      int pl = tid & 63;
      asm volatile("" : "+v"(pl));
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__float_as_uint(acc[mb][cb][4 * q]), __float_as_uint(acc[mb][cb][4 * q + 1]),
                      __float_as_uint(acc[mb][cb][4 * q + 2]), __float_as_uint(acc[mb][cb][4 * q + 3])},
                pr, static_cast<uint32_t>(pl) * 16u, wave * (MB * CB * 4096) + ((mb * CB + cb) * 4 + q) * 1024, 0);
      wait_vmcnt<0>();
      return;
    }
  }

  // Epilogue: acc[mb][cb] holds D[n][m] for n = n0 + WN*wave + 32*cb + 8*(r/4) + 4*h + r%4
  // and m = m0 + 32*mb + c. Bias is added in fp32 and the sum rounded once.
  // A tile past n_split holds GELU columns (uniform over the workgroup): the sum
  // is rounded to bf16 as it would be stored, GELU'd in fp32 and rounded again,
  // exactly what a separate GELU kernel reading the stored output computes.
  const bool gelu = n0 >= P.n_split;
  uint16_t *const Yo = gelu ? P.Y2 : Y;
  const int64_t ldo = gelu ? P.ldy2 : ldy;
  const int cs = gelu ? P.n_split : 0;  // column shift into Yo
  // GELU of the value rounded to bf16 as it would be stored (both roundings by the hardware convert).
  auto gelu1 = [](float v) {
    const uint32_t r = pack_bf16x2(v, 0.0f);
    return static_cast<uint16_t>(gelu_bf16x2(bf16_bits_to_f32(r & 0xffffu), 0.0f) & 0xffffu);
  };
  // The output goes through LDS when the wave's 64 columns lie inside N and the
  // output rows are 16-byte aligned (every full tile of the block linears).
  const bool staged = n0 + WN * (wave + 1) <= N && (ldo & 7) == 0 && (reinterpret_cast<uintptr_t>(Yo) & 15) == 0;
  // The staged path's bias: from the wave's LDS bias area when the prologue
  // loaded it there, else 2-byte buffer loads with no branches, all issued
  // before the drain below so that their latency overlaps it (a null bias is an
  // empty range and reads as zeros). Per-element guarded loads, each waited
  // for in turn, took ~1.5 us per tile; loads issued after the K loop, ~1 us.
  uint32_t bb[CB][4][4];
  if (staged && !bias_dma) {
    const __amdgpu_buffer_rsrc_t br = make_rsrc(bias, bias ? static_cast<uint32_t>(N) * 2u : 0u);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4)
          bb[cb][q][t4] = __builtin_amdgcn_raw_buffer_load_b16(
              br, static_cast<uint32_t>(n0 + WN * wave + 32 * cb + 8 * q + 4 * h + t4) * 2u, 0, 0);
  }
  // Every wave is done with the x stages before any wave stages its output
  // there: its own loads into LDS have landed (the last K blocks' look-ahead
  // DMAs may still be in flight; the workgroup barrier alone does not wait for
  // them) and the barrier then covers the other waves. It comes before the
  // per-wave choice of store path, so that every wave of the workgroup reaches
  // it, and it also leaves no DMA in flight when the workgroup ends.
  wait_vmcnt<0>();
  __syncthreads();
  if (staged) {
    if (bias_dma) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint2 v = *reinterpret_cast<const uint2 *>(bias_lds + 2 * (32 * cb + 8 * q + 4 * h));
          bb[cb][q][0] = v.x & 0xffffu;
          bb[cb][q][1] = v.x >> 16;
          bb[cb][q][2] = v.y & 0xffffu;
          bb[cb][q][3] = v.y >> 16;
        }
    }
    // Through LDS, so that every store writes whole 128-byte row segments: a
    // direct store from the MFMA layout writes 16 bytes into each of 32 rows,
    // and each partial line then reaches HBM as a write of its own. Each wave
    // stages HR*32 rows x WN columns at a time (row stride WN*2+8 bytes: the
    // 8-byte writes of 32 lanes then hit distinct banks), in its own region.
    // The GELU choice is made once for the whole tile: tested per value pair,
    // its branches took ~3 us per tile of the 256-row kernel.
    constexpr int RS = WN * 2 + 8;
    constexpr int HR = (MB % 2 == 0 && NW * (MB / 2) * 32 * RS <= STAGES * SB) ? MB / 2 : 1;
    static_assert(NW * HR * 32 * RS <= STAGES * SB && MB % HR == 0, "epilogue staging fits the x stages");
    uint8_t *ep = smem + wave * HR * 32 * RS;
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(Yo, static_cast<uint32_t>(min(static_cast<int64_t>(M) * ldo * 2,
                                                                              static_cast<int64_t>(0xffffffff))));
    // The lane index again, opaque to the compiler: values derived from it here
    // are then not shared with the prologue's, which the register-bound K loop
    // would spill (a reload before every store, each waiting for the stores
    // issued before it).
    int lo_lane = tid & 63;
    asm volatile("" : "+v"(lo_lane));
    const int ec = lo_lane & 31, eh = lo_lane >> 5;
    auto stage_out = [&](auto gelu_tag) {
      constexpr bool G = decltype(gelu_tag)::value;
#pragma unroll
      for (int piece = 0; piece < MB / HR; ++piece) {
#pragma unroll
        for (int mh = 0; mh < HR; ++mh) {
          const int mb = HR * piece + mh;
#pragma unroll
          for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              float v[4];
#pragma unroll
              for (int t4 = 0; t4 < 4; ++t4) v[t4] = acc[mb][cb][4 * q + t4] + bf16_bits_to_f32(bb[cb][q][t4]);
              uint32_t lo, hi;
              if constexpr (G) {
                const uint32_t r01 = pack_bf16x2(v[0], v[1]), r23 = pack_bf16x2(v[2], v[3]);
                lo = gelu_bf16x2(bf16_bits_to_f32(r01 & 0xffffu), bf16_bits_to_f32(r01 >> 16));
                hi = gelu_bf16x2(bf16_bits_to_f32(r23 & 0xffffu), bf16_bits_to_f32(r23 >> 16));
              } else {
                lo = pack_bf16x2(v[0], v[1]);
                hi = pack_bf16x2(v[2], v[3]);
              }
              *reinterpret_cast<uint2 *>(ep + (32 * mh + ec) * RS + 2 * (32 * cb + 8 * q + 4 * eh)) = make_uint2(lo, hi);
            }
        }
        // Row r of the staged block: WN/8 lanes x 16 bytes; a wave stores 512/WN rows per instruction.
        constexpr int LPR = WN / 8, RPI = 64 / LPR;
#pragma unroll
        for (int j = 0; j < HR * 32 / RPI; ++j) {
          const int r = RPI * j + lo_lane / LPR, col = 8 * (lo_lane % LPR);
          const uint8_t *src = ep + r * RS + 2 * col;
          const uint2 v0 = *reinterpret_cast<const uint2 *>(src), v1 = *reinterpret_cast<const uint2 *>(src + 8);
          const int m = m0 + 32 * HR * piece + r;
          // Rows past M fall outside the buffer range and are dropped.
          const uint32_t off = m < M ? static_cast<uint32_t>((static_cast<int64_t>(m) * ldo + n0 - cs + WN * wave + col) * 2)
                                     : 0xffffffffu;
          typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
          __builtin_amdgcn_raw_buffer_store_b128(u32x4{v0.x, v0.y, v1.x, v1.y}, yr, off, 0, 0);
        }
      }
    };
    if (gelu) stage_out(BoolTag<true>{});
    else stage_out(BoolTag<false>{});
    return;
  }
  // Direct stores (partial column tiles, unaligned outputs).
  float bv[CB][4][4];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const int n = n0 + WN * wave + 32 * cb + 8 * q + 4 * h + t4;
        bv[cb][q][t4] = (bias && n < N) ? bf16_bits_to_f32(bias[n]) : 0.0f;
      }
  auto out2 = [&](float a, float b) -> uint32_t {
    if (gelu) return gelu1(a) | (static_cast<uint32_t>(gelu1(b)) << 16);
    return pack_bf16x2(a, b);
  };
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + WN * wave + 32 * cb + 8 * q + 4 * h;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = m0 + 32 * mb + c;
        if (m >= M) continue;
        uint16_t *dst = Yo + static_cast<int64_t>(m) * ldo + (n - cs);
        const float v0 = acc[mb][cb][4 * q] + bv[cb][q][0], v1 = acc[mb][cb][4 * q + 1] + bv[cb][q][1];
        const float v2 = acc[mb][cb][4 * q + 2] + bv[cb][q][2], v3 = acc[mb][cb][4 * q + 3] + bv[cb][q][3];
        if (n + 3 < N) {
          *reinterpret_cast<uint2 *>(dst) = make_uint2(out2(v0, v1), out2(v2, v3));
        } else {
          const float v[4] = {v0, v1, v2, v3};
          for (int t4 = 0; t4 < 4 && n + t4 < N; ++t4)
            dst[t4] = gelu ? gelu1(v[t4]) : bf16_bits_rne(v[t4]);
        }
      }
    }
  }
}

template <int MB, int CB, int STAGES, int NW, bool SPLIT = false>
__global__ __launch_bounds__(64 * NW, 1) void nf4_gemm_kernel(GemmBatch batch, Code16 code) {
  qgemm_body<WCodec::kNF4, MB, CB, STAGES, NW, SPLIT>(batch, code);
}
template <int MB, int CB, int STAGES, int NW, bool SPLIT = false>
__global__ __launch_bounds__(64 * NW, 1) void int8_row_gemm_kernel(GemmBatch batch) {
  qgemm_body<WCodec::kInt8Row, MB, CB, STAGES, NW, SPLIT>(batch, Code16{});
}

// The outputs of the split tiles: each thread adds one 4-column group's K
// ranges in K order (range 0 first, so the sum is the same on every run) and
// finishes it as the tiled kernel's epilogue does: bias added in fp32 and the
// sum rounded once to bf16; GELU columns rounded, GELU'd and rounded again.
constexpr int kMaxSplit = 8;  // K ranges per split tile at most

template <int MB, int CB, int NW>
__global__ __launch_bounds__(256) void gemm_tail_sum(GemmBatch batch) {
  constexpr int TM = 32 * MB, WN = 32 * CB, TN = NW * WN, T4 = TM * TN / 4;
  const int e = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (e >= batch.tail * T4) return;
  // e = q * T4 + ((f * 4 + q4) * 64 + lane), f = (wave * MB + mb) * CB + cb: the split items' store order.
  const int q = e / T4, rem = e - q * T4;
  const int lane = rem & 63, q4 = (rem >> 6) & 3, f = rem >> 8;
  const int cb = f % CB, mb = (f / CB) % MB, wave = f / (CB * MB);
  // All ranges' loads first (up to kMaxSplit in flight), then the sums in K order.
  const float4 *src = reinterpret_cast<const float4 *>(batch.part) + static_cast<int64_t>(q) * T4 + rem;
  float4 p[kMaxSplit];
#pragma unroll
  for (int r = 0; r < kMaxSplit; ++r)
    if (r < batch.split) p[r] = src[static_cast<int64_t>(r) * batch.tail * T4];
  float4 v = p[0];
#pragma unroll
  for (int r = 1; r < kMaxSplit; ++r)
    if (r < batch.split) {
      v.x += p[r].x;
      v.y += p[r].y;
      v.z += p[r].z;
      v.w += p[r].w;
    }
  const int t = batch.tiles - batch.tail + q;
  const GemmProblem P = tile_problem(batch, t);
  int m0, n0;
  tile_origin<TM, TN>(P, t, m0, n0);
  const int m = m0 + 32 * mb + (lane & 31);
  const int n = n0 + WN * wave + 32 * cb + 8 * q4 + 4 * (lane >> 5);
  if (m >= P.M || n >= P.N) return;
  const bool gelu = n0 >= P.n_split;
  uint16_t *const dst = (gelu ? P.Y2 : P.Y) + static_cast<int64_t>(m) * (gelu ? P.ldy2 : P.ldy) + (n - (gelu ? P.n_split : 0));
  float a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int t4 = 0; t4 < 4; ++t4)
    a[t4] += (P.bias && n + t4 < P.N) ? bf16_bits_to_f32(P.bias[n + t4]) : 0.0f;
  // Each value rounded to bf16 by the hardware convert; for GELU columns that
  // rounded value GELU'd and rounded again.
  auto out1 = [&](float x) -> uint32_t {
    const uint32_t r = pack_bf16x2(x, 0.0f) & 0xffffu;
    return gelu ? gelu_bf16x2(bf16_bits_to_f32(r), 0.0f) & 0xffffu : r;
  };
  if (n + 3 < P.N) {
    *reinterpret_cast<uint2 *>(dst) = make_uint2(out1(a[0]) | (out1(a[1]) << 16), out1(a[2]) | (out1(a[3]) << 16));
  } else {
    for (int t4 = 0; t4 < 4 && n + t4 < P.N; ++t4) dst[t4] = static_cast<uint16_t>(out1(a[t4]));
  }
}

// fp32 partial tiles of a split launch: split * tail tiles of 256 x 256 floats.
constexpr int64_t kSplitTileBytes = 256 * 256 * 4;

// How a tiled batch runs: tile height 32 * mb, and whether the last round's
// `tail` tiles run as `split` K ranges each. Chosen from the shapes and the
// GPU's CU count only, so a call's bits never depend on anything else.
struct GemmPlan {
  int mb = 8;
  int split = 1;
  int64_t tail = 0;
  int64_t workspace_bytes() const { return split > 1 ? tail * split * kSplitTileBytes : 0; }
};

// `batch.p[0..count)` filled except tiles_n / tile0, which are set here. With
// split > 1 the last round's tiles (tiles % CUs of them, MB = 8) run as `split`
// K ranges each, their fp32 partial tiles in `part`.
template <int MB, int CB, int STAGES, int NW>
void launch_gemm(GemmBatch &batch, const Code16 &c, hipStream_t s, WCodec wc, int split, float *part) {
  int64_t tiles = 0;
  for (int i = 0; i < batch.count; ++i) {
    GemmProblem &p = batch.p[i];
    const int64_t tiles_m = cdiv(p.M, 32 * MB), tiles_n = cdiv(p.N, 32 * CB * NW);
    p.tiles_n = static_cast<int>(tiles_n);
    p.tile0 = static_cast<int>(tiles);
    tiles += tiles_m * tiles_n;
  }
  constexpr int64_t kTileBytes = 32 * MB * 32 * CB * NW * 4;
  static_assert(MB != 8 || kTileBytes == kSplitTileBytes, "split tile size");
  batch.tiles = static_cast<int>(tiles);
  batch.tail = MB == 8 && split > 1 ? static_cast<int>(tiles % cu_count()) : 0;
  batch.split = batch.tail ? split : 1;
  batch.part = batch.tail ? part : nullptr;
  batch.per_xcd = static_cast<int>(cdiv(tiles - batch.tail, 8));
  batch.dp_blocks = batch.per_xcd * 8;
  batch.tail_per_xcd = static_cast<int>(cdiv(static_cast<int64_t>(batch.tail) * batch.split, 8));
  const dim3 grid(static_cast<uint32_t>(batch.dp_blocks + 8 * batch.tail_per_xcd)), block(64 * NW);
  if (batch.tail == 0) {
    if (wc == WCodec::kInt8Row) int8_row_gemm_kernel<MB, CB, STAGES, NW><<<grid, block, 0, s>>>(batch);
    else nf4_gemm_kernel<MB, CB, STAGES, NW><<<grid, block, 0, s>>>(batch, c);
  } else if constexpr (MB == 8) {
    if (wc == WCodec::kInt8Row) int8_row_gemm_kernel<MB, CB, STAGES, NW, true><<<grid, block, 0, s>>>(batch);
    else nf4_gemm_kernel<MB, CB, STAGES, NW, true><<<grid, block, 0, s>>>(batch, c);
    const int64_t groups = static_cast<int64_t>(batch.tail) * (kTileBytes / 16);
    gemm_tail_sum<MB, CB, NW><<<dim3(static_cast<uint32_t>(cdiv(groups, 256))), dim3(256), 0, s>>>(batch);
  }
}

// Tiles of 4 waves side by side (each 64 columns), 3 LDS stages, and 256, 224
// or 192 rows (MB = 8, 7, 6). The tiles run in rounds of one per CU; a launch
// takes the height with the least rounds x relative tile time, the tile times
// measured on the 1536-token linear (M 1536, N 12288, K 3072: one 256-row tile
// 83 us, 224 rows 72 us, 192 rows 66 us; 128 rows measured slower again). There
// 192-row tiles fill two rounds (384 tiles) where 256-row ones leave the second
// round an eighth full: 165 -> 131 us. A launch of 216 256-row tiles (M 4608,
// N 3072) takes 252 224-row ones, the same single round.
// 128 x 512 tiles of 8 waves (128 x 64 each, two waves per SIMD) measured 15-25 %
// slower: each decoded weight fragment then serves 4 MFMAs instead of 8.
GemmPlan plan_gemm(const GemmBatch &batch, WCodec wc) {
  auto cost = [&](int mb, double tile_time) {
    int64_t tiles = 0;
    for (int i = 0; i < batch.count; ++i) tiles += cdiv(batch.p[i].M, 32 * mb) * cdiv(batch.p[i].N, 256);
    return static_cast<double>(cdiv(tiles, cu_count())) * tile_time;
  };
  // Smaller tiles only when they win by more than 2 % (ties keep the taller tile).
  const double c8 = cost(8, 1.0), c7 = cost(7, 0.87), c6 = cost(6, 0.80);
  // One round of 256-row tiles that keeps at least 3/4 of the CUs busy: the chip
  // is then power-bound, shorter tiles in one round finish no sooner, and the
  // taller tile does the same work with fewer tiles (4608 x 3072 x 15360: 374 us
  // with 256-row tiles, 390 us with 224, 574 us with 192). The int8 operand's
  // kernel keeps the cost model (256-row tiles made that shape slower).
  int64_t t8 = 0;
  for (int i = 0; i < batch.count; ++i) t8 += cdiv(batch.p[i].M, 256) * cdiv(batch.p[i].N, 256);
  const int64_t cu = cu_count();
  // Split tail (one K for the whole launch): the whole rounds of 256-row
  // tiles, then the last round's tiles as S K ranges each, so that the last
  // round takes ~1/S of a tile's K loop instead of all of it. Estimated in us: a
  // 256-row tile takes ~14 + 1.48 per K block (fit over K = 3072..15360), a split
  // item the same over its range, the partial tiles cost ~0.1 us each (written
  // and read back) and the summing launch ~3 us. Taken when the estimate beats
  // the best single height by 5 % (long K: 4 x 1536 tokens x 3072 x 15360, 288
  // tiles, 580 us with 192-row tiles).
  GemmPlan plan;
  bool one_k = true;
  for (int i = 1; i < batch.count; ++i) one_k = one_k && batch.p[i].K == batch.p[0].K;
  if (one_k && t8 > cu && t8 % cu) {
    const int64_t tail = t8 % cu, kb = batch.p[0].K / 64;
    const double tt = 14.0 + 1.48 * static_cast<double>(kb);
    const double best = std::min(c8, std::min(c7, c6)) * tt;
    double est = 0.0;
    int split = 0;
    for (int S = 2; S <= kMaxSplit && tail * S <= cu && kb >= 3 * S; ++S) {
      const double e = static_cast<double>(t8 / cu) * tt + 14.0 + 1.48 * static_cast<double>(kb) / S + 3.0 +
                       0.1 * static_cast<double>(tail * S);
      if (split == 0 || e < est) {
        est = e;
        split = S;
      }
    }
    if (split && est < 0.95 * best) {
      plan.split = split;
      plan.tail = tail;
      return plan;
    }
  }
  if (wc == WCodec::kNF4 && t8 <= cu && 4 * t8 >= 3 * cu) plan.mb = 8;
  else if (c6 < 0.98 * c7 && c6 < 0.98 * c8) plan.mb = 6;
  else if (c7 < 0.98 * c8) plan.mb = 7;
  return plan;
}

void launch_plan(GemmBatch &batch, const GemmPlan &plan, const Code16 &c, hipStream_t s, WCodec wc, float *part) {
  switch (plan.mb) {
    case 6: launch_gemm<6, 2, 3, 4>(batch, c, s, wc, 1, nullptr); break;
    case 7: launch_gemm<7, 2, 3, 4>(batch, c, s, wc, 1, nullptr); break;
    default: launch_gemm<8, 2, 3, 4>(batch, c, s, wc, plan.split, part); break;
  }
}

// Plans a batch and checks the caller's workspace against what the plan needs.
int plan_and_launch(const char *what, GemmBatch &batch, const Code16 &c, hipStream_t s, WCodec wc, void *workspace,
                    int64_t workspace_bytes) {
  const GemmPlan plan = plan_gemm(batch, wc);
  const int64_t need = plan.workspace_bytes();
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned(workspace, 16)))
    return set_error(SELAS_EINVAL,
                     "%s: this launch splits its last round of tiles over K and needs a 16-byte aligned workspace of "
                     "%lld bytes (selas_linear_workspace_bytes); got %lld bytes at %p",
                     what, (long long)need, (long long)workspace_bytes, workspace);
  launch_plan(batch, plan, c, s, wc, static_cast<float *>(workspace));
  return check_launch(what);
}

}  // namespace
}  // namespace selas

using namespace selas;

namespace {
// Validation shared by the single and batched entries: SELAS_OK when the fused
// kernels take the call, or the error (EUNSUPPORTED: the caller falls back).
// For int8_row weights `packed` is q [N, K] and `absmax` the N row scales;
// blocksize and code are not used.
int check_linear(const char *what, const void *x, int64_t M, int64_t K, int64_t ldx, const uint8_t *packed,
                 const float *absmax, int64_t blocksize, const float *code, int64_t N, const void *bias,
                 const void *y, int64_t ldy, int dtype, WCodec wc = WCodec::kNF4) {
  const bool i8 = wc == WCodec::kInt8Row;
  if (M < 0 || K <= 0 || N <= 0)
    return set_error(SELAS_EINVAL, "%s: bad shape M=%lld K=%lld N=%lld", what, (long long)M, (long long)K,
                     (long long)N);
  if (!valid_dtype(dtype)) return set_error(SELAS_EINVAL, "%s: bad dtype %d", what, dtype);
  if (ldx < K || ldy < N)
    return set_error(SELAS_EINVAL, "%s: row strides ldx=%lld ldy=%lld below K, N", what, (long long)ldx,
                     (long long)ldy);
  if (M == 0) return SELAS_OK;
  if (!x || !packed || !absmax || !y || (!code && !i8)) return set_error(SELAS_EINVAL, "%s: null pointer", what);
  if (dtype != SELAS_BF16)
    return set_error(SELAS_EUNSUPPORTED, "%s: fused kernels take bf16, got %s", what, dtype_name(dtype));
  if (i8 && K % 64)
    return set_error(SELAS_EUNSUPPORTED, "%s: fused kernels need K %% 64 == 0 (K %lld)", what, (long long)K);
  if (!i8 && (blocksize != 64 || K % 64))
    return set_error(SELAS_EUNSUPPORTED, "%s: fused kernels need blocksize 64 and K %% 64 == 0 (blocksize %lld, K %lld)",
                     what, (long long)blocksize, (long long)K);
  if (!aligned(x, 16) || ldx % 8 || !aligned(packed, 16) || !aligned(absmax, 4) || !aligned(y, 8) || ldy % 4 ||
      (bias && !aligned(bias, 2)))
    return set_error(SELAS_EUNSUPPORTED, "%s: fused kernels need 16-byte aligned x rows and codes, "
                                         "8-byte aligned y rows", what);
  // Buffer offsets are 32-bit: every operand (plus one tile of overhang) must span < 4 GiB.
  const int64_t lim = (1ll << 32) - 1;
  if ((M + 512) * ldx * 2 > lim || (N + 256) * (i8 ? K : K / 2) > lim || (N + 256) * (i8 ? 1 : K / 64) * 4 > lim ||
      M * ldy * 2 > lim)
    return set_error(SELAS_EUNSUPPORTED, "%s: operand above 4 GiB", what);
  return SELAS_OK;
}
}  // namespace

extern "C" int selas_nf4_linear(const void *x, int64_t M, int64_t K, int64_t ldx, const uint8_t *packed,
                                const float *absmax, int64_t blocksize, const float code[16], int64_t N,
                                const void *bias, void *y, int64_t ldy, int dtype, void *workspace,
                                int64_t workspace_bytes, void *stream) {
  if (int e = check_linear("nf4_linear", x, M, K, ldx, packed, absmax, blocksize, code, N, bias, y, ldy, dtype))
    return e;
  if (M == 0) return ok();
  Code16 c;
  for (int i = 0; i < 16; ++i) c.v[i] = code[i];
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t *xb = static_cast<const uint16_t *>(x);
  const uint16_t *bb = static_cast<const uint16_t *>(bias);
  uint16_t *yb = static_cast<uint16_t *>(y);
  if (M <= 32 && stream_k(K)) {
    const GemvDesc one{packed, absmax, bb, yb, N, ldy};
    return launch_gemv_stream(xb, ldx, M, K, nullptr, 1, one, N, c, s);
  }
  if (M <= 32) {
    const int64_t grid = cdiv(N, 32 * kGemvGroups);
    const size_t lds = kSplitTableWords * sizeof(uint32_t);
    nf4_gemv_kernel<<<dim3(static_cast<uint32_t>(grid)), dim3(kGemvThreads), lds, s>>>(
        xb, ldx, static_cast<int>(M), static_cast<int>(K), packed, absmax, c, static_cast<int>(N), bb, yb, ldy);
    return check_launch("nf4_linear (gemv)");
  }
  GemmBatch batch{};
  batch.count = 1;
  batch.p[0] = GemmProblem{xb, packed, absmax, bb, yb, nullptr, ldx, ldy, 0, static_cast<int>(M),
                           static_cast<int>(K), static_cast<int>(N), static_cast<int>(N), 0, 0};
  return plan_and_launch("nf4_linear (gemm)", batch, c, s, WCodec::kNF4, workspace, workspace_bytes);
}

namespace {
// Validates the problems of a batched call into `batch` (M = 0 problems left out).
int fill_batch(const char *what, WCodec wc, const selas_nf4_gemm_problem *problems, int64_t count,
               int64_t blocksize, const float *code, int dtype, GemmBatch &batch) {
  static_assert(kGemmMaxProblems == SELAS_MAX_BATCHED_LINEARS, "batch size");
  if (count < 0 || count > kGemmMaxProblems)
    return set_error(SELAS_EINVAL, "%s: count %lld outside [0, %d]", what, (long long)count, kGemmMaxProblems);
  if (count > 0 && !problems) return set_error(SELAS_EINVAL, "%s: null problems", what);
  for (int64_t i = 0; i < count; ++i) {
    const selas_nf4_gemm_problem &q = problems[i];
    const int64_t gc = q.gelu_cols;
    if (gc < 0 || gc > q.N)
      return set_error(SELAS_EINVAL, "%s: gelu_cols %lld outside [0, N=%lld]", what, (long long)gc, (long long)q.N);
    // y holds the first N - gelu_cols columns (row stride ldy >= that); with
    // every column GELU'd into y2 it is not written and may be NULL.
    const void *y = (gc == q.N && gc > 0 && !q.y) ? q.y2 : q.y;
    const int64_t ldy_chk = gc > 0 ? std::max<int64_t>(q.ldy, q.N) : q.ldy;
    if (int e = check_linear(what, q.x, q.M, q.K, q.ldx, q.packed, q.absmax, blocksize, code, q.N, q.bias, y, ldy_chk,
                             dtype, wc))
      return e;
    if (gc > 0 && gc < q.N && q.ldy < q.N - gc)
      return set_error(SELAS_EINVAL, "%s: ldy %lld below the %lld plain columns", what, (long long)q.ldy,
                       (long long)(q.N - gc));
    if (gc > 0) {
      if (!q.y2 || q.ldy2 < gc) return set_error(SELAS_EINVAL, "%s: gelu_cols needs y2 with ldy2 >= gelu_cols", what);
      if ((q.N - gc) % (32 * 2 * 4) || (gc < q.N && q.ldy % 4) || !aligned(q.y2, 8) || q.ldy2 % 4 ||
          q.M * q.ldy2 * 2 >= (1ll << 32))
        return set_error(SELAS_EUNSUPPORTED, "%s: the GELU columns must start at a multiple of 256, y and y2 "
                                             "rows 8-byte aligned and y2 below 4 GiB", what);
    }
    if (q.M == 0) continue;
    if (q.M <= 32)
      return set_error(SELAS_EUNSUPPORTED, "%s: M <= 32 runs the skinny kernel (M=%lld)", what, (long long)q.M);
    batch.p[batch.count++] = GemmProblem{static_cast<const uint16_t *>(q.x), q.packed, q.absmax,
                                         static_cast<const uint16_t *>(q.bias), static_cast<uint16_t *>(q.y),
                                         static_cast<uint16_t *>(q.y2), q.ldx, q.ldy, gc > 0 ? q.ldy2 : 0,
                                         static_cast<int>(q.M), static_cast<int>(q.K), static_cast<int>(q.N),
                                         static_cast<int>(q.N - gc), 0, 0};
  }
  return SELAS_OK;
}

int linear_batched(const char *what, WCodec wc, const selas_nf4_gemm_problem *problems, int64_t count,
                   int64_t blocksize, const float *code, int dtype, void *workspace, int64_t workspace_bytes,
                   void *stream) {
  GemmBatch batch{};
  if (int e = fill_batch(what, wc, problems, count, blocksize, code, dtype, batch)) return e;
  if (batch.count == 0) return ok();
  Code16 c{};
  if (wc == WCodec::kNF4)
    for (int i = 0; i < 16; ++i) c.v[i] = code[i];
  return plan_and_launch(what, batch, c, static_cast<hipStream_t>(stream), wc, workspace, workspace_bytes);
}
}  // namespace

extern "C" int selas_nf4_linear_batched(const selas_nf4_gemm_problem *problems, int64_t count, int64_t blocksize,
                                        const float code[16], int dtype, void *workspace, int64_t workspace_bytes,
                                        void *stream) {
  return linear_batched("nf4_linear_batched", WCodec::kNF4, problems, count, blocksize, code, dtype, workspace,
                        workspace_bytes, stream);
}

extern "C" int selas_int8_row_linear_batched(const selas_nf4_gemm_problem *problems, int64_t count, int dtype,
                                             void *workspace, int64_t workspace_bytes, void *stream) {
  return linear_batched("int8_row_linear_batched", WCodec::kInt8Row, problems, count, 0, nullptr, dtype, workspace,
                        workspace_bytes, stream);
}

extern "C" int selas_linear_workspace_bytes(const selas_nf4_gemm_problem *problems, int64_t count, int codec,
                                            int64_t *bytes) {
  if (!bytes) return set_error(SELAS_EINVAL, "linear_workspace_bytes: null result pointer");
  *bytes = 0;
  if (codec != SELAS_CODEC_NF4 && codec != SELAS_CODEC_INT8_ROW)
    return set_error(SELAS_EINVAL, "linear_workspace_bytes: unknown codec %d", codec);
  if (count < 0 || count > kGemmMaxProblems)
    return set_error(SELAS_EINVAL, "linear_workspace_bytes: count %lld outside [0, %d]", (long long)count,
                     kGemmMaxProblems);
  if (count > 0 && !problems) return set_error(SELAS_EINVAL, "linear_workspace_bytes: null problems");
  GemmBatch batch{};
  for (int64_t i = 0; i < count; ++i) {
    const selas_nf4_gemm_problem &q = problems[i];
    if (q.M < 0 || q.K <= 0 || q.N <= 0 || q.M > INT32_MAX || q.K > INT32_MAX || q.N > INT32_MAX)
      return set_error(SELAS_EINVAL, "linear_workspace_bytes: bad shape M=%lld K=%lld N=%lld", (long long)q.M,
                       (long long)q.K, (long long)q.N);
    if (q.M == 0) continue;
    if (q.M <= 32) return ok();  // the skinny kernels, or a batch that runs one by one: no workspace
    GemmProblem &p = batch.p[batch.count++];
    p.M = static_cast<int>(q.M);
    p.K = static_cast<int>(q.K);
    p.N = static_cast<int>(q.N);
  }
  if (batch.count == 0) return ok();
  *bytes = plan_gemm(batch, codec == SELAS_CODEC_NF4 ? WCodec::kNF4 : WCodec::kInt8Row).workspace_bytes();
  return ok();
}

extern "C" int selas_int8_row_linear(const void *x, int64_t M, int64_t K, int64_t ldx, const int8_t *q,
                                     const float *scale, int64_t N, const void *bias, void *y, int64_t ldy, int dtype,
                                     void *workspace, int64_t workspace_bytes, void *stream) {
  const uint8_t *qb = reinterpret_cast<const uint8_t *>(q);
  if (int e = check_linear("int8_row_linear", x, M, K, ldx, qb, scale, 0, nullptr, N, bias, y, ldy, dtype,
                           WCodec::kInt8Row))
    return e;
  if (M == 0) return ok();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t *xb = static_cast<const uint16_t *>(x);
  const uint16_t *bb = static_cast<const uint16_t *>(bias);
  uint16_t *yb = static_cast<uint16_t *>(y);
  if (M <= 32 && stream_k(K)) {
    const GemvDesc one{qb, scale, bb, yb, N, ldy};
    return launch_i8_gemv_stream(xb, ldx, M, K, nullptr, 1, one, N, s);
  }
  if (M <= 32) {
    const int64_t grid = cdiv(N, 32 * kI8G);
    int8_row_gemv_kernel<<<dim3(static_cast<uint32_t>(grid)), dim3(kI8GemvThreads), 0, s>>>(
        xb, ldx, static_cast<int>(M), static_cast<int>(K), q, scale, static_cast<int>(N), bb, yb, ldy);
    return check_launch("int8_row_linear (gemv)");
  }
  GemmBatch batch{};
  batch.count = 1;
  batch.p[0] = GemmProblem{xb, qb, scale, bb, yb, nullptr, ldx, ldy, 0, static_cast<int>(M),
                           static_cast<int>(K), static_cast<int>(N), static_cast<int>(N), 0, 0};
  return plan_and_launch("int8_row_linear (gemm)", batch, Code16{}, s, WCodec::kInt8Row, workspace,
                         workspace_bytes);
}

extern "C" int selas_nf4_linear_grouped(const void *x, int64_t M, int64_t K, int64_t ldx,
                                        const selas_nf4_gemv_desc *descs, int64_t count, int64_t total_n,
                                        int64_t blocksize, const float code[16], int dtype, void *stream) {
  static_assert(sizeof(selas_nf4_gemv_desc) == sizeof(GemvDesc), "descriptor layout");
  if (M < 0 || K <= 0 || count < 0 || total_n < 0)
    return set_error(SELAS_EINVAL, "nf4_linear_grouped: bad shape M=%lld K=%lld count=%lld", (long long)M,
                     (long long)K, (long long)count);
  if (M == 0 || count == 0) return ok();
  if (!x || !descs || !code) return set_error(SELAS_EINVAL, "nf4_linear_grouped: null pointer");
  if (ldx < K) return set_error(SELAS_EINVAL, "nf4_linear_grouped: ldx below K");
  if (dtype != SELAS_BF16) return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped: takes bf16");
  if (blocksize != 64 || !stream_k(K) || M > 32 || count > kSgMaxDescs)
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped: needs blocksize 64, K = 1024, 2048 or 3072, M <= 32, "
                                         "at most %d weights", kSgMaxDescs);
  if (!aligned(x, 16) || ldx % 8 || !aligned(descs, 8))
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped: x rows must be 16-byte aligned");
  if (((M - 1) * ldx + K) * 2 >= (1ll << 32))
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped: x spans 4 GiB or more");
  if (total_n <= 0 || total_n >= (1ll << 36))
    return set_error(SELAS_EINVAL, "nf4_linear_grouped: total_n must be the sum of the weights' row counts");
  if (total_n * (K / 2) >= (1ll << 32))
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped: a weight above 4 GiB");
  Code16 c;
  for (int i = 0; i < 16; ++i) c.v[i] = code[i];
  const GemvDesc none{nullptr, nullptr, nullptr, nullptr, 0, 0};
  return launch_gemv_stream(static_cast<const uint16_t *>(x), ldx, M, K,
                                reinterpret_cast<const GemvDesc *>(descs), static_cast<int>(count), none,
                                total_n, c, static_cast<hipStream_t>(stream));
}

extern "C" int selas_int8_row_linear_grouped(const void *x, int64_t M, int64_t K, int64_t ldx,
                                             const selas_nf4_gemv_desc *descs, int64_t count, int64_t total_n,
                                             int dtype, void *stream) {
  if (M < 0 || K <= 0 || count < 0 || total_n < 0)
    return set_error(SELAS_EINVAL, "int8_row_linear_grouped: bad shape M=%lld K=%lld count=%lld", (long long)M,
                     (long long)K, (long long)count);
  if (M == 0 || count == 0) return ok();
  if (!x || !descs) return set_error(SELAS_EINVAL, "int8_row_linear_grouped: null pointer");
  if (ldx < K) return set_error(SELAS_EINVAL, "int8_row_linear_grouped: ldx below K");
  if (dtype != SELAS_BF16) return set_error(SELAS_EUNSUPPORTED, "int8_row_linear_grouped: takes bf16");
  if (!stream_k(K) || M > 32 || count > kSgMaxDescs)
    return set_error(SELAS_EUNSUPPORTED, "int8_row_linear_grouped: needs K = 1024, 2048 or 3072, M <= 32, "
                                         "at most %d weights", kSgMaxDescs);
  if (!aligned(x, 16) || ldx % 8 || !aligned(descs, 8))
    return set_error(SELAS_EUNSUPPORTED, "int8_row_linear_grouped: x rows must be 16-byte aligned");
  if (((M - 1) * ldx + K) * 2 >= (1ll << 32))
    return set_error(SELAS_EUNSUPPORTED, "int8_row_linear_grouped: x spans 4 GiB or more");
  if (total_n <= 0 || total_n >= (1ll << 36))
    return set_error(SELAS_EINVAL, "int8_row_linear_grouped: total_n must be the sum of the weights' row counts");
  if (total_n * K >= (1ll << 32))
    return set_error(SELAS_EUNSUPPORTED, "int8_row_linear_grouped: a weight above 4 GiB");
  const GemvDesc none{nullptr, nullptr, nullptr, nullptr, 0, 0};
  return launch_i8_gemv_stream(static_cast<const uint16_t *>(x), ldx, M, K, reinterpret_cast<const GemvDesc *>(descs),
                               static_cast<int>(count), none, total_n, static_cast<hipStream_t>(stream));
}

// ------------------------------------------------ grouped skinny GEMM without caller memory
//
// selas_nf4_linear_grouped reads its weight descriptors from a device array the
// caller allocates. This variant takes them in host memory and stages them in
// descriptor tables of the library's own: `scratch`, a device array of the code
// object (one copy per GPU, held until the process ends) that holds
// kStaticStreams tables. Its device address comes from hipGetSymbolAddress once
// per device, on the first call there, and only that address is passed to
// kernels: the array's name in host code is a host-side stand-in, not a device
// address. Each (device, stream) pair that calls gets a table of its own, up to
// kStaticStreams per device; further streams are refused (SELAS_EUNSUPPORTED),
// so two streams never share a table. The descriptors reach the table as
// kernel arguments of a small copy kernel (kStageDescs per launch), so no copy
// from host memory and no allocation is made. A call's copies and its GEMM are
// enqueued under the table's lock, so host threads that share a stream cannot
// interleave them; the stream orders one call's GEMM before the next call's
// copies.
namespace {
constexpr int kStaticDescs = kSgMaxDescs;  // 1023 descriptors, 49,104 bytes per table
constexpr int kStaticStreams = 8;          // tables per GPU (392,832 bytes)
constexpr int kStageDescs = 64;            // descriptors per copy launch (3,072 bytes of arguments)
constexpr int kMaxDevices = 64;
static_assert(kStaticDescs == SELAS_STATIC_MAX_WEIGHTS, "scratch size");
static_assert(kStaticStreams == SELAS_STATIC_MAX_STREAMS, "scratch tables");

__device__ __align__(256) GemvDesc scratch[kStaticStreams * kStaticDescs];

struct DescChunk {
  GemvDesc d[kStageDescs];
  int first, count;
};

// Thread i copies descriptor i of the chunk to dst[first + i] (vector stores).
__global__ __launch_bounds__(kStageDescs) void stage_descs(DescChunk c, GemvDesc *dst) {
  const int i = threadIdx.x;
  if (i < c.count) dst[c.first + i] = c.d[i];
}

struct StaticDevice {
  GemvDesc *base = nullptr;  // device address of `scratch` on this device
  hipStream_t streams[kStaticStreams] = {};
  int used = 0;
  std::mutex table_mu[kStaticStreams];
};
std::mutex scratch_mu;
StaticDevice static_devices[kMaxDevices];

// The table of (current device, stream) and its lock; the device's scratch
// address is resolved on its first call.
int scratch_table(hipStream_t s, GemvDesc **out, std::mutex **lock) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(SELAS_EHIP, "nf4_linear_grouped_static: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped_static: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> g(scratch_mu);
  StaticDevice &d = static_devices[dev];
  if (!d.base) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(SELAS_EHIP, "nf4_linear_grouped_static: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                       hipGetErrorString(e));
    d.base = static_cast<GemvDesc *>(p);
  }
  int slot = 0;
  while (slot < d.used && d.streams[slot] != s) ++slot;
  if (slot == d.used) {
    if (d.used == kStaticStreams)
      return set_error(SELAS_EUNSUPPORTED,
                       "nf4_linear_grouped_static: %d streams on device %d already hold its descriptor tables",
                       kStaticStreams, dev);
    d.streams[d.used++] = s;
  }
  *out = d.base + static_cast<int64_t>(slot) * kStaticDescs;
  *lock = &d.table_mu[slot];
  return SELAS_OK;
}
}  // namespace

extern "C" int selas_nf4_linear_grouped_static(const void *x, int64_t M, int64_t K, int64_t ldx,
                                               const selas_nf4_gemv_desc *descs, int64_t count, int64_t blocksize,
                                               const float code[16], int dtype, void *stream) {
  if (M < 0 || K <= 0 || count < 0)
    return set_error(SELAS_EINVAL, "nf4_linear_grouped_static: bad shape M=%lld K=%lld count=%lld", (long long)M,
                     (long long)K, (long long)count);
  if (count > kStaticDescs)
    return set_error(SELAS_EINVAL, "nf4_linear_grouped_static: %lld weights, at most %d (SELAS_STATIC_MAX_WEIGHTS)",
                     (long long)count, kStaticDescs);
  if (M == 0 || count == 0) return ok();
  if (!x || !descs || !code) return set_error(SELAS_EINVAL, "nf4_linear_grouped_static: null pointer");
  if (ldx < K) return set_error(SELAS_EINVAL, "nf4_linear_grouped_static: ldx below K");
  if (dtype != SELAS_BF16) return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped_static: takes bf16");
  if (blocksize != 64 || !stream_k(K) || M > 32)
    return set_error(SELAS_EUNSUPPORTED,
                     "nf4_linear_grouped_static: needs blocksize 64, K = 1024, 2048 or 3072 and M <= 32");
  if (!aligned(x, 16) || ldx % 8)
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped_static: x rows must be 16-byte aligned");
  if (((M - 1) * ldx + K) * 2 >= (1ll << 32))
    return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped_static: x spans 4 GiB or more");
  int64_t total_n = 0;
  for (int64_t i = 0; i < count; ++i) {
    const selas_nf4_gemv_desc &d = descs[i];
    if (d.n <= 0 || d.ldy < d.n || !d.packed || !d.absmax || !d.y)
      return set_error(SELAS_EINVAL, "nf4_linear_grouped_static: descriptor %lld: n=%lld ldy=%lld or a null pointer",
                       (long long)i, (long long)d.n, (long long)d.ldy);
    if (!aligned(d.packed, 16) || !aligned(d.absmax, 4) || !aligned(d.y, 2) || (d.bias && !aligned(d.bias, 2)))
      return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped_static: descriptor %lld: misaligned codes or output",
                       (long long)i);
    if (d.n * (K / 2) >= (1ll << 32) || M * d.ldy * 2 >= (1ll << 32))
      return set_error(SELAS_EUNSUPPORTED, "nf4_linear_grouped_static: descriptor %lld: a weight above 4 GiB",
                       (long long)i);
    total_n += d.n;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  GemvDesc *table = nullptr;
  std::mutex *table_mu = nullptr;
  if (int e = scratch_table(s, &table, &table_mu)) return e;
  std::lock_guard<std::mutex> g(*table_mu);
  for (int64_t first = 0; first < count; first += kStageDescs) {
    DescChunk chunk{};
    chunk.first = static_cast<int>(first);
    chunk.count = static_cast<int>(std::min<int64_t>(kStageDescs, count - first));
    std::memcpy(chunk.d, descs + first, sizeof(GemvDesc) * chunk.count);
    stage_descs<<<dim3(1), dim3(kStageDescs), 0, s>>>(chunk, table);
    if (int e = check_launch("nf4_linear_grouped_static (descriptor copy)")) return e;
  }
  Code16 c;
  for (int i = 0; i < 16; ++i) c.v[i] = code[i];
  const GemvDesc none{nullptr, nullptr, nullptr, nullptr, 0, 0};
  return launch_gemv_stream(static_cast<const uint16_t *>(x), ldx, M, K, table, static_cast<int>(count), none, total_n,
                            c, s);
}
