// Fused attention forward of the FLUX blocks (head dim 128, no mask) for gfx950:
// softmax(q k^T / sqrt(128)) v for every (batch, head), written straight into the
// [B, L, H * 128] layout the projection linear reads.
//
// One workgroup = NWV waves (8 when L >= 3072, else 4) = 32 * NWV queries of
// one (batch, head); wave w owns queries 32w .. 32w+31. The keys stream through
// LDS in tiles of 64 (K rows and the matching V^T columns, double-buffered,
// loaded by buffer->LDS DMA, shared by all the workgroup's waves). Per tile:
//   * S^T = K Q^T on 32x32x16 MFMAs (16 per wave): K from LDS is the A operand,
//     Q (held in registers for the whole loop) the B operand, so lane l holds 32
//     scores of query l % 32 (lanes l and l^32 together hold its 64 keys);
//   * online softmax in the exp2 domain: the running maximum is raised only when
//     a tile's maximum exceeds it by more than 8 (2^8 headroom in fp32 and in the
//     bf16 probabilities), so the rescale of the output is rare;
//   * O^T += V^T P^T (16 MFMAs): the probabilities, rounded to bf16, are the B
//     operand straight from the score registers. For that, the K rows of a 32-key
//     block are loaded with bits 2 and 3 of the row index swapped: lane (q, h)
//     register r then holds key 16*(r/8) + 8*h + r%8, i.e. 8 consecutive keys per
//     MFMA k-step, and the V^T operand reads 8 consecutive keys (16 bytes).
// LDS tiles are XOR-swizzled in 16-byte chunks so that the fragment reads (16
// lanes per LDS cycle) hit 16 distinct 4-bank groups.
// Any sequence length: key and query rows past L read as zeros (buffer range),
// the last key tile's missing keys get score -inf, and query rows past L are not
// stored; v^T rows are padded with zeros to a multiple of 64 tokens.
//
// LDS bandwidth bounds this kernel: every MFMA reads a 1 KiB A fragment from LDS
// (halving those reads ran 24 % faster). Two query blocks per wave would share
// each fragment, but need about 500 registers (one wave per SIMD); that version
// ran 25 % slower, because a lone wave cannot overlap its softmax with MFMAs.
// Eight waves per workgroup (one workgroup per CU) share each tile's DMA among
// 256 queries instead of 128, which cuts the LDS traffic per query by a tenth.
#include <type_traits>
#include "common.h"

namespace selas {
namespace {

constexpr int kDh = 128;                   // head dim
constexpr int kKT = 64;                    // keys per tile
constexpr int kTileBytes = kKT * kDh * 2;  // one K tile or V^T tile: 16 KiB
constexpr int kStageBytes = 2 * kTileBytes;

// MFMA row rho of a 32-key block reads K row swap23(rho): bits 2 and 3 exchanged.
__device__ __forceinline__ int swap23(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// max / sum of v over lanes l and l ^ 32 (the two halves of one query's keys), by
// v_permlane32_swap: its first result holds lanes 0-31's v in every lane, the
// second lanes 32-63's.
__device__ __forceinline__ float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Two probabilities to packed bf16 (round to nearest even), one v_cvt_pk_bf16_f32.
// The caller materializes each probability once, where it is produced, and adds
// the same registers into the row sum; materializing again inside the pack made
// the compiler copy every value (32 moves per tile).
__device__ __forceinline__ uint32_t pack_probs(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

template <int NWV>
__global__ __launch_bounds__(64 * NWV, 2) void attn_fwd_kernel(const uint16_t *__restrict__ q,
                                                               const uint16_t *__restrict__ k,
                                                               const uint16_t *__restrict__ vt,
                                                               uint16_t *__restrict__ out, int64_t ldo, int H, int L,
                                                               int qtiles, int per_xcd, int total, float c2) {
  constexpr int kQT = 32 * NWV;  // queries per workgroup
  constexpr int KJ = 16 / NWV;   // DMA instructions per wave and tile, for K and for V^T each
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kStageBytes];
  // Work item t = (b % 8) * per_xcd + b / 8: each XCD takes a contiguous range,
  // so the query tiles of one head share that head's K and V^T in its L2.
  const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (t >= total) return;
  const int bh = t / qtiles, qt = t - bh * qtiles;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, c = lane & 31;
  // q, k: [B*H, L, 128]; v^T: [B*H, 128, Lp] with Lp = L rounded up to the 64-key tile
  // (zero-filled). Query and key rows past L read as zeros through the buffer range.
  const int Lp = (L + kKT - 1) / kKT * kKT;
  const int64_t head = static_cast<int64_t>(bh) * L * kDh;  // elements
  const uint32_t head_bytes = static_cast<uint32_t>(L) * kDh * 2;
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + head, head_bytes);
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(k + head, head_bytes);
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(vt + static_cast<int64_t>(bh) * Lp * kDh,
                                              static_cast<uint32_t>(Lp) * kDh * 2);

  // Q as the B operand of S^T = K Q^T: lane (query c of this wave, h) holds d = 16s + 8h .. +8.
  const int q_row = qt * kQT + 32 * wave + c;
  bf16x8 qf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
    qf[s] = __builtin_bit_cast(bf16x8, load_b128(qr, static_cast<uint32_t>(q_row) * 256u + (16 * s + 8 * h) * 2, 0));

  // DMA per tile: 16 instructions of 1 KiB for K (4 rows of 256 B each) and 16
  // for V^T (8 rows of 128 B), KJ + KJ per wave. Lane i of K instruction J fills
  // row r = 4J + i/16, physical chunk i%16, with logical chunk (i%16) ^ (r%16);
  // lane i of V^T instruction J fills row d = 8J + i/8, physical chunk i%8, with
  // logical chunk (i%8) ^ ((d/2)%8). The tile's first key goes in the scalar offset.
  uint32_t k_voff[KJ], v_voff[KJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) {
    const int J = KJ * wave + j;
    const int r = 4 * J + (lane >> 4);
    k_voff[j] = static_cast<uint32_t>(r) * 256u + ((static_cast<uint32_t>(lane & 15) ^ (r & 15)) << 4);
    const int d = 8 * J + (lane >> 3);
    v_voff[j] = static_cast<uint32_t>(d) * static_cast<uint32_t>(Lp) * 2u +
                ((static_cast<uint32_t>(lane & 7) ^ ((d >> 1) & 7)) << 4);
  }
  auto issue = [&](int stage, int kt) {
    uint8_t *base = smem + stage * kStageBytes;
    const uint32_t key0 = static_cast<uint32_t>(kt) * kKT;
#pragma unroll
    for (int j = 0; j < KJ; ++j) load_lds16(kr, base + (KJ * wave + j) * 1024, k_voff[j], key0 * 256u);
#pragma unroll
    for (int j = 0; j < KJ; ++j) load_lds16(vr, base + kTileBytes + (KJ * wave + j) * 1024, v_voff[j], key0 * 2u);
  };
  // A-operand fragments: K row of MFMA row c in key block kb, d-chunk 2s+h; V^T
  // row d = 32db + c, key chunk 4kb + 2t + h (keys 32kb + 16t + 8h .. +8).
  const int krow = swap23(c);
  auto kfrag = [&](int stage, int kb, int s) {
    const int r = 32 * kb + krow;
    const int cc = 2 * s + h;
    return *reinterpret_cast<const bf16x8 *>(smem + stage * kStageBytes + r * 256 + ((cc ^ (r & 15)) << 4));
  };
  auto vfrag = [&](int stage, int db, int kb, int t2) {
    const int d = 32 * db + c;
    const int cc = 4 * kb + 2 * t2 + h;
    return *reinterpret_cast<const bf16x8 *>(smem + stage * kStageBytes + kTileBytes + d * 128 +
                                             ((cc ^ ((d >> 1) & 7)) << 4));
  };

  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x16{};
  float m_run = -__builtin_inff(), l_run = 0.0f;
  const int ntiles = Lp / kKT;

  issue(0, 0);
  wait_vmcnt<0>();
  __syncthreads();

  // kMasked: the last tile of a sequence that is not a multiple of 64. The mask
  // is a separate instantiation so that full tiles carry no per-score selects
  // (a runtime test on every tile was turned into 93 selects and compares).
  auto tile = [&](int stage, int kt, auto masked) {
    constexpr bool kMasked = decltype(masked)::value;
    if (kt + 1 < ntiles) issue(stage ^ 1, kt + 1);
    // Scores: 16 MFMAs over (key block kb, d-chunk s) = (i / 8, i % 8). The K
    // fragments go through a ring of kKAhead registers, each read kKAhead MFMAs
    // before its use, so that no MFMA waits on a read issued just before it.
    constexpr int kKAhead = 4;
    f32x16 sc[2] = {f32x16{}, f32x16{}};
    bf16x8 kf[kKAhead];
#pragma unroll
    for (int i = 0; i < kKAhead; ++i) kf[i] = kfrag(stage, i / 8, i % 8);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sc[i / 8] = mfma32(kf[i % kKAhead], qf[i % 8], sc[i / 8]);
      if (i + kKAhead < 16) kf[i % kKAhead] = kfrag(stage, (i + kKAhead) / 8, (i + kKAhead) % 8);
    }
    // The same order for the scheduler, which otherwise issues the first key
    // block's reads right before their MFMAs where registers are tight.
    __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + kKAhead < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (kMasked) {
      // Keys past L do not exist. Register r of score block kb holds key
      // 32 kb + 16 (r/8) + 8 h + r % 8.
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * kKT + 32 * kb + 16 * (r >> 3) + 8 * h + (r & 7) >= L) sc[kb][r] = -__builtin_inff();
    }
    float mx = sc[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[kb][r]);
    mx = pair_max(mx) * c2;
    const bool raise = mx > m_run + 8.0f;
    // Skipped for the whole wave unless some query's maximum moved (rare after the
    // first tiles); lanes whose maximum stays multiply by exactly 1.
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float alpha = raise ? __builtin_amdgcn_exp2f(m_run - mx) : 1.0f;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
      l_run *= alpha;
      m_run = raise ? mx : m_run;
    }
    // V^T fragments of the second product (db, kb, t2) = (i / 4, (i / 2) % 2, i % 2),
    // the first kVAhead read before the exponentials, the rest kVAhead MFMAs ahead.
    constexpr int kVAhead = 8;
    bf16x8 vf[kVAhead];
#pragma unroll
    for (int i = 0; i < kVAhead; ++i) vf[i] = vfrag(stage, i / 4, (i / 2) % 2, i % 2);
    float ls = 0.0f;
    bf16x8 pb[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = materialize(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][8 * t2 + 2 * e], c2, -m_run)));
          const float p1 = materialize(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][8 * t2 + 2 * e + 1], c2, -m_run)));
          ls += p0 + p1;
          w[e] = pack_probs(p0, p1);
        }
        pb[kb][t2] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
      }
    l_run += ls;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o[i / 4] = mfma32(vf[i % kVAhead], pb[(i / 2) % 2][i % 2], o[i / 4]);
      const int j = i + kVAhead;
      if (j < 16) vf[i % kVAhead] = vfrag(stage, j / 4, (j / 2) % 2, j % 2);
    }
    // The next tile has landed for this wave; the barrier then covers every wave
    // and orders this tile's LDS reads before the DMA that reuses its stage.
    wait_vmcnt<0>();
    __syncthreads();
  };
  const std::integral_constant<bool, false> full{};
  const std::integral_constant<bool, true> last{};
  const int nfull = L / kKT;  // tiles whose 64 keys all exist
  int kt = 0;
  for (; kt + 2 <= nfull; kt += 2) {
    tile(0, kt, full);
    tile(1, kt + 1, full);
  }
  if (kt < nfull) tile(0, kt++, full);
  if (kt < ntiles) {  // a partial last tile, stage kt % 2
    if (kt & 1) tile(1, kt, last);
    else tile(0, kt, last);
  }

  // out[(b*L + q) * ldo + hh*128 + d] = O^T[d][q] / l, d = 32db + 8g + 4h + e for register 4g + e.
  const float inv = 1.0f / pair_sum(l_run);
  const int b = bh / H, hh = bh - b * H;
  if (q_row >= L) return;  // a last query tile past the sequence end
  uint16_t *orow = out + (static_cast<int64_t>(b) * L + q_row) * ldo + hh * kDh;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * h;
      *reinterpret_cast<uint2 *>(orow + d) = make_uint2(pack_bf16x2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                                                        pack_bf16x2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv));
    }
}

// vt[bh][d][l] = v[bh][l][d] for 64 tokens x 128 channels per workgroup, through LDS;
// vt rows hold Lp = L rounded up to 64 tokens, the ones past L zero. The tile is
// [token][channel] with a 65-word row: the row writes (lane = token r % 4, channel
// chunk) fall in 64 distinct banks, and the transposed 2-byte reads (lane = channel d,
// token chunk) in 32 distinct words, two lanes per word.
__global__ __launch_bounds__(256) void transpose_heads_kernel(const uint16_t *__restrict__ v, uint16_t *__restrict__ vt,
                                                              int L, int Lp) {
  constexpr int kRow = kDh + 2;  // 260-byte rows
  __shared__ __attribute__((aligned(16))) uint16_t tile[kKT * kRow];
  const int l0 = blockIdx.x * kKT;
  const int64_t head = static_cast<int64_t>(blockIdx.y) * L * kDh;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // token r, channels 8c .. 8c+7
    const int r = (tid >> 4) + 16 * i, ch = tid & 15;
    const uint4 x = l0 + r < L ? *reinterpret_cast<const uint4 *>(v + head + static_cast<int64_t>(l0 + r) * kDh + 8 * ch)
                               : make_uint4(0, 0, 0, 0);
    uint32_t *dst = reinterpret_cast<uint32_t *>(tile + r * kRow + 8 * ch);  // 4-byte aligned
    dst[0] = x.x;
    dst[1] = x.y;
    dst[2] = x.z;
    dst[3] = x.w;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // channel d, tokens 8c .. 8c+7
    const int d = (tid >> 3) + 32 * i, ch = tid & 7;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = static_cast<uint32_t>(tile[(8 * ch + 2 * e) * kRow + d]) |
             (static_cast<uint32_t>(tile[(8 * ch + 2 * e + 1) * kRow + d]) << 16);
    *reinterpret_cast<uint4 *>(vt + static_cast<int64_t>(blockIdx.y) * Lp * kDh + static_cast<int64_t>(d) * Lp + l0 +
                               8 * ch) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

}  // namespace
}  // namespace selas

using namespace selas;

namespace {
int check_heads(const char *what, int64_t B, int64_t H, int64_t L, int64_t Dh, int dtype) {
  if (B < 0 || H < 0 || L < 0 || Dh <= 0)
    return set_error(SELAS_EINVAL, "%s: bad shape B=%lld H=%lld L=%lld Dh=%lld", what, (long long)B, (long long)H,
                     (long long)L, (long long)Dh);
  if (!valid_dtype(dtype)) return set_error(SELAS_EINVAL, "%s: bad dtype %d", what, dtype);
  if (dtype != SELAS_BF16 || Dh != kDh)
    return set_error(SELAS_EUNSUPPORTED, "%s: fused attention takes bf16 and head_dim 128 (got %s, %lld)", what,
                     dtype_name(dtype), (long long)Dh);
  if ((L + kKT) * Dh * 2 >= (1ll << 32) || B * H >= (1ll << 31) / 64)
    return set_error(SELAS_EUNSUPPORTED, "%s: a head above 4 GiB", what);
  return SELAS_OK;
}
}  // namespace

extern "C" int selas_attention(const void *q, const void *k, const void *vt, int64_t B, int64_t H, int64_t L,
                               int64_t Dh, void *out, int64_t ldo, int dtype, void *stream) {
  if (int e = check_heads("attention", B, H, L, Dh, dtype)) return e;
  if (B == 0 || H == 0 || L == 0) return ok();
  if (!q || !k || !vt || !out) return set_error(SELAS_EINVAL, "attention: null pointer");
  if (ldo < H * Dh) return set_error(SELAS_EINVAL, "attention: out row stride %lld below H*Dh", (long long)ldo);
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(vt, 16) || !aligned(out, 8) || ldo % 4)
    return set_error(SELAS_EUNSUPPORTED, "attention: q, k, v^T must be 16-byte aligned, out rows 8-byte aligned");
  const float c2 = 1.4426950408889634f / sqrtf(static_cast<float>(Dh));  // log2(e) / sqrt(Dh)
  auto launch = [&](auto kernel, int nwv) {
    const int qtiles = static_cast<int>(cdiv(L, 32 * nwv));
    const int64_t total = B * H * qtiles;
    const int per_xcd = static_cast<int>(cdiv(total, 8));
    kernel<<<dim3(static_cast<uint32_t>(per_xcd * 8)), dim3(64 * nwv), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(vt),
        static_cast<uint16_t *>(out), ldo, static_cast<int>(H), static_cast<int>(L), qtiles, per_xcd,
        static_cast<int>(total), c2);
  };
  // Eight waves share each tile among more queries but run one workgroup per CU:
  // at L = 4608 (FLUX 1024^2) 282 us against 297 with four, at L = 1536 159 against
  // 151 (each workgroup's fixed costs weigh more over 24 key tiles than over 72).
  if (L >= 3072) launch(attn_fwd_kernel<8>, 8);
  else launch(attn_fwd_kernel<4>, 4);
  return check_launch("attention");
}

extern "C" int selas_transpose_heads(const void *v, int64_t BH, int64_t L, int64_t Dh, void *vt, int dtype,
                                     void *stream) {
  if (int e = check_heads("transpose_heads", 1, BH, L, Dh, dtype)) return e;
  if (BH == 0 || L == 0) return ok();
  if (!v || !vt) return set_error(SELAS_EINVAL, "transpose_heads: null pointer");
  if (!aligned(v, 16) || !aligned(vt, 16))
    return set_error(SELAS_EUNSUPPORTED, "transpose_heads: v and v^T must be 16-byte aligned");
  if (BH > 65535) return set_error(SELAS_EUNSUPPORTED, "transpose_heads: more than 65535 heads");
  const int64_t Lp = cdiv(L, kKT) * kKT;
  transpose_heads_kernel<<<dim3(static_cast<uint32_t>(Lp / kKT), static_cast<uint32_t>(BH)), dim3(256), 0,
                           static_cast<hipStream_t>(stream)>>>(static_cast<const uint16_t *>(v),
                                                               static_cast<uint16_t *>(vt), static_cast<int>(L),
                                                               static_cast<int>(Lp));
  return check_launch("transpose_heads");
}
