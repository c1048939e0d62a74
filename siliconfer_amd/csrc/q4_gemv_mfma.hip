// q4_gemv_mfma.hip — int4 decode GEMV for small batches with fp16 activations
// on MFMA (gfx950); same result contract as the VALU GEMV (q4_gemv_kernel.h).
//
// Why MFMA here: the VALU GEMV spends one dot2 per two weights per batch row,
// so from batch 4 up its arithmetic, and the batch rows of activations every
// lane holds, make it VALU- and register-bound instead of HBM-bound. On MFMA
// (v_mfma_f32_16x16x32_f16) the batch is the M side of the A operand (rows
// >= B read a valid row and only feed output rows that are never stored), each
// weight is dequantized once to an exact fp16 integer (q - z), and a lane needs
// 16 bytes of activations per MFMA.
//
// Layout: one workgroup per T x 16 weight rows (T row tiles per wave, 1 or
// 4); wave w covers the K blocks [w * BPW, (w + 1) * BPW) of every tile, so
// each activation fragment it loads feeds T MFMAs. Every workgroup reads the
// activations of the whole K from L2 (they do not stay in L1), so on wide
// matrices four tiles per wave cut that stream, which the L1/address path
// otherwise spends most of its cycles on (measured with TA/TCP counters),
// four times. Lanes of A rows >= B load nothing (a buffer load past the
// resource's end returns zero). A block is one scale group: lane l (row
// n = l % 16, k-group kg = l / 16) loads LW bytes of row n per block, LW = 16
// for group size 128 (four MFMAs per load) and 8 for group size 64 (two). The
// wider load halves the cache lines a wave instruction touches per byte: the
// MFMA operand layout puts a different row in each of 16 consecutive lanes, so
// one instruction reads 16 rows x 4 LW bytes.
// Load order per wave: the first activation blocks, every group's scale (and
// zero-point) bits, then every weight block, so nothing the first MFMAs need
// queues behind the weights (the load counter retires in issue order). The
// MFMA's k order inside a lane is the order the nibble magic produces
// (k0, k4, k1, k5, k2, k6, k3, k7); the activations are permuted to match,
// which leaves the dot product unchanged. Each group's partial is scaled by its
// fp16 scale in fp32 (exact weights, fp32 sums) and the waves' partials are
// summed through LDS in wave order. Blocks per wave (BPW) is compile-time, so
// group boundaries cost no selects and every register array stays in
// registers.
#include "q4_gemv_kernel.h"

namespace {

using sf_gemv::and_or;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kTileN = 16;
constexpr int kMaxWaves = 16;

// Per-lane weight load width LW (bytes): 16 when a group spans 128 k, else 8.
// A block is the K a wave instruction covers: 16 rows x (4 lanes x LW bytes),
// i.e. 8 LW k, LW / 4 MFMAs.
template <int LW> struct WLoad;
template <> struct WLoad<8> { typedef u32x2 T; static constexpr int kMaxBpw = 24; };
template <> struct WLoad<16> { typedef u32x4 T; static constexpr int kMaxBpw = 12; };

// Waves per workgroup a variant may use: 16 where its registers fit the
// 128-VGPR budget of a 1024-thread workgroup, else 8 (256 VGPRs); always 8
// for the folded RMSNorm, which holds a row norm's loads as well, and 16 for
// the folded SwiGLU only at the smaller block counts (its source ring).
__host__ __device__ constexpr int mfma_max_waves(int LW, bool asym, int bpw, int T, int pre = 0) {
  return pre == 1   ? 8
         : pre == 2 ? ((T > 1 ? bpw <= 2 : bpw * LW <= (asym ? 64 : 96)) ? 16 : 8)
                    : ((T > 1 || bpw * LW <= (asym ? 64 : 128)) ? 16 : 8);
}

// PRE folds the producer of the activations into their load, as the batch-1
// VALU GEMV does (x is then the fp32 source): PRE_RMSNORM x[b] = src[b] *
// inv_rms(src[b]) * pre_w with the norm of sf_row_inv_rms (the waves of a
// workgroup take the batch rows in turn and pass the norms through LDS),
// PRE_SILU x[b][k] = silu(src[b][k]) * src[b][K + k]; each value is rounded
// to fp16 as sf_rmsnorm / sf_silu_mul store it, so the result equals those
// kernels followed by this GEMV with the same plan. A lane loads the fp32
// sources of all its blocks ahead of the weights (so waiting for them never
// waits for the weight stream), which is why the host folds only plans of at
// most four MFMAs per lane; each block becomes fp16 operands just before its
// MFMAs.
template <int LW, bool ASYM, int BPW, int T, int PRE>
__global__ void __launch_bounds__(mfma_max_waves(LW, ASYM, BPW, T, PRE) * 64)
k_q4_gemv_mfma(const uint8_t *__restrict__ w, const f16 *__restrict__ stile,
               const uint8_t *__restrict__ ztile, const void *__restrict__ x, void *__restrict__ y,
               int ydt, float *__restrict__ y32, const void *__restrict__ bias, int bdt, int B,
               int N, int K, int G, int nblk, const float *__restrict__ pre_w, float eps) {
  constexpr int KB = 8 * LW;   // k per block
  constexpr int NM = LW / 4;   // MFMAs per block (one per weight dword)
  // activation ring: every block when they fit in 64 registers, else XR blocks
  // loaded XR - 1 ahead (folded producers: every block's sources)
  constexpr int XR = BPW * NM <= 16 ? BPW : 16 / NM;
  constexpr int XPRE = XR == BPW ? BPW : XR - 1;
  static_assert(PRE == sf_gemv::PRE_NONE || BPW * NM <= 4, "folded producers: four MFMAs per lane");
  typedef typename WLoad<LW>::T wvec_t;
  __shared__ float red[kMaxWaves][8][T * kTileN];

  const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wv_row0 = wave;  // RMSNorm: batch rows wave, wave + nw, ...
  __shared__ float inv_s[8];
  const int nl = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * T * kTileN;
  int nt[T];
#pragma unroll
  for (int t = 0; t < T; ++t) nt[t] = min(n0 + t * kTileN + nl, N - 1);  // rows past N re-read row N-1
  const int blk0 = wave * BPW;        // the host launches only waves with blk0 < nblk
  const int cnt = min(BPW, nblk - blk0);
  const int blast = blk0 + cnt - 1;   // blocks past the wave's own re-read its last one
  const int Kh = K >> 1;

  // lane (row n, k-group kg) covers k = KB blk + 2 LW kg .. + 2 LW - 1 of each block
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, B * K * 2, 0x00020000);
  const int xoff = nl < B ? (nl * K + kg * 2 * LW) * 2 : 0x40000000;
  u32x4 xs[XR][NM];
  auto xload = [&](int i) {
    if constexpr (PRE == sf_gemv::PRE_NONE) {
      const int o = xoff + min(blk0 + i, blast) * KB * 2;
#pragma unroll
      for (int j = 0; j < NM; ++j) xs[i % XR][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, o + j * 16, 0, 0);
    }
  };
  // folded producer: the lane's fp32 source (and norm weights / up half) of
  // every block, then (RMSNorm) the norm of the wave's first batch row
  float4_t fa[BPW][NM][2], fb[BPW][NM][2];
  SfRowNorm nrm;
  const float *srow = (const float *)x +
      (size_t)min(nl, B - 1) * (PRE == sf_gemv::PRE_SILU ? 2 * (size_t)K : (size_t)K);
  auto pload = [&](int i) {
    if constexpr (PRE != sf_gemv::PRE_NONE) {
#pragma unroll
      for (int j = 0; j < NM; ++j) {
        const int k = min(blk0 + i, blast) * KB + kg * 2 * LW + 8 * j;
        const float4_t *pa = (const float4_t *)(srow + k);
        const float4_t *pb = PRE == sf_gemv::PRE_SILU ? (const float4_t *)(srow + K + k)
                                                      : (const float4_t *)(pre_w + k);
        fa[i][j][0] = pa[0];
        fa[i][j][1] = pa[1];
        fb[i][j][0] = pb[0];
        fb[i][j][1] = pb[1];
      }
    }
  };
  if constexpr (PRE != sf_gemv::PRE_NONE) {
#pragma unroll
    for (int i = 0; i < BPW; ++i) pload(i);
    if constexpr (PRE == sf_gemv::PRE_RMSNORM)
      if (wv_row0 < B) nrm.issue<true>((const float *)x + (size_t)wv_row0 * K, nullptr, K);
  }
#pragma unroll
  for (int i = 0; i < XPRE; ++i) xload(i);

  uint32_t sbits[T][BPW], zbits[T][BPW];  // one group per block
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const size_t cell0 = (size_t)(nt[t] >> 3) * G;
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
      const size_t cell = cell0 + min(blk0 + q, G - 1);
      sbits[t][q] = ((const uint16_t *)stile)[cell * 8 + (nt[t] & 7)];
      if constexpr (ASYM) zbits[t][q] = ztile[cell * 4 + ((nt[t] & 7) >> 1)];
    }
  }

  wvec_t wv[T][BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i)
#pragma unroll
    for (int t = 0; t < T; ++t)
      wv[t][i] = __builtin_nontemporal_load((const wvec_t *)(w + (size_t)nt[t] * Kh + kg * LW +
                                                             (size_t)min(blk0 + i, blast) * 4 * LW));
  // keep every load above issued before any math (the scheduler would otherwise
  // interleave them with the MFMAs to save registers)
  __builtin_amdgcn_sched_barrier(0);

  float inv = 1.f;
  if constexpr (PRE == sf_gemv::PRE_RMSNORM) {
    const float *src = (const float *)x;
    for (int b = wv_row0; b < B; b += nw) {  // uniform per wave; all lanes active
      if (b != wv_row0) nrm.issue<true>(src + (size_t)b * K, nullptr, K);
      const float r = nrm.finish(src + (size_t)b * K, nullptr, K, eps);
      if (lane == 0) inv_s[b] = r;
    }
    __syncthreads();
    inv = inv_s[min(nl, B - 1)];
  }
  // block i's sources -> its fp16 operands (folded producers)
  auto pconvert = [&](int i) {
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      uint32_t pk[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v2[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int q = 2 * e + t;
          const float a = fa[i][j][q >> 2][q & 3], g = fb[i][j][q >> 2][q & 3];
          v2[t] = PRE == sf_gemv::PRE_RMSNORM ? sf_opaque(a * inv * g) : sf_silu_mul(a, g);
        }
        pk[e] = sf_bitcast<uint32_t>(half2_t{(f16)v2[0], (f16)v2[1]});
      }
      xs[i % XR][j] = u32x4{pk[0], pk[1], pk[2], pk[3]};
    }
  };

  const half2_t sixteenth = {(f16)0.0625f, (f16)0.0625f};
  const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  float4_t part[T];
  float acc[T][4];  // C rows b = 4 kg + r, column n
#pragma unroll
  for (int t = 0; t < T; ++t) {
    part[t] = zero4;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    if (i + XPRE < BPW) xload(i + XPRE);
    if constexpr (PRE != sf_gemv::PRE_NONE) pconvert(i);
    // blocks i >= cnt (only in a workgroup's last wave) are computed on re-read
    // data and dropped at the scale step by a select: a branch here would let
    // the compiler sink this block's loads into it, after the wait
    half2_t c1[T], c2[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint32_t z = 8u;  // offset-binary symmetric codes
      if constexpr (ASYM) {
        uint32_t zb = zbits[t][i];
        asm volatile("" : "+v"(zb));  // use the loaded bits here, not right after the load
        z = (zb >> (4 * (nt[t] & 1))) & 15u;
      }
      c1[t] = sf_bitcast<half2_t>((0xE400u | z) * 0x10001u);        // -(1024 + z)
      c2[t] = sf_bitcast<half2_t>((0xD400u + 16u * z) * 0x10001u);  // -(64 + z)
    }
#pragma unroll
    for (int j = 0; j < NM; ++j) {
      // A: x[k0, k4, k1, k5, k2, k6, k3, k7] of this lane's j-th 8-k group
      const u32x4 xv = xs[i % XR][j];
      const half2_t p0 = sf_bitcast<half2_t>(xv.x), p1 = sf_bitcast<half2_t>(xv.y);
      const half2_t p2 = sf_bitcast<half2_t>(xv.z), p3 = sf_bitcast<half2_t>(xv.w);
      const half8_t a = half8_t{p0.x, p2.x, p0.y, p2.y, p1.x, p3.x, p1.y, p3.y};
#pragma unroll
      for (int t = 0; t < T; ++t) {
        // B: the same 8 weights, q - z exact in fp16
        const uint32_t d = wv[t][i][j], d8 = d >> 8;
        const half2_t v0 = sf_bitcast<half2_t>(and_or(d, 0x000F000Fu, 0x64006400u)) + c1[t];
        const half2_t v1 = sf_bitcast<half2_t>(and_or(d, 0x00F000F0u, 0x64006400u)) * sixteenth + c2[t];
        const half2_t v2 = sf_bitcast<half2_t>(and_or(d8, 0x000F000Fu, 0x64006400u)) + c1[t];
        const half2_t v3 = sf_bitcast<half2_t>(and_or(d8, 0x00F000F0u, 0x64006400u)) * sixteenth + c2[t];
        const half8_t bw = half8_t{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
        part[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw, j == 0 ? zero4 : part[t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint32_t sb = sbits[t][i];
      asm volatile("" : "+v"(sb));  // convert at the point of use (keeps the load in flight)
      const float s = (float)sf_bitcast<f16>((uint16_t)sb);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][r] = i < cnt ? fmaf(part[t][r], s, acc[t][r]) : acc[t][r];
    }
  }

  // fold the waves (wave order) and store
  if (kg < 2) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][4 * kg + r][t * kTileN + nl] = acc[t][r];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < B * T * kTileN; e += blockDim.x) {
    const int b = e / (T * kTileN), c = e - b * (T * kTileN);
    const int row = n0 + c;
    if (row >= N) continue;
    float v = 0.f;
    for (int wi = 0; wi < nw; ++wi) v += red[wi][b][c];
    sf_gemv::store_out(y, ydt, y32, bias, bdt, (size_t)b * N + row, row, v);
  }
}

template <int LW, bool ASYM, int BPW, int T>
void launch_one(const sf_gemv::GemvArgs &a, int grid, int nw, int nblk, int pre,
                const float *pre_w, float eps) {
  using namespace sf_gemv;
  if constexpr (BPW * (LW / 4) <= 4) {
    if (pre == PRE_RMSNORM) {
      k_q4_gemv_mfma<LW, ASYM, BPW, T, PRE_RMSNORM><<<grid, nw * 64, 0, a.s>>>(
          a.w, a.st, a.zt, a.x, a.y, a.ydt, a.y32, a.bias, a.bdt, a.B, a.N, a.K, a.G, nblk, pre_w,
          eps);
      return;
    }
    if (pre == PRE_SILU) {
      k_q4_gemv_mfma<LW, ASYM, BPW, T, PRE_SILU><<<grid, nw * 64, 0, a.s>>>(
          a.w, a.st, a.zt, a.x, a.y, a.ydt, a.y32, a.bias, a.bdt, a.B, a.N, a.K, a.G, nblk, pre_w,
          eps);
      return;
    }
  }
  k_q4_gemv_mfma<LW, ASYM, BPW, T, PRE_NONE><<<grid, nw * 64, 0, a.s>>>(
      a.w, a.st, a.zt, a.x, a.y, a.ydt, a.y32, a.bias, a.bdt, a.B, a.N, a.K, a.G, nblk, nullptr,
      0.f);
}

// Compiled blocks-per-wave counts: 8-byte lanes {2, 4, 8, 12, 16, 24},
// 16-byte lanes {1, 2, 4, 6, 8, 12} (the same K per wave).
template <int LW> constexpr int kBucket[6] = {2, 4, 8, 12, 16, 24};
template <> constexpr int kBucket<16>[6] = {1, 2, 4, 6, 8, 12};

template <int LW, bool ASYM, int T>
void launch_bpw(const sf_gemv::GemvArgs &a, int grid, int nw, int nblk, int bpw, int pre,
                const float *pre_w, float eps) {
  constexpr const int *bk = kBucket<LW>;
#define SF_MB(I) launch_one<LW, ASYM, bk[I], T>(a, grid, nw, nblk, pre, pre_w, eps)
  if constexpr (T > 1) {  // four tiles per wave: the two smallest block counts only
    if (bpw == bk[0]) SF_MB(0);
    else SF_MB(1);
  } else {
    if (bpw == bk[0]) SF_MB(0);
    else if (bpw == bk[1]) SF_MB(1);
    else if (bpw == bk[2]) SF_MB(2);
    else if (bpw == bk[3]) SF_MB(3);
    else if (bpw == bk[4]) SF_MB(4);
    else SF_MB(5);
  }
#undef SF_MB
}

}  // namespace

// Waves per workgroup: enough that the grid holds about 3072 waves (three per
// SIMD: all of the matrix in flight at once), at most 16, and at least enough
// that no wave takes more than the largest block count. Blocks per wave: the
// smallest compiled count that covers the share, so only the last wave has a
// remainder. Wide matrices (>= 512 row tiles) whose K fits two blocks per
// wave at 16 waves run four row tiles per wave, so each activation fragment a
// wave loads feeds four MFMAs (the activation stream, which every workgroup
// reads whole from L2, shrinks four times).
struct MfmaPlan { int LW, T, grid, nw, nblk, bpw; };

static MfmaPlan mfma_plan(int N, int K, int g, bool asym) {
  MfmaPlan p;
  p.LW = g % 128 == 0 ? 16 : 8;
  p.nblk = K / (8 * p.LW);
  const int tiles = (N + kTileN - 1) / kTileN;
  const int *bk = p.LW == 16 ? kBucket<16> : kBucket<8>;
  const int maxb = p.LW == 16 ? WLoad<16>::kMaxBpw : WLoad<8>::kMaxBpw;
  {
    const int grid = (tiles + 3) / 4;
    int nw = 3072 / grid;
    nw = nw < 1 ? 1 : nw > kMaxWaves ? kMaxWaves : nw;
    const int need = (p.nblk + nw - 1) / nw;
    if (tiles >= 512 && need <= bk[1]) {
      p.T = 4;
      p.grid = grid;
      p.bpw = need <= bk[0] ? bk[0] : bk[1];
      p.nw = (p.nblk + p.bpw - 1) / p.bpw;
      return p;
    }
  }
  p.T = 1;
  p.grid = tiles;
  int nw = 3072 / p.grid;
  nw = nw < 1 ? 1 : nw > kMaxWaves ? kMaxWaves : nw;
  auto pick = [&](int waves) {
    int need = (p.nblk + waves - 1) / waves;
    if (need > maxb) need = (p.nblk + 7) / 8;
    int b = bk[5];
    for (int i = 0; i < 6; ++i)
      if (bk[i] >= need) { b = bk[i]; break; }
    return b;
  };
  p.bpw = pick(nw);
  if ((p.nblk + p.bpw - 1) / p.bpw > mfma_max_waves(p.LW, asym, p.bpw, 1)) p.bpw = pick(8);
  p.nw = (p.nblk + p.bpw - 1) / p.bpw;  // every launched wave has blocks
  return p;
}

template <int LW>
static void launch_plan(const sf_gemv::GemvArgs &a, const MfmaPlan &p, int pre,
                        const float *pre_w, float eps) {
  if (p.T == 4) {
    if (a.asym) launch_bpw<LW, true, 4>(a, p.grid, p.nw, p.nblk, p.bpw, pre, pre_w, eps);
    else launch_bpw<LW, false, 4>(a, p.grid, p.nw, p.nblk, p.bpw, pre, pre_w, eps);
  } else {
    if (a.asym) launch_bpw<LW, true, 1>(a, p.grid, p.nw, p.nblk, p.bpw, pre, pre_w, eps);
    else launch_bpw<LW, false, 1>(a, p.grid, p.nw, p.nblk, p.bpw, pre, pre_w, eps);
  }
}

namespace sf_gemv {

// Batch 3..8, fp16 activations, group size 64 or 128 (one 8- or 16-byte-lane
// block per group), K <= 8 waves x the largest block count.
bool mfma_gemv_applies(int B, int K, int g, int xdt) {
  const int lw = g % 128 == 0 ? 16 : 8;
  const int maxb = lw == 16 ? WLoad<16>::kMaxBpw : WLoad<8>::kMaxBpw;
  return xdt == SF_F16 && B >= 3 && B <= 8 && (g == 64 || g == 128) && K / (8 * lw) <= 8 * maxb;
}

// The folded producers run the plan of the plain GEMV (so the results agree
// bit for bit) when its waves hold at most four MFMAs' sources and fit the
// folded kernels' wave limit.
bool mfma_gemv_pre_applies(int B, int N, int K, int g, bool asym, int pre) {
  if (!mfma_gemv_applies(B, K, g, SF_F16)) return false;
  const MfmaPlan p = mfma_plan(N, K, g, asym);
  return p.bpw * (p.LW / 4) <= 4 && p.nw <= mfma_max_waves(p.LW, asym, p.bpw, p.T, pre);
}

int launch_mfma_gemv(const GemvArgs &a, int g, int pre, const float *pre_w, float eps) {
  const MfmaPlan p = mfma_plan(a.N, a.K, g, a.asym);
  if (p.LW == 16) launch_plan<16>(a, p, pre, pre_w, eps);
  else launch_plan<8>(a, p, pre, pre_w, eps);
  return SF_OK;
}

}  // namespace sf_gemv
