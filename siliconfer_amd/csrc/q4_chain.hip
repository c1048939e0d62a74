// q4_chain.hip — a chain of dependent int4 decode GEMVs (batch 1) in one
// persistent launch.
//
// A decoder layer at batch 1 is a sequence of GEMVs, each consuming the whole
// output of the one before (q|k|v -> o -> gate|up -> SwiGLU -> down, the
// reference's Attention / MLP call sites, /root/reference/siliconfer/model/
// layers.py:93-95, 133, 139-144). As separate launches every GEMV pays the
// launch gap and then waits one memory round trip for its activations before
// its weights stream; here one launch of one workgroup per CU runs every
// phase, and each workgroup issues its weight loads for a phase before it
// waits for that phase's input, so the weight stream continues across the
// hand-offs.
//
// Work split. Phase p's row tiles (16 rows, all of K) go round robin over the
// workgroups (tile t to workgroup t mod grid); within a workgroup wave w takes
// units [w U, w U + U) of K (U = ceil(units / 16)) of every tile, the tile's
// 16 waves' partials summed in LDS in wave order. Up to NBUF tiles of a
// workgroup are in flight (registers), NBUF - 1 of them issued before the
// input wait.
//
// Hand-off. A phase publishes its outputs as fp16 (the activation dtype its
// consumer stages anyway) in 8-byte words of two values and a 32-bit tag,
// written with agent-scope atomic stores; a phase feeding a SwiGLU publishes
// silu(gate) * up instead (sf_silu_mul, rounded to fp16): its workgroups own
// a gate tile and the matching up tile. When its outputs are out, a
// workgroup sets its own done word for the phase. A consumer's wave 0 polls
// the producing phase's done words (one dword per workgroup) until all carry
// the tag, then every thread reads its words with agent-scope atomic loads
// and accepts them when every tag matches (else reads them again; the done
// words are a cheap signal, the tags are what makes a value valid, since a
// value and its tag travel in one single-copy-atomic word). A phase's input
// is read before its first weight loads go out (a wave's vector loads
// complete in order, so the wait for the input then does not wait for the
// weights). Tags are launch epoch * 8 + phase + 1; each workgroup keeps the
// epoch in its own workspace slot, read at entry and advanced at exit, so the
// slots of all workgroups agree at every launch without any exchange. Every
// wait is bounded: after `spin_cap` rounds it records an error in the
// workspace and goes on (the results are then wrong, the kernel still
// exits), and the host reports it.
//
// Arithmetic per 1 KB weight unit as in the decode GEMV (q4_gemv_blk.h): the
// symmetric codes dequantized exactly into fp16 q - 8, four
// v_mfma_f32_16x16x32_f16 against the fp16 activations (A row 0; the other
// A rows repeat it and their outputs are dropped), each scale group's partial
// folded with its fp16 scale in fp32, the 16 waves' partials of a row summed
// in wave order. Activations are staged in LDS as fp16: the first phase's
// from the caller's fp16 vector, later phases' as their producer published
// them. The last phase writes fp32.
#include "q4_gemv_blk.h"
#include "sf_common.h"

namespace sf_chain {

using sf_gemv::DequantConsts;
using sf_gemv::dequant_f16;
using sf_gemv::half8_t;

constexpr int kWaves = 16, kThreads = kWaves * 64;
constexpr int kMaxUnits = 6;                       // units of K per wave: K <= 16 * 6 * 128
constexpr int kMaxK = kWaves * kMaxUnits * 128;    // 12288
constexpr int kLdsBytes = 96 * 1024;               // > half the CU's LDS: one workgroup per CU
constexpr size_t kHeaderBytes = 8192 + 4 * 1024 * 8;  // workspace: error word, epoch[1024] at 64, done[8][1024] at 8192
constexpr int kMaxTiles = 8;                       // row tiles per workgroup per phase
constexpr int kRing = 4;                           // unit loads in flight per lane
constexpr int kMaxGrid = 1024;                     // workgroups (one per CU)

enum { IN_X16 = 0, IN_LL = 1, IN_LL_SILU = 2 };

struct Phase {
  const uint8_t *w;  // blob codes
  const f16 *st;     // blob scales, tiled [ceil(N/8)][G][8]
  int N, K, G, gshift, nblk, ntiles, upw;  // g = 128 << gshift (or 64)
  int swiglu;        // publishes silu(gate) * up: gate rows [0, N/2), up rows [N/2, N)
  uint64_t *out_ll;  // published fp16 pairs (or null: the last phase)
  float *out;        // plain fp32 output [N] (the last phase)
};

struct Args {
  Phase ph[SF_CHAIN_MAX_PHASES];
  int nph;
  const f16 *x0;
  uint32_t *epoch;    // [grid] each workgroup's launch counter
  uint32_t *done;     // [phase][grid] the tag of the phase's last outputs of each workgroup
  int *err;           // 0, or the code of the first failed wait
  int spin_cap;
  int drop_phase;     // host test hook: this phase publishes nothing (-1: none)
};

__device__ __forceinline__ uint64_t ll_load(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// two values rounded to fp16 and the tag, as one word
__device__ __forceinline__ void ll_store2(uint64_t *p, float v0, float v1, uint32_t tag) {
  const uint32_t h = sf_bitcast<uint32_t>(half2_t{(f16)v0, (f16)v1});
  __hip_atomic_store(p, (uint64_t)h | ((uint64_t)tag << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void set_err(int *err, int code) {
  __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The workgroup barrier for LDS exchanges: this wave's LDS accesses complete,
// then s_barrier. __syncthreads' release fence would also wait for every
// outstanding global load of the wave, i.e. drain the ring of weight loads
// in flight; the asm clobbers keep the compiler from moving memory accesses
// across it.
#define CH_BARRIER()                                      \
  do {                                                    \
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");    \
    __builtin_amdgcn_s_barrier();                         \
    asm volatile("" ::: "memory");                        \
  } while (0)

// One phase's walk over this workgroup's units: step q = (tile j, unit slot i)
// with i < upw for every wave (the same steps in every wave, so the per-phase
// barriers line up); slots i >= cnt of the last waves are dummies whose loads
// re-read the tile's last unit (an L2 hit) and whose products are dropped.
// Every step issues its loads unconditionally (steps past the walk re-read
// its last unit): the count of loads in flight is then the same on every
// path, so each wait before a unit's use is an exact vmcnt, not a drain.
struct Walk {
  int u0, cnt, ub, cmax;           // first unit, real units, first unit clamped into K, last real slot
  int upw, mine, total, tpad;      // steps per tile, tiles, steps, steps padded to the ring size
  int qi;                          // steps issued
  int lj, li;                      // the next load's tile and slot
  const uint8_t *wt;               // tile lj's codes at unit 0, this lane's 16 bytes
  const uint32_t *sr;              // tile lj's scale pairs of this lane's row
};

// This workgroup's k-th tile of phase P: tiles t = blockIdx + k grid; for a
// SwiGLU phase, pairs (gate tile j, up tile j + ntiles / 2) with j =
// blockIdx + (k / 2) grid, gate first.
__device__ __forceinline__ int tile_of(const Phase &P, int k, int grid) {
  if (P.swiglu) return (int)blockIdx.x + (k >> 1) * grid + (k & 1) * (P.ntiles >> 1);
  return (int)blockIdx.x + k * grid;
}

// point W at its tile k (steps past the walk stay on the last tile; a
// workgroup with no tile in the phase reads tile 0, never below it)
__device__ __forceinline__ void walk_tile(const Phase &P, Walk &W, int k, int grid, int lane) {
  const int t = max(0, min(tile_of(P, min(k, W.mine - 1), grid), P.ntiles - 1));
  W.wt = P.w + (size_t)t * P.nblk * 1024 + lane * 16;
  // the scale cell's aligned pair of rows (row & ~1, row | 1) as one dword
  const int row = min(t * 16 + (lane & 15), P.N - 1);
  W.sr = (const uint32_t *)P.st + ((size_t)(row >> 3) * P.G * 8 + (row & 6)) / 2;
}

template <int NS>
__device__ __forceinline__ Walk walk_of(const Phase &P, int wave, int grid, int lane) {
  Walk w;
  w.upw = P.upw;
  w.u0 = wave * P.upw;
  w.cnt = max(0, min(P.upw, P.nblk - w.u0));
  w.ub = min(w.u0, P.nblk - 1);
  w.cmax = max(w.cnt - 1, 0);  // slots past it re-read the wave's last real unit
  const int n = P.swiglu ? P.ntiles >> 1 : P.ntiles;
  w.mine = n > (int)blockIdx.x ? (n - 1 - (int)blockIdx.x) / grid + 1 : 0;
  if (P.swiglu) w.mine *= 2;
  w.total = w.mine * P.upw;
  w.tpad = (w.total + NS - 1) / NS * NS;
  w.qi = 0;
  w.lj = 0;
  w.li = 0;
  walk_tile(P, w, 0, grid, lane);
  return w;
}

template <int NS, int GK>
__global__ void __launch_bounds__(kThreads) k_q4_chain(Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  f16 *const xs = (f16 *)smem;                      // staged activations [kMaxK]
  float *const red = (float *)(smem + kMaxK * 2);   // [kMaxTiles][kWaves][16] wave partials
  __shared__ uint32_t vote[kWaves];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, kg = lane >> 4;
  const int grid = gridDim.x;

  const DequantConsts dk;
  // all_ok: every thread's `ok`, through one LDS word per wave (stamped with
  // the round, so no reset is needed) and two bare barriers
  auto all_ok = [&](bool ok, int round) {
    const bool w_ok = __builtin_amdgcn_ballot_w64(!ok) == 0;
    if (lane == 0) vote[wave] = (uint32_t)w_ok | ((uint32_t)round << 1);
    CH_BARRIER();
    bool r = true;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) r &= vote[w] == (1u | ((uint32_t)round << 1));
    CH_BARRIER();  // every wave has read the votes before the next round writes them
    return r;
  };
  // the ring of unit loads: NS per lane (16 bytes of one unit each, NS KB per
  // wave in flight), and each unit's fp16 scale bits (g == 64: the groups of
  // MFMAs 0-1 and 2-3, kept apart until their use so that no load is waited
  // for at issue)
  u32x4 ring[NS];
  uint32_t rs0[NS], rs1[NS];
  // issue the next load of walk W (phase P) into one ring slot: the unit's
  // 16 bytes of this lane and its scale pair(s); the scale group of unit u is
  // u >> gshift (g = 128 << gshift) or 2u and 2u + 1 (g = 64)
  auto issue = [&](const Phase &P, Walk &W, u32x4 &wv, uint32_t &sv0, uint32_t &sv1) {
    const int u = W.ub + min(W.li, W.cmax);
    wv = __builtin_nontemporal_load((const u32x4 *)(W.wt + (size_t)u * 1024));
    if constexpr (GK == 0) {
      sv0 = W.sr[(size_t)(u >> P.gshift) * 4];
    } else {
      sv0 = W.sr[(size_t)(2 * u) * 4];
      sv1 = W.sr[(size_t)(2 * u + 1) * 4];
    }
    if (++W.li == W.upw) {
      W.li = 0;
      walk_tile(P, W, ++W.lj, grid, lane);
    }
  };
  // The ring is one stream of unit loads over every phase: the load walk
  // (phase pl, walk Wl) runs NS - 1 steps ahead of the compute, so the next
  // phase's first units go out while this one computes. Each phase's steps
  // are padded to a multiple of NS (the padding re-reads the phase's last
  // unit and computes nothing), so every phase starts at ring slot 0; a
  // phase with no tile in this workgroup has no steps. Past the last phase
  // the walk keeps re-reading its last unit (loads left in flight at exit).
  int pl = 0;
  Phase Pl = a.ph[0];
  Walk Wl = walk_of<NS>(Pl, wave, grid, lane);
  auto issue_next = [&](u32x4 &wv, uint32_t &sv0, uint32_t &sv1) {
    while (Wl.qi >= Wl.tpad && pl + 1 < a.nph) {
      Pl = a.ph[++pl];
      Wl = walk_of<NS>(Pl, wave, grid, lane);
    }
    issue(Pl, Wl, wv, sv0, sv1);
    ++Wl.qi;
  };
  // The launch epoch: this workgroup's slot holds the epoch after the last
  // launch's (every workgroup of a launch writes its own slot at exit, so all
  // slots agree once the previous launch has finished; the scalar load waits
  // on no vector load).
  uint32_t epoch;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(epoch)
               : "s"(a.epoch + blockIdx.x) : "memory");

  // A phase's input is read before its first weight loads go out, so that
  // waiting for the input does not wait for them (a wave's vector loads
  // complete in order): x0 for the first phase, the producer's words for the
  // others (a first attempt; if a tag is stale the phase falls back to
  // polling the done words and reading again). Words w = tid + i kThreads of
  // K / 2 (two fp16 each); the loads are unconditional (clamped), so the
  // waits before their use are exact counts.
  constexpr int kWpt = kMaxK / 2 / kThreads;  // 6
  uint64_t win[kWpt];
  auto read_input = [&](int p, const Phase &P) {
    const int nwv = P.K / 2;
#pragma unroll
    for (int i = 0; i < kWpt; ++i) {
      const int w = min((int)tid + i * kThreads, nwv - 1);
      if (p == 0) win[i] = ((const uint32_t *)a.x0)[w];
      else win[i] = ll_load(a.ph[p - 1].out_ll + w);
    }
  };

  Phase P = a.ph[0];  // the computing phase's descriptor held in registers
  read_input(0, P);
#pragma unroll
  for (int s = 0; s + 1 < NS; ++s) issue_next(ring[s], rs0[s], rs1[s]);
  for (int p = 0; p < a.nph; ++p) {
    if (p > 0) P = a.ph[p];
    const Walk W = walk_of<NS>(P, wave, grid, lane);
    const uint32_t tag_out = epoch * SF_CHAIN_MAX_PHASES + p + 1;
    const uint32_t tag_in = epoch * SF_CHAIN_MAX_PHASES + p;  // the producing phase's tag

    // ---- the phase's input, staged in LDS as fp16 (zero past K)
    // (straight-line: every word register is consumed here, so no later reuse
    // of its register waits on a load; the kThreads * kWpt words are exactly
    // the staging buffer, and words past K stage zeros)
    const int nwv = P.K / 2;  // words of K
    bool ok = true;
#pragma unroll
    for (int i = 0; i < kWpt; ++i) {
      const int w = (int)tid + i * kThreads;
      ok &= p == 0 || w >= nwv || (uint32_t)(win[i] >> 32) == tag_in;
      ((uint32_t *)xs)[w] = w < nwv ? (uint32_t)win[i] : 0u;
    }
    if (p > 0 && !all_ok(ok, 0)) {
      // slow path: wave 0 waits for every workgroup's done word of the
      // producing phase, then every thread reads its words again until all
      // tags are this launch's
      const uint64_t *src = a.ph[p - 1].out_ll;
      if (wave == 0) {
        const uint32_t *dn = a.done + (size_t)(p - 1) * kMaxGrid;
        int rounds = 0;
        for (;;) {
          bool dok = true;
          for (int i = lane; i < grid; i += 64) dok &= ld_agent(dn + i) == tag_in;
          if (__builtin_amdgcn_ballot_w64(!dok) == 0) break;
          if (++rounds >= a.spin_cap) {
            if (lane == 0) set_err(a.err, 1 + p);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
      CH_BARRIER();
      for (int rounds = 1;; ++rounds) {
        bool rok = true;
        for (int w = tid; w < nwv; w += kThreads) {
          const uint64_t v = ll_load(src + w);
          rok &= (uint32_t)(v >> 32) == tag_in;
          ((uint32_t *)xs)[w] = (uint32_t)v;
        }
        if (all_ok(rok, rounds)) break;
        if (rounds >= a.spin_cap) {
          if (tid == 0) set_err(a.err, 1 + p);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    CH_BARRIER();

    // ---- the units: MFMAs over the staged activations; each tile's wave
    // partial goes to LDS when its last unit is done
    const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
    const int shalf = 16 * (nl & 1);  // the lane's row within its scale pair (tiles start at even rows)
    int cj = 0, ci = 0;
    float acc = 0.f;
    for (int q0 = 0; q0 < W.tpad; q0 += NS) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int q = q0 + s;
        issue_next(ring[(s + NS - 1) % NS], rs0[(s + NS - 1) % NS], rs1[(s + NS - 1) % NS]);
        if (q < W.total) {
          if (ci < W.cnt) {
            const int kb = (W.u0 + ci) * 128;
            float4_t part[2] = {zero4, zero4};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const u32x4 av = *(const u32x4 *)(xs + kb + 32 * j + 8 * kg);
              const u32x4 bw = dequant_f16(ring[s][j], 8u, dk);
              const int sl = GK == 0 ? 0 : j >> 1;
              part[sl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sf_bitcast<half8_t>(av),
                                                                sf_bitcast<half8_t>(bw), part[sl], 0, 0, 0);
            }
            // the scale bits are used here and only here (a conversion moved up
            // to the load would wait for every load issued before it)
            uint32_t s0 = rs0[s];
            asm volatile("" : "+v"(s0));
            acc = fmaf(part[0][0], (float)sf_bitcast<f16>((uint16_t)(s0 >> shalf)), acc);
            if constexpr (GK != 0) {
              uint32_t s1 = rs1[s];
              asm volatile("" : "+v"(s1));
              acc = fmaf(part[1][0], (float)sf_bitcast<f16>((uint16_t)(s1 >> shalf)), acc);
            }
          }
          if (++ci == W.upw) {
            if (lane < 16) red[(cj * kWaves + wave) * 16 + lane] = acc;  // A row 0, weight row `lane`
            acc = 0.f;
            ci = 0;
            ++cj;
          }
        }
      }
    }
    const int mine = W.mine;
    const int N_out = P.N, half_tiles = P.ntiles >> 1, swiglu = P.swiglu;
    float *const out = P.out;
    uint64_t *const out_ll = P.out_ll;
    CH_BARRIER();
    // ---- fold: each output sums its 16 wave partials in wave order
    auto wsum = [&](int k, int r) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += red[(k * kWaves + w) * 16 + r];
      return v;
    };
    if (out) {  // the last phase: fp32
      for (int idx = tid; idx < mine * 16; idx += kThreads) {
        const int k = idx >> 4, r = idx & 15;
        const int row = tile_of(a.ph[p], k, grid) * 16 + r;
        if (row < N_out) out[row] = wsum(k, r);
      }
    } else if (p != a.drop_phase) {
      if (swiglu) {  // silu(gate) * up of rows (r, r + 1) of each pair, one word
        for (int idx = tid; idx < (mine >> 1) * 8; idx += kThreads) {
          const int m = idx >> 3, r = 2 * (idx & 7);
          const int j = (int)blockIdx.x + m * grid;
          const float a0 = sf_silu_mul(wsum(2 * m, r), wsum(2 * m + 1, r));
          const float a1 = sf_silu_mul(wsum(2 * m, r + 1), wsum(2 * m + 1, r + 1));
          if (j < half_tiles) ll_store2(out_ll + (j * 16 + r) / 2, a0, a1, tag_out);
        }
      } else {  // rows (r, r + 1), one word (a row past N publishes 0)
        for (int idx = tid; idx < mine * 8; idx += kThreads) {
          const int k = idx >> 3, r = 2 * (idx & 7);
          const int row = ((int)blockIdx.x + k * grid) * 16 + r;
          if (row < N_out) ll_store2(out_ll + row / 2, wsum(k, r), row + 1 < N_out ? wsum(k, r + 1) : 0.f, tag_out);
        }
      }
      CH_BARRIER();
      if (tid == 0) st_agent(a.done + (size_t)p * kMaxGrid + blockIdx.x, tag_out);
    }
    // the next phase's input (first attempt), once this phase is published
    if (p + 1 < a.nph) read_input(p + 1, a.ph[p + 1]);
  }
  if (tid == 0) st_agent(a.epoch + blockIdx.x, epoch + 1);  // the next launch's epoch
}

}  // namespace sf_chain

using namespace sf_chain;

extern "C" size_t sf_q4_chain_workspace_bytes(const int *N, int nph) {
  if (!N || nph < 1 || nph > SF_CHAIN_MAX_PHASES) return 0;
  size_t b = kHeaderBytes;  // error word, epoch[1024], done[8][1024]
  for (int p = 0; p + 1 < nph; ++p) b += sf_align256((size_t)(N[p] + 1) / 2 * 8);  // published words
  return b;
}

extern "C" int sf_q4_chain(const void *const *blobs, const int *N, const int *K, const int *group,
                           const int *in_kind, int nph, const void *x0_f16, float *y_f32,
                           void *workspace, size_t ws_bytes, int spin_cap, int drop_phase,
                           void *stream) {
  SF_REQUIRE(blobs && N && K && group && in_kind && x0_f16 && y_f32 && workspace, SF_EINVAL,
             "sf_q4_chain: null argument");
  SF_REQUIRE(nph >= 1 && nph <= SF_CHAIN_MAX_PHASES, SF_EINVAL, "sf_q4_chain: %d phases (1..%d)", nph,
             SF_CHAIN_MAX_PHASES);
  SF_REQUIRE(ws_bytes >= sf_q4_chain_workspace_bytes(N, nph), SF_EINVAL,
             "sf_q4_chain: workspace of %zu bytes, need %zu", ws_bytes, sf_q4_chain_workspace_bytes(N, nph));
  SF_REQUIRE(((uintptr_t)workspace & 255) == 0 && ((uintptr_t)x0_f16 & 15) == 0, SF_EINVAL,
             "sf_q4_chain: workspace must be 256-byte and x0 16-byte aligned");
  SF_REQUIRE(spin_cap >= 1, SF_EINVAL, "sf_q4_chain: spin_cap must be >= 1");
  int dev = 0, cus = 0;
  SF_REQUIRE(hipGetDevice(&dev) == hipSuccess, SF_EHIP, "sf_q4_chain: hipGetDevice failed");
  SF_REQUIRE(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0,
             SF_EHIP, "sf_q4_chain: no CU count");
  SF_REQUIRE(cus <= 1024, SF_EUNSUPPORTED, "sf_q4_chain: %d CUs (at most 1024)", cus);
  Args a{};
  a.nph = nph;
  uint8_t *ws = (uint8_t *)workspace;
  a.err = (int *)ws;
  a.epoch = (uint32_t *)(ws + 64);
  a.done = (uint32_t *)(ws + 8192);
  size_t off = kHeaderBytes;
  for (int p = 0; p < nph; ++p) {
    const int g = group[p];
    SF_REQUIRE(N[p] > 0 && K[p] > 0 && blobs[p], SF_EINVAL, "sf_q4_chain: phase %d: empty", p);
    SF_REQUIRE(K[p] % 128 == 0 && K[p] <= kMaxK, SF_EUNSUPPORTED,
               "sf_q4_chain: phase %d: K=%d (a multiple of 128 up to %d)", p, K[p], kMaxK);
    SF_REQUIRE(g == 64 || (g % 128 == 0 && K[p] % g == 0), SF_EUNSUPPORTED,
               "sf_q4_chain: phase %d: group %d (64 or a multiple of 128)", p, g);
    SF_REQUIRE(in_kind[p] >= IN_X16 && in_kind[p] <= IN_LL_SILU && (in_kind[p] == IN_X16) == (p == 0),
               SF_EINVAL, "sf_q4_chain: phase %d: input kind %d (the first phase reads x0, the others "
               "the previous phase)", p, in_kind[p]);
    const bool swiglu = p + 1 < nph && in_kind[p + 1] == IN_LL_SILU;  // this phase feeds a SwiGLU
    BlobLayout L;
    sf_blob_layout(N[p], K[p], g, 0, &L);
    SF_REQUIRE(swiglu ? N[p] % 32 == 0 && 2 * ((L.NTI / 2 + cus - 1) / cus) <= kMaxTiles
                      : L.NTI <= kMaxTiles * cus,
               SF_EUNSUPPORTED, "sf_q4_chain: phase %d: %d rows (at most %d%s)", p, N[p], kMaxTiles * cus * 16,
               swiglu ? ", a multiple of 32 for a gate|up phase" : "");
    Phase &P = a.ph[p];
    P.w = (const uint8_t *)blobs[p];
    P.st = (const f16 *)((const uint8_t *)blobs[p] + L.s_off);
    P.N = N[p];
    P.K = K[p];
    P.G = L.G;
    P.nblk = L.NB;
    P.ntiles = L.NTI;
    P.upw = (L.NB + kWaves - 1) / kWaves;
    int gs = 0;
    while (g >= 128 && (128 << gs) < g) ++gs;
    SF_REQUIRE(g == 64 || (128 << gs) == g, SF_EUNSUPPORTED,
               "sf_q4_chain: phase %d: group %d (64, or 128 times a power of two)", p, g);
    P.gshift = gs;
    SF_REQUIRE((g == 64) == (group[0] == 64), SF_EUNSUPPORTED,
               "sf_q4_chain: phase %d: group %d; a chain runs groups of 64 or multiples of 128, not both", p, g);
    P.swiglu = swiglu;
    if (p > 0) {
      const bool sw_in = in_kind[p] == IN_LL_SILU;
      SF_REQUIRE(sw_in ? N[p - 1] == 2 * K[p] : N[p - 1] >= K[p], SF_EINVAL,
                 "sf_q4_chain: phase %d takes %s%d inputs, phase %d gives %d", p, sw_in ? "2 x " : "",
                 K[p], p - 1, N[p - 1]);
    }
    P.out_ll = p + 1 < nph ? (uint64_t *)(ws + off) : nullptr;
    P.out = p + 1 == nph ? y_f32 : nullptr;
    if (p + 1 < nph) off += sf_align256((size_t)(N[p] + 1) / 2 * 8);
  }
  a.x0 = (const f16 *)x0_f16;
  a.spin_cap = spin_cap;
  a.drop_phase = drop_phase;
  const bool g64 = group[0] == 64;
  const void *kfn = g64 ? (const void *)k_q4_chain<kRing, 1> : (const void *)k_q4_chain<kRing, 0>;
  static bool attr[2] = {false, false};
  if (!attr[g64]) {
    SF_REQUIRE(hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes) == hipSuccess,
               SF_EHIP, "sf_q4_chain: LDS attribute");
    attr[g64] = true;
  }
  int per_cu = 0;
  SF_REQUIRE(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kfn, kThreads, kLdsBytes) == hipSuccess &&
                 per_cu >= 1,
             SF_EHIP, "sf_q4_chain: the kernel does not fit a CU");
  if (g64) k_q4_chain<kRing, 1><<<cus, kThreads, kLdsBytes, (hipStream_t)stream>>>(a);
  else k_q4_chain<kRing, 0><<<cus, kThreads, kLdsBytes, (hipStream_t)stream>>>(a);
  return sf_check_launch("sf_q4_chain");
}

extern "C" int sf_q4_chain_error(const void *workspace, int *err_out, void *stream) {
  SF_REQUIRE(workspace && err_out, SF_EINVAL, "sf_q4_chain_error: null argument");
  int v = 0;
  SF_REQUIRE(hipMemcpyAsync(&v, workspace, 4, hipMemcpyDeviceToHost,
                            (hipStream_t)stream) == hipSuccess &&
                 hipStreamSynchronize((hipStream_t)stream) == hipSuccess,
             SF_EHIP, "sf_q4_chain_error: copy failed");
  *err_out = v;
  return 0;
}
