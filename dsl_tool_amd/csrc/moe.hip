// MoE glue on either side of the grouped FP8 GEMM:
//   route         top-k expert ids -> group offsets, each assignment's row in
//                 the expert-sorted order, and each sorted row's token;
//   permute_quant gather token rows into that order, quantized per row to
//                 E4M3 with scale amax/448 (the grouped GEMM's X and sx);
//   combine       out[t] = sum_j w[t, j] * Y[dest[t, j]] in slot order.
// The sorted order is stable: rows of one expert follow the flattened
// assignment order a = t * topk + j.  Ids outside [0, E) are dropped
// (dest = -1, no row).  Every step is deterministic (no float atomics, no
// order that depends on scheduling).
#include <type_traits>

#include "launch.h"
#include "quant_core.h"

namespace dsl {

constexpr int kRouteChunk = 256;      // assignments per block in the count and scatter passes
constexpr int kFusedScan = 16384;     // histogram ints each scatter block may read itself

// Pass 1: per-block expert histograms, counts[b][e].
__global__ __launch_bounds__(256) void moe_count_kernel(const int32_t *__restrict__ ids, int n,
                                                        int E, int32_t *__restrict__ counts) {
  extern __shared__ int hist[];
  for (int e = threadIdx.x; e < E; e += 256) hist[e] = 0;
  __syncthreads();
  const int a0 = blockIdx.x * kRouteChunk;
  for (int i = threadIdx.x; i < kRouteChunk && a0 + i < n; i += 256) {
    const int e = ids[a0 + i];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) counts[(int64_t)blockIdx.x * E + e] = hist[e];
}

// Scan for many blocks (one block of 16 x 64 threads): offsets[e] = rows of experts < e;
// counts[b][e] is replaced by the first sorted row of block b's expert-e
// assignments.  Experts go in runs of 64; thread (part, l) owns expert
// e0 + l over a contiguous range of blocks, so the column sums, the prefix
// over the 16 ranges, the wave scan over the 64 experts and the rewrite
// are each a few steps deep however many blocks there are.
__global__ __launch_bounds__(1024) void moe_scan_kernel(int32_t *__restrict__ counts, int nb, int E,
                                                       int32_t *__restrict__ offsets) {
  constexpr int PARTS = 16;
  __shared__ int psum[PARTS][64];      // a range's count of each expert, then its prefix
  __shared__ int first[64];            // first sorted row of each expert of the run
  const int l = threadIdx.x & 63, part = threadIdx.x >> 6;
  const int bpp = (nb + PARTS - 1) / PARTS;
  const int b0 = part * bpp, b1 = min(nb, b0 + bpp);
  int carry = 0;                       // wave 0: rows of the experts of earlier runs
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + l;
    int s = 0;
    if (e < E)
      for (int b = b0; b < b1; ++b) s += counts[(int64_t)b * E + e];
    psum[part][l] = s;
    __syncthreads();
    if (part == 0) {
      // exclusive prefix over the ranges, then over the experts (one wave)
      int tot = 0;
      for (int q = 0; q < PARTS; ++q) {
        const int c = psum[q][l];
        psum[q][l] = tot;
        tot += c;
      }
      int incl = tot;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        incl += l >= d ? v : 0;
      }
      first[l] = carry + incl - tot;
      if (e < E) offsets[e] = first[l];
      carry += __shfl(incl, 63, 64);
    }
    __syncthreads();
    if (e < E) {
      int r = first[l] + psum[part][l];
      for (int b = b0; b < b1; ++b) {
        const int c = counts[(int64_t)b * E + e];
        counts[(int64_t)b * E + e] = r;
        r += c;
      }
    }
    __syncthreads();                   // first[] and psum are rewritten by the next run
  }
  if (threadIdx.x == 0) offsets[E] = carry;
}

// Pass 2: bases and stable scatter, one block of four waves per chunk.
// With a small histogram (nb x E <= kFusedScan ints) the four waves first
// form, for each expert e (in runs of 64, thread (q, l) owning expert e0 + l
// over a quarter of the blocks), the rows of experts < e (offsets[e],
// written by block 0 for the grouped GEMM) plus the rows of expert e in
// blocks before this one: the chunk's first sorted row per expert.  Every
// block reads the whole histogram (L2-resident) instead of waiting for a
// separate scan launch.  Larger histograms take moe_scan_kernel first
// (scanned = 1: counts then holds each block's first rows).  Then wave 0 walks the
// chunk 64 assignments at a time; the lanes holding the same expert are
// found with one ballot per expert-id bit, so a lane's rank among the
// step's earlier same-expert lanes is a popcount, and the step's last such
// lane advances the expert's next row in LDS (a single wave: LDS operations
// stay in program order).
__global__ __launch_bounds__(256) void moe_scatter_kernel(const int32_t *__restrict__ ids, int n,
                                                         int E, int topk,
                                                         const int32_t *__restrict__ counts, int nb,
                                                         int scanned, int32_t *__restrict__ offsets,
                                                         int32_t *__restrict__ dest,
                                                         int32_t *__restrict__ src_token) {
  extern __shared__ int run[];          // [E] next sorted row per expert
  __shared__ int qbefore[4][64], qtot[4][64];
  const int l = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int blk = blockIdx.x;
  if (scanned) {                        // the bases are in counts already
    if (q != 0) return;
    for (int e = l; e < E; e += 64) run[e] = counts[(int64_t)blk * E + e];
  } else {
  const int bpq = (nb + 3) / 4, qb0 = q * bpq, qb1 = min(nb, qb0 + bpq);
  int carry = 0;                        // wave 0: rows of the experts of earlier runs
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + l;
    int before = 0, tot = 0;
    if (e < E) {
      // eight loads in flight per thread (the sums are integers: any order)
      int b = qb0;
      for (; b + 8 <= qb1; b += 8) {
        int c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) c[u] = counts[(int64_t)(b + u) * E + e];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          tot += c[u];
          before += b + u < blk ? c[u] : 0;
        }
      }
      for (; b < qb1; ++b) {
        const int c = counts[(int64_t)b * E + e];
        tot += c;
        before += b < blk ? c : 0;
      }
    }
    qbefore[q][l] = before;
    qtot[q][l] = tot;
    __syncthreads();
    if (q == 0) {
      const int bef = qbefore[0][l] + qbefore[1][l] + qbefore[2][l] + qbefore[3][l];
      const int tt = qtot[0][l] + qtot[1][l] + qtot[2][l] + qtot[3][l];
      int incl = tt;                    // inclusive scan over the run's 64 experts
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        incl += l >= d ? v : 0;
      }
      const int off = carry + incl - tt;
      if (e < E) {
        run[e] = off + bef;
        if (blk == 0) offsets[e] = off;
      }
      carry += __shfl(incl, 63, 64);
    }
    __syncthreads();                    // qbefore / qtot are rewritten by the next run
  }
  if (q != 0) return;
  if (blk == 0 && l == 0) offsets[E] = carry;
  }
  __builtin_amdgcn_wave_barrier();      // wave 0 alone from here: run[] is its own
  const int lane = l;
  int bits = 0;
  while ((1 << bits) < E + 1) ++bits;   // ids -1 map to E: bits cover 0..E
  const uint64_t below = (1ull << lane) - 1ull;
  const int a0 = blk * kRouteChunk;
  constexpr int STEPS = kRouteChunk / 64;
  int idv[STEPS];                       // the chunk's ids, all loads in flight at once
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int a = a0 + st * 64 + lane;
    idv[st] = a < n ? ids[a] : -1;
  }
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int s0 = st * 64;
    if (a0 + s0 >= n) break;            // uniform
    const int a = a0 + s0 + lane;
    const int e = idv[st];
    const bool valid = e >= 0 && e < E;
    const int key = valid ? e : E;      // dropped and past-the-end lanes share key E
    uint64_t same = ~0ull;
    for (int b = 0; b < bits; ++b) {
      const uint64_t m = __ballot((key >> b) & 1);
      same &= ((key >> b) & 1) ? m : ~m;
    }
    const int rank = __popcll(same & below);
    const bool last = (same >> lane) == 1ull;  // no higher lane holds this key
    int row = -1;
    if (valid) row = run[e] + rank;
    __builtin_amdgcn_s_waitcnt(0xc07f);        // lgkmcnt(0): every lane's read of run is back
    __builtin_amdgcn_wave_barrier();
    if (valid && last) run[e] = row + 1;
    if (a < n) {
      dest[a] = row;
      if (valid) src_token[row] = a / topk;
    }
  }
}

// Whole route in one wave (decode-size batches, up to 64 * kWaveSteps
// assignments): the ballot ranking of moe_scatter_kernel over the
// assignments step by step with per-expert counts in LDS, the exclusive
// scan over the experts (64 at a time, wave shuffles), then each lane writes
// the rows of the assignments it holds in registers.  One wave keeps its LDS
// operations in program order, so there is no barrier.
constexpr int kWaveSteps = 16;         // steps of 64: up to 1024 assignments

__global__ __launch_bounds__(64) void moe_route_wave_kernel(const int32_t *__restrict__ ids, int n,
                                                           int E, int topk,
                                                           int32_t *__restrict__ offsets,
                                                           int32_t *__restrict__ dest,
                                                           int32_t *__restrict__ src_token) {
  extern __shared__ int cnt[];           // [E] counts, then first rows
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) cnt[e] = 0;
  int bits = 0;
  while ((1 << bits) < E + 1) ++bits;
  const uint64_t below = (1ull << lane) - 1ull;
  const int steps = (n + 63) / 64;
  int kr[kWaveSteps];                    // key (12 bits, E for dropped) | rank << 12
#pragma unroll
  for (int st = 0; st < kWaveSteps; ++st) {
    kr[st] = E;
    if (st < steps) {                    // uniform
      const int a = st * 64 + lane;
      const int e = a < n ? ids[a] : -1;
      kr[st] = (e >= 0 && e < E) ? e : E;
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): the zeroed counts are in LDS
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int st = 0; st < kWaveSteps; ++st) {
    if (st < steps) {                    // uniform
      const int k = kr[st];
      uint64_t same = ~0ull;
      for (int b = 0; b < bits; ++b) {
        const uint64_t m = __ballot((k >> b) & 1);
        same &= ((k >> b) & 1) ? m : ~m;
      }
      int r = 0;
      if (k < E) r = cnt[k] + __popcll(same & below);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // every lane's read of cnt is back
      __builtin_amdgcn_wave_barrier();
      if (k < E && (same >> lane) == 1ull) cnt[k] = r + 1;
      kr[st] = k | (r << 12);
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {   // exclusive scan over the experts
    const int e = e0 + lane;
    const int c = e < E ? cnt[e] : 0;
    int incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(incl, d, 64);
      if (lane >= d) incl += t;
    }
    if (e < E) {
      cnt[e] = carry + incl - c;
      offsets[e] = carry + incl - c;
    }
    carry += __shfl(incl, 63, 64);
  }
  if (lane == 0) offsets[E] = carry;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int st = 0; st < kWaveSteps; ++st) {
    const int a = st * 64 + lane;
    if (st < steps && a < n) {
      const int k = kr[st] & 0xfff, r = kr[st] >> 12;
      const int row = k < E ? cnt[k] + r : -1;
      dest[a] = row;
      if (row >= 0) src_token[row] = a / topk;
    }
  }
}

// Whole route in one workgroup of 16 waves (small n; up to 16 * kOneSteps * 64):
// wave w ranks its contiguous range of assignments step by step with the
// ballot scheme of moe_scatter_kernel, keeping per-expert counts in LDS;
// the expert and wave prefix sums follow in LDS, and each lane then writes
// the final rows of the assignments it holds in registers.
constexpr int kOneSteps = 64;          // steps of 64 per wave: up to 65536 assignments

__global__ __launch_bounds__(1024) void moe_route_one_kernel(const int32_t *__restrict__ ids, int n,
                                                            int E, int topk,
                                                            int32_t *__restrict__ offsets,
                                                            int32_t *__restrict__ dest,
                                                            int32_t *__restrict__ src_token) {
  extern __shared__ int cnt[];           // [16][E] per-wave counts, then wave bases
  __shared__ int tot[kMaxGroups + 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 16 * E; i += 1024) cnt[i] = 0;
  __syncthreads();
  const int per_wave = (n + 15) / 16;
  const int steps = (per_wave + 63) / 64;
  const int a0 = w * per_wave, a1 = min(n, a0 + per_wave);
  int bits = 0;
  while ((1 << bits) < E + 1) ++bits;
  const uint64_t below = (1ull << lane) - 1ull;
  // key (12 bits, E for dropped) and rank within the wave (20 bits), packed
  int kr[kOneSteps];
  int *mine = cnt + w * E;
#pragma unroll
  for (int st = 0; st < kOneSteps; ++st) {
    kr[st] = E;
    if (st < steps) {                    // uniform
      const int a = a0 + st * 64 + lane;
      const int e = a < a1 ? ids[a] : -1;
      kr[st] = (e >= 0 && e < E) ? e : E;
    }
  }
#pragma unroll
  for (int st = 0; st < kOneSteps; ++st) {
    if (st < steps) {                    // uniform
      const int k = kr[st];
      uint64_t same = ~0ull;
      for (int b = 0; b < bits; ++b) {
        const uint64_t m = __ballot((k >> b) & 1);
        same &= ((k >> b) & 1) ? m : ~m;
      }
      int r = 0;
      if (k < E) r = mine[k] + __popcll(same & below);
      __builtin_amdgcn_wave_barrier();
      if (k < E && (same >> lane) == 1ull) mine[k] = r + 1;
      kr[st] = k | (r << 12);
    }
  }
  __syncthreads();
  // per expert: total and the prefix over waves (cnt becomes the wave base)
  for (int e = threadIdx.x; e < E; e += 1024) {
    int s = 0;
    for (int ww = 0; ww < 16; ++ww) {
      const int c = cnt[ww * E + e];
      cnt[ww * E + e] = s;
      s += c;
    }
    tot[e] = s;
  }
  __syncthreads();
  if (w == 0) {                          // exclusive scan over experts, 64 at a time
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int c = e < E ? tot[e] : 0;
      int incl = c;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
      }
      if (e < E) {
        tot[e] = carry + incl - c;
        offsets[e] = carry + incl - c;
      }
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) offsets[E] = carry;
  }
  __syncthreads();
#pragma unroll
  for (int st = 0; st < kOneSteps; ++st) {
    const int a = a0 + st * 64 + lane;
    if (st < steps && a < a1) {
      const int k = kr[st] & 0xfff, r = kr[st] >> 12;
      const int row = k < E ? tot[k] + cnt[w * E + k] + r : -1;
      dest[a] = row;
      if (row >= 0) src_token[row] = a / topk;
    }
  }
}

// Per-token E4M3 scattered to every routed slot: one workgroup per token,
// thread t holding chunks t + 256 j of the row.  The token is read and
// quantized once and its codes and scale are written to each sorted row
// dest[t * topk + j] that lies in [0, rows); dropped slots (-1) are skipped.
template <int CPL>
__global__ __launch_bounds__(256) void moe_permute_quant_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, int k_dim, const int32_t *__restrict__ dest,
    int topk, int rows, uint8_t *__restrict__ qx, float *__restrict__ sx, int tok_major) {
  __shared__ float sh[4];
  const int t = blockIdx.x;
  const int nch = k_dim >> 3;
  const uint16_t *xr = x + (int64_t)t * ldx;
  uint4 xa[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = threadIdx.x + 256 * j;
    xa[j] = c < nch ? reinterpret_cast<const uint4 *>(xr)[c] : make_uint4(0, 0, 0, 0);
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(xa[j], f);
    m = fmaxf(m, amax8(f));
  }
  const float s = fp8_scale_of(block_max(m, sh));
  const float r = rcp_approx(s);
  uint2 q[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(xa[j], f);
    q[j] = e4m3_quot8(f, s, r);
  }
  for (int slot = 0; slot < topk; ++slot) {
    const int row = dest[(int64_t)t * topk + slot];
    if (row < 0 || row >= rows) continue;                // uniform across the block
    if (threadIdx.x == 0) sx[row] = s;
    if (tok_major) continue;
    uint8_t *qr = qx + (int64_t)row * k_dim;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = threadIdx.x + 256 * j;
      if (c < nch) *reinterpret_cast<uint2 *>(qr + (int64_t)c * 8) = q[j];
    }
  }
  if (tok_major) {                                       // codes once, at the token's row
    uint8_t *qr = qx + (int64_t)t * k_dim;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = threadIdx.x + 256 * j;
      if (c < nch) *reinterpret_cast<uint2 *>(qr + (int64_t)c * 8) = q[j];
    }
  }
}

// The same with 16 elements per thread (k % 16 == 0): 128 threads, each
// chunk read as two 16-byte loads and written as one 16-byte store of codes
// per routed row.  Per element it is the same arithmetic, so the codes and
// scales are identical.
template <int CPL>
__global__ __launch_bounds__(128) void moe_permute_quant16_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, int k_dim, const int32_t *__restrict__ dest,
    int topk, int rows, uint8_t *__restrict__ qx, float *__restrict__ sx, int tok_major) {
  __shared__ float sh[2];
  const int t = blockIdx.x;
  const int nch = k_dim >> 4;
  const uint4 *xr = reinterpret_cast<const uint4 *>(x + (int64_t)t * ldx);
  uint4 xa[CPL][2];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = threadIdx.x + 128 * j;
    xa[j][0] = c < nch ? xr[2 * c] : make_uint4(0, 0, 0, 0);
    xa[j][1] = c < nch ? xr[2 * c + 1] : make_uint4(0, 0, 0, 0);
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float f[8];
      unpack8(xa[j][h], f);
      m = fmaxf(m, amax8(f));
    }
  const float s = fp8_scale_of(block_max(m, sh));
  const float r = rcp_approx(s);
  uint4 q[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(xa[j][0], f);
    const uint2 lo = e4m3_quot8(f, s, r);
    unpack8(xa[j][1], f);
    const uint2 hi = e4m3_quot8(f, s, r);
    q[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
  for (int slot = 0; slot < topk; ++slot) {
    const int row = dest[(int64_t)t * topk + slot];
    if (row < 0 || row >= rows) continue;                // uniform across the block
    if (threadIdx.x == 0) sx[row] = s;
    if (tok_major) continue;
    uint4 *qr = reinterpret_cast<uint4 *>(qx + (int64_t)row * k_dim);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = threadIdx.x + 128 * j;
      if (c < nch) qr[c] = q[j];
    }
  }
  if (tok_major) {                                       // codes once, at the token's row
    uint4 *qr = reinterpret_cast<uint4 *>(qx + (int64_t)t * k_dim);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = threadIdx.x + 128 * j;
      if (c < nch) qr[c] = q[j];
    }
  }
}

// Token-major quantize for rows of up to 2048 elements (k % 8 == 0): one
// wave per token (four per workgroup), lane l holding chunks l + 64 j, the
// amax by wave reduction alone; codes to the token's row, the scale to each
// routed row by the lanes j < topk.  Same arithmetic as above, so the same
// codes and scales.
template <int CPL>
__global__ __launch_bounds__(256) void moe_quant_tokens_wave_kernel(
    const uint16_t *__restrict__ x, int64_t ldx, int k_dim, int tokens,
    const int32_t *__restrict__ dest, int topk, int rows, uint8_t *__restrict__ qx,
    float *__restrict__ sx) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;                       // whole waves: no barrier below
  const int lane = threadIdx.x & 63;
  const int nch = k_dim >> 3;
  const uint4 *xr = reinterpret_cast<const uint4 *>(x + (int64_t)t * ldx);
  uint4 d[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    d[j] = c < nch ? xr[c] : make_uint4(0, 0, 0, 0);
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(d[j], f);
    m = fmaxf(m, amax8(f));
  }
  const float s = fp8_scale_of(wave_max(m));
  const float r = rcp_approx(s);
  uint2 *qr = reinterpret_cast<uint2 *>(qx + (int64_t)t * k_dim);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c < nch) {
      float f[8];
      unpack8(d[j], f);
      qr[c] = e4m3_quot8(f, s, r);
    }
  }
  for (int slot = lane; slot < topk; slot += 64) {
    const int row = dest[(int64_t)t * topk + slot];
    if (row >= 0 && row < rows) sx[row] = s;
  }
}

// Route and per-token quantize in one launch for decode-size batches (up to
// 64 * kWaveSteps assignments, k <= 2048): one wave per token, four per
// workgroup.  Every wave ranks all the assignments exactly as
// moe_route_wave_kernel does (ballots per step, per-expert counts in its own
// LDS slice, the exclusive scan over the experts) -- a few hundred
// instructions at these sizes, issued while the token's row is loading --
// and then writes its own token's part only: dest and src_token of the
// token's assignments, the token's codes (as moe_quant_tokens_wave_kernel),
// and its scale at each of the token's sorted rows.  Token 0's wave writes
// the offsets.  So the tables, codes and scales are those of the two
// launches it replaces, bit for bit.
template <int CPL>
__global__ __launch_bounds__(256) void moe_route_quant_wave_kernel(
    const int32_t *__restrict__ ids, int n, int E, int topk, const uint16_t *__restrict__ x,
    int64_t ldx, int k_dim, int tokens, int32_t *__restrict__ offsets,
    int32_t *__restrict__ dest, int32_t *__restrict__ src_token, uint8_t *__restrict__ qx,
    float *__restrict__ sx) {
  extern __shared__ int slices[];        // [4 waves][E] counts, then first rows
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;               // whole waves: no barrier below
  const int lane = threadIdx.x & 63;
  int *cnt = slices + (threadIdx.x >> 6) * E;
  // the token's row first: its loads are in flight during the ranking
  const int nch = k_dim >> 3;
  const uint4 *xr = reinterpret_cast<const uint4 *>(x + (int64_t)t * ldx);
  uint4 d[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    d[j] = c < nch ? xr[c] : make_uint4(0, 0, 0, 0);
  }
  for (int e = lane; e < E; e += 64) cnt[e] = 0;
  int bits = 0;
  while ((1 << bits) < E + 1) ++bits;
  const uint64_t below = (1ull << lane) - 1ull;
  const int steps = (n + 63) / 64;
  int kr[kWaveSteps];                    // key (12 bits, E for dropped) | rank << 12
#pragma unroll
  for (int st = 0; st < kWaveSteps; ++st) {
    kr[st] = E;
    if (st < steps) {                    // uniform
      const int a = st * 64 + lane;
      const int e = a < n ? ids[a] : -1;
      kr[st] = (e >= 0 && e < E) ? e : E;
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): the zeroed counts are in LDS
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int st = 0; st < kWaveSteps; ++st) {
    if (st < steps) {                    // uniform
      const int k = kr[st];
      uint64_t same = ~0ull;
      for (int b = 0; b < bits; ++b) {
        const uint64_t m = __ballot((k >> b) & 1);
        same &= ((k >> b) & 1) ? m : ~m;
      }
      int r = 0;
      if (k < E) r = cnt[k] + __popcll(same & below);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // every lane's read of cnt is back
      __builtin_amdgcn_wave_barrier();
      if (k < E && (same >> lane) == 1ull) cnt[k] = r + 1;
      kr[st] = k | (r << 12);
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {   // exclusive scan over the experts
    const int e = e0 + lane;
    const int c = e < E ? cnt[e] : 0;
    int incl = c;
#pragma unroll
    for (int dd = 1; dd < 64; dd <<= 1) {
      const int v = __shfl_up(incl, dd, 64);
      if (lane >= dd) incl += v;
    }
    if (e < E) {
      cnt[e] = carry + incl - c;
      if (t == 0) offsets[e] = carry + incl - c;
    }
    carry += __shfl(incl, 63, 64);
  }
  if (t == 0 && lane == 0) offsets[E] = carry;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  // the token's codes and scale (moe_quant_tokens_wave_kernel's arithmetic)
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float f[8];
    unpack8(d[j], f);
    m = fmaxf(m, amax8(f));
  }
  const float s = fp8_scale_of(wave_max(m));
  const float rq = rcp_approx(s);
  uint2 *qr = reinterpret_cast<uint2 *>(qx + (int64_t)t * k_dim);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c < nch) {
      float f[8];
      unpack8(d[j], f);
      qr[c] = e4m3_quot8(f, s, rq);
    }
  }
  // the token's assignments t*topk .. t*topk+topk-1, held by lane a % 64 at
  // step a / 64: their rows, and the scale at each
#pragma unroll
  for (int st = 0; st < kWaveSteps; ++st) {
    const int a = st * 64 + lane;
    if (st < steps && a < n && a / topk == t) {
      const int k = kr[st] & 0xfff, r = kr[st] >> 12;
      const int row = k < E ? cnt[k] + r : -1;
      dest[a] = row;
      if (row >= 0) {
        src_token[row] = t;
        sx[row] = s;
      }
    }
  }
}

// out[t] = sum_j w[t, j] * y[dest[t, j]] (dropped slots skipped), fp32 in
// slot order with separate multiply and add, then bf16 or fp32.
template <int CPL>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const uint16_t *__restrict__ y, int rows_y, int64_t ldy, int n, const int32_t *__restrict__ dest,
    const float *__restrict__ w, int topk, void *__restrict__ out, int64_t ldo, int out_f32) {
#pragma clang fp contract(off)   // one rounding per multiply and per add, as specified
  const int t = blockIdx.x;
  const int nch = n >> 3;
  float acc[CPL][8];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
  // slots in groups of up to 8: every row load of a group in flight before
  // its adds, which stay in slot order
  constexpr int G = CPL <= 2 ? 8 : (CPL <= 4 ? 4 : 1);
  for (int s0 = 0; s0 < topk; s0 += G) {
    uint4 yv[G][CPL];
    float wsv[G];
    bool ok[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int s = s0 + g;
      const int row = s < topk ? dest[(int64_t)t * topk + s] : -1;
      ok[g] = row >= 0 && row < rows_y;                 // uniform across the block
      wsv[g] = ok[g] ? w[(int64_t)t * topk + s] : 0.f;
      const uint4 *yr = reinterpret_cast<const uint4 *>(y + (int64_t)(ok[g] ? row : 0) * ldy);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = threadIdx.x + 256 * j;
        yv[g][j] = (ok[g] && c < nch) ? yr[c] : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (!ok[g]) continue;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        float f[8];
        unpack8(yv[g][j], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = acc[j][e] + wsv[g] * f[e];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = threadIdx.x + 256 * j;
    if (c >= nch) continue;
    if (out_f32) {
      float *o = static_cast<float *>(out) + (int64_t)t * ldo + (int64_t)c * 8;
      reinterpret_cast<float4 *>(o)[0] = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
      reinterpret_cast<float4 *>(o)[1] = make_float4(acc[j][4], acc[j][5], acc[j][6], acc[j][7]);
    } else {
      uint4 o;
      o.x = pack_bf16x2(acc[j][0], acc[j][1]);
      o.y = pack_bf16x2(acc[j][2], acc[j][3]);
      o.z = pack_bf16x2(acc[j][4], acc[j][5]);
      o.w = pack_bf16x2(acc[j][6], acc[j][7]);
      reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + (int64_t)t * ldo)[c] = o;
    }
  }
}

size_t moe_route_workspace_bytes(int64_t assignments, int64_t num_experts) {
  const int64_t nb = (assignments + kRouteChunk - 1) / kRouteChunk;
  return (size_t)(nb < 1 ? 1 : nb) * (size_t)num_experts * sizeof(int32_t);
}

hipError_t launch_moe_route(const int32_t *ids, int n, int topk, int E, int32_t *offsets,
                            int32_t *dest, int32_t *src_token, int32_t *ws, hipStream_t st) {
  // one launch for small batches (decode-time routing); the two-pass form
  // (histograms, then bases + scatter per chunk) spreads the scattered row
  // writes over many CUs and wins beyond that (32768 assignments: 20 us for
  // the earlier three passes against 38 us in one workgroup)
  if (n <= 64 * kWaveSteps && E <= 2047) {
    moe_route_wave_kernel<<<1, 64, (size_t)E * sizeof(int), st>>>(ids, n, E, topk, offsets, dest,
                                                                  src_token);
    return hipGetLastError();
  }
  if (n <= 4096 && E <= 2047 && 16 * E * (int)sizeof(int) <= 64 * 1024) {
    moe_route_one_kernel<<<1, 1024, (size_t)16 * E * sizeof(int), st>>>(ids, n, E, topk, offsets,
                                                                        dest, src_token);
    return hipGetLastError();
  }
  // at least one block: with no assignments it still writes the zero offsets
  const int nb = n > 0 ? (n + kRouteChunk - 1) / kRouteChunk : 1;
  const size_t lds = (size_t)E * sizeof(int);
  moe_count_kernel<<<nb, 256, lds, st>>>(ids, n, E, ws);
  const int scanned = (int64_t)nb * E > kFusedScan;
  if (scanned) moe_scan_kernel<<<1, 1024, 0, st>>>(ws, nb, E, offsets);
  moe_scatter_kernel<<<nb, 256, lds, st>>>(ids, n, E, topk, ws, nb, scanned, offsets, dest,
                                           src_token);
  return hipGetLastError();
}

template <class F>
static void by_cpl(int cols, F &&f) {
  const int per = (cols / 8 + 255) / 256;
  if (per <= 1) f(std::integral_constant<int, 1>{});
  else if (per <= 2) f(std::integral_constant<int, 2>{});
  else if (per <= 4) f(std::integral_constant<int, 4>{});
  else if (per <= 8) f(std::integral_constant<int, 8>{});
  else f(std::integral_constant<int, 16>{});
}

hipError_t launch_moe_permute_quant(const uint16_t *x, int64_t ldx, int k_dim, int tokens,
                                    const int32_t *dest, int topk, int rows, uint8_t *qx, float *sx,
                                    bool tok_major, hipStream_t st) {
  if (tokens == 0 || (rows == 0 && !tok_major)) return hipSuccess;
  if (tok_major && k_dim <= 2048 && ldx % 8 == 0) {
    const unsigned g = (unsigned)((tokens + 3) / 4);
    const int per = (k_dim / 8 + 63) / 64;
    if (per <= 1)
      moe_quant_tokens_wave_kernel<1><<<g, 256, 0, st>>>(x, ldx, k_dim, tokens, dest, topk, rows, qx, sx);
    else if (per <= 2)
      moe_quant_tokens_wave_kernel<2><<<g, 256, 0, st>>>(x, ldx, k_dim, tokens, dest, topk, rows, qx, sx);
    else
      moe_quant_tokens_wave_kernel<4><<<g, 256, 0, st>>>(x, ldx, k_dim, tokens, dest, topk, rows, qx, sx);
    return hipGetLastError();
  }
  if (k_dim % 16 == 0 && ldx % 8 == 0) {
    // 16-element chunks over 128 threads: the chunk count per thread is
    // that of 8-element chunks over 256
    by_cpl(k_dim, [&](auto cpl) {
      moe_permute_quant16_kernel<decltype(cpl)::value><<<tokens, 128, 0, st>>>(x, ldx, k_dim, dest,
                                                                               topk, rows, qx, sx,
                                                                               tok_major ? 1 : 0);
    });
  } else {
    by_cpl(k_dim, [&](auto cpl) {
      moe_permute_quant_kernel<decltype(cpl)::value><<<tokens, 256, 0, st>>>(x, ldx, k_dim, dest,
                                                                             topk, rows, qx, sx,
                                                                             tok_major ? 1 : 0);
    });
  }
  return hipGetLastError();
}

hipError_t launch_moe_route_quant(const int32_t *ids, int n, int topk, int E,
                                  const uint16_t *x, int64_t ldx, int k_dim, int tokens,
                                  int32_t *offsets, int32_t *dest, int32_t *src_token,
                                  uint8_t *qx, float *sx, hipStream_t st) {
  static_assert(moe_route_quant_max_assignments == 64 * kWaveSteps, "one wave ranks them all");
  if (tokens < 1 || n < 1 || n > moe_route_quant_max_assignments || E < 1 || E > 2047 ||
      k_dim < 8 || k_dim > 2048 || k_dim % 8 != 0 || ldx % 8 != 0)
    return hipErrorInvalidValue;
  const unsigned g = (unsigned)((tokens + 3) / 4);
  const size_t lds = (size_t)4 * E * sizeof(int);
  const int per = (k_dim / 8 + 63) / 64;
  if (per <= 1)
    moe_route_quant_wave_kernel<1><<<g, 256, lds, st>>>(ids, n, E, topk, x, ldx, k_dim, tokens,
                                                        offsets, dest, src_token, qx, sx);
  else if (per <= 2)
    moe_route_quant_wave_kernel<2><<<g, 256, lds, st>>>(ids, n, E, topk, x, ldx, k_dim, tokens,
                                                        offsets, dest, src_token, qx, sx);
  else
    moe_route_quant_wave_kernel<4><<<g, 256, lds, st>>>(ids, n, E, topk, x, ldx, k_dim, tokens,
                                                        offsets, dest, src_token, qx, sx);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const uint16_t *y, int rows_y, int64_t ldy, int n, const int32_t *dest,
                              const float *w, int tokens, int topk, void *out, int64_t ldo,
                              int out_f32, hipStream_t st) {
  if (tokens == 0) return hipSuccess;
  by_cpl(n, [&](auto cpl) {
    moe_combine_kernel<decltype(cpl)::value><<<tokens, 256, 0, st>>>(y, rows_y, ldy, n, dest, w, topk,
                                                                     out, ldo, out_f32);
  });
  return hipGetLastError();
}

}  // namespace dsl
