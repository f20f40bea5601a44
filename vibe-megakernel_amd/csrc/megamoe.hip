// megamoe.hip — FP8 (E4M3, 128x128 block-scaled) MoE decode layer for MI355X (gfx950).
//
// The layer, as five stream-ordered kernel launches (one process, one GPU):
//   k_router                  router logits on fp64 MFMA as split partials over H
//   k_select                  adds the split partials in order and rounds once to fp32, then
//                             per token (one wavefront each): sigmoid/softmax gate,
//                             group-limited top-k with a (value desc, index asc) total order;
//                             its extra workgroups quantize x (E4M3, one fp32 scale per token
//                             per 128)
//   k_permute                 one workgroup: expert histogram, exclusive scan, stable
//                             (token, slot)-ordered permutation, and the expert work lists
//                             (chunks of <= 64 rows, heaviest first)
//   k_experts                 one persistent kernel draining a work queue of gate/up units
//                             (chunk, 128-row block of I), then down units (chunk, 128-row
//                             block of H): weights streamed from HBM into fp8 MFMA
//                             (16x16x128, weights as the M operand, tokens as N), 128x128
//                             block scales applied per K block, SwiGLU and the per-128 E4M3
//                             requantization of h fused into gate/up; a down unit starts
//                             as soon as the gate/up units of its rows are done
//   k_combine                 slot-order fp32 sum of bf16(d)*w plus the shared expert,
//                             rounded once to bf16 (and, in the block form, the residual add)
//
// The block form (megamoe_block_forward) adds the steps either side of the layer in the
// reference's decoder block (frontier.py:335,354): k_norm, the RMSNorm of x that the router
// and the experts read, as a sixth launch before k_router, and the residual add in k_combine.
//
// Reference math (all eager PyTorch in the reference): megabench/tasks/frontier.py:180-186
// (linear), :229-242 (route), :335-354 (MoE block); megabench/tasks/quantization.py:57-131
// (FP8 formats); megabench/tasks/references/moe.py:66-78 and distributed.py:174-176
// (softmax routing); megabench/tasks/megamoe.py:131-150,161-168 (expert grouping order).

#include <hip/hip_runtime.h>
#include <math.h>
#include <mutex>
#include <stdlib.h>
#include <stddef.h>
#include <type_traits>
#include <stdint.h>
#include <string.h>

#include "megamoe.h"


namespace {

constexpr int kBlock = 128;  // quantization block edge (weights 128x128, activations 1x128)

// Row stride (in floats) of the h scale rows: whole 128-byte lines, so rows of different
// chunks never share a cache line (see the hand-over notes of the expert kernel).
__host__ __device__ constexpr int scale_ld(int blocks) { return (blocks + 31) / 32 * 32; }

// Bound of one readiness wait, in ticks of the 100 MHz real-time clock (s_memrealtime):
// past it (or once any wait has given up) the wait ends and flags an error, and the
// combine then writes NaN to every output element.
constexpr uint64_t kWaitTicks = 20000000;  // 0.2 s

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------------------
// Scalar numerics shared by the kernels
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// float -> bf16 bits, round to nearest even; NaN becomes the canonical quiet NaN 0x7fc0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// float -> E4M3FN code, round to nearest even. Callers clamp to [-448, 448] first, as
// quantization.py:106,125 do; NaN maps to 0x7f with its sign.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  uint32_t code;
  if (a > 0x7f800000u) {
    code = 0x7fu;
  } else if (a < 0x3c800000u) {
    // Below 2^-6 the E4M3 grid is uniform with step 2^-9; the product is exact and
    // rint rounds half to even. A result of 8 is the smallest normal, code 0x08.
    code = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  } else {
    const uint32_t e = (a >> 23) - 120u;  // E4M3 biased exponent (bias 7)
    const uint32_t keep = (a >> 20) & 7u, rest = a & 0xfffffu;
    code = (e << 3) | keep;
    code += (rest > 0x80000u) || (rest == 0x80000u && (keep & 1u));
  }
  return sign | code;
}

__device__ __forceinline__ float clamp448(float v) { return v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v); }

// Four floats in [-448, 448] (or NaN) -> four E4M3FN codes in bytes 0..3, by gfx950's
// v_cvt_pk_fp8_f32 (OCP E4M3, round to nearest even), two per instruction. It gives
// f32_to_e4m3's code for every fp32 value in [-448, 448] of either sign (the whole range a
// clamped value can take; megamoe_e4m3_selftest compares the two on all of them); for a
// positive NaN it gives 0xff, which is set to 0x7f here, as f32_to_e4m3 (and torch) code it.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  const float v[4] = {a, b, c, d};
  uint32_t pos_nan = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) pos_nan |= (__float_as_uint(v[i]) - 0x7f800001u < 0x7fffffu ? 0x80u : 0u) << (8 * i);
  return w & ~pos_nan;
}

// Activation scale of one 128-block: max(amax, 1e-4) / 448 (quantization.py:57-58), or
// the smallest power of two not below it when pow2 is set (quantization.py:59).
__device__ __forceinline__ float act_scale(float amax, int pow2) {
  float s = fmaxf(amax, 1e-4f) / 448.0f;
  if (pow2) {
    const uint32_t b = __float_as_uint(s);
    if (b & 0x7fffffu) s = __uint_as_float(((b >> 23) + 1u) << 23);
  }
  return s;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// threadIdx.x % 64 behind an empty asm: what the persistent kernels' units derive from it is computed
// where it is used, not hoisted out of the persistent loop and held (or spilled) across it.
__device__ __forceinline__ int opaque_lane() {
  int l = threadIdx.x & 63;
  asm volatile("" : "+v"(l));
  return l;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Device-coherent stores: relaxed agent-scope atomic stores, which write through the XCD's
// L2 to memory, so a workgroup on another XCD that has not read the line before reads the
// new value (the hand-over rule of the expert and layer kernels below).
__device__ __forceinline__ void store_coherent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(int64_t* p, int64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(double* p, double v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(int4* p, int4 v) {
  store_coherent(reinterpret_cast<uint64_t*>(p), (uint64_t)(uint32_t)v.x | ((uint64_t)(uint32_t)v.y << 32));
  store_coherent(reinterpret_cast<uint64_t*>(p) + 1, (uint64_t)(uint32_t)v.z | ((uint64_t)(uint32_t)v.w << 32));
}
// All of this wavefront's memory operations complete (vmcnt, expcnt and lgkmcnt zero).
__device__ __forceinline__ void publish_fence() { __builtin_amdgcn_s_waitcnt(0); }

// A store that another workgroup of the same kernel reads (CO: device-coherent, as above)
// or that only later kernels read (a plain store; kernel boundaries order it).
template <bool CO, class T>
__device__ __forceinline__ void store_out(T* p, T v) {
  if constexpr (CO)
    store_coherent(p, v);
  else
    *p = v;
}

// ---------------------------------------------------------------------------------------
// Dynamic E4M3 quantization of one full 128-wide block by one wavefront (two values per
// lane): scale = max(amax, 1e-4)/448, code = RNE(clamp(v / scale, +-448)).
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ void quant_block(const uint16_t* src, uint8_t* dst, float* scale, int pow2, int lane) {
  const uint32_t two = *reinterpret_cast<const uint32_t*>(src + 2 * lane);
  const float v0 = bf16_bits_to_f32(two & 0xffffu), v1 = bf16_bits_to_f32(two >> 16);
  const float s = act_scale(wave_max(fmaxf(fabsf(v0), fabsf(v1))), pow2);
  const uint32_t q = e4m3x4(clamp448(v0 / s), clamp448(v1 / s), 0.0f, 0.0f);
  *reinterpret_cast<uint16_t*>(dst + 2 * lane) = (uint16_t)q;
  if (lane == 0) *scale = s;
}

// Ragged rows (any column count): one wavefront per (row, 128-column block).
__global__ __launch_bounds__(256) void k_quant_rows(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                    float* __restrict__ scales, int rows, int cols, int pow2) {
  const int nb = (cols + kBlock - 1) / kBlock;
  const int lane = threadIdx.x & 63;
  const long nwaves = (long)gridDim.x * 4;
  for (long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6); b < (long)rows * nb; b += nwaves) {
    const int r = (int)(b / nb), cb = (int)(b % nb);
    const int c = cb * kBlock + 2 * lane;
    const uint16_t* src = x + (size_t)r * cols;
    const float v0 = c < cols ? bf16_bits_to_f32(src[c]) : 0.0f;
    const float v1 = c + 1 < cols ? bf16_bits_to_f32(src[c + 1]) : 0.0f;
    const float amax = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
    const float s = act_scale(amax, pow2);
    uint8_t* dst = q + (size_t)r * cols;
    const uint32_t code = e4m3x4(clamp448(v0 / s), clamp448(v1 / s), 0.0f, 0.0f);
    if (c < cols) dst[c] = (uint8_t)code;
    if (c + 1 < cols) dst[c + 1] = (uint8_t)(code >> 8);
    if (lane == 0) scales[(size_t)r * nb + cb] = s;
  }
}

// Self-test of e4m3x4 against f32_to_e4m3 on the magnitudes [first, first + count) as fp32
// bit patterns, each with both signs and in each of the four code slots: the mismatches are
// added to *bad.
__global__ __launch_bounds__(256) void k_e4m3_selftest(uint32_t first, uint32_t count,
                                                       unsigned long long* __restrict__ bad) {
  unsigned long long n = 0;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < count; i += gridDim.x * 256u) {
#pragma unroll
    for (int sgn = 0; sgn < 2; ++sgn) {
      const float f = __uint_as_float((first + i) | (sgn ? 0x80000000u : 0u));
      const uint32_t want = f32_to_e4m3(f) * 0x01010101u;
      n += e4m3x4(f, f, f, f) != want;
    }
  }
  if (n) atomicAdd(bad, n);
}

// ---------------------------------------------------------------------------------------
// RMSNorm of bf16 rows (megabench/tasks/common.py:13-21, weight_in_fp32 as there), one
// workgroup per row:
//   s = sum of x^2 (fp64: each square of a bf16 value is exact, and the sum of a row's
//       squares stays exact unless its magnitudes span more than 2^37),
//   m = fp32(s / H), r = 1 / sqrt(m + eps) (fp32, each operation correctly rounded),
//   n = fp32(x) * r, out = bf16(n * w) (weight_in_fp32) or bf16(bf16(n) * w).
// The reference's fp32 mean and rsqrt round in torch's order; the band absorbs the
// difference (an ulp of r at most moves a bf16 output by one ulp).
// ---------------------------------------------------------------------------------------

constexpr int kNormChunks = 8;                     // 4-element chunks per thread and pass
constexpr int kNormPass = 256 * 4 * kNormChunks;  // elements of a row per pass (8192)

struct NormChunks {
  uint2 x[kNormChunks], w[kNormChunks];
};

// Chunk k of a pass is elements 4 * (tid + 256 k) .. +3 from `base`; past H reads nothing.
__device__ __forceinline__ void norm_load(NormChunks& c, const uint16_t* xr, const uint16_t* w, int base, int H,
                                          int tid) {
#pragma unroll
  for (int k = 0; k < kNormChunks; ++k) {
    const int e = base + 4 * (tid + 256 * k);
    const bool in = e < H;
    c.x[k] = in ? *reinterpret_cast<const uint2*>(xr + e) : make_uint2(0u, 0u);
    c.w[k] = in ? *reinterpret_cast<const uint2*>(w + e) : make_uint2(0u, 0u);
  }
}

__device__ __forceinline__ double norm_squares(const NormChunks& c) {
  double s = 0.0;
#pragma unroll
  for (int k = 0; k < kNormChunks; ++k) {
    const uint32_t q[2] = {c.x[k].x, c.x[k].y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const double a = bf16_bits_to_f32(q[i] & 0xffffu), b = bf16_bits_to_f32(q[i] >> 16);
      s += a * a;
      s += b * b;
    }
  }
  return s;
}

template <bool CO>
__device__ __forceinline__ void norm_store(const NormChunks& c, uint16_t* orow, int base, int H, int tid, float r,
                                           int weight_in_fp32) {
#pragma unroll
  for (int k = 0; k < kNormChunks; ++k) {
    const int e = base + 4 * (tid + 256 * k);
    const uint32_t q[2] = {c.x[k].x, c.x[k].y}, gw[2] = {c.w[k].x, c.w[k].y};
    uint32_t o[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float n0 = __fmul_rn(bf16_bits_to_f32(q[i] & 0xffffu), r), n1 = __fmul_rn(bf16_bits_to_f32(q[i] >> 16), r);
      if (!weight_in_fp32) {
        n0 = round_bf16(n0);
        n1 = round_bf16(n1);
      }
      const float w0 = bf16_bits_to_f32(gw[i] & 0xffffu), w1 = bf16_bits_to_f32(gw[i] >> 16);
      o[i] = f32_to_bf16_bits(__fmul_rn(n0, w0)) | (f32_to_bf16_bits(__fmul_rn(n1, w1)) << 16);
    }
    if (e < H) store_out<CO>(reinterpret_cast<uint64_t*>(orow + e), (uint64_t)o[0] | ((uint64_t)o[1] << 32));
  }
}

// Every thread issues the loads of its chunks of x and gamma at once; a row of up to
// kNormPass elements stays in registers from the sum of squares to the output (longer rows
// reload their later passes).
template <bool CO>
__device__ __forceinline__ void norm_row(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int row,
                                         int H, float eps, int weight_in_fp32, uint16_t* __restrict__ out,
                                         double* part) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint16_t* xr = x + (size_t)row * H;
  uint16_t* orow = out + (size_t)row * H;
  NormChunks first;
  norm_load(first, xr, w, 0, H, tid);
  double s = norm_squares(first);
  for (int base = kNormPass; base < H; base += kNormPass) {
    NormChunks more;
    norm_load(more, xr, w, base, H, tid);
    s += norm_squares(more);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) part[wv] = s;
  __syncthreads();
  s = (part[0] + part[1]) + (part[2] + part[3]);
  const float m = (float)(s / (double)H);
  // sqrtf and / are correctly rounded in HIP device code by default
  // (-fhip-fp32-correctly-rounded-divide-sqrt); __fsqrt_rn is the ~1 ulp hardware sqrt.
  const float r = 1.0f / __builtin_sqrtf(__fadd_rn(m, eps));
  norm_store<CO>(first, orow, 0, H, tid, r, weight_in_fp32);
  for (int base = kNormPass; base < H; base += kNormPass) {
    NormChunks more;
    norm_load(more, xr, w, base, H, tid);
    norm_store<CO>(more, orow, base, H, tid, r, weight_in_fp32);
  }
}

__global__ __launch_bounds__(256) void k_norm(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                              int rows, int H, float eps, int weight_in_fp32,
                                              uint16_t* __restrict__ out) {
  __shared__ double part[4];
  norm_row<false>(x, w, blockIdx.x, H, eps, weight_in_fp32, out, part);
}

// ---------------------------------------------------------------------------------------
// Router logits on fp64 MFMA: partial[split][t][e] = sum over one split of H of
// x[t,h] * W[e,h]. v_mfma_f64_16x16x4f64 multiplies a 16-expert x 4-channel tile of W by
// a 4-channel x 16-token tile of x; products of a bf16 and an fp32 value are exact in
// fp64, so after the splits are added in order (k_select) and rounded once to fp32 the
// logits are the correctly rounded dot products except when an fp64 sum lands within
// ~2^-50 of an fp32 rounding boundary.
//
// A workgroup owns one 16-expert x 16-token tile and one split of H; its four
// wavefronts take consecutive quarters of the split and their tiles are added in
// wavefront order through LDS. Splits number up to four, so a DeepSeek-V3-sized router
// keeps about a thousand wavefronts busy and routing sums at most four partials.
//
// Operand layout of the 16x16x4 f64 MFMA: lane l supplies A[l%16][k] and B[k][l%16] for
// its k = l/16; the result holds row l/16 + 4v, column l%16 in element v (measured on
// gfx950; the fp8 MFMA below puts row 4*(l/16) + v there instead). Over a 16-channel
// step, lane group g feeds channels 4g .. 4g+3 in four MFMAs (one 16-byte W load and one
// 8-byte x load per lane), the same channel order for A and B.
//
// Workgroups past the router tiles (blockIdx.x >= n_router) quantize x instead,
// kQuantPerWave 128-blocks per wavefront.
// ---------------------------------------------------------------------------------------

typedef double f64x4 __attribute__((ext_vector_type(4)));

constexpr int kRouterTile = 16;   // experts per workgroup tile, tokens per accumulator tile
constexpr int kRouterWaves = 4;   // wavefronts per router workgroup (split of its H range)
constexpr int kMaxSplits = 16;    // router splits of H over workgroups (router_splits)
constexpr int kQuantPerWave = 2;  // x blocks quantized per wavefront by the quantizing workgroups
constexpr int kRouterDepth = 8;   // 16-channel steps per wavefront, all in flight at once

// Splits of H over workgroups: the smallest power of two <= 16 that leaves each wavefront
// at most kRouterDepth 16-channel steps (a whole number of them), else the largest that
// divides H evenly (the wavefronts then stream their slices in rounds of kRouterDepth).
inline int router_splits(int H) {
  int best = 1;
  for (int n = 1; n <= kMaxSplits; n *= 2) {
    if (H % (n * kRouterWaves * 16)) break;
    best = n;
    if (H / (n * kRouterWaves * 16) <= kRouterDepth) break;
  }
  return best;
}

inline int router_quant_groups(int T, int H) {
  return (T * (H / kBlock) + 4 * kQuantPerWave - 1) / (4 * kQuantPerWave);
}

// x quantization for the expert GEMMs, kQuantPerWave 128-blocks per wavefront; run by
// extra workgroups of k_select (k_select is latency-bound on a few CUs, the router is not).
__device__ __forceinline__ void quant_x_group(int group, const uint16_t* __restrict__ x, uint8_t* __restrict__ xq,
                                              float* __restrict__ xs, int T, int H, int pow2) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nbh = H / kBlock;
  const int first = (group * 4 + wv) * kQuantPerWave;
#pragma unroll
  for (int q = 0; q < kQuantPerWave; ++q) {
    const int it = first + q;
    if (it < T * nbh) {
      const int t = it / nbh, cb = it % nbh;
      const size_t o = (size_t)t * H + (size_t)cb * kBlock;
      quant_block(x + o, xq + o, xs + (size_t)t * nbh + cb, pow2, lane);
    }
  }
}

// Router partials. Workgroup (expert tile et, split, pass) of kRouterWaves wavefronts
// covers 16 experts, H range [split * H/nsplit, +H/nsplit) and tokens [pass * 16 * NTT,
// +16 * NTT): wavefront w takes the w-th of kRouterWaves equal slices of the range, keeps
// NTT 16x16 fp64 accumulators (one per token tile) and streams its slice in 16-channel
// steps, all of them in flight at once (at most kRouterDepth). The router weights of the
// slice are read once per pass, x once per expert tile. The wavefronts' sums are added in
// wavefront order through LDS and the split's partial is stored in fp64. Passes are
// workgroups of their own, so every workgroup does the same work and the grid spreads
// evenly over the CUs.
template <int NTT, bool CO>
__device__ __forceinline__ void router_tile(const uint16_t* __restrict__ x, const float* __restrict__ w,
                                            double* __restrict__ partial, int T, int H, int E, int n_et, int nsplit,
                                            int unit, f64x4* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int et = unit % n_et, split = (unit / n_et) % nsplit, pass = unit / (n_et * nsplit);
  const int span = H / nsplit / kRouterWaves;  // channels per wavefront, a multiple of 16
  const int k0 = split * (H / nsplit) + wv * span;
  const int g = lane >> 4;
  const int e = et * kRouterTile + (lane & 15);
  const bool e_ok = e < E;
  // Rows past E or T read row 0 and are zeroed after the load: the loads themselves stay
  // unconditional so the compiler keeps all of them in flight.
  const float* wp = w + (size_t)(e_ok ? e : 0) * H + k0 + 4 * g;
  const int steps = span / 16;
  {
    const int tp = pass * 16 * NTT;
    const uint16_t* xp[NTT];
    bool t_ok[NTT];
#pragma unroll
    for (int i = 0; i < NTT; ++i) {
      const int t = tp + 16 * i + (lane & 15);
      t_ok[i] = t < T;
      xp[i] = x + (size_t)(t_ok[i] ? t : 0) * H + k0 + 4 * g;
    }
    f64x4 acc[NTT];
#pragma unroll
    for (int i = 0; i < NTT; ++i) acc[i] = f64x4{0.0, 0.0, 0.0, 0.0};
    for (int c0 = 0; c0 < steps; c0 += kRouterDepth) {
    float4 a[kRouterDepth];
    uint2 b[kRouterDepth][NTT];
#pragma unroll
    for (int u = 0; u < kRouterDepth; ++u) {
      const int k = min(c0 + u, steps - 1) * 16;
      a[u] = *reinterpret_cast<const float4*>(wp + k);
#pragma unroll
      for (int i = 0; i < NTT; ++i) b[u][i] = *reinterpret_cast<const uint2*>(xp[i] + k);
    }
#pragma unroll
    for (int u = 0; u < kRouterDepth; ++u) {
      const bool live = c0 + u < steps;  // steps past the end contribute zero
      const bool ok_a = e_ok && live;
      const float av[4] = {a[u].x, a[u].y, a[u].z, a[u].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const double ac = ok_a ? (double)av[c] : 0.0;
#pragma unroll
        for (int i = 0; i < NTT; ++i) {
          const uint32_t word = c < 2 ? b[u][i].x : b[u][i].y;
          const float xv = bf16_bits_to_f32((c & 1) ? (word >> 16) : (word & 0xffffu));
          const double bc = (t_ok[i] && live) ? (double)xv : 0.0;
          acc[i] = __builtin_amdgcn_mfma_f64_16x16x4f64(ac, bc, acc[i], 0, 0, 0);
        }
      }
    }
    }
    // Slices of the split, added in wavefront order.
    if (wv > 0) {
#pragma unroll
      for (int i = 0; i < NTT; ++i) red[((wv - 1) * NTT + i) * 64 + lane] = acc[i];
    }
    __syncthreads();
    if (wv == 0) {
#pragma unroll
      for (int q = 0; q < kRouterWaves - 1; ++q)
#pragma unroll
        for (int i = 0; i < NTT; ++i) {
          const f64x4 o = red[(q * NTT + i) * 64 + lane];
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[i][v] += o[v];
        }
#pragma unroll
      for (int i = 0; i < NTT; ++i) {
        const int t = tp + 16 * i + (lane & 15);
        if (t < T) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int eo = et * kRouterTile + g + 4 * v;
            if (eo < E) store_out<CO>(&partial[((size_t)split * T + t) * E + eo], acc[i][v]);
          }
        }
      }
    }
  }
}

template <int NTT>
__global__ __launch_bounds__(kRouterWaves * 64) void k_router(const uint16_t* __restrict__ x,
                                                              const float* __restrict__ w,
                                                              double* __restrict__ partial, int T, int H, int E,
                                                              int n_et, int nsplit) {
  __shared__ f64x4 red[(kRouterWaves - 1) * NTT * 64];
  router_tile<NTT, false>(x, w, partial, T, H, E, n_et, nsplit, blockIdx.x, red);
}

// logits[t][e] = fp32(sum of the splits in split order); used by megamoe_router_logits.
__global__ __launch_bounds__(256) void k_logits(const double* __restrict__ partial, int nsplit, int T, int E,
                                                float* __restrict__ logits) {
  const size_t n = (size_t)T * E;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const double* p = partial + i;
  double s = 0.0;
#pragma unroll 4
  for (int q = 0; q < nsplit; ++q) s += p[(size_t)q * n];
  logits[i] = (float)s;
}

// ---------------------------------------------------------------------------------------
// Routing, one wavefront per token; lane l holds experts l, l+64, ... (VPL per lane).
// Selection order is (score descending, expert index ascending), the order a stable
// descending argsort produces (frontier.py:236,240; distributed.py:174).
//
// The K picks come out in selection order from K rounds of a wavefront-wide maximum over
// 64-bit keys (score code, complemented index); each round's winner drops its key.
// ---------------------------------------------------------------------------------------

constexpr int kMaxTopK = 32;
constexpr int kMaxExperts = 1024;
constexpr int kMaxGroups = 64;

// Order-preserving code of a float (larger float, larger code); -0 and +0 coincide.
__device__ __forceinline__ uint32_t order_code(float f) {
  const uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long lanes_below() {
  const int lane = threadIdx.x & 63;
  return lane ? (~0ull >> (64 - lane)) : 0ull;
}

// Cross-lane butterfly steps without LDS: DPP within rows of 16 lanes (quad_perm [1,0,3,2]
// and [2,3,0,1], row_half_mirror, row_mirror), then the permlane16/32 swaps across rows.
// Applied smallest first, step s leaves every lane with the max (or merged top-2) of its
// aligned group of 2^(s+1) lanes. They need every lane of the wavefront active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

// The value of the partner lane at butterfly step `step` (0..5); for steps 4 and 5 the two
// halves of the swap are returned as (mine, other) in lane order.
template <int STEP>
__device__ __forceinline__ void lane_pair(uint32_t v, uint32_t& a, uint32_t& b) {
  if constexpr (STEP == 0) {
    a = v; b = dpp_u32<0xB1>(v);
  } else if constexpr (STEP == 1) {
    a = v; b = dpp_u32<0x4E>(v);
  } else if constexpr (STEP == 2) {
    a = v; b = dpp_u32<0x141>(v);
  } else if constexpr (STEP == 3) {
    a = v; b = dpp_u32<0x140>(v);
  } else if constexpr (STEP == 4) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = p[0]; b = p[1];
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = p[0]; b = p[1];
  }
}

template <int STEP>
__device__ __forceinline__ uint32_t max_step_u32(uint32_t v) {
  uint32_t a, b;
  lane_pair<STEP>(v, a, b);
  return a > b ? a : b;
}

// Largest 32-bit value over the wavefront (every lane gets it).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max_step_u32<0>(v);
  v = max_step_u32<1>(v);
  v = max_step_u32<2>(v);
  v = max_step_u32<3>(v);
  v = max_step_u32<4>(v);
  return max_step_u32<5>(v);
}

// Largest magnitude among the four bf16 values of `four`, as bf16 bits. Non-negative floats
// order as their bits do, so the block maximum below is an integer maximum; NaN counts as 0
// (as fmaxf drops it).
__device__ __forceinline__ uint32_t bf16x4_absmax_bits(uint2 four) {
  const uint32_t w[2] = {four.x, four.y};
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t lo = w[i] & 0x7fffu, hi = (w[i] >> 16) & 0x7fffu;
    m = max(m, lo <= 0x7f80u ? lo : 0u);
    m = max(m, hi <= 0x7f80u ? hi : 0u);
  }
  return m;
}

// Largest 32-bit value over each half of the wavefront (lanes 0..31 and 32..63 separately).
__device__ __forceinline__ uint32_t half_wave_max_u32(uint32_t v) {
  v = max_step_u32<0>(v);
  v = max_step_u32<1>(v);
  v = max_step_u32<2>(v);
  v = max_step_u32<3>(v);
  return max_step_u32<4>(v);
}

// One row of x (nbh blocks) in E4M3 per 128 by the workgroup's four wavefronts, wavefront wv
// taking blocks wv, wv + 4, ... in batches of up to 8, two blocks at a time: each half of the
// wavefront holds one block, four values per lane, so every instruction works on two blocks.
// A batch's block maxima are reduced together (independent DPP and permlane chains over each
// half, no LDS), then scale = max(amax, 1e-4)/448 and code = RNE(clamp(v / scale, +-448)) per
// value (e4m3x4), as quant_block; each lane writes its four codes as one 4-byte device-
// coherent store (the single-launch kernel's expert units read them from other workgroups),
// a whole line per block. The scales gather in LDS (`lds`, nbh floats) and leave as one
// contiguous store per 64 blocks. Blocks past the row's end are loaded from its last block
// and not stored. Called by the whole workgroup.
__device__ __forceinline__ void quant_row(const uint16_t* x, uint8_t* xq, float* xs, int nbh, int pow2, int lane,
                                          int wv, float* lds) {
  constexpr int kPairs = 4;  // blocks per wavefront and batch: 2 * kPairs
  const int l = lane & 31, half = lane >> 5;
  for (int b0 = wv; b0 < nbh; b0 += 4 * 2 * kPairs) {
    uint2 four[kPairs];
#pragma unroll
    for (int j = 0; j < kPairs; ++j) {
      const int b = min(b0 + 4 * (2 * j + half), nbh - 1);
      four[j] = *reinterpret_cast<const uint2*>(x + (size_t)b * kBlock + 4 * l);
    }
    uint32_t m[kPairs];
#pragma unroll
    for (int j = 0; j < kPairs; ++j) m[j] = half_wave_max_u32(bf16x4_absmax_bits(four[j]));
#pragma unroll
    for (int j = 0; j < kPairs; ++j) {
      const int b = b0 + 4 * (2 * j + half);
      const float s = act_scale(__uint_as_float(m[j] << 16), pow2);
      const uint32_t q = e4m3x4(clamp448(bf16_bits_to_f32(four[j].x & 0xffffu) / s),
                                clamp448(bf16_bits_to_f32(four[j].x >> 16) / s),
                                clamp448(bf16_bits_to_f32(four[j].y & 0xffffu) / s),
                                clamp448(bf16_bits_to_f32(four[j].y >> 16) / s));
      if (b < nbh) {
        store_coherent(reinterpret_cast<uint32_t*>(xq + (size_t)b * kBlock + 4 * l), q);
        if (l == 0) lds[b] = s;
      }
    }
  }
  __syncthreads();
  if (wv == 0)
    for (int b = lane; b < nbh; b += 64) store_coherent(xs + b, lds[b]);
  __syncthreads();
}

// Merges the (largest, second largest) pairs of lanes at butterfly step STEP.
template <int STEP>
__device__ __forceinline__ void top2_step(float& b1, float& b2) {
  uint32_t a1, o1, a2, o2;
  lane_pair<STEP>(__float_as_uint(b1), a1, o1);
  lane_pair<STEP>(__float_as_uint(b2), a2, o2);
  const float x1 = __uint_as_float(a1), y1 = __uint_as_float(o1);
  const float x2 = __uint_as_float(a2), y2 = __uint_as_float(o2);
  b2 = fmaxf(fminf(x1, y1), fmaxf(x2, y2));
  b1 = fmaxf(x1, y1);
}

// Top-2 merge over aligned lane segments of `len` lanes (a power of two, 1..64).
__device__ __forceinline__ void top2_segment(float& b1, float& b2, int len) {
  if (len >= 2) top2_step<0>(b1, b2);
  if (len >= 4) top2_step<1>(b1, b2);
  if (len >= 8) top2_step<2>(b1, b2);
  if (len >= 16) top2_step<3>(b1, b2);
  if (len >= 32) top2_step<4>(b1, b2);
  if (len >= 64) top2_step<5>(b1, b2);
}

// Selection key of an expert: the order code of its score above, the complement of its
// index below, so a larger key is a larger score or, on equal scores, a lower index.
__device__ __forceinline__ unsigned long long select_key(float score, int e) {
  return ((unsigned long long)order_code(score) << 32) | (0xffffffffu - (uint32_t)e);
}

// Tokens per workgroup: one. Its four wavefronts load and sum the split partials of the
// token's logits (one entry, all splits, per thread for up to 256 experts), then
// wavefront 0 routes the token.
constexpr int kSelectTokens = 1;


// LDS of one token's routing.
struct SelectLds {
  float logit[kSelectTokens][kMaxExperts];
  float choice[kSelectTokens][kMaxExperts];
  unsigned long long key[kSelectTokens][kMaxExperts];  // VPL >= 8: keys of lane l at [64j + l]
  float bias[kMaxExperts];                             // the router bias (sigmoid gate)
  float gscore[kSelectTokens][kMaxGroups];
  int pick_id[kSelectTokens][kMaxTopK];
  float pick_val[kSelectTokens][kMaxTopK];
};

// The gate's probability of a logit (sigmoid), or the logit itself (softmax, whose weights
// come from the picked logits).
__device__ __forceinline__ float gate_prob(float logit, int gate) {
  return gate == MEGAMOE_GATE_SIGMOID ? 1.0f / (1.0f + expf(-logit)) : logit;
}

// Wavefront `wv` routes token t from the logits in LDS (one wavefront per token, no barrier).
// The logits and the choices stay in LDS and are read again where needed (a probability is
// recomputed from its logit by the same expression, so it has the same bits). The selection
// keys of the lane's VPL experts stay in registers up to VPL 4; from VPL 8 (over 256 experts)
// they go to LDS and the lane keeps only its largest: with 8 or 16 keys of 64 bits per lane
// held in registers, the single-launch kernel, whose register budget the expert units set,
// spilled them to scratch.
template <int VPL, bool CO>
__device__ __forceinline__ void route_token(SelectLds& L, int lane, int wv, int t, bool token_ok, int E, int K,
                                            int G, int TG, int gate,
                                            int renorm, float scaling, int64_t* __restrict__ ids_out,
                                            float* __restrict__ w_out) {
  const float* logit_lds = L.logit[wv];
  float* choice_lds = L.choice[wv];
  auto& gscore = L.gscore;
  int* pick_id = L.pick_id[wv];
  float* pick_val = L.pick_val[wv];
  // Selection keys of the lane's experts (0: not selectable), built from the choices
  // (sigmoid + bias, or the logit).
  constexpr bool kKeysInLds = VPL >= 8;
  constexpr int VR = kKeysInLds ? 1 : VPL;  // keys held in registers
  unsigned long long* key_lds = L.key[wv];
  unsigned long long key[VR];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    const bool valid = token_ok && e < E;
    const float logit = valid ? logit_lds[e] : -INFINITY;
    const float choice = gate == MEGAMOE_GATE_SIGMOID ? gate_prob(logit, gate) + L.bias[min(e, E - 1)] : logit;
    if (G > 1 && valid) choice_lds[e] = choice;
    const unsigned long long k = valid ? select_key(choice, e) : 0ull;
    if constexpr (kKeysInLds)
      key_lds[e] = k;
    else
      key[j] = k;
  }
  if (G > 1) {
    // Group score: the sum of the two largest choices of the group (frontier.py:234). A
    // group is scanned by lpg lanes (the largest power of two <= 64 / G), whose top-2
    // pairs are then merged with shuffles inside the lane segment. Each wavefront works
    // on its own LDS rows from here on.
    const int gs = E / G;
    int lpg = 1;
    while (lpg * 2 * G <= 64) lpg *= 2;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the choices are in LDS
    __builtin_amdgcn_wave_barrier();
    const int grp = lane / lpg, sub = lane % lpg;
    float b1 = -INFINITY, b2 = -INFINITY;
    if (grp < G && token_ok) {
      for (int i = sub; i < gs; i += lpg) {
        const float v = choice_lds[grp * gs + i];
        b2 = fmaxf(b2, fminf(b1, v));
        b1 = fmaxf(b1, v);
      }
    }
    top2_segment(b1, b2, lpg);
    if (grp < G && sub == 0 && token_ok) gscore[wv][grp] = gs >= 2 ? b1 + b2 : b1;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    // Keep the TG best groups, ties to the lower group index (frontier.py:235).
    bool keep = false;
    if (lane < G && token_ok) {
      const float mine = gscore[wv][lane];
      int rank = 0;
      for (int h = 0; h < G; ++h) {
        const float o = gscore[wv][h];
        rank += (o > mine) || (o == mine && h < lane);
      }
      keep = rank < TG;
    }
    const unsigned long long kept = __ballot(keep);
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (!((kept >> ((lane + 64 * j) / gs)) & 1ull)) {
        if constexpr (kKeysInLds)
          key_lds[lane + 64 * j] = 0ull;
        else
          key[j] = 0ull;
      }
  }
  // With the keys in LDS, the lane's largest one.
  auto lane_best = [&]() {
    unsigned long long b = 0ull;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const unsigned long long k = key_lds[lane + 64 * j];
      b = k > b ? k : b;
    }
    return b;
  };
  if constexpr (kKeysInLds) key[0] = lane_best();
  // K rounds: the wavefront's largest remaining key is the next pick (selection order,
  // frontier.py:236; distributed.py:174); its owner records it and drops it. The maximum
  // is taken over the score codes (the keys' upper halves) first; only when several lanes
  // hold that code does a second maximum over their index parts pick the lowest index.
  for (int r = 0; r < K && token_ok; ++r) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int j = 0; j < VR; ++j) best = key[j] > best ? key[j] : best;
    const uint32_t hi = (uint32_t)(best >> 32), lo = (uint32_t)best;
    const uint32_t top = wave_max_u32(hi);
    unsigned long long owner = __ballot(hi == top);
    if (__popcll(owner) > 1) {
      const uint32_t top_lo = wave_max_u32(hi == top ? lo : 0u);
      owner = __ballot(hi == top && lo == top_lo);
    }
    if (lane == __ffsll((long long)owner) - 1) {
      // The key's index part is the complement of its expert.
      pick_id[r] = (int)(0xffffffffu - lo);
      if constexpr (kKeysInLds) {
        key_lds[0xffffffffu - lo] = 0ull;
        key[0] = lane_best();
      } else {
#pragma unroll
        for (int j = 0; j < VR; ++j)
          if (key[j] == best) key[j] = 0ull;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  if (!token_ok) return;
  int my_id = 0;
  float my_val = 0.0f;
  if (lane < K) {
    my_id = pick_id[lane];
    my_val = gate_prob(logit_lds[my_id], gate);
    pick_val[lane] = my_val;
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  // Weights; sums run in slot order.
  float w = 0.0f;
  if (gate == MEGAMOE_GATE_SIGMOID) {
    if (renorm) {
      float s = 0.0f;
      for (int r = 0; r < K; ++r) s += pick_val[r];
      w = my_val / (s + 1e-20f) * scaling;
    } else {
      w = my_val * scaling;
    }
  } else if (renorm) {
    const float m = pick_val[0];  // the first pick holds the largest logit
    float s = 0.0f;
    for (int r = 0; r < K; ++r) s += expf(pick_val[r] - m);
    w = expf(my_val - m) / s * scaling;
  } else {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (lane + 64 * j < E) m = fmaxf(m, logit_lds[lane + 64 * j]);
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if (lane + 64 * j < E) s += expf(logit_lds[lane + 64 * j] - m);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    w = expf(my_val - m) / s * scaling;
  }
  if (lane < K) {
    store_out<CO>(&ids_out[(size_t)t * K + lane], (int64_t)my_id);
    store_out<CO>(&w_out[(size_t)t * K + lane], w);
  }
}

// Routing of token `token` (kSelectTokens = 1) by the workgroup's 256 threads: all load and
// sum the split partials, wavefront 0 routes. ids and weights go out as device-coherent
// stores (a later workgroup of the single-launch kernel reads them).
template <int VPL, bool CO>
__device__ __forceinline__ void select_token(const double* __restrict__ partial, int nsplit,
                                             const float* __restrict__ logits_in, const float* __restrict__ bias,
                                             int T, int E, int K, int G, int TG, int gate, int renorm, float scaling,
                                             int64_t* __restrict__ ids_out, float* __restrict__ w_out, int token,
                                             SelectLds& L) {
  auto& lds_logit = L.logit;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int t0 = token * kSelectTokens, t = t0 + wv;
  const bool token_ok = t < T;

  // The bias into LDS (thread i: entries i, i+256, ...), loaded beside the logits' loads.
  constexpr int NB = (64 * VPL + 255) / 256;
  float bias_e[NB];
#pragma unroll
  for (int r = 0; r < NB; ++r) bias_e[r] = bias ? bias[min((int)threadIdx.x + 256 * r, E - 1)] : 0.0f;

  // Logits of the workgroup's tokens into LDS: thread i sums the splits (in split order)
  // of entries i, i+256, ... (kSelectTokens * E <= 64 * VPL of them, up to kMaxSplits
  // splits each), every load issued before the first add.
  const int n_here = min(kSelectTokens, T - t0) * E;
  if (logits_in) {
#pragma unroll
    for (int r = 0; r < (kSelectTokens * 64 * VPL + 255) / 256; ++r) {
      const int i = threadIdx.x + 256 * r;
      const float v = logits_in[(size_t)t0 * E + min(i, n_here - 1)];
      if (i < n_here) lds_logit[i / E][i % E] = v;
    }
  } else {
    const size_t stride = (size_t)T * E;
    const double* p = partial + (size_t)t0 * E;
    constexpr int NE = (kSelectTokens * 64 * VPL + 255) / 256;  // entries per thread
    constexpr int R = NE < 2 ? NE : 2;                           // entries per round of loads
#pragma unroll
    for (int r0 = 0; r0 < NE; r0 += R) {
      double part[R][kMaxSplits];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + 256 * (r0 + r);
#pragma unroll
        for (int q = 0; q < kMaxSplits; ++q)  // clamped, unconditional loads
          part[r][q] = p[(size_t)min(q, nsplit - 1) * stride + min(i, n_here - 1)];
      }
      // Every load of the round is issued before the first add: short of registers in the
      // single-launch kernel, the compiler otherwise sinks each load to its add and waits
      // for each in turn (one round trip per split instead of one per round).
      static_assert(kMaxSplits == 16, "one asm operand per split");
#pragma unroll
      for (int r = 0; r < R; ++r)
        asm volatile(""
                     : "+v"(part[r][0]), "+v"(part[r][1]), "+v"(part[r][2]), "+v"(part[r][3]), "+v"(part[r][4]),
                       "+v"(part[r][5]), "+v"(part[r][6]), "+v"(part[r][7]), "+v"(part[r][8]), "+v"(part[r][9]),
                       "+v"(part[r][10]), "+v"(part[r][11]), "+v"(part[r][12]), "+v"(part[r][13]),
                       "+v"(part[r][14]), "+v"(part[r][15])
                     :
                     : "memory");
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < kMaxSplits; ++q)
          if (q >= nsplit) part[r][q] = 0.0;  // entries past the end are dropped below
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + 256 * (r0 + r);
        double s = 0.0;
#pragma unroll
        for (int q = 0; q < kMaxSplits; ++q)
          if (q < nsplit) s += part[r][q];
        if (i < n_here) lds_logit[i / E][i % E] = (float)s;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NB; ++r)
    if ((int)threadIdx.x + 256 * r < E) L.bias[threadIdx.x + 256 * r] = bias_e[r];
  __syncthreads();
  // The lane behind an empty asm: the experts' indices derived from it are computed here, not
  // hoisted out of the single-launch kernel's persistent loop and held (or spilled) across it.
  if (wv < kSelectTokens) route_token<VPL, CO>(L, opaque_lane(), wv, t, token_ok, E, K, G, TG, gate, renorm, scaling,
                                           ids_out, w_out);
}

template <int VPL>
__global__ __launch_bounds__(256) void k_select(const double* __restrict__ partial, int nsplit,
                                                const float* __restrict__ logits_in, const float* __restrict__ bias,
                                                int T, int E, int K, int G, int TG, int gate, int renorm,
                                                float scaling, int64_t* __restrict__ ids_out,
                                                float* __restrict__ w_out, int n_sel, const uint16_t* __restrict__ x,
                                                uint8_t* __restrict__ xq, float* __restrict__ xs, int H, int pow2) {
  if ((int)blockIdx.x >= n_sel) {
    quant_x_group((int)blockIdx.x - n_sel, x, xq, xs, T, H, pow2);
    return;
  }
  __shared__ SelectLds lds;
  select_token<VPL, false>(partial, nsplit, logits_in, bias, T, E, K, G, TG, gate, renorm, scaling, ids_out, w_out,
                           blockIdx.x, lds);
}


// ---------------------------------------------------------------------------------------
// Histogram, scan, stable permutation and the expert work lists, in one workgroup.
//
// Rows of expert e are its (token, slot) entries in increasing token order
// (megamoe.py:138-149); each token picks an expert at most once, so an entry's rank is
// the number of earlier tokens that picked the same expert: a popcount over a
// per-expert token bitmap.
//
// Work lists: each expert's rows split into chunks of at most 64 (the most one pass of
// the expert kernels multiplies); chunks are listed heaviest class first (33-64 rows,
// then 17-32, then 1-16) so the dynamic work queues of the expert kernels start the
// long units first. The shared expert (all T tokens) is listed like a routed expert;
// in the gate/up list it appears once per I-sized slice of its S*I rows.
// ---------------------------------------------------------------------------------------

// The 64-bit value of the lane N below in the same row of 16 lanes (DPP row_shr:N), 0 for the
// lanes below N of each row. Needs every lane of the wavefront active.
template <int N>
__device__ __forceinline__ unsigned long long row_shr_u64(unsigned long long x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)x, 0x110 + N, 0xF, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(x >> 32), 0x110 + N, 0xF, 0xF, true);
  return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long x, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
  return ((unsigned long long)hi << 32) | lo;
}

// Exclusive scan over the workgroup (at most 16 wavefronts, all lanes active) of a value
// packing four counters: bits 0-20 rows, 21-35 chunks of 33-64 rows, 36-46 chunks of 17-32,
// 47-57 chunks of 1-16. Within a wavefront: DPP shifts inside each row of 16 lanes, then the
// rows' totals read from lanes 15, 31 and 47 (no LDS round trips: the LDS shuffles took ~2
// us on the single launch's critical path); across wavefronts: every thread adds the totals
// of the wavefronts below it from LDS. `tmp` (16 entries) is written before the barrier and
// read after it.
// Sum over the wavefront of a small non-negative v, from two ballots per bit of the largest
// v: a few instructions. An atomic add of a lane-varying value to one address would have
// the compiler's atomic optimizer fold the lanes in a scalar loop, one active lane per trip
// (the permute's hit count spent ~1.8 us there with 64 lanes).
__device__ __forceinline__ int wave_sum_small(int v) {
  int sum = 0;
  for (int b = 0; __ballot(v >> b) != 0ull; ++b) sum += __popcll(__ballot((v >> b) & 1)) << b;
  return sum;
}

__device__ unsigned long long block_exclusive_scan(unsigned long long v, unsigned long long* tmp,
                                                   unsigned long long* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  unsigned long long x = v;
  x += row_shr_u64<1>(x);
  x += row_shr_u64<2>(x);
  x += row_shr_u64<4>(x);
  x += row_shr_u64<8>(x);
  const unsigned long long r0 = readlane_u64(x, 15), r1 = readlane_u64(x, 31), r2 = readlane_u64(x, 47);
  const int row = lane >> 4;
  x += (row >= 1 ? r0 : 0ull) + (row >= 2 ? r1 : 0ull) + (row >= 3 ? r2 : 0ull);
  if (lane == 63) tmp[wid] = x;
  __syncthreads();
  unsigned long long base = 0ull, all = 0ull;
  for (int q = 0; q < nw; ++q) {
    const unsigned long long t = tmp[q];
    base += q < wid ? t : 0ull;
    all += t;
  }
  *total = all;
  return base + x - v;
}

// Ints of the meta block. The error flag has a 128-byte line of its own, apart from the
// queue counter that every workgroup updates.
constexpr int kMetaHit = 0, kMetaUnitsGU = 1, kMetaUnitsDN = 2, kMetaQueueGU = 3, kMetaQueueDN = 4,
              kMetaWide = 5, kMetaError = 32, kMetaInts = 64;
constexpr int kChunkRows = 64;     // rows per chunk of the fp8 form (column tiles of up to 4)
constexpr int kChunkRowsA16 = 32;  // of its W8A16 form (bf16 activations: column tiles of up to 2)
constexpr int kChunkRowsMx = 128;  // of the MXFP4 form: wide units over 33-128 rows, narrow up to 32

struct PermuteOut {
  int* counts;   // [E]
  int* offsets;  // [E+1]
  int* meta;     // kMeta*
  int* perm;     // [T*K] grouped row -> token*K + slot
  int* inv;      // [T*K] token*K + slot -> grouped row
  int4* gu;      // gate/up chunks {expert (E = shared), first grouped row, rows, first 128-block}
  int4* dn;      // down chunks
  int* dn_of_gu; // gate/up chunk -> down chunk of the same rows
  int* ready;    // [down chunks, stride ready_stride] zeroed here, counted by the expert kernel
  int* pairs;    // [gate/up chunks * nbI] zeroed here (NULL: none), counted by the expert kernel
  int ready_stride = 1;  // ints between two chunks' counters
  int* xcd = nullptr;    // the batch form's per-XCD queues (kXcdInts; NULL: none)
  int ready_min = 0;     // readiness counters zeroed at least (the dense schedule's down chunks)
};

// The batch form's work split over the XCDs (the lists in expert order, `wide` 2): XCD x
// takes the chunks [bound x, bound x+1) first (8 ranges of about equal chunk counts, cut at
// expert boundaries), so the units of an expert, which read the same weights, run on one
// XCD and meet in its L2. One queue counter per XCD and phase (gate/up, down), each on a
// 128-byte line of its own, then the 9 bounds.
constexpr int kXcds = 8, kXcdStride = 32, kXcdBound = 2 * kXcds * kXcdStride, kXcdInts = kXcdBound + kXcds + 1;

// The XCD this workgroup runs on (hardware register XCC_ID), as a queue index.
__device__ __forceinline__ int my_xcd() {
  return __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) % kXcds;
}

// Readiness counters of the fp8 form (one per down chunk): the down units poll them while
// the gate/up units run, hundreds at a time early in the down phase. Each counter gets a
// line of its own, 4352 bytes from the next (different cache and memory channels; the
// same reasoning as the signals of the single-launch kernel), when there are at most
// kReadySpreadChunks chunks, else one 128-byte line: Qwen3-30B-A3B's layer 142.9 -> 138.2 us,
// Mixtral 286.2 -> 282.4, Kimi-K2 2057 -> 2048 (single launch; 3 us on the stream-ordered
// form), DeepSeek-V3 unchanged.
constexpr int kReadySpread = (4096 + 256) / 4, kReadyLine = 32, kReadySpreadChunks = 2048;

__device__ __forceinline__ int chunk_class(int rows) { return rows > 32 ? 0 : (rows > 16 ? 1 : 2); }

// Ids from the caller (the MXFP4 form takes its routing as an input) may be out of range or
// repeat an expert within a token; either sets the error flag, and the permutation, the
// work lists and every later kernel's work are skipped (the combine writes NaN). Expert
// e here is id e + base (a rank's local experts under expert parallelism).
//
// With `wide` 1 (the MXFP4 form, no shared expert), a chunk of more than 32 rows is worked by
// wide units, 4 per 128-channel block of gate/up and 2 per 128-row block of down (times
// the K parts); those chunks lead the lists, and meta[kMetaWide] counts them. With `wide` 2
// (the batch form, no shared expert) the lists are in expert order instead: each expert's
// chunks in a row, each record's .w holding its index in that group and the group's size
// (bits 16 up), so the batch kernel can hand out a weight block's units for every chunk of
// the expert one after another.

// Part `part` of `parts` of the 128-byte lines of three matrices of `bytes` each (a multiple
// of 128), touched by a workgroup of NT threads: one 4-byte load per line, the values folded
// and kept by an empty asm, so the lines land in the caches for a later reader.
template <int NT>
__device__ __forceinline__ void touch_lines(const uint8_t* m0, const uint8_t* m1, const uint8_t* m2, size_t bytes,
                                            int part, int parts) {
  const size_t per_mat = bytes / 128, lines = 3 * per_mat, per = (lines + parts - 1) / parts;
  const size_t l0 = (size_t)part * per, l1 = l0 + per < lines ? l0 + per : lines;
  int acc = 0;
#pragma unroll 4
  for (size_t l = l0 + threadIdx.x; l < l1; l += NT) {
    const size_t m = l / per_mat, o = (l % per_mat) * 128;
    const uint8_t* base = m == 0 ? m0 : (m == 1 ? m1 : m2);
    acc ^= *reinterpret_cast<const int*>(base + o);
  }
  asm volatile("" ::"v"(acc));
}

// The permute by one workgroup of any size (a multiple of 64, at least 256): thread i owns
// the contiguous experts [i*ept, i*ept + ept) (ept = ceil(E / threads)), so the scan over
// threads runs in expert order. Every output goes out as a device-coherent store: the
// single-launch kernel's expert units read them from other workgroups.
//
// An entry's row within its expert is its rank among the entries of that expert in (token,
// slot) order, i.e. the number of earlier entries of the flat [T*K] id array with the same
// expert (a token picks an expert at most once). Two ways to count it:
//   tile_waves == 0: a per-expert token bitmap in LDS and a popcount (32 + E + E*ceil(T/32)
//     ints of `smem`);
//   tile_waves > 0: without the bitmap, for any T: the entries in tiles of 64*tile_waves,
//     each wavefront of a tile ranking its 64 entries with a ballot per distinct expert,
//     the tile's waves added per expert in wave order through LDS, and a running count per
//     expert across tiles (32 + E + E*tile_waves ints). Repeated ids within a token are
//     found by comparing each entry with its token's other slots.
// flags[0..1] are two more LDS ints.
template <bool CO>
__device__ __forceinline__ void permute_block(const int64_t* __restrict__ ids, int64_t base, int T, int K, int E,
                                              int S, int nbI, int nbH, int ks, int chunk, int wide,
                                              const PermuteOut& out, int* smem, int* flags, int tile_waves = 0,
                                              bool prefix = false) {
  int* bad = flags;
  int* hits = flags + 1;
  unsigned long long* tmp = (unsigned long long*)smem;  // 16
  int* cnt = smem + 32;                                  // E
  unsigned* bm = (unsigned*)(cnt + E);                   // E * words (bitmap), or tile_waves * E (tiles)
  const int words = (T + 31) / 32;
  const int tid = threadIdx.x, nt = blockDim.x, n = T * K;
  for (int i = tid; i < E; i += nt) cnt[i] = 0;
  if (!tile_waves)
    for (int i = tid; i < E * words; i += nt) bm[i] = 0u;
  if (tid == 0) {
    *bad = 0;
    *hits = 0;
  }
  __syncthreads();
  // Each thread's first kKeep entries stay in registers for the rank loop below (one load of
  // the ids on the critical path instead of two).
  constexpr int kKeep = 4;
  int keep[kKeep];
#pragma unroll
  for (int j = 0; j < kKeep; ++j) keep[j] = 0;
  for (int i = tid, j = 0; i < n; i += nt, ++j) {
    const int64_t e64 = ids[i] - base;
    const int t = i / K;
#pragma unroll
    for (int q = 0; q < kKeep; ++q)
      if (q == j) keep[q] = (int)e64;
    if (e64 < 0 || e64 >= E) {
      *bad = 1;
      continue;
    }
    const int e = (int)e64;
    atomicAdd(&cnt[e], 1);
    if (!tile_waves) {
      if (atomicOr(&bm[e * words + (t >> 5)], 1u << (t & 31)) & (1u << (t & 31))) *bad = 1;
    } else {
      for (int k2 = 0; k2 < K; ++k2)
        if (t * K + k2 != i && ids[t * K + k2] == ids[i]) *bad = 1;
    }
  }
  __syncthreads();
  if (*bad) {
    if (tid == 0) {
      store_out<CO>(&out.meta[kMetaUnitsGU], 0);
      store_out<CO>(&out.meta[kMetaUnitsDN], 0);
      store_out<CO>(&out.meta[kMetaQueueGU], 0);
      store_out<CO>(&out.meta[kMetaError], 1);
    }
    return;
  }
  const int ept = (E + nt - 1) / nt, e_lo = min(E, tid * ept), e_hi = min(E, e_lo + ept);
  auto classes = [chunk](int c, int& a4, int& a2, int& a1) {
    const int full = c / chunk, rem = c % chunk;
    a4 = full + (rem > 32 ? 1 : 0);
    a2 = (rem > 16 && rem <= 32) ? 1 : 0;
    a1 = (rem > 0 && rem <= 16) ? 1 : 0;
  };
  unsigned long long mine = 0ull;
  int my_hits = 0;
  for (int e = e_lo; e < e_hi; ++e) {
    const int c = cnt[e];
    int a4, a2, a1;
    classes(c, a4, a2, a1);
    mine += (unsigned long long)c | ((unsigned long long)a4 << 21) | ((unsigned long long)a2 << 36) |
            ((unsigned long long)a1 << 47);
    my_hits += c > 0;
  }
  {
    const int wave_hits = wave_sum_small(my_hits);
    if ((tid & 63) == 0 && wave_hits) atomicAdd(hits, wave_hits);
  }
  unsigned long long tot = 0;
  const unsigned long long packed = block_exclusive_scan(mine, tmp, &tot);
  int off = (int)(packed & 0x1fffffu), p4 = (int)((packed >> 21) & 0x7fffu), p2 = (int)((packed >> 36) & 0x7ffu),
      p1 = (int)((packed >> 47) & 0x7ffu);
  const int total = (int)(tot & 0x1fffffu), t4 = (int)((tot >> 21) & 0x7fffu), t2 = (int)((tot >> 36) & 0x7ffu),
            t1 = (int)((tot >> 47) & 0x7ffu);
  // Shared expert chunks of T rows.
  const int sf = T / chunk, sr = T % chunk;
  const int s4 = S ? sf + (sr > 32 ? 1 : 0) : 0, s2 = S ? ((sr > 16 && sr <= 32) ? 1 : 0) : 0,
            s1 = S ? ((sr > 0 && sr <= 16) ? 1 : 0) : 0;
  // gate/up list: [S*s4 | t4 | S*s2 | t2 | S*s1 | t1]; down list: [s4 | t4 | s2 | t2 | s1 | t1]
  const int gbase[3] = {0, S * s4 + t4, S * s4 + t4 + S * s2 + t2};
  const int dbase[3] = {0, s4 + t4, s4 + t4 + s2 + t2};
  const int gshared[3] = {S * s4, S * s2, S * s1};
  const int dshared[3] = {s4, s2, s1};
  for (int e = e_lo; e < e_hi; ++e) {
    const int c = cnt[e];
    int a4, a2, a1;
    classes(c, a4, a2, a1);
    const int full = c / chunk, rem = c % chunk;
    store_out<CO>(&out.counts[e], c);
    store_out<CO>(&out.offsets[e], off);
    if (wide == 2) {
      // Lists in expert order: expert e's chunks at the prefix of every class's chunks over
      // the experts before it, .w = the chunk's index in its expert's group | group size << 16.
      const int nch = a4 + a2 + a1, first = p4 + p2 + p1;
      for (int i = 0; i < nch; ++i) {
        const int4 ch = make_int4(e, off + chunk * i, min(chunk, c - chunk * i), i | (nch << 16));
        store_out<CO>(&out.gu[first + i], ch);
        store_out<CO>(&out.dn[first + i], ch);
        store_out<CO>(&out.dn_of_gu[first + i], first + i);
      }
      // The XCD bounds inside this expert's group: bound x is the first group start at or
      // past x * total / 8 (rounded up), so this group owns the targets in [first, first + nch).
      if (out.xcd) {
        const int total_ch = t4 + t2 + t1;
        for (int x = 1; x < kXcds; ++x) {
          const int target = (x * total_ch + kXcds - 1) / kXcds;
          if (first <= target && target < first + nch)
            store_out<CO>(&out.xcd[kXcdBound + x], target == first ? first : first + nch);
        }
      }
    } else {
      for (int i = 0; i < a4; ++i) {
        const int4 ch = make_int4(e, off + chunk * i, min(chunk, c - chunk * i), 0);
        store_out<CO>(&out.gu[gbase[0] + gshared[0] + p4 + i], ch);
        store_out<CO>(&out.dn[dbase[0] + dshared[0] + p4 + i], ch);
        store_out<CO>(&out.dn_of_gu[gbase[0] + gshared[0] + p4 + i], dbase[0] + dshared[0] + p4 + i);
      }
      if (a2) {
        const int4 ch = make_int4(e, off + chunk * full, rem, 0);
        store_out<CO>(&out.gu[gbase[1] + gshared[1] + p2], ch);
        store_out<CO>(&out.dn[dbase[1] + dshared[1] + p2], ch);
        store_out<CO>(&out.dn_of_gu[gbase[1] + gshared[1] + p2], dbase[1] + dshared[1] + p2);
      }
      if (a1) {
        const int4 ch = make_int4(e, off + chunk * full, rem, 0);
        store_out<CO>(&out.gu[gbase[2] + gshared[2] + p1], ch);
        store_out<CO>(&out.dn[dbase[2] + dshared[2] + p1], ch);
        store_out<CO>(&out.dn_of_gu[gbase[2] + gshared[2] + p1], dbase[2] + dshared[2] + p1);
      }
    }
    cnt[e] = off;  // the expert's first row, for the ranks below (only this thread reads cnt[e] above)
    off += c;
    p4 += a4;
    p2 += a2;
    p1 += a1;
  }
  if (tid == 0) {
    if (S > 0) {
      for (int i = 0; i * chunk < T; ++i) {
        const int rows = min(chunk, T - chunk * i);
        const int cls = rows == chunk ? 0 : chunk_class(rows);  // a full chunk is counted in s4 (sf)
        const int idx = cls == 0 ? i : 0;        // index within the shared part of the class
        const int per_copy = cls == 0 ? s4 : 1;  // shared chunks of this class per copy
        for (int s = 0; s < S; ++s) {
          store_out<CO>(&out.gu[gbase[cls] + s * per_copy + idx], make_int4(E, chunk * i, rows, s * nbI));
          store_out<CO>(&out.dn_of_gu[gbase[cls] + s * per_copy + idx], dbase[cls] + idx);
        }
        store_out<CO>(&out.dn[dbase[cls] + idx], make_int4(E, chunk * i, rows, 0));
      }
    }
    store_out<CO>(&out.offsets[E], total);
    store_out<CO>(&out.meta[kMetaHit], *hits);
    const int wf = wide == 1 ? 4 : 1, wfd = wide == 1 ? 2 : 1;  // units per block of a chunk of over 32 rows
    store_out<CO>(&out.meta[kMetaUnitsGU], (S * (s4 + s2 + s1) + wf * t4 + t2 + t1) * nbI);
    store_out<CO>(&out.meta[kMetaUnitsDN], (s4 + s2 + s1 + wfd * t4 + t2 + t1) * nbH * ks);
    store_out<CO>(&out.meta[kMetaWide], wide == 1 ? t4 : 0);
    if (out.xcd) {
      const int total_ch = t4 + t2 + t1;
      for (int q = 0; q < 2 * kXcds; ++q) store_out<CO>(&out.xcd[q * kXcdStride], 0);
      store_out<CO>(&out.xcd[kXcdBound], 0);
      for (int x = 1; x <= kXcds; ++x)  // targets no group holds: past the last chunk
        if ((x * total_ch + kXcds - 1) / kXcds >= total_ch) store_out<CO>(&out.xcd[kXcdBound + x], total_ch);
    }
    store_out<CO>(&out.meta[kMetaQueueGU], 0);
    store_out<CO>(&out.meta[kMetaQueueDN], 0);
    store_out<CO>(&out.meta[kMetaError], 0);
  }
  const int dtot = max(s4 + s2 + s1 + t4 + t2 + t1, out.ready_min);
  for (int i = tid; i < dtot; i += nt) store_out<CO>(&out.ready[(size_t)i * out.ready_stride], 0);
  if (out.pairs)
    for (int i = tid; i < (S * (s4 + s2 + s1) + t4 + t2 + t1) * nbI; i += nt) store_out<CO>(&out.pairs[i], 0);
  __syncthreads();
  if (!tile_waves) {
    // With `prefix` (long rows: the stream-ordered permute of many rows), each expert's row
    // first gets the exclusive popcount prefix of its words (E * words more ints after the
    // bitmap; one wavefront a row, a scan over its lanes), so a rank is one prefix and one
    // masked popcount instead of a walk over up to T/32 words.
    const unsigned* pre = bm + E * words;
    if (!CO && prefix) {
      unsigned* pw = bm + E * words;
      const int lane = tid & 63, nw = nt >> 6;
      for (int r = tid >> 6; r < E; r += nw) {
        int carry = 0;
        for (int q0 = 0; q0 < words; q0 += 64) {
          const int q = q0 + lane;
          const int v = q < words ? __popc(bm[r * words + q]) : 0;
          int incl = v;
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
          }
          if (q < words) pw[r * words + q] = (unsigned)(carry + incl - v);
          carry += __shfl(incl, 63);
        }
      }
      __syncthreads();
    }
    for (int i = tid, j = 0; i < n; i += nt, ++j) {
      int e = 0;
#pragma unroll
      for (int q = 0; q < kKeep; ++q)
        if (q == j) e = keep[q];
      if (j >= kKeep) e = (int)(ids[i] - base);
      const int t = i / K;
      const unsigned* row = bm + e * words;
      int rank = __popc(row[t >> 5] & ((1u << (t & 31)) - 1u));
      if (!CO && prefix)
        rank += (int)pre[e * words + (t >> 5)];
      else
        for (int q = 0; q < (t >> 5); ++q) rank += __popc(row[q]);
      const int pos = cnt[e] + rank;
      store_out<CO>(&out.perm[pos], i);
      store_out<CO>(&out.inv[i], pos);
    }
    return;
  }
  // Tiles of 64 * tile_waves entries (cnt[e] holds the running first free row of expert e).
  int* wcount = reinterpret_cast<int*>(bm);  // [tile_waves][E]
  const int lane = tid & 63, w = tid >> 6, tile = 64 * tile_waves;
  for (int b0 = 0; b0 < n; b0 += tile) {
    for (int q = tid; q < tile_waves * E; q += nt) wcount[q] = 0;
    __syncthreads();
    const int i = b0 + tid;
    const bool live = w < tile_waves && i < n;
    const int e = live ? (int)(ids[i] - base) : -1;
    int my_rank = 0;
    if (w < tile_waves) {
      unsigned long long rest = __ballot(live);
      while (rest) {
        const int leader = __ffsll((long long)rest) - 1;
        const int le = __shfl(e, leader);
        const unsigned long long m = __ballot(live && e == le);
        if (live && e == le) my_rank = __popcll(m & lanes_below());
        if (lane == 0) wcount[w * E + le] = __popcll(m);
        rest &= ~m;
      }
    }
    __syncthreads();
    if (live) {
      int pos = cnt[e] + my_rank;
      for (int q = 0; q < w; ++q) pos += wcount[q * E + e];
      store_out<CO>(&out.perm[pos], i);
      store_out<CO>(&out.inv[i], pos);
    }
    __syncthreads();
    for (int q = tid; q < E; q += nt) {
      int add = 0;
      for (int v = 0; v < tile_waves; ++v) add += wcount[v * E + q];
      cnt[q] += add;
    }
    __syncthreads();
  }
}

// LDS ints of permute_block: the bitmap form when it fits in `capacity` ints, else the tiled
// form with as many waves per tile as fit (up to the workgroup's). Returns the tile waves
// (0: bitmap) or -1 if neither fits.
__host__ __device__ inline int permute_tile_waves(int T, int E, int threads, int capacity) {
  const size_t words = ((size_t)T + 31) / 32;
  if ((size_t)E * (1 + words) + 32 <= (size_t)capacity) return 0;
  const int fit = (capacity - 32 - E) / E, waves = threads / 64;
  return fit >= 1 ? (fit < waves ? fit : waves) : -1;
}
constexpr int kPermuteLdsInts = 16384;  // 64 KB

__global__ __launch_bounds__(1024) void k_permute(const int64_t* __restrict__ ids, int64_t base, int T, int K, int E,
                                                  int S, int nbI, int nbH, int ks, int chunk, int wide,
                                                  PermuteOut out, int tile_waves, int prefix,
                                                  const uint8_t* t0, const uint8_t* t1, const uint8_t* t2,
                                                  size_t tbytes) {
  extern __shared__ int smem[];
  __shared__ int flags[2];
  if (blockIdx.x > 0) {
    // The workgroups after the first touch the three matrices' lines (the shared expert's
    // weights, which the expert kernel's first units read) while the permute runs.
    touch_lines<1024>(t0, t1, t2, tbytes, (int)blockIdx.x - 1, (int)gridDim.x - 1);
    return;
  }
  permute_block<false>(ids, base, T, K, E, S, nbI, nbH, ks, chunk, wide, out, smem, flags, tile_waves, prefix != 0);
}

// Workgroups of k_permute that touch the lines of three matrices while the permute runs.
constexpr int kTouchGroups = 128;

// Launches k_permute with the LDS its form needs; with `touch` (three matrices of tbytes
// each), kTouchGroups more workgroups pull their lines into the caches meanwhile (the fp8
// form's shared expert: the stream-ordered expert kernel's first units read them).
int launch_permute(const int64_t* ids, int64_t base, int T, int K, int E, int S, int nbI, int nbH, int ks, int chunk,
                   int wide, const PermuteOut& po, hipStream_t st, const uint8_t* const* touch = nullptr,
                   size_t tbytes = 0) {
  const int tw = permute_tile_waves(T, E, 1024, kPermuteLdsInts);
  if (tw < 0) return MEGAMOE_ERR_UNSUPPORTED;
  // The bitmap form ranks from popcount prefixes when its rows are long (8 words or more)
  // and the prefixes fit beside the bitmap.
  const size_t words = ((size_t)T + 31) / 32;
  const bool prefix = !tw && words >= 8 && 32 + (size_t)E * (1 + 2 * words) <= (size_t)kPermuteLdsInts;
  const size_t ints = tw ? 32 + (size_t)E * (1 + tw) : 32 + (size_t)E * (1 + (prefix ? 2 : 1) * words);
  const bool touching = touch && tbytes > 0;
  hipLaunchKernelGGL(k_permute, dim3(touching ? 1 + kTouchGroups : 1), dim3(1024), ints * 4, st, ids, base, T, K, E,
                     S, nbI, nbH, ks, chunk, wide, po, tw, prefix ? 1 : 0, touching ? touch[0] : nullptr,
                     touching ? touch[1] : nullptr, touching ? touch[2] : nullptr, touching ? tbytes : (size_t)0);
  return hipGetLastError() == hipSuccess ? MEGAMOE_OK : MEGAMOE_ERR_HIP;
}

// ---------------------------------------------------------------------------------------
// Cross-workgroup hand-over inside the expert kernel (h from gate/up units to down
// units). h and its scales are written with device-coherent stores (relaxed agent-scope
// atomic stores, which write through the XCD's L2 to memory), so publishing them takes
// only a wait for the stores to complete, not a writeback of the whole L2. Readers use
// ordinary loads, which cannot return a stale line: every cache is coherent when the
// kernel starts (kernel-boundary acquire); each 128-byte line of h is written by exactly
// one unit, and each padded scale row (one line) by the gate/up units of its chunk, each
// storing only its own 4 bytes; and no workgroup reads a line before the counts of all its
// writers have landed, so no cache holds a copy of a line from before its last write.
// ---------------------------------------------------------------------------------------


// ---------------------------------------------------------------------------------------
// Expert GEMM core. One wavefront multiplies RT row tiles (16 weight rows each) by NCT
// column tiles (16 activation rows each) over the whole reduction axis with
// v_mfma_scale_f32_16x16x128_f8f6f4 (E4M3 x E4M3, unit E8M0 scales): one MFMA per
// (row tile, column tile, 128-wide K block), so each 128x128 weight scale block and each
// 1x128 activation scale block meets exactly one MFMA result, which is scaled in fp32
// and added to the accumulator.
//
// MFMA operand layout: lane l supplies row (l % 16) of its tile and the 32 K bytes
// [16*(l/16), +16) and [64 + 16*(l/16), +16) of the block (16-byte chunks g and g + 4,
// g = l/16), the same byte positions for the weight (A) and the activation (B) operand.
// Result layout: lane l holds rows 4*(l/16) .. +3 of column (l % 16).
//
// Weights stream HBM -> LDS with non-temporal global_load_lds_dwordx4: one instruction
// moves 8 whole 128-byte K-block rows of a tile, lane l fetching chunk (l%8) ^ (l/8) of
// row l/8 into the instruction's LDS slot l, so the chunks of each row sit XOR-swizzled by
// the row index. Two ds_read_b128 per tile give the MFMA layout back (chunk c of row r is
// at slot position c ^ (r % 8)). Full-line requests stream close to the HBM peak where
// 64-byte half lines loaded straight into the MFMA layout do not, and the stages in
// flight take no registers. Each wavefront owns a private ring of D stages in LDS, so no
// barrier is involved: the wait for a stage is an explicit vmcnt (below).
//
// Activations and scales are loaded into registers D-1 stages ahead.
// ---------------------------------------------------------------------------------------

constexpr int kTileBytes = 16 * kBlock;  // one 16-row tile of one K block
constexpr int kRingWave = 16384;         // LDS ring bytes per wavefront

constexpr int kNonTemporal = 2;          // cache policy of the weight loads

__device__ __forceinline__ f32x4 mfma_e4m3(const i32x8& a, const i32x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

__device__ __forceinline__ i32x8 load_k32(const uint8_t* p) {
  const i32x4 lo = *reinterpret_cast<const i32x4*>(p);
  const i32x4 hi = *reinterpret_cast<const i32x4*>(p + 64);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Waits until at most N vector memory operations of this wavefront are outstanding.
// The memory clobber keeps the compiler from moving loads across the wait.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N <= 63, "vmcnt holds 6 bits");
  // gfx9 s_waitcnt immediate: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
  asm volatile("" ::: "memory");
}

// This lane's byte offsets for one tile: `dma` in global memory relative to the tile's
// row 0 (row l/8, swizzled chunk), rd0/rd1 of its two MFMA chunks in the LDS tile.
struct LaneTile {
  int dma, rd0, rd1;
};


__device__ __forceinline__ LaneTile lane_tile(int lda) {
  const int lane = opaque_lane();
  const int lr = lane >> 3, row = lane & 15, rr = row & 7, g = lane >> 4;
  const int base = (row >> 3) * 1024 + rr * kBlock;
  return LaneTile{lr * lda + (((lane & 7) ^ lr) << 4), base + ((g ^ rr) << 4), base + (((g + 4) ^ rr) << 4)};
}

template <int NCT, int SG, bool A16 = false>
struct Stage {
  i32x8 b[NCT];
  float sw[SG];
  float sx[NCT];
};

// The stage of the W8A16 form (frontier.py:180-183, quantize=False): bf16 activations, no
// activation scale. Column tile c's 32 K values of the lane come as four chunks of eight
// (K 16g .. 16g+7, 16g+8 .., 64+16g .., 72+16g .. for lane group g = lane / 16: the K
// values the fp8 weight operand of the lane holds, in the same order).
template <int NCT, int SG>
struct Stage<NCT, SG, true> {
  i32x4 b[NCT][4];
  float sw[SG];
};

template <int RT, int NCT, int SG>
struct Operands {
  const uint8_t* a[RT];    // row 0 of each 16-row weight tile (wave-uniform)
  int lda;                 // weight row length in bytes
  const uint8_t* spare;    // 16 * lda bytes that loads past the last K block read instead
  const float* sw[SG];     // per-K-block weight scales of scale group g (wave-uniform)
  const uint8_t* b[NCT];   // lane's activation row at its K byte offset
  const float* sx[NCT];    // lane's activation scale row
};

// 2*RT weight loads of K block kb into one ring slot, or (live == false, past the last
// block) the same number of loads from the spare region, which has the shape of one tile
// (16 rows of lda bytes): only the wave-uniform base changes, the lane offsets do not.
template <int RT, int NCT, int SG>
__device__ __forceinline__ void issue_a(uint8_t* slot, const Operands<RT, NCT, SG>& op, const LaneTile& lt, int kb,
                                        bool live) {
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint8_t* base = live ? op.a[t] + (size_t)kb * kBlock : op.spare;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(base +
                                                                                     (uint32_t)(lt.dma + 8 * i * op.lda)),
                                       (__attribute__((address_space(3))) void*)(slot + t * kTileBytes + i * 1024),
                                       16, 0, kNonTemporal);
  }
}

// At least 3*NCT vector loads: two 16-byte loads and one scale per column tile.
template <int RT, int NCT, int SG>
__device__ __forceinline__ void load_stage_b(Stage<NCT, SG>& s, const Operands<RT, NCT, SG>& op, int kb) {
  const size_t o = (size_t)kb * kBlock;
#pragma unroll
  for (int c = 0; c < NCT; ++c) s.b[c] = load_k32(op.b[c] + o);
#pragma unroll
  for (int c = 0; c < NCT; ++c) s.sx[c] = op.sx[c][kb];
#pragma unroll
  for (int g = 0; g < SG; ++g) s.sw[g] = op.sw[g][kb];
}

// W8A16: 4*NCT vector loads, four 16-byte bf16 chunks per column tile (op.b[c] points at
// the lane's first chunk of K block 0: 2 * kBlock bytes a block, chunks at +0, +16, +128,
// +144).
template <int RT, int NCT, int SG>
__device__ __forceinline__ void load_stage_b(Stage<NCT, SG, true>& s, const Operands<RT, NCT, SG>& op, int kb) {
  const size_t o = (size_t)kb * 2 * kBlock;
#pragma unroll
  for (int c = 0; c < NCT; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      s.b[c][q] = *reinterpret_cast<const i32x4*>(op.b[c] + o + (q >> 1) * 128 + (q & 1) * 16);
#pragma unroll
  for (int g = 0; g < SG; ++g) s.sw[g] = op.sw[g][kb];
}

// A count another workgroup raises, and the value the work needs from it.
struct ReadyWait {
  const int* count;  // NULL: nothing to wait for
  int need;
  int* error;        // set to 1 if the bounded wait gives up
  uint64_t ticks = kWaitTicks;  // the bound, in 100 MHz ticks
  bool patient = false;         // many workgroups wait on this count: poll less often
  int max_naps = 2;             // patient waits: naps of ~1000 cycles between polls, doubling up to this
  int* claim = nullptr;         // the queue word the workgroup claims its next unit from (NULL: none)
  int* ticket = nullptr;        // thread 0: where the claimed index goes (read after the unit)
};

// Claims a unit: thread 0 adds one to the queue word and gets the old value. The address goes
// through an empty asm into vector registers, which keeps the compiler's atomic optimizer off
// this atomic: for a uniform address it combines the lanes and reads the result back at once,
// so the wavefront would wait for the atomic's round trip (1-5 us while hundreds of workgroups
// claim from the one word) right where it is issued. The pointer stays in the global address
// space: a flat atomic would also count in lgkmcnt, which every LDS read of the ring waits on.
__device__ __forceinline__ int claim_ticket(int* queue) {
  __attribute__((address_space(1))) int* q = (__attribute__((address_space(1))) int*)queue;
  asm volatile("" : "+v"(q));
  return __hip_atomic_fetch_add(q, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The claim of the next unit, issued inside a unit's weight stream once its first weight
// stages are requested (stream_gemm, stream_gemm_shared): its round trip then overlaps the
// first loads, which the unit waits for anyway. Issued at the start of the unit, the claim's
// round trip came before the unit's own first loads (its work-list entries, whose wait covers
// every load issued before them); the gap between two units of a workgroup was ~2 us.
__device__ __forceinline__ void issue_claim(const ReadyWait& w) {
  if (w.claim && threadIdx.x == 0) *w.ticket = claim_ticket(w.claim);
}

__device__ __forceinline__ ReadyWait claiming(ReadyWait w, int* queue, int* ticket) {
  w.claim = queue;
  w.ticket = ticket;
  return w;
}

// The acquire that ends a wait for data another workgroup of the same launch wrote. Workgroup
// scope: the data is written through to memory and no workgroup reads one of its lines before
// the line's last write, so no cache holds a stale copy; an agent-scope acquire would add a
// cache invalidation per wait, hundreds of waits per call while other workgroups stream
// through the same L2s. A build with MEGAMOE_AGENT_ACQUIRE=1 takes agent scope instead: a
// check build, in which the bit-exactness tests of the single launch must pass unchanged.
#ifndef MEGAMOE_AGENT_ACQUIRE
#define MEGAMOE_AGENT_ACQUIRE 0
#endif
__device__ __forceinline__ void acquire_after_wait() {
  if constexpr (MEGAMOE_AGENT_ACQUIRE)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  else
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Thread 0 polls the count (bounded in time), then the workgroup passes a barrier. The barrier
// carries no release fence (this workgroup publishes nothing here, and a release would
// wait for the weight loads in flight); the acquire fence after it keeps the loads that
// follow from moving above it.
__device__ __forceinline__ void wait_ready(const ReadyWait& w) {
  if (!w.count) return;
  if (threadIdx.x == 0) {
    const uint64_t t0 = wall_clock64();
    int naps = 1;  // patient waits: 1, 2, ... max_naps naps of ~1000 cycles between polls
    for (int polls = 0; __hip_atomic_load(w.count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < w.need; ++polls) {
      if ((polls & 15) == 15 && (__hip_atomic_load(w.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
                                 wall_clock64() - t0 > w.ticks)) {
        atomicExch(w.error, 1);
        break;
      }
      if (w.patient) {
        // Hundreds of workgroups wait on one word at once (the router's, the permute's and
        // the down units' counts): each poll is a load at the memory channel that holds the
        // word, which every weight stream also crosses, so the polls back off.
        for (int k = 0; k < naps; ++k) __builtin_amdgcn_s_sleep(16);
        naps = 2 * naps < w.max_naps ? 2 * naps : w.max_naps;
      } else {
        __builtin_amdgcn_s_sleep(2);
      }
    }
  }
  __builtin_amdgcn_s_barrier();
  acquire_after_wait();
}


// The RT tiles of one ring slot in MFMA layout. The reads are inline asm: the compiler
// takes any LDS read that follows a global_load_lds as depending on the most recent one
// and would wait for every load in flight (vmcnt 0) before it, while the ring's own vmcnt
// wait already covers the slot read here. The lgkmcnt wait names the results as operands,
// so no use of them can be scheduled before it.
template <int RT>
__device__ __forceinline__ void read_slot(i32x8 (&a)[RT], uint32_t p0, uint32_t p1) {
  i32x4 lo[RT], hi[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3"
                 : "=&v"(lo[r]), "=&v"(hi[r])
                 : "v"(p0 + r * kTileBytes), "v"(p1 + r * kTileBytes)
                 : "memory");
  if constexpr (RT == 2) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo[0]), "+v"(hi[0]), "+v"(lo[1]), "+v"(hi[1]));
  } else {
    static_assert(RT == 4, "two or four row tiles");
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(lo[0]), "+v"(hi[0]), "+v"(lo[1]), "+v"(hi[1]), "+v"(lo[2]), "+v"(hi[2]), "+v"(lo[3]),
                   "+v"(hi[3]));
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) a[r] = __builtin_shufflevector(lo[r], hi[r], 0, 1, 2, 3, 4, 5, 6, 7);
}

// `slot` is the LDS byte address of the ring slot.
template <int RT, int NCT, int SG>
__device__ __forceinline__ void compute_stage(uint32_t slot, const LaneTile& lt, const Stage<NCT, SG>& s,
                                              f32x4 (&acc)[RT][NCT]) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  i32x8 at[RT];
  read_slot<RT>(at, slot + lt.rd0, slot + lt.rd1);
  // The scales pass through an empty asm first, which keeps their products where the
  // stage is consumed: hoisted next to the loads of a later stage, a product would need
  // those loads to have landed, and the compiler, which does not take vmcnt to count them
  // in order once LDS DMA is in flight, would wait for vmcnt 0 there, every stage.
  float sw[SG], sx[NCT];
#pragma unroll
  for (int g = 0; g < SG; ++g) {
    sw[g] = s.sw[g];
    asm volatile("" : "+v"(sw[g]));
  }
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    sx[c] = s.sx[c];
    asm volatile("" : "+v"(sx[c]));
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const i32x8& a = at[r];
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      const f32x4 p = mfma_e4m3(a, s.b[c], zero);
      const float k = sw[r * SG / RT] * sx[c];
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[r][c][v] = __builtin_fmaf(p[v], k, acc[r][c][v]);
    }
  }
}

// Eight e4m3 values (two dwords, lowest byte first) as eight bf16: the conversion is exact
// (every e4m3 value is a bf16 value), two values per instruction.
__device__ __forceinline__ i32x4 e4m3x8_to_bf16(int lo, int hi) {
  i32x4 r;
  r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
  r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
  r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
  r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
  return r;
}

// W8A16 stage: each weight tile's 32 e4m3 values of the lane become four bf16 chunks, and
// four 16x16x32 bf16 MFMAs (chunk q of the weights against chunk q of the activations, the
// same K values) give the block's product, which the block's weight scale multiplies into
// the fp32 sum, as in the W8A8 stage (frontier.py:180-183: dequant(W, s) @ fp32(x)).
template <int RT, int NCT, int SG>
__device__ __forceinline__ void compute_stage(uint32_t slot, const LaneTile& lt, const Stage<NCT, SG, true>& s,
                                              f32x4 (&acc)[RT][NCT]) {
  i32x8 at[RT];
  read_slot<RT>(at, slot + lt.rd0, slot + lt.rd1);
  float sw[SG];
#pragma unroll
  for (int g = 0; g < SG; ++g) {
    sw[g] = s.sw[g];
    asm volatile("" : "+v"(sw[g]));
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    i32x4 a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = e4m3x8_to_bf16(at[r][2 * q], at[r][2 * q + 1]);
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      f32x4 p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[q]),
                                                    __builtin_bit_cast(bf16x8, s.b[c][q]), p, 0, 0, 0);
      const float k = sw[r * SG / RT];
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[r][c][v] = __builtin_fmaf(p[v], k, acc[r][c][v]);
    }
  }
}

// Streams nkb K blocks through the wavefront's LDS ring (D slots) with D-1 stages of loads
// in flight. With a ReadyWait, the weights of the first stages are requested before the
// wait and the activations (which another workgroup produces) after it, so the wait's
// round trip overlaps the first weight loads; the claim of the workgroup's next unit, if the
// ReadyWait carries one, is issued between them (one more vector memory operation after the
// first weights, which only makes the first stage's vmcnt wait below more conservative).
//
// The stream starts at K block `rot` and wraps around (any rot in [0, nkb); callers derive
// it from the unit index). Units that run at the same time then read different K blocks of
// their weight rows: with every workgroup at the same K block, the addresses in flight
// differ only in their high bits (multiples of the row length, 4 KiB for some models), and
// the HBM channels serve them unevenly (about 6% slower on a Mixtral-shaped layer). The
// fp32 sum over K blocks then runs in a rotated order; it depends on the work list only,
// so results are still the same on every call.
//
// The wait for stage s: a wavefront's vector memory loads (to LDS or to registers)
// complete in issue order, and the compiler's own counters do not cover the LDS that
// global_load_lds writes. When stage s is consumed, each of stages s+1 .. s+D-1 has been
// issued after stage s's weights, as a group of 2*RT weight loads and at least 3*NCT
// activation loads (4*NCT in the W8A16 form), so vmcnt <= (D-1)*(2*RT + 3*NCT) (or 4*NCT)
// implies stage s has landed.
// Loads past the last K block are not skipped: a branch around them would merge paths with
// different load counts, and the compiler then waits for vmcnt 0 before the next MFMA,
// which drains the pipeline at every stage. They read the spare region instead (every
// workgroup reads it, so it stays in L2; re-reading the last weight block would go to HBM,
// since non-temporal lines do not stay in L2) into slots nothing reads any more, and they
// land before any later load into the ring (issue order). The slot a stage overwrites was
// read (ds_read, issued in program order before the overwriting load) one stage earlier.
template <int RT, int NCT, int SG, int D, bool A16 = false>
__device__ __forceinline__ void stream_gemm(const Operands<RT, NCT, SG>& op, int nkb, int rot, uint8_t* ring,
                                            f32x4 (&acc)[RT][NCT],
                                            const ReadyWait& ready = ReadyWait{nullptr, 0, nullptr}) {
  // K block i of the stream is block (i + rot) mod nkb of the operands.
  auto phys = [nkb, rot](int kb) {
    const int p = kb + rot;
    return p >= nkb ? p - nkb : p;
  };
  constexpr int kSlot = RT * kTileBytes;
  constexpr int kAfter = (D - 1) * (2 * RT + (A16 ? 4 : 3) * NCT);
  static_assert(D >= 2 && D * kSlot <= kRingWave, "LDS ring");
  const LaneTile lt = lane_tile(op.lda);
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < NCT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  Stage<NCT, SG, A16> st[D];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) issue_a(ring + s * kSlot, op, lt, phys(min(s, nkb - 1)), s < nkb);
  issue_claim(ready);
  wait_ready(ready);
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load_stage_b(st[s], op, phys(min(s, nkb - 1)));
  for (int kb0 = 0; kb0 < nkb; kb0 += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int kb = kb0 + s, kn = phys(min(kb + D - 1, nkb - 1));
      load_stage_b(st[(s + D - 1) % D], op, kn);
      issue_a(ring + ((s + D - 1) % D) * kSlot, op, lt, kn, kb + D - 1 < nkb);
      wait_vmem<kAfter>();
      if (kb < nkb) compute_stage(ring_lds + s * kSlot, lt, st[s], acc);
    }
  }
}

// The stream of a down unit over 33-64 activation rows (four column tiles), with the
// activation tiles shared by the workgroup's four wavefronts: wave w moves only column
// tile w of each stage, HBM/L2 -> LDS by DMA (two 1 KB instructions, the weight tiles'
// swizzle), into one of two slots; a barrier per stage makes all four tiles visible, and
// every wave reads them from LDS. Each wave so moves a quarter of stream_gemm's
// activation bytes through the vector L1. The slots are the last 4 KB of the four waves'
// rings (a three-slot weight ring of 4 KB leaves them free): tiles 0-1 of slot q in wave
// 2q's ring, tiles 2-3 in wave 2q+1's. Weights run two stages ahead (as stream_gemm with
// D = 3), activations and scales one: iteration kb waits for its activation tile (issued
// after the barrier of stage kb - 1) with only the weights of stage kb + 1 issued after
// it, passes the barrier, requests the tile of stage kb + 1 into the other slot (read by
// every wave before this barrier), reads stage kb and requests the weights of kb + 2.
struct StageShared {
  float sx[4];
  float sw;
};

__device__ __forceinline__ void issue_shared(uint32_t slot_tile, const uint8_t* const (&xrow)[2], int kb,
                                             StageShared& st, const Operands<2, 4, 1>& op) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(xrow[i] + (size_t)kb * kBlock),
                                     (__attribute__((address_space(3))) void*)(uintptr_t)(slot_tile + i * 1024), 16, 0,
                                     0);
#pragma unroll
  for (int c = 0; c < 4; ++c) st.sx[c] = op.sx[c][kb];
  st.sw = op.sw[0][kb];
}

// xrow[i]: this lane's DMA source row for rows 8i .. 8i+7 of column tile w (clamped to
// the chunk), at its swizzled 16-byte chunk of a K block, K part start included.
__device__ __forceinline__ void stream_gemm_shared(const Operands<2, 4, 1>& op, const uint8_t* const (&xrow)[2],
                                                   int nkb, int rot, uint8_t* ring, f32x4 (&acc)[2][4],
                                                   const ReadyWait& ready) {
  constexpr int RT = 2, NCT = 4, D = 3;
  constexpr int kSlot = RT * kTileBytes;
  static_assert(D * kSlot + 2 * kTileBytes <= kRingWave, "LDS ring and activation slots");
  auto phys = [nkb, rot](int kb) {
    const int p = kb + rot;
    return p >= nkb ? p - nkb : p;
  };
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const LaneTile lt = lane_tile(op.lda);
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;
  const uint32_t rings_lds = ring_lds - (uint32_t)(w * kRingWave);
#define MEGAMOE_XTILE(q, c) \
  (rings_lds + (uint32_t)((2 * (q) + ((c) >> 1)) * kRingWave + (kRingWave - 2 * kTileBytes) + ((c) & 1) * kTileBytes))
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < NCT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  StageShared st[2];
  // Issue order W0, A0, W1, then per stage kb: A(kb+1), W(kb+2). When stage kb is waited
  // for, only W(kb+1) was issued after A(kb), and W(kb) before it: vmcnt <= 2*RT. Every
  // stage, live or not, issues the same loads and passes the same barrier (a branch around
  // loads would make the compiler drain every load); only the MFMAs of stages past the
  // end are skipped.
  issue_a(ring, op, lt, phys(0), true);
  issue_claim(ready);
  wait_ready(ready);
  issue_shared(MEGAMOE_XTILE(0, w), xrow, phys(0), st[0], op);
  issue_a(ring + kSlot, op, lt, phys(min(1, nkb - 1)), 1 < nkb);
  for (int kb0 = 0; kb0 < nkb; kb0 += 2 * D) {
#pragma unroll
    for (int s = 0; s < 2 * D; ++s) {  // 2*D: slot indices of both rings are compile-time
      const int kb = kb0 + s;
      wait_vmem<2 * RT>();
      __builtin_amdgcn_s_barrier();
      issue_shared(MEGAMOE_XTILE((s + 1) & 1, w), xrow, phys(min(kb + 1, nkb - 1)), st[(s + 1) & 1], op);
      i32x8 at[RT];
      read_slot<RT>(at, ring_lds + (s % D) * kSlot + lt.rd0, ring_lds + (s % D) * kSlot + lt.rd1);
      i32x8 bt[NCT];
#pragma unroll
      for (int c = 0; c < NCT; ++c) {
        i32x4 lo, hi;
        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3"
                     : "=&v"(lo), "=&v"(hi)
                     : "v"(MEGAMOE_XTILE(s & 1, c) + lt.rd0), "v"(MEGAMOE_XTILE(s & 1, c) + lt.rd1)
                     : "memory");
        bt[c] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(bt[0]), "+v"(bt[1]), "+v"(bt[2]), "+v"(bt[3]));
      issue_a(ring + ((s + 2) % D) * kSlot, op, lt, phys(min(kb + 2, nkb - 1)), kb + 2 < nkb);
      float sw = st[s & 1].sw, sx[NCT];
      asm volatile("" : "+v"(sw));
#pragma unroll
      for (int c = 0; c < NCT; ++c) {
        sx[c] = st[s & 1].sx[c];
        asm volatile("" : "+v"(sx[c]));
      }
      if (kb < nkb) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NCT; ++c) {
          const float k = sw * sx[c];
#pragma unroll
          for (int r = 0; r < RT; ++r) {
            const f32x4 pr = mfma_e4m3(at[r], bt[c], zero);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[r][c][v] = __builtin_fmaf(pr[v], k, acc[r][c][v]);
          }
        }
      }
    }
  }
  // The last stage requested one more activation tile into another wave's ring: every wave
  // waits for its loads and the workgroup passes a barrier before any ring is reused.
  wait_vmem<0>();
  __builtin_amdgcn_s_barrier();
#undef MEGAMOE_XTILE
}

// Rows of one chunk: rows r = 0 .. n-1 map to grouped buffer row row0 + r and to token
// perm[row0 + r] / K (routed) or row0 + r (shared expert, perm == NULL).
struct ChunkRows {
  int n;
  int row0;
  const int* perm;
  int K;
  int by_token;  // 0: the unit's h and d rows are row0 + r (grouped); 1: out_base + row r's token
  int out_base;  // (the dense schedule: expert e's rows e*T + t)
};

// Row r's token: perm[row0 + r] / K (grouped rows), else row0 + r.
__device__ __forceinline__ int row_token(const ChunkRows& cr, int r) {
  return cr.perm ? cr.perm[cr.row0 + r] / cr.K : cr.row0 + r;
}

// The row of the unit's h and d where row r goes.
__device__ __forceinline__ int out_row(const ChunkRows& cr, int r) {
  return cr.by_token ? cr.out_base + row_token(cr, r) : cr.row0 + r;
}

// The dense schedule (the host's dense_experts): lists of every expert's gate/up and down
// units, known before the routing is. Gate/up chunk c: the shared expert's copies first
// (c < S, its block offset c * nbI), then routed expert c - S; down chunk c: the shared
// expert first (if any), then the routed experts. Routed expert e's h and d rows are rows
// e*T + t of the routed rows, t the token. A unit that starts before the routing is known
// works every token (dense_rows); one that starts after works the expert's routed rows
// (routed_rows), or nothing if no token picked the expert. Each row's values are the same
// either way: every MFMA output column depends only on its own row.
__device__ __forceinline__ int4 dense_gu_chunk(int c, int E, int S, int T, int nbI) {
  return c < S ? make_int4(E, 0, T, c * nbI) : make_int4(c - S, 0, T, 0);
}
__device__ __forceinline__ int4 dense_dn_chunk(int c, int E, int S, int T) {
  const int sh = S > 0 ? 1 : 0;
  return c < sh ? make_int4(E, 0, T, 0) : make_int4(c - sh, 0, T, 0);
}
__device__ __forceinline__ ChunkRows dense_rows(int e, int T, int K) { return ChunkRows{T, 0, nullptr, K, 1, e * T}; }
__device__ __forceinline__ ChunkRows routed_rows(int e, int T, int K, const int* offsets, const int* perm) {
  const int o = offsets[e];
  return ChunkRows{offsets[e + 1] - o, o, perm, K, 1, e * T};
}
// The down chunk a dense gate/up chunk feeds, and the gate/up units a dense down chunk needs.
__device__ __forceinline__ int dense_dn_of_gu(int c, int S) { return c < S ? 0 : c - S + (S > 0 ? 1 : 0); }
__device__ __forceinline__ int dense_dn_need(int c, int S, int nbI) { return S > 0 && c == 0 ? S * nbI : nbI; }


struct GateUpArgs {
  const uint8_t* xq;   // [T, H] e4m3
  const float* xs;     // [T, H/128]
  const uint8_t* gate; const float* gate_scale;
  const uint8_t* up; const float* up_scale;
  const uint8_t* sgate; const float* sgate_scale;
  const uint8_t* sup; const float* sup_scale;
  const int* offsets; const int* perm; const int4* chunks;
  int* meta;
  uint8_t* hq_r; float* hs_r;   // routed rows [T*K, I], [T*K, I/128]
  uint8_t* hq_s; float* hs_s;   // shared rows [T, S*I], [T, S*I/128]
  uint16_t* st_r;               // bf16 gate and up outputs of routed rows, [2][T*K, I]
  uint16_t* st_s;               // of shared rows, [2][T, S*I]
  int* pairs;                   // per (gate/up chunk, 128-row block): halves finished
  const uint8_t* spare;         // 16 rows of the longest weight row, in the workspace
  int T, H, I, K, S, E, pow2;
  int swiglu;                   // 0: fp32 product rounded once; 1: bf16 silu, bf16 product
  float limit;                  // > 0: SwiGLU clamp (gate above, up both sides)
  int dense;                    // the dense schedule: units from dense_gu_chunk, h rows e*T + t
  int pad_;
  const uint16_t* x16;          // W8A16: the bf16 rows [T, H] the experts read (x, or the normalized x)
  uint16_t* h16_r;              // W8A16: bf16 h of the routed rows [rows_r, I]
  uint16_t* h16_s;              // W8A16: of the shared rows [T, S*I]
};

// One gate/up unit: rows [jb*128, jb*128+128) of gate and of up against the chunk's
// activation rows (at most 16*NCT). Wave w owns gate and up rows 32w .. 32w+31 of the
// block, so SwiGLU pairs matching registers; the per-row amax over the 128-block for the
// requantization of h is reduced across the four wavefronts through LDS.
template <int NCT>
__device__ __forceinline__ void gateup_unit(const GateUpArgs& a, const uint8_t* wg, const uint8_t* wu, const float* sg,
                            const float* su, const ChunkRows& cr, int jb, uint8_t* hq, float* hs, int ldh,
                            int rot, float (*red)[64], uint8_t* ring, const ReadyWait& ready) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kofs = 16 * (lane >> 4);
  const int H = a.H, nkb = H / kBlock, nbh = scale_ld(ldh / kBlock);
  Operands<4, NCT, 2> op;
  op.lda = H;
  op.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const size_t row = (size_t)(32 * w + 16 * r);
    op.a[r] = wg + row * H;
    op.a[r + 2] = wu + row * H;
  }
  op.sw[0] = sg;
  op.sw[1] = su;
  int orow[NCT];  // the h row of each column (a padding column's is never stored)
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = min(16 * c + (lane & 15), cr.n - 1);  // padding columns repeat a valid row
    const int tok = row_token(cr, r);
    op.b[c] = a.xq + (size_t)tok * H + kofs;
    op.sx[c] = a.xs + (size_t)tok * nkb;
    orow[c] = cr.by_token ? cr.out_base + tok : cr.row0 + r;
  }
  f32x4 acc[4][NCT];
  stream_gemm<4, NCT, 2, 2>(op, nkb, rot, ring, acc, ready);

  // g, u = bf16 (frontier.py:184-186), clamped at the SwiGLU limit if one is set
  // (glm53.py:175); h = bf16(silu(fp32 g) * fp32 u) (frontier.py:337, DeepSeek) or
  // bf16(bf16(silu(g)) * u) (frontier.py:338, glm53.py:174-175).
  const bool bf16_silu = a.swiglu != 0;
  const float L = a.limit > 0.0f ? a.limit : INFINITY;
  float hv[NCT][2][4];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float g = fminf(round_bf16(acc[p][c][v]), L);
        const float u = fminf(fmaxf(round_bf16(acc[p + 2][c][v]), -L), L);
        const float h = bf16_silu ? round_bf16(round_bf16(silu(g)) * u) : round_bf16(silu(g) * u);
        hv[c][p][v] = h;
        amax = fmaxf(amax, fabsf(h));
      }
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    if (lane < 16) red[w][16 * c + lane] = amax;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int col = 16 * c + (lane & 15);
    const float amax = fmaxf(fmaxf(red[0][col], red[1][col]), fmaxf(red[2][col], red[3][col]));
    const float s = act_scale(amax, a.pow2);
    if (col < cr.n) {
      uint8_t* dst = hq + (size_t)orow[c] * ldh + (size_t)jb * kBlock + 32 * w + 4 * (lane >> 4);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint32_t packed = e4m3x4(clamp448(hv[c][p][0] / s), clamp448(hv[c][p][1] / s),
                                       clamp448(hv[c][p][2] / s), clamp448(hv[c][p][3] / s));
        store_coherent(reinterpret_cast<uint32_t*>(dst + 16 * p), packed);
      }
      if (w == 0 && lane < 16) store_coherent(hs + (size_t)orow[c] * nbh + jb, s);
    }
  }
}

// The W8A16 gate/up unit (frontier.py:180-183 with quantize=False, the expert GEMMs of the
// DeepSeek family at frontier.py:265-270): gateup_unit's rows and waves, with the bf16 rows
// of x as the activations; g and u are rounded to bf16 (frontier.py:183), clamped if a
// SwiGLU limit is set, and h = bf16(silu(fp32 g) * fp32 u) (frontier.py:337) or
// bf16(bf16(silu(g)) * u) (glm53.py:174-175) stays in bf16 for the down units (no
// requantization).
template <int NCT>
__device__ __forceinline__ void gateup_unit16(const GateUpArgs& a, const uint8_t* wg, const uint8_t* wu,
                                              const float* sg, const float* su, const ChunkRows& cr, int jb,
                                              uint16_t* h, int ldh, int rot, uint8_t* ring, const ReadyWait& ready) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.H;
  Operands<4, NCT, 2> op;
  op.lda = H;
  op.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const size_t row = (size_t)(32 * w + 16 * r);
    op.a[r] = wg + row * H;
    op.a[r + 2] = wu + row * H;
  }
  op.sw[0] = sg;
  op.sw[1] = su;
  int orow[NCT];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = min(16 * c + (lane & 15), cr.n - 1);  // padding columns repeat a valid row
    const int tok = row_token(cr, r);
    op.b[c] = reinterpret_cast<const uint8_t*>(a.x16 + (size_t)tok * H) + 32 * (lane >> 4);
    op.sx[c] = nullptr;
    orow[c] = cr.by_token ? cr.out_base + tok : cr.row0 + r;
  }
  f32x4 acc[4][NCT];
  stream_gemm<4, NCT, 2, 2, true>(op, H / kBlock, rot, ring, acc, ready);
  const bool bf16_silu = a.swiglu != 0;
  const float L = a.limit > 0.0f ? a.limit : INFINITY;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    if (16 * c + (lane & 15) >= cr.n) continue;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      uint32_t bits[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float g = fminf(round_bf16(acc[p][c][v]), L);
        const float u = fminf(fmaxf(round_bf16(acc[p + 2][c][v]), -L), L);
        bits[v] = f32_to_bf16_bits(bf16_silu ? round_bf16(silu(g)) * u : silu(g) * u);
      }
      uint16_t* dst = h + (size_t)orow[c] * ldh + (size_t)jb * kBlock + 32 * w + 16 * p + 4 * (lane >> 4);
      store_coherent(reinterpret_cast<uint64_t*>(dst),
                     (uint64_t)(bits[0] | (bits[1] << 16)) | ((uint64_t)(bits[2] | (bits[3] << 16)) << 32));
    }
  }
}

// Gate/up unit u of the work list (of the dense schedule's lists): chunk u / nbI, 128-row
// block u % nbI of the chunk's expert (plus the slice offset of a shared-expert copy).
// `ready`: a count to wait for before the activation rows are read (the quantized x of the
// single launch's dense schedule), after the unit's first weight stages are requested.
// In the dense schedule, `known`: the routing is known (the unit works its expert's routed
// rows; else every token).
template <bool A16 = false>
__device__ __forceinline__ void gateup_work(const GateUpArgs& a, int u, float (*red)[64], uint8_t* ring,
                                            const ReadyWait& ready = ReadyWait{nullptr, 0, nullptr},
                                            bool known = true) {
  const int nbI = a.I / kBlock, nkb = a.H / kBlock;
  const int4 ch = a.dense ? dense_gu_chunk(u / nbI, a.E, a.S, a.T, nbI) : a.chunks[u / nbI];
  const int j = u % nbI, jb = ch.w + j;
  const int rot = u % nkb;  // concurrent units start at different K blocks
  const uint8_t *wg, *wu;
  const float *sg, *su;
  uint8_t* hq;
  float* hs;
  int ldh;
  ChunkRows cr;
  if (ch.x == a.E) {  // shared expert: rows of its S*I-row gate/up matrices
    wg = a.sgate + (size_t)jb * kBlock * a.H;
    wu = a.sup + (size_t)jb * kBlock * a.H;
    sg = a.sgate_scale + (size_t)jb * nkb;
    su = a.sup_scale + (size_t)jb * nkb;
    cr = ChunkRows{ch.z, ch.y, nullptr, a.K};
    hq = a.hq_s;
    hs = a.hs_s;
    ldh = a.S * a.I;
  } else {
    const size_t rowblk = (size_t)ch.x * nbI + jb;
    wg = a.gate + rowblk * kBlock * a.H;
    wu = a.up + rowblk * kBlock * a.H;
    sg = a.gate_scale + rowblk * nkb;
    su = a.up_scale + rowblk * nkb;
    cr = !a.dense ? ChunkRows{ch.z, ch.y, a.perm, a.K}
                  : (known ? routed_rows(ch.x, a.T, a.K, a.offsets, a.perm) : dense_rows(ch.x, a.T, a.K));
    hq = a.hq_r;
    hs = a.hs_r;
    ldh = a.I;
  }
  if constexpr (A16) {
    // Chunks of at most 32 rows (the W8A16 form's permute).
    uint16_t* h = ch.x == a.E ? a.h16_s : a.h16_r;
    if (cr.n <= 16)
      gateup_unit16<1>(a, wg, wu, sg, su, cr, jb, h, ldh, rot, ring, ready);
    else
      gateup_unit16<2>(a, wg, wu, sg, su, cr, jb, h, ldh, rot, ring, ready);
  } else if (cr.n <= 16) {
    gateup_unit<1>(a, wg, wu, sg, su, cr, jb, hq, hs, ldh, rot, red, ring, ready);
  } else if (cr.n <= 32) {
    gateup_unit<2>(a, wg, wu, sg, su, cr, jb, hq, hs, ldh, rot, red, ring, ready);
  } else {
    gateup_unit<4>(a, wg, wu, sg, su, cr, jb, hq, hs, ldh, rot, red, ring, ready);
  }
}

// One half of a gate/up block: rows [jb*128, jb*128+128) of gate (half 0) or of up (half 1)
// against the chunk's activation rows (at most 16*NCT). Wave w owns rows 32w .. 32w+31 of
// the block. The half rounds its outputs to bf16 (frontier.py:184-186), clamps them at the
// SwiGLU limit if one is set (glm53.py:175: gate above, up on both sides) and stores them
// to the staging rows with device-coherent stores; then it counts itself in the block's
// pair counter. The half that finishes second reads the other half's values back (the same
// elements its own lanes hold), forms h = bf16(silu(fp32 g) * fp32 u) (frontier.py:337,
// DeepSeek) or bf16(bf16(silu(g)) * u) (frontier.py:338, glm53.py:174-175), reduces the
// per-row amax over the 128-block across the four wavefronts through LDS and requantizes h
// to E4M3 per 128. Returns true for that half (the block of h is complete).
//
// Staging hand-over: every staged line is written by exactly one half, read only by the
// other half of its block after the counter has shown the writer done (the writer's
// stores complete before its increment), and never read earlier in the kernel, so no
// cache can hold a stale copy of it.
template <int NCT>
__device__ __forceinline__ bool gateup_half(const GateUpArgs& a, const uint8_t* wt, const float* sc, const ChunkRows& cr, int jb,
                            int half, uint8_t* hq, float* hs, uint16_t* st_mine, const uint16_t* st_other, int ldh,
                            int* pair, int rot, float (*red)[64], int* flag, uint8_t* ring,
                            const ReadyWait& claim) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kofs = 16 * (lane >> 4);
  const int H = a.H, nkb = H / kBlock, nbh = scale_ld(ldh / kBlock);
  Operands<2, NCT, 1> op;
  op.lda = H;
  op.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 2; ++r) op.a[r] = wt + (size_t)(32 * w + 16 * r) * H;
  op.sw[0] = sc;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = min(16 * c + (lane & 15), cr.n - 1);  // padding columns repeat a valid row
    const int tok = row_token(cr, r);
    op.b[c] = a.xq + (size_t)tok * H + kofs;
    op.sx[c] = a.xs + (size_t)tok * nkb;
  }
  f32x4 acc[2][NCT];
  stream_gemm<2, NCT, 1, NCT == 4 ? 3 : 4>(op, nkb, rot, ring, acc, claim);

  const float L = a.limit > 0.0f ? a.limit : INFINITY;
  const float lo = half ? -L : -INFINITY;  // up is clamped on both sides, gate above only
  float mine[NCT][2][4];
  // Lane element (c, p, v): output channel jb*128 + 32w + 16p + 4*(lane/16) + v of token
  // row 16c + lane%16; four consecutive channels per lane go out as one 8-byte store.
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int col = 16 * c + (lane & 15);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      uint32_t bits[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float x = fminf(fmaxf(round_bf16(acc[p][c][v]), lo), L);
        mine[c][p][v] = x;
        bits[v] = f32_to_bf16_bits(x);
      }
      if (col < cr.n) {
        uint16_t* dst = st_mine + (size_t)(cr.row0 + col) * ldh + (size_t)jb * kBlock + 32 * w + 16 * p +
                        4 * (lane >> 4);
        store_coherent(reinterpret_cast<uint64_t*>(dst),
                       (uint64_t)(bits[0] | (bits[1] << 16)) | ((uint64_t)(bits[2] | (bits[3] << 16)) << 32));
      }
    }
  }
  publish_fence();
  __syncthreads();
  if (threadIdx.x == 0) *flag = atomicAdd(pair, 1);
  __syncthreads();
  if (*flag == 0) return false;  // the other half finishes the block
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  const bool bf16_silu = a.swiglu != 0;
  float hv[NCT][2][4];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int col = 16 * c + (lane & 15);
    const int rr = min(col, cr.n - 1);
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint2 o = *reinterpret_cast<const uint2*>(st_other + (size_t)(cr.row0 + rr) * ldh +
                                                      (size_t)jb * kBlock + 32 * w + 16 * p + 4 * (lane >> 4));
      const float ov[4] = {bf16_bits_to_f32(o.x & 0xffffu), bf16_bits_to_f32(o.x >> 16),
                           bf16_bits_to_f32(o.y & 0xffffu), bf16_bits_to_f32(o.y >> 16)};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float g = half ? ov[v] : mine[c][p][v];
        const float u = half ? mine[c][p][v] : ov[v];
        const float h = bf16_silu ? round_bf16(round_bf16(silu(g)) * u) : round_bf16(silu(g) * u);
        hv[c][p][v] = h;
        amax = fmaxf(amax, fabsf(h));
      }
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    if (lane < 16) red[w][16 * c + lane] = amax;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int col = 16 * c + (lane & 15);
    const float amax = fmaxf(fmaxf(red[0][col], red[1][col]), fmaxf(red[2][col], red[3][col]));
    const float s = act_scale(amax, a.pow2);
    if (col < cr.n) {
      uint8_t* dst = hq + (size_t)(cr.row0 + col) * ldh + (size_t)jb * kBlock + 32 * w + 4 * (lane >> 4);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint32_t packed = e4m3x4(clamp448(hv[c][p][0] / s), clamp448(hv[c][p][1] / s),
                                       clamp448(hv[c][p][2] / s), clamp448(hv[c][p][3] / s));
        store_coherent(reinterpret_cast<uint32_t*>(dst + 16 * p), packed);
      }
      if (w == 0 && lane < 16) store_coherent(hs + (size_t)(cr.row0 + col) * nbh + jb, s);
    }
  }
  return true;
}

// Gate/up unit u of the work list: block pair u / 2 (chunk (u/2) / nbI, 128-row block
// (u/2) % nbI of the chunk's expert, plus the slice offset of a shared-expert copy), half
// u % 2 (gate, then up). Returns true if this unit completed the block of h.
// `claim`: the claim of the workgroup's next unit, issued inside the weight stream.
__device__ __forceinline__ bool gateup_work_split(const GateUpArgs& a, int u, float (*red)[64], int* flag, uint8_t* ring,
                                                  const ReadyWait& claim) {
  const int nbI = a.I / kBlock, nkb = a.H / kBlock;
  const int pair = u >> 1, half = u & 1;
  const int4 ch = a.chunks[pair / nbI];
  const int j = pair % nbI, jb = ch.w + j;
  const int rot = pair % nkb;  // concurrent units start at different K blocks
  const uint8_t* wt;
  const float* sc;
  uint8_t* hq;
  float* hs;
  uint16_t* st;
  int ldh;
  size_t st_half;
  ChunkRows cr;
  if (ch.x == a.E) {  // shared expert: rows of its S*I-row gate/up matrices
    wt = (half ? a.sup : a.sgate) + (size_t)jb * kBlock * a.H;
    sc = (half ? a.sup_scale : a.sgate_scale) + (size_t)jb * nkb;
    cr = ChunkRows{ch.z, ch.y, nullptr, a.K};
    hq = a.hq_s;
    hs = a.hs_s;
    ldh = a.S * a.I;
    st = a.st_s;
    st_half = (size_t)a.T * ldh;
  } else {
    const size_t rowblk = (size_t)ch.x * nbI + jb;
    wt = (half ? a.up : a.gate) + rowblk * kBlock * a.H;
    sc = (half ? a.up_scale : a.gate_scale) + rowblk * nkb;
    cr = ChunkRows{ch.z, ch.y, a.perm, a.K};
    hq = a.hq_r;
    hs = a.hs_r;
    ldh = a.I;
    st = a.st_r;
    st_half = (size_t)a.T * a.K * ldh;
  }
  uint16_t* mine = st + (half ? st_half : 0);
  const uint16_t* other = st + (half ? 0 : st_half);
  int* ctr = a.pairs + pair;
  if (cr.n <= 16)
    return gateup_half<1>(a, wt, sc, cr, jb, half, hq, hs, mine, other, ldh, ctr, rot, red, flag, ring, claim);
  else if (cr.n <= 32)
    return gateup_half<2>(a, wt, sc, cr, jb, half, hq, hs, mine, other, ldh, ctr, rot, red, flag, ring, claim);
  else
    return gateup_half<4>(a, wt, sc, cr, jb, half, hq, hs, mine, other, ldh, ctr, rot, red, flag, ring, claim);
}

struct DownArgs {
  const uint8_t* down; const float* down_scale;
  const uint8_t* sdown; const float* sdown_scale;
  const int* offsets; const int* perm; const int4* chunks;
  int* meta;
  const uint8_t* hq_r; const float* hs_r;
  const uint8_t* hq_s; const float* hs_s;
  uint16_t* d_r;  // [T*K, H] bf16, grouped rows
  uint16_t* d_s;  // [T, H] bf16
  float* p_r;     // ks > 1: [ks, T*K, H] fp32 partial d of each K part
  float* p_s;     // ks > 1: [ks, T, H]
  const uint8_t* spare;  // 16 rows of the longest weight row, in the workspace
  int T, H, I, K, S, E, ks;
  int dense;      // the dense schedule: units from dense_dn_chunk, rows e*T + t
  int rows_r;     // routed rows of d_r and of each part of p_r: T*K, or E*T in the dense schedule
  const uint16_t* h16_r;  // W8A16: bf16 h of the routed rows [rows_r, I]
  const uint16_t* h16_s;  // W8A16: of the shared rows [T, S*I]
};

// One down unit: rows [j*128, j*128+128) of a down matrix [H, ldk] against the chunk's
// requantized h rows, over K part kp of a.ks (K blocks [kp*nkb/ks, (kp+1)*nkb/ks)). Wave w
// owns rows 32w .. 32w+31. With one part the result is d in bf16; with several, each part
// stores its fp32 partial to pd and the combine adds the parts in order before rounding.
// A16: the W8A16 form; hq then holds the bf16 h rows (2 * ldk bytes a row), hs is unused.
template <int NCT, bool CO, bool A16 = false>
__device__ __forceinline__ void down_unit(const DownArgs& a, const uint8_t* wd, const float* sd, int ldk, const uint8_t* hq,
                          const float* hs, const ChunkRows& cr, int j, int kp, uint16_t* d, float* pd,
                          int rot, const ReadyWait& ready, uint8_t* ring) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kofs = 16 * (lane >> 4);
  const int nkb = ldk / kBlock, nkbp = nkb / a.ks, kb0 = kp * nkbp;
  Operands<2, NCT, 1> op;
#pragma unroll
  for (int r = 0; r < 2; ++r) op.a[r] = wd + (size_t)(32 * w + 16 * r) * ldk + (size_t)kb0 * kBlock;
  op.lda = ldk;
  op.spare = a.spare;
  op.sw[0] = sd + kb0;
  int orow[NCT];  // the h (and d) row of each column
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = min(16 * c + (lane & 15), cr.n - 1);
    orow[c] = out_row(cr, r);
    if constexpr (A16) {
      op.b[c] = hq + ((size_t)orow[c] * ldk + (size_t)kb0 * kBlock) * 2 + 2 * kofs;
      op.sx[c] = nullptr;
    } else {
      op.b[c] = hq + (size_t)orow[c] * ldk + (size_t)kb0 * kBlock + kofs;
      op.sx[c] = hs + (size_t)orow[c] * scale_ld(nkb) + kb0;
    }
  }
  f32x4 acc[2][NCT];
  if constexpr (A16) {
    static_assert(NCT <= 2, "W8A16 chunks hold at most 32 rows");
    stream_gemm<2, NCT, 1, 4, true>(op, nkbp, rot, ring, acc, ready);
  } else if constexpr (NCT == 4) {
    // DMA sources of this wave's column tile: lane l moves chunk (l % 8) ^ (l / 8) of row
    // 8i + l / 8 (clamped to the chunk's rows), as the weight tiles.
    const int lr = lane >> 3;
    const uint8_t* xrow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      xrow[i] = hq + (size_t)out_row(cr, min(16 * w + 8 * i + lr, cr.n - 1)) * ldk + (size_t)kb0 * kBlock +
                (((lane & 7) ^ lr) << 4);
    stream_gemm_shared(op, xrow, nkbp, rot, ring, acc, ready);
  } else {
    stream_gemm<2, NCT, 1, 4>(op, nkbp, rot, ring, acc, ready);
  }
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = 16 * c + (lane & 15);
    if (r < cr.n) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const size_t o = (size_t)orow[c] * a.H + (size_t)j * kBlock + 32 * w + 16 * p + 4 * (lane >> 4);
        // Device-coherent stores: the combine (a later kernel, or a later unit of the
        // single-launch kernel on another XCD) reads them.
        if (a.ks == 1) {
          const uint32_t lo = f32_to_bf16_bits(acc[p][c][0]) | (f32_to_bf16_bits(acc[p][c][1]) << 16);
          const uint32_t hi = f32_to_bf16_bits(acc[p][c][2]) | (f32_to_bf16_bits(acc[p][c][3]) << 16);
          store_out<CO>(reinterpret_cast<uint64_t*>(d + o), (uint64_t)lo | ((uint64_t)hi << 32));
        } else {
          uint64_t* q = reinterpret_cast<uint64_t*>(pd + o);
          store_out<CO>(q, (uint64_t)__float_as_uint(acc[p][c][0]) | ((uint64_t)__float_as_uint(acc[p][c][1]) << 32));
          store_out<CO>(q + 1, (uint64_t)__float_as_uint(acc[p][c][2]) | ((uint64_t)__float_as_uint(acc[p][c][3]) << 32));
        }
      }
    }
  }
}

// Down unit v of the work list: chunk v / (nbH*ks), then 128-row block j of the down
// matrix and K part kp (v % (nbH*ks) = j*ks + kp).
// In the dense schedule, `known`: the routing is known (the unit works its expert's routed
// rows; else every token).
template <bool CO, bool A16 = false>
__device__ __forceinline__ void down_work(const DownArgs& a, int v, const ReadyWait& ready, uint8_t* ring,
                                          bool known = true) {
  const int nbH = a.H / kBlock, nbI = a.I / kBlock;
  const int c = v / (nbH * a.ks);
  const int4 ch = a.dense ? dense_dn_chunk(c, a.E, a.S, a.T) : a.chunks[c];
  const int rem = v % (nbH * a.ks), j = rem / a.ks, kp = rem % a.ks;
  const int rot = v % (nbI / a.ks);  // concurrent units start at different K blocks
  float* pd_s = a.p_s + (size_t)kp * a.T * a.H;
  float* pd_r = a.p_r + (size_t)kp * a.rows_r * a.H;
  if (ch.x == a.E) {
    const int ldk = a.S * a.I;
    const ChunkRows cr{ch.z, ch.y, nullptr, a.K};
    const uint8_t* wd = a.sdown + (size_t)j * kBlock * ldk;
    const float* sd = a.sdown_scale + (size_t)j * (ldk / kBlock);
    if constexpr (A16) {
      const uint8_t* h = reinterpret_cast<const uint8_t*>(a.h16_s);
      if (cr.n <= 16)
        down_unit<1, CO, true>(a, wd, sd, ldk, h, nullptr, cr, j, kp, a.d_s, pd_s, rot, ready, ring);
      else
        down_unit<2, CO, true>(a, wd, sd, ldk, h, nullptr, cr, j, kp, a.d_s, pd_s, rot, ready, ring);
      return;
    }
    if (cr.n <= 16)
      down_unit<1, CO>(a, wd, sd, ldk, a.hq_s, a.hs_s, cr, j, kp, a.d_s, pd_s, rot, ready, ring);
    else if (cr.n <= 32)
      down_unit<2, CO>(a, wd, sd, ldk, a.hq_s, a.hs_s, cr, j, kp, a.d_s, pd_s, rot, ready, ring);
    else
      down_unit<4, CO>(a, wd, sd, ldk, a.hq_s, a.hs_s, cr, j, kp, a.d_s, pd_s, rot, ready, ring);
  } else {
    const ChunkRows cr = !a.dense ? ChunkRows{ch.z, ch.y, a.perm, a.K}
                                  : (known ? routed_rows(ch.x, a.T, a.K, a.offsets, a.perm)
                                           : dense_rows(ch.x, a.T, a.K));
    const size_t rowblk = (size_t)ch.x * nbH + j;
    const uint8_t* wd = a.down + rowblk * kBlock * a.I;
    const float* sd = a.down_scale + rowblk * nbI;
    if constexpr (A16) {
      const uint8_t* h = reinterpret_cast<const uint8_t*>(a.h16_r);
      if (cr.n <= 16)
        down_unit<1, CO, true>(a, wd, sd, a.I, h, nullptr, cr, j, kp, a.d_r, pd_r, rot, ready, ring);
      else
        down_unit<2, CO, true>(a, wd, sd, a.I, h, nullptr, cr, j, kp, a.d_r, pd_r, rot, ready, ring);
      return;
    }
    if (cr.n <= 16)
      down_unit<1, CO>(a, wd, sd, a.I, a.hq_r, a.hs_r, cr, j, kp, a.d_r, pd_r, rot, ready, ring);
    else if (cr.n <= 32)
      down_unit<2, CO>(a, wd, sd, a.I, a.hq_r, a.hs_r, cr, j, kp, a.d_r, pd_r, rot, ready, ring);
    else
      down_unit<4, CO>(a, wd, sd, a.I, a.hq_r, a.hs_r, cr, j, kp, a.d_r, pd_r, rot, ready, ring);
  }
}

// y[t, h0 .. h0+7] = bf16( sum_slot fp32(d[t,slot]) * w[t,slot]  (slot order, each product
//                          rounded) + fp32(shared[t]) )          frontier.py:349-354
//
// Slots are worked eight at a time: their rows (inv) and weights first (SlotRows; the
// single-launch kernel loads them before it waits for the down units, since the permute and
// the routing wrote them), then every d load of the eight at once.
struct SlotRows {
  int row[8];
  float w[8];
};

// Where slot s of token t left its d row: row inv[t*K + s] of the grouped rows, or in the
// dense schedule (dense_t = T > 0) row ids[t*K + s] * T + t, its expert's row of the token.
struct SlotMap {
  const int* inv;
  const int64_t* ids;
  int dense_t;
};

__device__ __forceinline__ void load_slots(const SlotMap& m, const float* __restrict__ wts, int K, int t, int s0,
                                           SlotRows& r) {
  if (m.dense_t) {
#pragma unroll
    for (int u = 0; u < 8; ++u) r.row[u] = (int)m.ids[t * K + min(s0 + u, K - 1)] * m.dense_t + t;
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) r.row[u] = m.inv[t * K + min(s0 + u, K - 1)];  // clamped, unconditional loads
  }
#pragma unroll
  for (int u = 0; u < 8; ++u)
    r.w[u] = wts ? wts[t * K + min(s0 + u, K - 1)] : 1.0f;  // no weights: already applied (the MXFP4 form)
}

__device__ __forceinline__ void combine8(const uint16_t* __restrict__ d_r, const uint16_t* __restrict__ d_s,
                                         const SlotMap& inv, const float* __restrict__ wts, int H, int K,
                                         int S, int t, int h0, float (&acc)[8], const SlotRows& first, bool use_first) {
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int s0 = 0; s0 < K; s0 += 8) {
    SlotRows r;
    if (s0 == 0 && use_first)
      r = first;
    else
      load_slots(inv, wts, K, t, s0, r);
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const uint4*>(d_r + (size_t)r.row[u] * H + h0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (s0 + u < K) {
        const uint32_t q[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(bf16_bits_to_f32(q[i] & 0xffffu), r.w[u]));
          acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(bf16_bits_to_f32(q[i] >> 16), r.w[u]));
        }
      }
    }
  }
  if (S > 0) {
    const uint4 v = *reinterpret_cast<const uint4*>(d_s + (size_t)t * H + h0);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = __fadd_rn(acc[2 * i], bf16_bits_to_f32(q[i] & 0xffffu));
      acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], bf16_bits_to_f32(q[i] >> 16));
    }
  }
}

// d = bf16(the sum of the KS fp32 parts of a row, in part order) for the 8 outputs at `src`
// (parts `part` floats apart): every part's load is issued before the first add.
template <int KS>
__device__ __forceinline__ void sum_parts8(const float* __restrict__ src, size_t part, float (&dv)[8]) {
  f32x4 lo[KS], hi[KS];
#pragma unroll
  for (int kp = 0; kp < KS; ++kp) {
    lo[kp] = *reinterpret_cast<const f32x4*>(src + kp * part);
    hi[kp] = *reinterpret_cast<const f32x4*>(src + kp * part + 4);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) dv[i] = 0.0f;
#pragma unroll
  for (int kp = 0; kp < KS; ++kp) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dv[i] = __fadd_rn(dv[i], lo[kp][i]);
      dv[4 + i] = __fadd_rn(dv[4 + i], hi[kp][i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) dv[i] = round_bf16(dv[i]);
}

__device__ __forceinline__ void sum_parts8(const float* __restrict__ src, size_t part, int ks, float (&dv)[8]) {
  if (ks == 2)
    sum_parts8<2>(src, part, dv);
  else if (ks == 4)
    sum_parts8<4>(src, part, dv);
  else
    sum_parts8<8>(src, part, dv);  // down_splits gives 2, 4 or 8 parts when it splits
}

// The same combine when the down GEMMs were split over ks K parts: d = bf16(sum of the
// fp32 parts in part order) for every slot row and for the shared row, then as combine8.
__device__ __forceinline__ void combine8_parts(const float* __restrict__ p_r, const float* __restrict__ p_s, int ks,
                                               const SlotMap& inv, const float* __restrict__ wts, int T,
                                               int rows_r, int H, int K, int S, int t, int h0, float (&acc)[8],
                                               const SlotRows& first, bool use_first) {
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int s0 = 0; s0 < K; s0 += 8) {
    SlotRows r;
    if (s0 == 0 && use_first)
      r = first;
    else
      load_slots(inv, wts, K, t, s0, r);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (s0 + u < K) {
        float dv[8];
        sum_parts8(p_r + (size_t)r.row[u] * H + h0, (size_t)rows_r * H, ks, dv);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(dv[i], r.w[u]));
      }
    }
  }
  if (S > 0) {
    float dv[8];
    sum_parts8(p_s + (size_t)t * H + h0, (size_t)T * H, ks, dv);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __fadd_rn(acc[i], dv[i]);
  }
}

// If a readiness wait of the expert kernel gave up, every element of y is NaN. With a
// residual (the block form), y = bf16(residual + bf16(layer output)) (frontier.py:354).
__global__ __launch_bounds__(256) void k_combine(const uint16_t* __restrict__ d_r, const uint16_t* __restrict__ d_s,
                                                 const float* __restrict__ p_r, const float* __restrict__ p_s, int ks,
                                                 SlotMap inv, int rows_r, const float* __restrict__ wts, int T,
                                                 int H, int K, int S, const int* __restrict__ meta,
                                                 const uint16_t* __restrict__ residual, uint16_t* __restrict__ y,
                                                 int* __restrict__ status) {
  const int i = blockIdx.x * 256 + threadIdx.x, per_row = H / 8;
  if (status && i == 0) *status = meta[kMetaError];  // the call's outcome, kept after it
  if (i >= T * per_row) return;
  if (meta[kMetaError]) {
    *reinterpret_cast<uint4*>(y + (size_t)i * 8) = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
    return;
  }
  const int t = i / per_row, h0 = (i % per_row) * 8;
  float acc[8];
  if (ks > 1)
    combine8_parts(p_r, p_s, ks, inv, wts, T, rows_r, H, K, S, t, h0, acc, SlotRows{}, false);
  else
    combine8(d_r, d_s, inv, wts, H, K, S, t, h0, acc, SlotRows{}, false);
  uint32_t o[4];
  if (residual) {
    const uint4 v = *reinterpret_cast<const uint4*>(residual + (size_t)t * H + h0);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = __fadd_rn(bf16_bits_to_f32(q[j] & 0xffffu), round_bf16(acc[2 * j]));
      const float hi = __fadd_rn(bf16_bits_to_f32(q[j] >> 16), round_bf16(acc[2 * j + 1]));
      o[j] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16_bits(acc[2 * j]) | (f32_to_bf16_bits(acc[2 * j + 1]) << 16);
  }
  *reinterpret_cast<uint4*>(y + (size_t)t * H + h0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// ---------------------------------------------------------------------------------------
// The expert stage as one persistent kernel. One work queue lists every gate/up unit,
// then every down unit; each workgroup claims its units from the queue, so workgroups
// that run out of gate/up work go straight on to down units instead of idling through
// the gate/up tail.
//
// A down unit of chunk c needs the h rows of chunk c, i.e. every gate/up unit of the
// chunk: ready[c] counts them (nbI per routed chunk, S*nbI for the shared expert), and
// the down unit's workgroup waits for the count after requesting its first weight
// stages (the weights do not depend on it). Every gate/up unit precedes every down unit
// in the queue, so when a down unit is claimed, each unit it waits for has been claimed
// by a workgroup that is running it (gate/up units wait for nothing): the wait ends
// however many workgroups are resident. It is also bounded in time. The combine runs
// as its own small kernel after this one.
// ---------------------------------------------------------------------------------------


struct ExpertArgs {
  GateUpArgs gu;
  DownArgs dn;
  const int* dn_of_gu;  // gate/up chunk -> down chunk
  int* ready;           // [down chunks, stride ready_stride] finished gate/up units
  int ready_stride;
  int pad_;
};

// SPLIT: each 128-row block of gate/up is worked as two units, gate and up, and the one
// that finishes second forms h (gateup_half); otherwise one unit multiplies both
// (gateup_unit). The two give the same bits; the host picks one from the geometry.
// A16: the W8A16 form (bf16 activations and h; whole-block gate/up units, chunks of at most
// 32 rows).
template <bool SPLIT, bool A16 = false>
__global__ __launch_bounds__(256, 2) void k_experts(ExpertArgs args) {
  typedef const __attribute__((address_space(4))) ExpertArgs* ArgsPtr;
  __shared__ float red[4][64];
  __shared__ __attribute__((aligned(16))) uint8_t rings[4 * kRingWave];  // one weight ring per wavefront
  __shared__ int slot, flag;
  static_assert(sizeof(ExpertArgs) % 8 == 0, "argument segment layout");
  int* meta = args.gu.meta;
  // The dense schedule's lists come from the geometry (the permute has run: its counts say
  // which experts no token picked, and their units are skipped).
  const bool dense = args.gu.dense != 0;
  const int nbI0 = args.gu.I / kBlock, sh = args.gu.S > 0 ? 1 : 0;
  const int total_gu = dense ? (args.gu.S + args.gu.E) * nbI0 : (SPLIT ? 2 : 1) * meta[kMetaUnitsGU];
  const int total = total_gu + (dense ? (args.gu.E + sh) * (args.dn.H / kBlock) * args.dn.ks : meta[kMetaUnitsDN]);
  // Every unit, the first included, is claimed from the queue: a unit that a down unit
  // waits for is then always held by a running workgroup (one that has not started yet
  // holds nothing), whatever number of workgroups the device keeps resident.
  if (threadIdx.x == 0) slot = atomicAdd(&meta[kMetaQueueGU], 1);
  __syncthreads();
  int u = slot;
  while (u < total) {
    // The arguments are re-read from the kernel argument segment (where `args`, the only
    // argument, sits at offset 0) through a pointer behind an empty asm, so each unit
    // derives its addresses afresh instead of every path's values being hoisted out of
    // this loop and held (or spilled) across it.
    ArgsPtr ap = (ArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    ExpertArgs a;
    __builtin_memcpy(&a, (const ExpertArgs*)ap, sizeof(a));
    const int nbI = a.gu.I / kBlock, nbH = a.dn.H / kBlock;
    uint8_t* ring = rings + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * kRingWave;
    __syncthreads();
    // Thread 0 claims the next unit inside this unit's weight stream (issue_claim) and hands
    // it out after this unit; a unit that streams nothing claims at its end. A workgroup on
    // a down unit can only hold later (down) units this way, so no gate/up unit waits behind
    // a waiting workgroup.
    int ticket = -1;
    if (u < total_gu) {
      bool done = true;
      if constexpr (SPLIT) {
        done = gateup_work_split(a.gu, u, red, &flag, ring,
                                 claiming(ReadyWait{nullptr, 0, nullptr}, &meta[kMetaQueueGU], &ticket));
      } else {
        const int c = u / nbI;
        if (!(dense && c >= a.gu.S && a.gu.offsets[c - a.gu.S + 1] == a.gu.offsets[c - a.gu.S]))
          gateup_work<A16>(a.gu, u, red, ring,
                           claiming(ReadyWait{nullptr, 0, nullptr}, &meta[kMetaQueueGU], &ticket));
      }
      if (done) {
        publish_fence();
        __syncthreads();
        const int dc = dense ? dense_dn_of_gu(u / nbI, a.gu.S) : a.dn_of_gu[(SPLIT ? u >> 1 : u) / nbI];
        if (threadIdx.x == 0) atomicAdd(&a.ready[(size_t)dc * a.ready_stride], 1);
      }
    } else {
      const int v = u - total_gu, c = v / (nbH * a.dn.ks), e = c - (a.dn.S > 0 ? 1 : 0);
      if (!(dense && e >= 0 && a.gu.offsets[e + 1] == a.gu.offsets[e])) {
        const int need = dense ? dense_dn_need(c, a.dn.S, nbI) : (a.dn.chunks[c].x == a.dn.E ? a.dn.S * nbI : nbI);
        down_work<false, A16>(a.dn, v,
                              claiming(ReadyWait{&a.ready[(size_t)c * a.ready_stride], need, &meta[kMetaError]},
                                       &meta[kMetaQueueGU], &ticket),
                              ring);
      }
    }
    if (threadIdx.x == 0) slot = ticket >= 0 ? ticket : claim_ticket(&meta[kMetaQueueGU]);
    __syncthreads();
    u = slot;
  }
}

// =======================================================================================
// The whole layer as one launch (megamoe_layer_forward). One persistent kernel drains one
// queue whose order is the layer's dependency order:
//
//   norm units     one per token row (block form only): RMSNorm of x into the workspace
//   router units   the router tiles of k_router (expert tile, split of H, token pass)
//   select units   one per token: quantize the token's row of x (it needs nothing), wait
//                  for every router unit, then sum the partials and route the token as
//                  k_select does; the select unit that finishes last runs the permute
//                  (histogram, scan, permutation, work lists) in its own workgroup
//   expert units   the gate/up and down units of k_experts, from the permute's lists
//   combine units  2048 outputs each, once every down unit is done
//
// A unit waits only for units earlier in the queue, each of which was claimed by a
// workgroup that is running it, so every wait ends whatever number of workgroups the
// device keeps resident (waits are also bounded in time, as in k_experts; a wait that
// gives up sets the error word and the combine writes NaN). The hand-overs between units
// follow k_experts' rule: data crosses workgroups as device-coherent stores, is published
// by a counter raised after the stores completed, and no workgroup reads a line before
// its last write. The waits on a whole phase (norm, router, permute, down units) poll the
// spread flags of a signal instead of the counter itself (see kSigLines).
//
// The control words (queue, counters, flags, error) must be zero when a call starts: the
// workspace is zeroed once when it is allocated, and the last workgroup to leave a call
// zeroes them again, so a call is exactly one launch.
// =======================================================================================

// kCtlStatus is not zeroed: it keeps the last call's outcome (1: a bounded wait gave up and y
// is NaN) for megamoe_layer_status; the stream-ordered form's combine writes it too.
constexpr int kCtlQueue = 0, kCtlNormed = 32, kCtlRouted = 64, kCtlSelected = 96, kCtlQuant = 128, kCtlDown = 160,
              kCtlExited = 192, kCtlError = 224, kCtlStatus = 256;  // one 128-byte line each
constexpr int kCombineUnit = 256 * 8;  // outputs per combine unit

// Signals: "every norm unit is done", "every router unit is done", "the work lists are
// written", "every down unit is done", "every row of x is quantized" (the dense schedule's
// gate/up units wait for it). Hundreds of workgroups wait on each at once. Polled
// through one word, the waits slowed the workgroups still working by up to 3x (the last
// DeepSeek-V3 down units took 37-55 us instead of 12-16; measured per unit): every poll is a
// device-coherent load at the one memory line that holds the word, which every weight stream
// crosses too. So a signal is kSigLines flag words on lines of their own (4352 bytes apart,
// which differ in the low and the high address bits that pick a cache and memory channel):
// the workgroup whose increment completes a count raises all of them, and each waiting
// workgroup polls the one its index picks.
constexpr int kSigNormed = 0, kSigRouted = 1, kSigPermuted = 2, kSigDown = 3, kSigQuant = 4, kSignals = 5;
constexpr int kSigLines = 16, kSigStride = (4096 + 256) / 4;  // flags per signal; ints between flags
constexpr int kCtlSig = 512;                                  // the first flag
// Start flags of the router units that workgroups take by index (LayerArgs::n_first), one
// per 128-byte line: 0 not started, 1 taken by its workgroup, 2 taken by a rescuing one.
constexpr int kStartStride = 32, kMaxStartUnits = 1024;
constexpr int kCtlStart = kCtlSig + kSignals * kSigLines * kSigStride;
constexpr int kCtlInts = kCtlStart + kMaxStartUnits * kStartStride;

struct LayerArgs {
  ExpertArgs ex;
  const uint16_t* x_in;     // the layer's (or block's) input x [T, H]
  const uint16_t* x;        // the rows the router and the experts read: x_in, or the normalized rows
  const uint16_t* norm_w;   // bf16 gamma [H]; NULL: no normalization
  uint16_t* xn;             // normalized rows [T, H] (workspace)
  const float* router;
  const float* bias;
  double* partial;
  int64_t* ids;
  float* wts;
  uint8_t* xq;
  float* xs;
  PermuteOut po;
  uint16_t* y;
  const uint16_t* residual;  // NULL: no residual add
  int* ctl;
  float eps, scaling;
  int weight_in_fp32;
  int T, H, E, K, S, G, TG, gate, renorm, pow2;
  int nsplit, n_et, ntt, vpl, ks;
  int n_norm, n_router;
  int force_timeout;  // test hook: the combine units wait for a flag value never raised, 20 us at most
  int n_first;        // router units [0, n_first) go to the workgroup of the same index (0: none)
  int force_rescue;   // test hook: odd workgroups leave their router unit to the routing units
  int dense;          // the dense schedule (host: dense_experts); ex.ready then points at counters
                      // of this kernel's own, zeroed by the last workgroup of each call
  int n_ready;        // dense: readiness counters to zero at the end (down chunks)
  int pad_;
};

__device__ __forceinline__ int* signal_flag(int* ctl, int sig, int line) {
  return ctl + kCtlSig + (sig * kSigLines + line) * kSigStride;
}

// The flag of signal `sig` this workgroup polls (workgroups are dealt to the 8 XCDs in turn,
// so the bits above the lowest three spread each XCD's waiters over the lines).
__device__ __forceinline__ int* my_signal_flag(int* ctl, int sig) {
  return signal_flag(ctl, sig, (blockIdx.x >> 3) & (kSigLines - 1));
}

// Raises signal `sig`, by the workgroup whose count increment completed it (after the atomic
// returned, so every unit's stores, completed before its own increment, are in memory).
__device__ __forceinline__ void raise_signal(int* ctl, int sig) {
  if (threadIdx.x < kSigLines)
    __hip_atomic_store(signal_flag(ctl, sig, threadIdx.x), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0 waits (bounded in time) until this workgroup's flag of `sig` reaches `need` (1;
// more only for the timeout test hook), then the workgroup passes a barrier; the acquire
// keeps the loads that follow below it.
__device__ __forceinline__ void wait_signal(int* ctl, int sig, int need = 1, uint64_t ticks = kWaitTicks) {
  wait_ready(ReadyWait{my_signal_flag(ctl, sig), need, &ctl[kCtlError], ticks, true});
}

__device__ __forceinline__ int load_count(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// After a unit's stores: they complete, then thread 0 adds `add` to ctl[word]; the
// workgroup whose addition brings it to `need` raises `sig` (if sig >= 0). Returns the
// count before the addition (in every thread).
__device__ __forceinline__ int publish_count(int* ctl, int word, int add, int need, int sig, int* old_lds) {
  publish_fence();
  __syncthreads();
  if (threadIdx.x == 0) *old_lds = atomicAdd(&ctl[word], add);
  __syncthreads();
  const int old = *old_lds;
  if (sig >= 0 && old + add == need) raise_signal(ctl, sig);
  return old;
}

template <int NTT>
__device__ __forceinline__ void layer_router(const LayerArgs& a, int unit, uint8_t* lds) {
  router_tile<NTT, true>(a.x, a.router, a.partial, a.T, a.H, a.E, a.n_et, a.nsplit, unit,
                         reinterpret_cast<f64x4*>(lds));
}

__device__ __forceinline__ void layer_router_unit(const LayerArgs& a, int r, uint8_t* lds) {
  if (a.ntt == 1)
    layer_router<1>(a, r, lds);
  else if (a.ntt == 2)
    layer_router<2>(a, r, lds);
  else
    layer_router<4>(a, r, lds);
}

// A routing unit waits this long for the router signal before it looks for router units
// that were never started (see rescue_router_unit): 100 us, several times the router phase
// of any config, so with every workgroup resident it never looks.
constexpr uint64_t kRescueTicks = 10000;

// Thread 0 polls signal `sig` for at most `ticks` (as wait_ready, without giving up for the
// call); returns, in every thread, whether it came. When it did, the acquire after the
// barrier keeps the loads that follow below it.
__device__ __forceinline__ bool wait_signal_for(int* ctl, int sig, uint64_t ticks, int* lds) {
  if (threadIdx.x == 0) {
    const int* f = my_signal_flag(ctl, sig);
    const uint64_t t0 = wall_clock64();
    int came = 0, naps = 1;
    while (!(came = load_count(f) != 0) && wall_clock64() - t0 < ticks) {
      for (int k = 0; k < naps; ++k) __builtin_amdgcn_s_sleep(16);
      naps = naps < 2 ? 2 * naps : 2;
    }
    *lds = came;
  }
  __syncthreads();
  acquire_after_wait();
  const bool came = *lds != 0;
  __syncthreads();
  return came;
}

// Takes (start flag 0 -> 2) the lowest router unit in [0, n_first) whose workgroup has not
// started it, for this workgroup to run; -1 if every one has started. In every thread.
__device__ __forceinline__ int rescue_router_unit(int n_first, int* ctl, int* lds) {
  for (;;) {
    if (threadIdx.x == 0) lds[0] = n_first;
    __syncthreads();
    for (int b = threadIdx.x; b < n_first; b += 256)
      if (load_count(&ctl[kCtlStart + b * kStartStride]) == 0) atomicMin(&lds[0], b);
    __syncthreads();
    const int b = lds[0];
    if (b == n_first) return -1;
    if (threadIdx.x == 0) lds[1] = atomicCAS(&ctl[kCtlStart + b * kStartStride], 0, 2) == 0;
    __syncthreads();
    if (lds[1]) return b;
  }
}

template <int VPL>
__device__ __forceinline__ void layer_select(const LayerArgs& a, int token, uint8_t* lds) {
  select_token<VPL, true>(a.partial, a.nsplit, nullptr, a.bias, a.T, a.E, a.K, a.G, a.TG, a.gate, a.renorm, a.scaling,
                    a.ids, a.wts, token, *reinterpret_cast<SelectLds*>(lds));
}

// Where the combine finds each slot's d row: the permute's inverse, or in the dense schedule
// the row of the slot's expert for the token.
__device__ __forceinline__ SlotMap layer_slots(const LayerArgs& a) {
  return a.dense ? SlotMap{nullptr, a.ids, a.T} : SlotMap{a.po.inv, nullptr, 0};
}

// Combine unit c: outputs [c * kCombineUnit, +kCombineUnit) of y, as k_combine (with
// `use_first`, `first` holds the thread's first eight slots, loaded already). The slots pass by
// value: behind a pointer that may be null they were kept in scratch memory.
__device__ __forceinline__ void layer_combine(const LayerArgs& a, int c, const SlotRows& first, bool use_first) {
  const DownArgs& dn = a.ex.dn;
  const int i = c * (kCombineUnit / 8) + threadIdx.x, per_row = a.H / 8;
  if (i >= a.T * per_row) return;
  if (load_count(&a.ctl[kCtlError])) {
    *reinterpret_cast<uint4*>(a.y + (size_t)i * 8) = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
    return;
  }
  const int t = i / per_row, h0 = (i % per_row) * 8;
  float acc[8];
  const SlotMap m = layer_slots(a);
  if (a.ks > 1)
    combine8_parts(dn.p_r, dn.p_s, a.ks, m, a.wts, a.T, dn.rows_r, a.H, a.K, a.S, t, h0, acc, first, use_first);
  else
    combine8(dn.d_r, dn.d_s, m, a.wts, a.H, a.K, a.S, t, h0, acc, first, use_first);
  uint32_t o[4];
  if (a.residual) {
    const uint4 v = *reinterpret_cast<const uint4*>(a.residual + (size_t)t * a.H + h0);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = __fadd_rn(bf16_bits_to_f32(q[j] & 0xffffu), round_bf16(acc[2 * j]));
      const float hi = __fadd_rn(bf16_bits_to_f32(q[j] >> 16), round_bf16(acc[2 * j + 1]));
      o[j] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16_bits(acc[2 * j]) | (f32_to_bf16_bits(acc[2 * j + 1]) << 16);
  }
  *reinterpret_cast<uint4*>(a.y + (size_t)t * a.H + h0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// While the routing units and the permute run, most workgroups only wait for the work lists
// and HBM is mostly idle. The shared expert's weights need no routing: each waiting workgroup
// touches its share of their 128-byte lines (one 4-byte load per line, the values folded and
// kept by an empty asm), so the shared expert's units, which lead the lists, find them in the
// caches (the memory-side cache above all: the lines come from every XCD) instead of HBM.
// Measured (A/B, four runs each): DeepSeek-V3 -2.8 us, GLM-5.3-Flash -6.6, Kimi-K2 -4.3.
__device__ __forceinline__ void touch_shared_weights(const ExpertArgs& ex, int part, int parts) {
  touch_lines<256>(ex.gu.sgate, ex.gu.sup, ex.dn.sdown, (size_t)ex.gu.S * ex.gu.I * ex.gu.H, part, parts);
}

// In every thread, for a unit of routed expert e in the dense schedule: 0, the routing is not
// known yet (the permute's signal has not come): the unit works every token; 1, known and some
// token picked e: the unit works e's routed rows; 2, known and no token picked e: the unit is
// skipped (no combine reads its rows). Thread 0 decides and the workgroup takes its answer
// (the units have barriers, so every wavefront must take the same branch).
__device__ __forceinline__ int dense_state(int* ctl, const int* offsets, int e, int* lds) {
  if (threadIdx.x == 0) {
    int st = 0;
    if (load_count(my_signal_flag(ctl, kSigPermuted)) != 0)
      st = load_count(&offsets[e + 1]) == load_count(&offsets[e]) ? 2 : 1;
    *lds = st;
  }
  __syncthreads();
  acquire_after_wait();
  const int st = *lds;
  __syncthreads();
  return st;
}

// A16: the W8A16 form (bf16 activations into the expert units, chunks of at most 32 rows).
template <bool SPLIT, bool A16 = false>
__global__ __launch_bounds__(256, 2) void k_layer(LayerArgs args) {
  typedef const __attribute__((address_space(4))) LayerArgs* ArgsPtr;
  typedef const __attribute__((address_space(4))) ExpertArgs* ExArgsPtr;
  __shared__ float red[4][64];
  __shared__ __attribute__((aligned(16))) uint8_t rings[4 * kRingWave];  // weight rings; front-end scratch
  __shared__ int slot, flag, flags[2], units[2];
  __shared__ double part[4];
  static_assert(sizeof(LayerArgs) % 8 == 0 && offsetof(LayerArgs, ex) == 0, "argument segment layout");
  static_assert(sizeof(SelectLds) <= sizeof(rings) && (kRouterWaves - 1) * 4 * 64 * sizeof(f64x4) <= sizeof(rings),
                "front-end scratch in the rings");
  int* ctl = args.ctl;
  const int fixed = args.n_norm + args.n_router + args.T;  // units listed before the routing is known
  // Router units [0, n_first) go to the workgroup of the same index, the rest through the
  // queue, whose first entry is unit n_first: 512 workgroups claiming their first unit from
  // one counter at once took ~10 us to be served, and the router phase waited for the last.
  // A workgroup taking unit b by index marks its start flag; if a routing unit took the unit
  // meanwhile (rescue_router_unit: its workgroup had not started in 100 us), this one runs it
  // anyway (same values) but does not count it.
  const int n_first = args.n_first;
  int counts = 1;  // thread 0: whether this workgroup counts its router unit
  if (threadIdx.x == 0) {
    if ((int)blockIdx.x < n_first && !(args.force_rescue && (blockIdx.x & 1))) {
      counts = atomicCAS(&ctl[kCtlStart + blockIdx.x * kStartStride], 0, 1) == 0;
      slot = blockIdx.x;
    } else {
      // The workgroups past the front-end units (with the routed lists) will most likely claim
      // an expert unit, which cannot start before the permute has published the lists (15-60
      // us away), so they claim one after another, ~27 ns apart by index, instead of all at
      // once: hundreds of claims arriving together at the one counter queued for ~5 us, and
      // the router and routing units' own claims and start flags waited behind them (the
      // router phase of a Qwen3-30B-A3B-shaped layer ended at ~9 us instead of ~5). A
      // workgroup that does get a front-end unit runs it as before.
      if (!args.dense && (int)blockIdx.x >= fixed)
        for (int k = (int)blockIdx.x - fixed; k > 0; --k) __builtin_amdgcn_s_sleep(1);
      slot = n_first + atomicAdd(&ctl[kCtlQueue], 1);
    }
  }
  __syncthreads();
  int u = slot, next = 0;
  int resume = -1;  // a routing unit to return to after running a rescued router unit

  // Phase 1: the front-end units (claims only grow, so a workgroup never comes back here).
  // A workgroup claims its next unit only when it has finished this one: the front-end units
  // are short and every routing unit waits for the slowest router unit, so a unit must not be
  // reserved by a busy workgroup while an idle one could start it.
  while (u < fixed) {
    // The arguments are re-read per unit (as in k_experts) so each unit derives its
    // addresses afresh instead of every path's values being held across the loop.
    ArgsPtr ap = (ArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    LayerArgs a;
    __builtin_memcpy(&a, (const LayerArgs*)ap, sizeof(a));
    if (u < a.n_norm) {
      norm_row<true>(a.x_in, a.norm_w, u, a.H, a.eps, a.weight_in_fp32, a.xn, part);
      publish_count(ctl, kCtlNormed, 1, a.n_norm, kSigNormed, &units[0]);
    } else if (u < a.n_norm + a.n_router) {
      if (a.n_norm) wait_signal(ctl, kSigNormed);
      const int r = u - a.n_norm;
      layer_router_unit(a, r, rings);
      // Counted unless a rescuing workgroup took it first (then that one counts it).
      publish_fence();
      __syncthreads();
      if (threadIdx.x == 0) units[0] = counts ? atomicAdd(&ctl[kCtlRouted], 1) : -2;
      if (threadIdx.x == 0) counts = 1;
      __syncthreads();
      if (units[0] == a.n_router - 1) raise_signal(ctl, kSigRouted);
    } else {
      const int t = u - a.n_norm - a.n_router;
      if (a.n_norm) wait_signal(ctl, kSigNormed);
      // This token's row of x in E4M3 per 128 (needs nothing else; runs while the router does).
      const int nbh = a.H / kBlock, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
      const bool back = resume >= 0;  // after a rescued router unit: look again at once
      if (!back) {
        // The W8A16 form quantizes nothing: its experts read the bf16 rows, and the region of
        // the quantized x holds its bf16 h. A write-through store of x there would leave the
        // line in this XCD's L2, where a down unit on the same XCD, reading the h row that a
        // gate/up unit on another XCD wrote later, would find the stale copy.
        if constexpr (!A16)
          quant_row(a.x + (size_t)t * a.H, a.xq + (size_t)t * a.H, a.xs + (size_t)t * nbh, nbh, a.pow2, lane, wv,
                    reinterpret_cast<float*>(rings));
        // The dense schedule's gate/up units read every token's row once all are quantized
        // (W8A16: once every routing unit has passed its wait for the normalized rows).
        if (a.dense) publish_count(ctl, kCtlQuant, 1, a.T, kSigQuant, &units[0]);
      }
      resume = -1;
      bool routed = false;  // the router signal came (and was acquired) in the wait below
      if (n_first) {
        if (!back) routed = wait_signal_for(ctl, kSigRouted, kRescueTicks, flags);
        if (!routed) {
          // A router unit whose workgroup never started: run it (and count it), then come back.
          const int b = rescue_router_unit(n_first, ctl, flags);
          if (b >= 0) {
            resume = u;
            u = a.n_norm + b;
            continue;
          }
        }
      }
      if (!routed) wait_signal(ctl, kSigRouted);
      if (a.vpl == 1)
        layer_select<1>(a, t, rings);
      else if (a.vpl == 2)
        layer_select<2>(a, t, rings);
      else if (a.vpl == 4)
        layer_select<4>(a, t, rings);
      else if (a.vpl == 8)
        layer_select<8>(a, t, rings);
      else
        layer_select<16>(a, t, rings);
      if (publish_count(ctl, kCtlSelected, 1, a.T, -1, &units[0]) == a.T - 1) {
        // Every token is routed: this workgroup runs the permute, then publishes the lists.
        acquire_after_wait();
        permute_block<true>(a.ids, 0, a.T, a.K, a.E, a.S, a.ex.gu.I / kBlock, a.H / kBlock, a.ks,
                            A16 ? kChunkRowsA16 : kChunkRows, 0,
                            a.po, reinterpret_cast<int*>(rings), flags,
                            permute_tile_waves(a.T, a.E, 256, kPermuteLdsInts));
        publish_fence();
        __syncthreads();
        raise_signal(ctl, kSigPermuted);
      }
    }
    if (resume >= 0) {  // back to the routing unit that ran a rescued router unit
      __syncthreads();
      u = resume;
      continue;
    }
    __syncthreads();
    if (threadIdx.x == 0) slot = n_first + atomicAdd(&ctl[kCtlQueue], 1);
    __syncthreads();
    u = slot;
  }

  // Phase 2: the work lists, once the permute has run (its meta words were never read before
  // in this call). If the wait gave up (error word set), the lists are not read: no expert
  // units, only the combine units, which then write NaN. Most workgroups wait here while the
  // routing units and the permute, the critical path, run: their polls back off to ~3.6 us
  // apart (8 naps) instead of ~0.9 (DeepSeek-V3 -1.7 us, Mixtral -2.2, Qwen3-30B-A3B -0.6,
  // Kimi-K2 0, over two A/B runs; 16 naps measured no better).
  // The dense schedule's lists are known from the geometry: no wait (its units wait for the
  // quantized x and for each other instead; the combine for the routing).
  const bool dense = args.dense != 0;
  if (!dense) {
    if (args.ex.gu.S > 0) touch_shared_weights(args.ex, blockIdx.x, gridDim.x);
    wait_ready(ReadyWait{my_signal_flag(ctl, kSigPermuted), 1, &ctl[kCtlError], kWaitTicks, true, 8});
  }
  if (threadIdx.x == 0) {
    const int nbI = args.ex.gu.I / kBlock, S = args.ex.gu.S, E = args.E;
    if (dense) {
      units[0] = (S + E) * nbI;
      units[1] = (E + (S > 0 ? 1 : 0)) * (args.H / kBlock) * args.ks;
    } else {
      const bool lists = load_count(my_signal_flag(ctl, kSigPermuted)) != 0;
      units[0] = lists ? (SPLIT ? 2 : 1) * load_count(&args.po.meta[kMetaUnitsGU]) : 0;
      units[1] = lists ? load_count(&args.po.meta[kMetaUnitsDN]) : 0;
    }
  }
  __syncthreads();
  const int n_gu = units[0], n_dn = units[1];
  const int experts_end = fixed + n_gu + n_dn;
  const int total = experts_end + (args.T * args.H + kCombineUnit - 1) / kCombineUnit;

  // Phase 3: the expert units, as k_experts runs them (its loop, over the permute's lists).
  int my_down = 0;  // down units this workgroup finished and has not yet counted
  while (u < experts_end) {
    ExArgsPtr ap = (ExArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();  // LayerArgs::ex is at offset 0
    asm volatile("" : "+s"(ap));
    ExpertArgs a;
    __builtin_memcpy(&a, (const ExpertArgs*)ap, sizeof(a));
    const int nbI = a.gu.I / kBlock, nbH = a.dn.H / kBlock;
    uint8_t* ring = rings + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * kRingWave;
    __syncthreads();
    // The next unit is claimed inside this unit's weight stream, as in k_experts.
    int ticket = -1;
    int* const queue = &ctl[kCtlQueue];
    if (u < fixed + n_gu) {
      const int g = u - fixed;
      bool done = true;
      if constexpr (SPLIT) {
        done = gateup_work_split(a.gu, g, red, &flag, ring, claiming(ReadyWait{nullptr, 0, nullptr}, queue, &ticket));
      } else if (dense) {
        // Every expert's units from the start: before the routing is known a unit works every
        // token and waits only for the quantized x; after, its expert's routed rows, or
        // nothing if no token picked the expert.
        const int c = g / nbI;
        const int st = c >= a.gu.S ? dense_state(ctl, a.gu.offsets, c - a.gu.S, &flags[0]) : 0;
        if (st != 2)
          gateup_work<A16>(a.gu, g, red, ring,
                           claiming(ReadyWait{my_signal_flag(ctl, kSigQuant), 1, &ctl[kCtlError], kWaitTicks, true, 2},
                                    queue, &ticket),
                           st == 1);
      } else {
        gateup_work<A16>(a.gu, g, red, ring, claiming(ReadyWait{nullptr, 0, nullptr}, queue, &ticket));
      }
      if (done) {
        publish_fence();
        __syncthreads();
        const int dc = dense ? dense_dn_of_gu(g / nbI, a.gu.S) : a.dn_of_gu[(SPLIT ? g >> 1 : g) / nbI];
        if (threadIdx.x == 0) atomicAdd(&a.ready[(size_t)dc * a.ready_stride], 1);
      }
    } else {
      const int v = u - fixed - n_gu, c = v / (nbH * a.dn.ks);
      const int sh = a.dn.S > 0 ? 1 : 0;
      const int st = dense && c >= sh ? dense_state(ctl, a.gu.offsets, c - sh, &flags[0]) : 0;
      if (st != 2) {
        const int need = dense ? dense_dn_need(c, a.dn.S, nbI) : (a.dn.chunks[c].x == a.dn.E ? a.dn.S * nbI : nbI);
        down_work<true, A16>(a.dn, v,
                             claiming(ReadyWait{&a.ready[(size_t)c * a.ready_stride], need, &ctl[kCtlError]}, queue,
                                      &ticket),
                             ring, st == 1);
      }
      ++my_down;
    }
    if (threadIdx.x == 0) slot = n_first + (ticket >= 0 ? ticket : claim_ticket(queue));
    __syncthreads();
    u = slot;
  }
  // Down units are counted once per workgroup, when it moves past them: their d rows (device-
  // coherent stores) complete first. (An agent-scope release after plain stores instead
  // writes back the XCD's whole L2, once per workgroup: measured far slower.) The workgroup
  // whose count completes the down units raises the signal the combine units wait for.
  if (my_down) publish_count(ctl, kCtlDown, my_down, n_dn, kSigDown, &units[0]);

  // Phase 4: the combine units, once every down unit is counted (no down units: the lists
  // were not written, the error word is set and the combine writes NaN).
  if (u < total) {
    ArgsPtr ap = (ArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    LayerArgs a;
    __builtin_memcpy(&a, (const LayerArgs*)ap, sizeof(a));
    // The first unit's slot rows and weights (written before the lists were published) load
    // while the down units finish. The dense schedule's expert units did not wait for the
    // routing: the combine does.
    if (a.dense) wait_signal(ctl, kSigPermuted);
    SlotRows first;
    {
      const int i = (u - experts_end) * (kCombineUnit / 8) + threadIdx.x, per_row = a.H / 8;
      load_slots(layer_slots(a), a.wts, a.K, min(i, a.T * per_row - 1) / per_row, 0, first);
    }
    if (n_dn) wait_signal(ctl, kSigDown, 1 + a.force_timeout, a.force_timeout ? (uint64_t)2000 : kWaitTicks);
    bool use_first = true;
    while (u < total) {
      __syncthreads();
      if (threadIdx.x == 0) next = n_first + claim_ticket(&ctl[kCtlQueue]);
      layer_combine(a, u - experts_end, first, use_first);
      use_first = false;
      if (threadIdx.x == 0) slot = next;
      __syncthreads();
      u = slot;
    }
  }
  // Leaving: the last workgroup out (every other one has finished its last wait and unit)
  // keeps the call's outcome in the status word and zeroes the counters and the signal flags
  // for the next call.
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = atomicAdd(&ctl[kCtlExited], 1) == (int)gridDim.x - 1;
    if (last)
      __hip_atomic_store(&ctl[kCtlStatus], load_count(&ctl[kCtlError]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    slot = last;
  }
  __syncthreads();
  if (slot) {
    constexpr int words[] = {kCtlQueue, kCtlNormed, kCtlRouted, kCtlSelected, kCtlQuant, kCtlDown, kCtlError,
                             kCtlExited};
    constexpr int n_words = sizeof(words) / sizeof(words[0]);
    static_assert(n_words + kSignals * kSigLines <= 256, "one store per thread");
    const int i = threadIdx.x;
    if (i < n_words)
      __hip_atomic_store(&ctl[words[i]], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else if (i < n_words + kSignals * kSigLines)
      __hip_atomic_store(signal_flag(ctl, (i - n_words) / kSigLines, (i - n_words) % kSigLines), 0,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int b = i; b < n_first; b += 256)
      __hip_atomic_store(&ctl[kCtlStart + b * kStartStride], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int c = i; c < args.n_ready; c += 256)  // the dense schedule's readiness counters
      __hip_atomic_store(&args.ex.ready[(size_t)c * args.ex.ready_stride], 0, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

// =======================================================================================
// The MXFP4 form (megamoe.py:116-182, serial): E2M1 expert weights with one E8M0 scale per
// 32 input channels, activations in E4M3 with E8M0 scales per 32, routing as an input.
// gfx950's scaled MFMA takes both formats and both scales natively: in
// v_mfma_scale_f32_16x16x128_f8f6f4 with an E2M1 A operand, lane r + 16g holds row r and
// K elements [32g, 32g+32) in 16 bytes (the even element in the low nibble), so one lane's
// operand is one stored 32-block; the E4M3 B operand keeps the layout of the fp8 form; and
// the E8M0 byte of lane r + 16g scales row (or column) r over K elements [32g, 32g+32)
// (layouts measured on gfx950). Products and power-of-two scales are exact and the MFMA
// sums in fp32, so no scale multiplies follow it.
//
// A ring stage covers 256 K elements: one 128-byte line of each weight row, two MFMAs per
// tile (the first and second 16 bytes of each 32-byte LDS read). The scale bytes of a stage
// come with one 8-byte load per lane and operand row, shifted to the lane's block.
// =======================================================================================

constexpr int kMxStageK = 256;

// Calls f(std::integral_constant<int, I>{}) for I = B .. E-1 (a loop whose index is a
// compile-time constant in the body).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

__device__ __forceinline__ f32x4 mfma_e2m1_e4m3(const i32x4& a, const i32x8& b, f32x4 c, int sa, int sb) {
  const i32x8 a8 = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b, c, 4, 0, 0, sa, 0, sb);
}

// Biased E8M0 exponent that maps `amax` (>= 0) into E4M3: the fp32 exponent, one up where
// the mantissa exceeds 1.75's, less 448's exponent (8), floored at 2^-22 (1e-4 / 448);
// quantization.py:67-78.
__device__ __forceinline__ uint32_t e8m0_exponent(float amax) {
  const int r = (int)((__float_as_uint(amax) + (0x7FFFFFu - 0x600000u)) >> 23);
  return (uint32_t)(max(r, 105 + 8) - 8);
}

template <int RT, int NCT>
struct StageMx {
  i32x8 b[NCT][2];  // activations of the stage's two 128-K steps
  uint2 sb[NCT];    // activation E8M0 bytes [8p, 8p+8) of the lane's token row
  uint2 sa[RT];     // weight E8M0 bytes [8p, 8p+8) of the lane's row in each tile (per-stage loads)
};

template <int RT, int NCT>
struct OperandsMx {
  const uint8_t* a[RT];    // row 0 of each 16-row weight tile (E2M1, lda bytes per row)
  int lda;
  const uint8_t* spare;    // 16 * lda bytes that loads past the last stage read instead
  const uint8_t* sa[RT];   // lane's weight scale row in each tile
  const uint8_t* b[NCT];   // lane's activation row at its K byte offset
  const uint8_t* sb[NCT];  // lane's activation scale row
};

template <int CPOL, int RT, int NCT>
__device__ __forceinline__ void issue_a_mx(uint8_t* slot, const OperandsMx<RT, NCT>& op, const LaneTile& lt, int p,
                                           bool live) {
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const uint8_t* base = live ? op.a[t] + (size_t)p * kBlock : op.spare;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(base +
                                                                                     (uint32_t)(lt.dma + 8 * i * op.lda)),
                                       (__attribute__((address_space(3))) void*)(slot + t * kTileBytes + i * 1024),
                                       16, 0, CPOL);
  }
}

// 4*NCT vector loads, plus NCT + RT for the scales of stage p when SCALES.
template <bool SCALES, int RT, int NCT>
__device__ __forceinline__ void load_stage_mx(StageMx<RT, NCT>& s, const OperandsMx<RT, NCT>& op, int p) {
  const size_t o = (size_t)p * kMxStageK;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    s.b[c][0] = load_k32(op.b[c] + o);
    s.b[c][1] = load_k32(op.b[c] + o + 128);
  }
  if constexpr (SCALES) {
#pragma unroll
    for (int c = 0; c < NCT; ++c) s.sb[c] = *reinterpret_cast<const uint2*>(op.sb[c] + 8 * p);
#pragma unroll
    for (int t = 0; t < RT; ++t) s.sa[t] = *reinterpret_cast<const uint2*>(op.sa[t] + 8 * p);
  }
}

// The weight and activation scales of the stage pair starting at the even stage pa
// (RT + NCT vector loads).
template <int RT, int NCT>
struct PairMx {
  uint4 sa[RT];
  uint4 sb[NCT];
};

template <int RT, int NCT>
__device__ __forceinline__ void load_pair_mx(PairMx<RT, NCT>& q, const OperandsMx<RT, NCT>& op, int pa) {
#pragma unroll
  for (int c = 0; c < NCT; ++c) q.sb[c] = *reinterpret_cast<const uint4*>(op.sb[c] + 8 * pa);
#pragma unroll
  for (int t = 0; t < RT; ++t) q.sa[t] = *reinterpret_cast<const uint4*>(op.sa[t] + 8 * pa);
}

template <int RT>
__device__ __forceinline__ void read_slot_mx(i32x4 (&lo)[RT], i32x4 (&hi)[RT], uint32_t p0, uint32_t p1) {
#pragma unroll
  for (int r = 0; r < RT; ++r)
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3"
                 : "=&v"(lo[r]), "=&v"(hi[r])
                 : "v"(p0 + r * kTileBytes), "v"(p1 + r * kTileBytes)
                 : "memory");
  if constexpr (RT == 2) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo[0]), "+v"(hi[0]), "+v"(lo[1]), "+v"(hi[1]));
  } else {
    static_assert(RT == 4, "two or four row tiles");
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(lo[0]), "+v"(hi[0]), "+v"(lo[1]), "+v"(hi[1]), "+v"(lo[2]), "+v"(hi[2]), "+v"(lo[3]),
                   "+v"(hi[3]));
  }
}

// `shift` = 8 * (lane / 16): the lane's byte in each scale word; `saw` and `sbw` hold the
// weight and activation scale words of the stage. The scale bytes pass an empty asm (as in mfma_stage) so their
// extraction stays after the stage's wait.
template <int RT, int NCT>
__device__ __forceinline__ void mfma_stage_mx(const i32x4 (&lo)[RT], const i32x4 (&hi)[RT], const StageMx<RT, NCT>& s,
                                              const uint2 (&saw)[RT], const uint2 (&sbw)[NCT], int shift,
                                              f32x4 (&acc)[RT][NCT]) {
  int sa0[RT], sa1[RT], sb0[NCT], sb1[NCT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    uint2 w = saw[r];
    asm volatile("" : "+v"(w.x), "+v"(w.y));
    sa0[r] = (int)((w.x >> shift) & 0xffu);
    sa1[r] = (int)((w.y >> shift) & 0xffu);
  }
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    uint2 w = sbw[c];
    asm volatile("" : "+v"(w.x), "+v"(w.y));
    sb0[c] = (int)((w.x >> shift) & 0xffu);
    sb1[c] = (int)((w.y >> shift) & 0xffu);
  }
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < NCT; ++c) acc[r][c] = mfma_e2m1_e4m3(lo[r], s.b[c][0], acc[r][c], sa0[r], sb0[c]);
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < NCT; ++c) acc[r][c] = mfma_e2m1_e4m3(hi[r], s.b[c][1], acc[r][c], sa1[r], sb1[c]);
}

// The fp8 form's stream (D slots, loads in issue order, the spare region for loads past
// the end, a rotated start) over nst stages of 256 K elements. The per-lane scale loads
// touch one line per row (or token) and tile per stage; with PAIR (nst and rot even,
// D = 2) one 16-byte load per lane and tile brings the scales of a stage pair, issued
// with the even stage's loads into one of two pair buffers (stage p reads buffer (p / 2) % 2, so the
// loop is unrolled by four and no register copy crosses the back edge: a copy of loaded
// registers there makes the compiler wait for vmcnt 0). CPOL is the weight loads' cache
// policy: non-temporal where each line is read once, cached where the four wavefronts of a
// wide unit request the same lines.
template <int RT, int NCT, int D, bool PAIR, int CPOL = kNonTemporal>
__device__ __forceinline__ void stream_gemm_mx(const OperandsMx<RT, NCT>& op, int nst, int rot, uint8_t* ring,
                                               f32x4 (&acc)[RT][NCT],
                                               const ReadyWait& ready = ReadyWait{nullptr, 0, nullptr}) {
  constexpr int kSlot = RT * kTileBytes;
  constexpr int U = PAIR ? 4 : D;  // stages per loop trip
  constexpr int kAfter = PAIR ? (D - 1) * (2 * RT + 4 * NCT) : (D - 1) * (3 * RT + 5 * NCT);
  static_assert(D >= 2 && D * kSlot <= kRingWave && kAfter <= 63, "LDS ring and vmcnt range");
  static_assert(!PAIR || D == 2, "paired scale loads use two pair buffers and a two-slot ring");
  auto phys = [nst, rot](int p) {
    const int q = p + rot;
    return q >= nst ? q - nst : q;
  };
  const LaneTile lt = lane_tile(op.lda);
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring;
  const int shift = 8 * (opaque_lane() >> 4);
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < NCT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  StageMx<RT, NCT> st[D];
  PairMx<RT, NCT> pair[2];
  // The loads of stage i (logical index; its parity is a compile-time fact at each call).
  // The pair load's address stays inside the rows: its even stage is at most nst - 2.
  auto load = [&](auto ic, int i) {
    constexpr int c = decltype(ic)::value;  // i modulo U
    const int pi = phys(min(i, nst - 1));
    load_stage_mx<!PAIR>(st[c % D], op, pi);
    if constexpr (PAIR && c % 2 == 0) load_pair_mx(pair[(c / 2) % 2], op, phys(min(i, nst - 2)));
  };
  auto half = [](const uint4& q, auto odd) {
    return decltype(odd)::value ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y);
  };
  auto scales = [&](auto sc, uint2 (&saw)[RT], uint2 (&sbw)[NCT]) {
    constexpr int c = decltype(sc)::value;
    const std::integral_constant<bool, c % 2 == 1> odd{};
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      if constexpr (!PAIR)
        saw[r] = st[c % D].sa[r];
      else
        saw[r] = half(pair[(c / 2) % 2].sa[r], odd);
    }
#pragma unroll
    for (int k = 0; k < NCT; ++k) {
      if constexpr (!PAIR)
        sbw[k] = st[c % D].sb[k];
      else
        sbw[k] = half(pair[(c / 2) % 2].sb[k], odd);
    }
  };
#pragma unroll
  for (int s = 0; s < D - 1; ++s) issue_a_mx<CPOL>(ring + s * kSlot, op, lt, phys(min(s, nst - 1)), s < nst);
  wait_ready(ready);
  static_for<0, D - 1>([&](auto si) { load(si, (int)decltype(si)::value); });
  for (int p0 = 0; p0 < nst; p0 += U) {
    static_for<0, U>([&](auto si) {
      constexpr int s = decltype(si)::value;
      const int p = p0 + s;
      load(std::integral_constant<int, (s + D - 1) % U>{}, p + D - 1);
      issue_a_mx<CPOL>(ring + ((s + D - 1) % D) * kSlot, op, lt, phys(min(p + D - 1, nst - 1)), p + D - 1 < nst);
      wait_vmem<kAfter>();
      if (p < nst) {
        i32x4 lo[RT], hi[RT];
        uint2 saw[RT], sbw[NCT];
        read_slot_mx<RT>(lo, hi, ring_lds + (s % D) * kSlot + lt.rd0, ring_lds + (s % D) * kSlot + lt.rd1);
        scales(si, saw, sbw);
        mfma_stage_mx(lo, hi, st[s % D], saw, sbw, shift, acc);
      }
    });
  }
}

struct GateUpMxArgs {
  const uint8_t* x;    // [T, H] e4m3
  const uint8_t* xs;   // [T, H/32] e8m0
  const float* wts;    // [T*K] routing weights
  const uint8_t* l1;   // [E, 2I, H/2] e2m1 (rows 0..I-1 gate, I..2I-1 up)
  const uint8_t* l1s;  // [E, 2I, H/32] e8m0
  const int* offsets; const int* perm; const int4* chunks;
  int* meta;
  uint8_t* hq;         // [T*K, I] e4m3, grouped rows
  uint8_t* hs;         // [T*K, hs_ld] e8m0 (one 128-byte line per row)
  const uint8_t* spare;
  int T, H, I, K, E, hs_ld;
  int ebase;  // id of expert 0 (a rank's first local expert)
  float limit;
};

// Gate/up unit: rows [jb*128, +128) of the expert's gate and up matrices. Wave w owns
// gate rows 32w .. 32w+31 and the same up rows, i.e. one 32-channel block of h: its E8M0
// requantization needs no reduction across wavefronts.
//   gate, up = bf16(l1); gate = min(gate, limit); up = clamp(up, +-limit)
//   a = gate / (1 + exp(-gate)) * up * w_slot (fp32, megamoe.py:116-122)
//   h = E4M3(a * 2^(127-e)), e = E8M0 exponent of the block's amax (megamoe.py:125-128)
template <int NCT>
__device__ void gateup_mx_epilogue(const GateUpMxArgs& a, int jb, const ChunkRows& cr, const f32x4 (&acc)[4][NCT],
                                   uint8_t (*red8)[64]);

template <int NCT, bool PAIR>
__device__ void gateup_mx_unit(const GateUpMxArgs& a, int e, int jb, const ChunkRows& cr, int rot, uint8_t (*red8)[64],
                               uint8_t* ring) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;
  const int H = a.H, lda = H / 2, sld = H / 32;
  const size_t gate0 = (size_t)e * 2 * a.I + (size_t)jb * kBlock + 32 * w, up0 = gate0 + a.I;
  OperandsMx<4, NCT> op;
  op.lda = lda;
  op.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    op.a[r] = a.l1 + (gate0 + 16 * r) * lda;
    op.a[r + 2] = a.l1 + (up0 + 16 * r) * lda;
    op.sa[r] = a.l1s + (gate0 + 16 * r + lr) * sld;
    op.sa[r + 2] = a.l1s + (up0 + 16 * r + lr) * sld;
  }
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int tok = row_token(cr, min(16 * c + lr, cr.n - 1));
    op.b[c] = a.x + (size_t)tok * H + 16 * (lane >> 4);
    op.sb[c] = a.xs + (size_t)tok * sld;
  }
  f32x4 acc[4][NCT];
  stream_gemm_mx<4, NCT, 2, PAIR>(op, H / kMxStageK, rot, ring, acc);
  gateup_mx_epilogue<NCT>(a, jb, cr, acc, red8);
}

// The epilogue of a 128-channel gate/up unit whose wave w holds gate and up channels
// [32w, 32w + 32) of block jb for column tiles 0 .. NCT-1: SwiGLU, the E8M0 scale of each
// row's 32 channels (within the wavefront), E4M3 h, and the four waves' scale bytes of a
// row gathered into one dword.
template <int NCT>
__device__ void gateup_mx_epilogue(const GateUpMxArgs& a, int jb, const ChunkRows& cr, const f32x4 (&acc)[4][NCT],
                                   uint8_t (*red8)[64]) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;
  const float L = a.limit;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int col = 16 * c + lr;
    const float wrow = a.wts[cr.perm[cr.row0 + min(col, cr.n - 1)]];
    float hv[2][4];
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float g = fminf(round_bf16(acc[p][c][v]), L);
        const float u = fminf(fmaxf(round_bf16(acc[p + 2][c][v]), -L), L);
        const float act = __fmul_rn(__fmul_rn(g / __fadd_rn(1.0f, expf(-g)), u), wrow);
        hv[p][v] = act;
        amax = fmaxf(amax, fabsf(act));
      }
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const uint32_t ex = e8m0_exponent(amax);
    const float inv = __uint_as_float((254u - ex) << 23);
    if (col < cr.n) {
      uint8_t* dst = a.hq + (size_t)(cr.row0 + col) * a.I + (size_t)jb * kBlock + 32 * w + 4 * (lane >> 4);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint32_t packed = e4m3x4(clamp448(__fmul_rn(hv[p][0], inv)), clamp448(__fmul_rn(hv[p][1], inv)),
                                       clamp448(__fmul_rn(hv[p][2], inv)), clamp448(__fmul_rn(hv[p][3], inv)));
        store_coherent(reinterpret_cast<uint32_t*>(dst + 16 * p), packed);
      }
      if (lane < 16) red8[w][col] = (uint8_t)ex;
    }
  }
  __syncthreads();
  if (w == 0) {
    for (int col = lane; col < 16 * NCT && col < cr.n; col += 64) {
      const uint32_t word = red8[0][col] | (red8[1][col] << 8) | (red8[2][col] << 16) | (red8[3][col] << 24);
      store_coherent(reinterpret_cast<uint32_t*>(a.hs + (size_t)(cr.row0 + col) * a.hs_ld + 4 * jb), word);
    }
  }
}

__device__ __forceinline__ void store_coherent_byte(uint8_t* p, uint8_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wide gate/up unit, for a chunk of 33-128 rows: gate rows [32 blk, +32) and the same up
// rows (one 32-channel block of h) for every row of the chunk; wave w takes column tiles
// [w NCT, w NCT + NCT). Every wave streams the same 64 weight rows into its own ring, with
// cached loads so that L2 can serve the four requests for a line; the LDS-DMA requests
// themselves are four times the weight bytes, which bounds these units below the HBM rate.
// A wave past the chunk's last tile streams a copy of it and stores nothing (all waves take
// the same path and barriers).
template <int NCT, bool PAIR>
__device__ void gateup_mx_wide(const GateUpMxArgs& a, int e, int blk, const ChunkRows& cr, int rot, uint8_t* ring) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;
  const int H = a.H, lda = H / 2, sld = H / 32;
  const size_t gate0 = (size_t)e * 2 * a.I + (size_t)blk * 32, up0 = gate0 + a.I;
  OperandsMx<4, NCT> op;
  op.lda = lda;
  op.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    op.a[r] = a.l1 + (gate0 + 16 * r) * lda;
    op.a[r + 2] = a.l1 + (up0 + 16 * r) * lda;
    op.sa[r] = a.l1s + (gate0 + 16 * r + lr) * sld;
    op.sa[r + 2] = a.l1s + (up0 + 16 * r + lr) * sld;
  }
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int tok = row_token(cr, min(16 * (w * NCT + c) + lr, cr.n - 1));
    op.b[c] = a.x + (size_t)tok * H + 16 * (lane >> 4);
    op.sb[c] = a.xs + (size_t)tok * sld;
  }
  f32x4 acc[4][NCT];
  stream_gemm_mx<4, NCT, 2, PAIR, 0>(op, H / kMxStageK, rot, ring, acc);

  const float L = a.limit;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int col = 16 * (w * NCT + c) + lr;
    const float wrow = a.wts[cr.perm[cr.row0 + min(col, cr.n - 1)]];
    float hv[2][4];
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float g = fminf(round_bf16(acc[p][c][v]), L);
        const float u = fminf(fmaxf(round_bf16(acc[p + 2][c][v]), -L), L);
        const float act = __fmul_rn(__fmul_rn(g / __fadd_rn(1.0f, expf(-g)), u), wrow);
        hv[p][v] = act;
        amax = fmaxf(amax, fabsf(act));
      }
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const uint32_t ex = e8m0_exponent(amax);
    const float inv = __uint_as_float((254u - ex) << 23);
    if (col < cr.n) {
      uint8_t* dst = a.hq + (size_t)(cr.row0 + col) * a.I + (size_t)blk * 32 + 4 * (lane >> 4);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint32_t packed = e4m3x4(clamp448(__fmul_rn(hv[p][0], inv)), clamp448(__fmul_rn(hv[p][1], inv)),
                                       clamp448(__fmul_rn(hv[p][2], inv)), clamp448(__fmul_rn(hv[p][3], inv)));
        store_coherent(reinterpret_cast<uint32_t*>(dst + 16 * p), packed);
      }
      if (lane < 16) store_coherent_byte(a.hs + (size_t)(cr.row0 + col) * a.hs_ld + blk, (uint8_t)ex);
    }
  }
}

// Gate/up units: `nwide` wide chunks first (4 nbI units each, one per 32-channel block),
// then narrow chunks (nbI units each). Returns the unit's chunk. CALLER: each kernel
// instantiates its own copy, so the inliner sees one call site per copy (one copy shared by
// k_experts_mx and k_layer_mx compiled k_experts_mx to 256 VGPRs with spills and scratch,
// against 237 and none, and slowed it by 40%).
template <int CALLER>
__device__ int gateup_mx_work(const GateUpMxArgs& a, int u, int nwide, uint8_t (*red8)[64], uint8_t* ring) {
  const int nbI = a.I / kBlock;
  const int nst = a.H / kMxStageK;
  if (u < nwide * 4 * nbI) {
    const int c = u / (4 * nbI), blk = u % (4 * nbI);
    const int4 ch = a.chunks[c];
    const ChunkRows cr{ch.z, ch.y, a.perm, a.K};
    const int key = (ch.x + a.ebase) * nbI + blk / 4;  // as the narrow unit of the same 128 channels
    const bool two = cr.n > 64;
    if (nst % 2 == 0) {
      const int rot = 2 * (key % (nst / 2));
      if (two)
        gateup_mx_wide<2, true>(a, ch.x, blk, cr, rot, ring);
      else
        gateup_mx_wide<1, true>(a, ch.x, blk, cr, rot, ring);
    } else {
      const int rot = key % nst;
      if (two)
        gateup_mx_wide<2, false>(a, ch.x, blk, cr, rot, ring);
      else
        gateup_mx_wide<1, false>(a, ch.x, blk, cr, rot, ring);
    }
    return c;
  }
  u -= nwide * 4 * nbI;
  const int c = nwide + u / nbI;
  const int4 ch = a.chunks[c];
  const int jb = u % nbI;
  const ChunkRows cr{ch.z, ch.y, a.perm, a.K};
  // The rotation (the first of the nst stages, which sets the fp32 accumulation order)
  // follows the global expert and the 128-channel block, not the unit's place in the queue
  // or its kind, so a row's result does not depend on which other rows share its chunk or
  // rank.
  const int key = (ch.x + a.ebase) * nbI + jb;
  if (nst % 2 == 0) {  // paired scale loads: an even rotation keeps the pairs aligned
    const int rot = 2 * (key % (nst / 2));
    if (cr.n <= 16)
      gateup_mx_unit<1, true>(a, ch.x, jb, cr, rot, red8, ring);
    else
      gateup_mx_unit<2, true>(a, ch.x, jb, cr, rot, red8, ring);
  } else {
    const int rot = key % nst;
    if (cr.n <= 16)
      gateup_mx_unit<1, false>(a, ch.x, jb, cr, rot, red8, ring);
    else
      gateup_mx_unit<2, false>(a, ch.x, jb, cr, rot, red8, ring);
  }
  return c;
}

struct DownMxArgs {
  const uint8_t* l2;   // [E, H, I/2] e2m1
  const uint8_t* l2s;  // [E, H, I/32] e8m0
  const int* offsets; const int* perm; const int4* chunks;
  int* meta;
  const uint8_t* hq; const uint8_t* hs;
  uint16_t* d;  // [T*K, H] bf16, grouped rows
  float* pd;    // ks > 1: [ks, T*K, H] fp32 partial d of each K part
  uint16_t* y;  // K == 1 and ks == 1: d straight into the output, row perm[r] (token order)
  const uint8_t* spare;
  int T, H, I, K, E, hs_ld, ks;
  int ebase;
};

// A down unit's output: bf16 d (four values) or the fp32 part (four values). CO: device-
// coherent stores, for a combine unit of the same launch (as store_out); a compile-time
// choice, so the expert kernel's epilogue carries no second store path.
template <bool CO>
__device__ __forceinline__ void store_d_mx(uint16_t* p, uint32_t lo, uint32_t hi) {
  if constexpr (CO)
    store_coherent(reinterpret_cast<uint64_t*>(p), (uint64_t)lo | ((uint64_t)hi << 32));
  else
    *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

template <bool CO>
__device__ __forceinline__ void store_part_mx(float* p, const f32x4& v) {
  if constexpr (CO) {
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    store_coherent(q, (uint64_t)__float_as_uint(v[0]) | ((uint64_t)__float_as_uint(v[1]) << 32));
    store_coherent(q + 1, (uint64_t)__float_as_uint(v[2]) | ((uint64_t)__float_as_uint(v[3]) << 32));
  } else {
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

// Where a down unit's bf16 d row goes: grouped row r of the workspace, or with one slot per
// token and no K split, the token's output row (y = bf16(fp32(d)) = d needs no combine).
__device__ __forceinline__ uint16_t* down_row_mx(const DownMxArgs& a, const ChunkRows& cr, int r) {
  return a.y ? a.y + (size_t)cr.perm[cr.row0 + r] * a.H : a.d + (size_t)(cr.row0 + r) * a.H;
}

// Down unit: rows [j*128, +128) of the expert's down matrix over K part kp of ks.
template <int NCT, bool PAIR, bool CO>
__device__ void down_mx_unit(const DownMxArgs& a, int e, int j, int kp, const ChunkRows& cr, int rot,
                             const ReadyWait& ready, uint8_t* ring) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;
  const int I = a.I, lda = I / 2, sld = I / 32, nstp = I / kMxStageK / a.ks, p0 = kp * nstp;
  OperandsMx<2, NCT> op;
  op.lda = lda;
  op.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const size_t row = (size_t)e * a.H + (size_t)j * kBlock + 32 * w + 16 * r;
    op.a[r] = a.l2 + row * lda + (size_t)p0 * kBlock;
    op.sa[r] = a.l2s + (row + lr) * sld + 8 * p0;
  }
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int rr = cr.row0 + min(16 * c + lr, cr.n - 1);
    op.b[c] = a.hq + (size_t)rr * I + (size_t)p0 * kMxStageK + 16 * (lane >> 4);
    op.sb[c] = a.hs + (size_t)rr * a.hs_ld + 8 * p0;
  }
  f32x4 acc[2][NCT];
  stream_gemm_mx<2, NCT, PAIR ? 2 : (NCT == 2 ? 3 : 4), PAIR>(op, nstp, rot, ring, acc, ready);
  float* pd = a.pd + (size_t)kp * a.T * a.K * a.H;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = 16 * c + lr;
    if (r < cr.n) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const size_t col = (size_t)j * kBlock + 32 * w + 16 * p + 4 * (lane >> 4);
        if (a.ks == 1) {
          const uint32_t lo = f32_to_bf16_bits(acc[p][c][0]) | (f32_to_bf16_bits(acc[p][c][1]) << 16);
          const uint32_t hi = f32_to_bf16_bits(acc[p][c][2]) | (f32_to_bf16_bits(acc[p][c][3]) << 16);
          store_d_mx<CO>(down_row_mx(a, cr, r) + col, lo, hi);
        } else {
          store_part_mx<CO>(pd + (size_t)(cr.row0 + r) * a.H + col, acc[p][c]);
        }
      }
    }
  }
}

// Wide down unit, for a chunk of 33-128 rows: down rows [64 j64, +64) over K part kp, for
// every row of the chunk; wave w takes column tiles [w NCT, w NCT + NCT), every wave
// streaming the same weight rows (as gateup_mx_wide).
template <int NCT, bool PAIR, bool CO>
__device__ void down_mx_wide(const DownMxArgs& a, int e, int j64, int kp, const ChunkRows& cr, int rot,
                             const ReadyWait& ready, uint8_t* ring) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;
  const int I = a.I, lda = I / 2, sld = I / 32, nstp = I / kMxStageK / a.ks, p0 = kp * nstp;
  OperandsMx<4, NCT> op;
  op.lda = lda;
  op.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const size_t row = (size_t)e * a.H + (size_t)j64 * 64 + 16 * r;
    op.a[r] = a.l2 + row * lda + (size_t)p0 * kBlock;
    op.sa[r] = a.l2s + (row + lr) * sld + 8 * p0;
  }
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int rr = cr.row0 + min(16 * (w * NCT + c) + lr, cr.n - 1);
    op.b[c] = a.hq + (size_t)rr * I + (size_t)p0 * kMxStageK + 16 * (lane >> 4);
    op.sb[c] = a.hs + (size_t)rr * a.hs_ld + 8 * p0;
  }
  f32x4 acc[4][NCT];
  stream_gemm_mx<4, NCT, 2, PAIR, 0>(op, nstp, rot, ring, acc, ready);
  float* pd = a.pd + (size_t)kp * a.T * a.K * a.H;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = 16 * (w * NCT + c) + lr;
    if (r < cr.n) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const size_t col = (size_t)j64 * 64 + 16 * p + 4 * (lane >> 4);
        if (a.ks == 1) {
          const uint32_t lo = f32_to_bf16_bits(acc[p][c][0]) | (f32_to_bf16_bits(acc[p][c][1]) << 16);
          const uint32_t hi = f32_to_bf16_bits(acc[p][c][2]) | (f32_to_bf16_bits(acc[p][c][3]) << 16);
          store_d_mx<CO>(down_row_mx(a, cr, r) + col, lo, hi);
        } else {
          store_part_mx<CO>(pd + (size_t)(cr.row0 + r) * a.H + col, acc[p][c]);
        }
      }
    }
  }
}

// Down units: `nwide` wide chunks first (2 nbH ks units each), then narrow chunks (nbH ks
// each). A unit waits for every gate/up unit of its chunk: 4 nbI for a wide chunk, nbI
// for a narrow one. CO: d as device-coherent stores (a unit of the same launch reads it).
template <bool CO>
__device__ void down_mx_work(const DownMxArgs& a, int v, int nwide, int* ready_counts, int* error,
                             uint8_t* ring) {
  const int nbH = a.H / kBlock, nbI = a.I / kBlock;
  const int nstp = a.I / kMxStageK / a.ks;
  if (v < nwide * 2 * nbH * a.ks) {
    const int c = v / (2 * nbH * a.ks), rem = v % (2 * nbH * a.ks), j64 = rem / a.ks, kp = rem % a.ks;
    const int4 ch = a.chunks[c];
    const ChunkRows cr{ch.z, ch.y, a.perm, a.K};
    const ReadyWait ready{&ready_counts[c], 4 * nbI, error};
    const int key = ((ch.x + a.ebase) * (nbH / 2) + j64 / 4) * a.ks + kp;  // as every unit of these rows
    const bool two = cr.n > 64;
    if (nstp % 2 == 0) {
      const int rot = 2 * (key % (nstp / 2));
      if (two)
        down_mx_wide<2, true, CO>(a, ch.x, j64, kp, cr, rot, ready, ring);
      else
        down_mx_wide<1, true, CO>(a, ch.x, j64, kp, cr, rot, ready, ring);
    } else {
      const int rot = key % nstp;
      if (two)
        down_mx_wide<2, false, CO>(a, ch.x, j64, kp, cr, rot, ready, ring);
      else
        down_mx_wide<1, false, CO>(a, ch.x, j64, kp, cr, rot, ready, ring);
    }
    return;
  }
  v -= nwide * 2 * nbH * a.ks;
  const int c = nwide + v / (nbH * a.ks);
  const int4 ch = a.chunks[c];
  const int rem = v % (nbH * a.ks), j = rem / a.ks, kp = rem % a.ks;
  const ChunkRows cr{ch.z, ch.y, a.perm, a.K};
  const ReadyWait ready{&ready_counts[c], nbI, error};
  // Keyed by 256-row block, as the batch units (k_experts_mx_batch) of the same rows.
  const int key = ((ch.x + a.ebase) * (nbH / 2) + j / 2) * a.ks + kp;
  if (nstp % 2 == 0) {
    const int rot = 2 * (key % (nstp / 2));
    if (cr.n <= 16)
      down_mx_unit<1, true, CO>(a, ch.x, j, kp, cr, rot, ready, ring);
    else
      down_mx_unit<2, true, CO>(a, ch.x, j, kp, cr, rot, ready, ring);
  } else {
    const int rot = key % nstp;
    if (cr.n <= 16)
      down_mx_unit<1, false, CO>(a, ch.x, j, kp, cr, rot, ready, ring);
    else
      down_mx_unit<2, false, CO>(a, ch.x, j, kp, cr, rot, ready, ring);
  }
}


// ---------------------------------------------------------------------------------------
// Batch mode of the MXFP4 experts (tens of rows per expert, e.g. a rank's share under
// expert parallelism): one workgroup per CU, every operand through LDS DMA.
//   * weights: wave w streams its own 4 tiles (gate/up: 32 gate + 32 up rows of a
//     128-channel block; down: 64 rows of a 256-row block) into a private ring of
//     kBatchSlots stages, and their E8M0 scale rows (4-byte DMA) beside them;
//   * activations: the chunk's (up to) 64 rows in 4 tiles of 16, tile w requested by wave w
//     into a slot shared by the workgroup, with their E8M0 scale rows; each wave multiplies
//     its weight tiles by all four tiles (64 MFMA accumulators);
//   * one barrier per stage: after it every tile of the stage is in LDS and every wave has
//     read the previous stage's slots, which the stage kBatchSlots - 1 ahead then refills.
// No register load is in flight across the loop, so the compiler's wait counting cannot
// force a drain; the LDS reads are inline asm, ordered by their own lgkmcnt wait. The K
// rotation and the MFMA sequence of every output are the decode units', so a row's result
// does not depend on the mode either.
// ---------------------------------------------------------------------------------------

constexpr int kBatchSlots = 3;
constexpr int kBatchA = 4 * kTileBytes;      // a wave's four weight tiles of one stage (8 KB)
constexpr int kBatchAs = 1024;               // their scale rows for a stage pair: 64 rows x 16 bytes
constexpr int kBatchB = 4 * 2 * kTileBytes;  // four 16-row activation tiles x 256 bytes (16 KB)
constexpr int kBatchBs = 1024;               // their scale rows for a stage pair: 64 rows x 16 bytes
constexpr int kBatchRows = 64;               // rows per chunk
constexpr int kBatchMinRows = 24;            // average rows per expert from which batch mode runs

struct BatchLds {
  uint8_t a[4][kBatchSlots][kBatchA];
  uint8_t as[4][kBatchSlots][kBatchAs];
  uint8_t b[kBatchSlots][kBatchB];
  uint8_t bs[kBatchSlots][kBatchBs];
};

// The per-lane addresses of one wave's loads, at stage 0 of the unit's K range.
struct BatchOps {
  OperandsMx<4, 1> w;        // weight tiles (a[], lda, spare); sa/b/sb unused
  const uint8_t* as;         // scale row of tile lane/16, row lane%16 (16 bytes: a stage pair)
  const uint8_t* b[2];       // activation rows 8i + lane/8 of this wave's tile, at its swizzled chunk
  const uint8_t* bs;         // lanes 0-15: scale row of this wave's tile row lane (a stage pair)
  int bstage;                // activation bytes per stage (256)
};

// One LDS DMA instruction: SIZE bytes per lane from src into dst + lane * SIZE (cached).
template <int SIZE>
__device__ __forceinline__ void lds_dma(const uint8_t* src, uint8_t* dst) {
  static_assert(SIZE == 4 || SIZE == 16, "dword or dwordx4");
  if constexpr (SIZE == 16)
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
  else
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
}

// The weight tiles of stage pp (8 DMA instructions) into weight slot s; with `scales`, also
// the E8M0 rows of the stage pair starting at the even stage pq (one 16-byte DMA: lane l
// fetches row l % 16 of tile l / 16) into scale slot ss.
__device__ __forceinline__ void batch_issue_w(BatchLds& L, const BatchOps& o, const LaneTile& lt, int w, int s, int pp,
                                              bool live, bool scales, int ss, int pq) {
  issue_a_mx<kNonTemporal>(L.a[w][s], o.w, lt, pp, live);
  if (scales) lds_dma<16>(o.as + 8 * pq, L.as[w][ss]);
}

// This wave's activation tile of stage pp (4 DMA instructions) into activation slot s;
// with `scales`, also its tile's E8M0 rows for the stage pair at pq (lanes 0-15 only, each
// 16 bytes) into scale slot ss.
__device__ __forceinline__ void batch_issue_x(BatchLds& L, const BatchOps& o, int w, int s, int pp, bool scales, int ss,
                                              int pq) {
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      lds_dma<16>(o.b[q] + (size_t)pp * o.bstage + 128 * h, L.b[s] + w * 2 * kTileBytes + h * kTileBytes + q * 1024);
  if (scales && opaque_lane() < 16) lds_dma<16>(o.bs + 8 * pq, L.bs[ss] + 256 * w);
}

// Weights run three stages ahead and activations two, in rings of three slots; the E8M0
// rows of both come per stage pair (one 16-byte DMA per row and pair, halving the
// scattered scale requests), in rings of three pairs, issued with the pair's even stage.
// Iteration p: wait for stage p; barrier (every wave's activation tile of stage p is in LDS
// and every wave has read the activation slot of stage p - 1); request activations p + 2
// into that slot; read stage p; request weights p + 3 into the weight slot just read; the
// MFMAs. The loads go out in the order x(p+2), w(p+3) and those issued after x(p) are w(p+1),
// x(p+1), w(p+2): 21 instructions for even p and 22 for odd p (a pair's scales ride with its
// even stage), 4 and 13 at p = 0 and 1 after the prologue's w0 w1 w2 x0 x1. Waiting for x(p)
// also completes w(p) and both scale pairs of stage p, issued before it. The unroll of six
// keeps every slot index a compile-time constant. The stage count and the rotation are even
// (the host runs batch mode only then), so a pair never wraps.
__device__ __forceinline__ void stream_gemm_mx_batch(BatchLds& L, const BatchOps& o, int nst, int rot,
                                                     f32x4 (&acc)[4][4],
                                                     const ReadyWait& ready = ReadyWait{nullptr, 0, nullptr}) {
  constexpr int S = kBatchSlots, U = 6;
  static_assert(S == 3, "three-slot rings: weights three stages ahead, activations two");
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = opaque_lane(), r = lane & 15;
  auto phys = [nst, rot](int p) {
    const int q = p + rot;
    return q >= nst ? q - nst : q;
  };
  // First stage of the pair holding stage q, clamped into the range (loads past the end
  // re-read the last pair).
  auto pair_of = [&](int q) { return phys(2 * min(q / 2, nst / 2 - 1)); };
  const LaneTile lt = lane_tile(o.w.lda);
  const int shift = 8 * (lane >> 4);
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Weights (and their scales) first: they do not depend on the readiness wait.
#pragma unroll
  for (int i = 0; i < 3; ++i)
    batch_issue_w(L, o, lt, w, i, phys(min(i, nst - 1)), i < nst, i % 2 == 0, (i / 2) % S, pair_of(i));
  wait_ready(ready);
#pragma unroll
  for (int i = 0; i < 2; ++i) batch_issue_x(L, o, w, i, phys(min(i, nst - 1)), i % 2 == 0, (i / 2) % S, pair_of(i));
  const uint32_t a_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)&L.a[w][0][0];
  const uint32_t as_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)&L.as[w][0][0];
  const uint32_t b_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)&L.b[0][0];
  const uint32_t bs_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)&L.bs[0][0];
  const int rr = r & 7, g = lane >> 4;
  const uint32_t brow = (uint32_t)((r >> 3) * 1024 + rr * kBlock);
  const uint32_t c0 = (uint32_t)((g ^ rr) << 4), c1 = (uint32_t)(((g + 4) ^ rr) << 4);
  for (int p0 = 0; p0 < nst; p0 += U) {
    static_for<0, U>([&](auto si) {
      constexpr int s = decltype(si)::value;
      const int p = p0 + s;
      if (p >= 2) {
        if constexpr (s % 2 == 0)
          wait_vmem<21>();
        else
          wait_vmem<22>();
      } else if (p == 1) {
        wait_vmem<13>();
      } else {
        wait_vmem<4>();
      }
      __builtin_amdgcn_s_barrier();
      batch_issue_x(L, o, w, (s + 2) % S, phys(min(p + 2, nst - 1)), s % 2 == 0, ((s + 2) / 2) % S, pair_of(p + 2));
      i32x4 lo[4], hi[4];
      uint2 saw[4], sbw[4];
      StageMx<4, 4> st;
      if (p < nst) {
        read_slot_mx<4>(lo, hi, a_lds + (s % S) * kBatchA + lt.rd0, a_lds + (s % S) * kBatchA + lt.rd1);
        const uint32_t half = 8 * (s % 2);
        const uint32_t asb = as_lds + ((s / 2) % S) * kBatchAs + 16 * r + half;
        const uint32_t bsb = bs_lds + ((s / 2) % S) * kBatchBs + 16 * r + half;
        const uint32_t bb = b_lds + (s % S) * kBatchB + brow;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          asm volatile("ds_read_b64 %0, %1" : "=v"(saw[t]) : "v"(asb + 256 * t) : "memory");
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          asm volatile("ds_read_b64 %0, %1" : "=v"(sbw[c]) : "v"(bsb + 256 * c) : "memory");
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            i32x4 x0, x1;
            const uint32_t base = bb + c * 2 * kTileBytes + h * kTileBytes;
            asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3"
                         : "=&v"(x0), "=&v"(x1)
                         : "v"(base + c0), "v"(base + c1)
                         : "memory");
            st.b[c][h] = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(saw[0]), "+v"(saw[1]), "+v"(saw[2]), "+v"(saw[3]), "+v"(sbw[0]), "+v"(sbw[1]),
                       "+v"(sbw[2]), "+v"(sbw[3]));
#pragma unroll
        for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(st.b[c][0]), "+v"(st.b[c][1]));
      }
      // The weight slot of stage p is read (its lgkmcnt wait is above): refill it.
      batch_issue_w(L, o, lt, w, s % S, phys(min(p + 3, nst - 1)), p + 3 < nst, (s + 3) % 2 == 0, ((s + 3) / 2) % S,
                    pair_of(p + 3));
      if (p < nst) mfma_stage_mx(lo, hi, st, saw, sbw, shift, acc);
    });
  }
}

// Batch gate/up unit: 128-channel block jb of gate and up for the chunk's rows (at most 64):
// wave w holds gate and up channels [32w, 32w + 32), as the decode unit.
__device__ void gateup_mx_batch(const GateUpMxArgs& a, int e, int jb, const ChunkRows& cr, int rot, BatchLds& L,
                                uint8_t (*red8)[64]) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.H, lda = H / 2, sld = H / 32;
  const size_t gate0 = (size_t)e * 2 * a.I + (size_t)jb * kBlock + 32 * w, up0 = gate0 + a.I;
  BatchOps o;
  o.w.lda = lda;
  o.w.spare = a.spare;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    o.w.a[r] = a.l1 + (gate0 + 16 * r) * lda;
    o.w.a[r + 2] = a.l1 + (up0 + 16 * r) * lda;
  }
  {
    const int t = lane >> 4;
    const size_t row = (t < 2 ? gate0 + 16 * t : up0 + 16 * (t - 2)) + (lane & 15);
    o.as = a.l1s + row * sld;
  }
  const int chunk16 = ((lane & 7) ^ (lane >> 3)) << 4;
#pragma unroll
  for (int q = 0; q < 2; ++q)
    o.b[q] = a.x + (size_t)row_token(cr, min(16 * w + 8 * q + (lane >> 3), cr.n - 1)) * H + chunk16;
  o.bs = a.xs + (size_t)row_token(cr, min(16 * w + (lane & 15), cr.n - 1)) * sld;
  o.bstage = kMxStageK;
  f32x4 acc[4][4];
  stream_gemm_mx_batch(L, o, H / kMxStageK, rot, acc);
  gateup_mx_epilogue<4>(a, jb, cr, acc, red8);
}

// Batch down unit: down rows [256 j2, +256) over K part kp for the chunk's rows; wave w
// holds rows 64w .. 64w+63 of the block.
__device__ void down_mx_batch(const DownMxArgs& a, int e, int j2, int kp, const ChunkRows& cr, int rot,
                              const ReadyWait& ready, BatchLds& L) {
  const int lane = opaque_lane(), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15;
  const int I = a.I, lda = I / 2, sld = I / 32, nstp = I / kMxStageK / a.ks, p0 = kp * nstp;
  const size_t row0 = (size_t)e * a.H + (size_t)j2 * 256 + 64 * w;
  BatchOps o;
  o.w.lda = lda;
  o.w.spare = a.spare;
#pragma unroll
  for (int t = 0; t < 4; ++t) o.w.a[t] = a.l2 + (row0 + 16 * t) * lda + (size_t)p0 * kBlock;
  o.as = a.l2s + (row0 + 16 * (lane >> 4) + (lane & 15)) * sld + 8 * p0;
  const int chunk16 = ((lane & 7) ^ (lane >> 3)) << 4;
#pragma unroll
  for (int q = 0; q < 2; ++q)
    o.b[q] = a.hq + (size_t)(cr.row0 + min(16 * w + 8 * q + (lane >> 3), cr.n - 1)) * I + (size_t)p0 * kMxStageK +
             chunk16;
  o.bs = a.hs + (size_t)(cr.row0 + min(16 * w + (lane & 15), cr.n - 1)) * a.hs_ld + 8 * p0;
  o.bstage = kMxStageK;
  f32x4 acc[4][4];
  stream_gemm_mx_batch(L, o, nstp, rot, acc, ready);
  float* pd = a.pd + (size_t)kp * a.T * a.K * a.H;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int col = 16 * c + lr;
    if (col < cr.n) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const size_t h0 = (size_t)j2 * 256 + 64 * w + 16 * t + 4 * (lane >> 4);
        if (a.ks == 1) {
          const uint32_t lo = f32_to_bf16_bits(acc[t][c][0]) | (f32_to_bf16_bits(acc[t][c][1]) << 16);
          const uint32_t hi = f32_to_bf16_bits(acc[t][c][2]) | (f32_to_bf16_bits(acc[t][c][3]) << 16);
          *reinterpret_cast<uint2*>(down_row_mx(a, cr, col) + h0) = make_uint2(lo, hi);
        } else {
          *reinterpret_cast<f32x4*>(pd + (size_t)(cr.row0 + col) * a.H + h0) = acc[t][c];
        }
      }
    }
  }
}

// The rotation of the decode units of the same block (their paired scale loads keep it
// even when the stage count is).
__device__ __forceinline__ int mx_rotation(int key, int nst) {
  return nst % 2 == 0 ? 2 * (key % (nst / 2)) : key % nst;
}

struct ExpertMxArgs {
  GateUpMxArgs gu;
  DownMxArgs dn;
  const int* dn_of_gu;
  int* ready;
  int* xcd;  // the batch kernel's per-XCD queues (PermuteOut::xcd)
};

// Thread 0 of a batch workgroup on XCD x: its next unit, from x's gate/up queue, else from
// the other XCDs' in turn, then from the down queues likewise (a down unit only once every
// gate/up unit is taken, so the units a down unit waits for are held by running workgroups).
// Queue y of a phase hands out the units of chunks [bnd[y], bnd[y+1]) in list order (`per`
// units a chunk); `done` marks the queues this workgroup found empty (a queue only empties).
// `total` once every queue is empty.
__device__ __forceinline__ int claim_xcd(int* q, const int* bnd, int x, int nbI, int per, int total_gu, int total,
                                         unsigned& done) {
  for (int phase = 0; phase < 2; ++phase)
    for (int k = 0; k < kXcds; ++k) {
      const int y = (x + k) % kXcds, id = phase * kXcds + y;
      if ((done >> id) & 1u) continue;
      const int first = bnd[y] * (phase ? per : nbI), size = bnd[y + 1] * (phase ? per : nbI) - first;
      if (size > 0) {
        const int i = atomicAdd(&q[id * kXcdStride], 1);
        if (i < size) return phase ? total_gu + first + i : first + i;
      }
      done |= 1u << id;
    }
  return total;
}

// The persistent expert kernel of the MXFP4 form: the queue, claims and readiness waits
// of k_experts, with the MXFP4 units.
__global__ __launch_bounds__(256, 2) void k_experts_mx(ExpertMxArgs args) {
  typedef const __attribute__((address_space(4))) ExpertMxArgs* ArgsPtr;
  __shared__ uint8_t red8[4][64];
  __shared__ __attribute__((aligned(16))) uint8_t rings[4 * kRingWave];
  __shared__ int slot;
  static_assert(sizeof(ExpertMxArgs) % 8 == 0, "argument segment layout");
  int* meta = args.gu.meta;
  const int total_gu = meta[kMetaUnitsGU];
  const int total = total_gu + meta[kMetaUnitsDN];
  const int nwide = meta[kMetaWide];
  if (threadIdx.x == 0) slot = atomicAdd(&meta[kMetaQueueGU], 1);
  __syncthreads();
  int u = slot, next = 0;
  while (u < total) {
    ArgsPtr ap = (ArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    ExpertMxArgs a;
    __builtin_memcpy(&a, (const ExpertMxArgs*)ap, sizeof(a));
    uint8_t* ring = rings + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * kRingWave;
    __syncthreads();
    if (threadIdx.x == 0) next = atomicAdd(&meta[kMetaQueueGU], 1);
    if (u < total_gu) {
      const int c = gateup_mx_work<0>(a.gu, u, nwide, red8, ring);
      publish_fence();
      __syncthreads();
      if (threadIdx.x == 0) atomicAdd(&a.ready[a.dn_of_gu[c]], 1);
    } else {
      down_mx_work<false>(a.dn, u - total_gu, nwide, a.ready, &meta[kMetaError], ring);
    }
    if (threadIdx.x == 0) slot = next;
    __syncthreads();
    u = slot;
  }
}


// The batch-mode expert kernel: the queue, claims and readiness waits of k_experts_mx, one
// workgroup per CU, with the batch units (chunks of at most 64 rows; down units of 256 rows).
__global__ __launch_bounds__(256, 1) void k_experts_mx_batch(ExpertMxArgs args) {
  typedef const __attribute__((address_space(4))) ExpertMxArgs* ArgsPtr;
  __shared__ uint8_t red8[4][64];
  __shared__ __attribute__((aligned(16))) BatchLds lds;
  __shared__ int slot, bnd[kXcds + 1];
  int* meta = args.gu.meta;
  const int total_gu = meta[kMetaUnitsGU];
  const int total = total_gu + meta[kMetaUnitsDN];
  // Units are claimed from the queue of this workgroup's XCD first (claim_xcd).
  const int xcd = my_xcd(), cnbI = args.gu.I / kBlock, cper = args.dn.H / 256 * args.dn.ks;
  unsigned done = 0;
  if (threadIdx.x == 0) {
    for (int i = 0; i <= kXcds; ++i) bnd[i] = args.xcd[kXcdBound + i];
    slot = claim_xcd(args.xcd, bnd, xcd, cnbI, cper, total_gu, total, done);
  }
  __syncthreads();
  int u = slot, next = 0;
  while (u < total) {
    ArgsPtr ap = (ArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    ExpertMxArgs a;
    __builtin_memcpy(&a, (const ExpertMxArgs*)ap, sizeof(a));
    const int nbI = a.gu.I / kBlock, nbH2 = a.dn.H / 256;
    __syncthreads();
    if (threadIdx.x == 0) next = claim_xcd(a.xcd, bnd, xcd, cnbI, cper, total_gu, total, done);
    if (u < total_gu) {
      // Units in expert order, block-major within the expert: the units of one weight block
      // for each chunk of the expert (its group of chunks, .w) are handed out one after
      // another and start at the same K stage, so the weights streamed for the first are
      // still cached when the others read them.
      const int w0 = a.gu.chunks[u / nbI].w, cg = u / nbI - (w0 & 0xffff), ng = w0 >> 16, r = u - cg * nbI;
      const int c = cg + r % ng, jb = r / ng;
      const int4 ch = a.gu.chunks[c];
      const ChunkRows cr{ch.z, ch.y, a.gu.perm, a.gu.K};
      const int nst = a.gu.H / kMxStageK;
      gateup_mx_batch(a.gu, ch.x, jb, cr, mx_rotation((ch.x + a.gu.ebase) * nbI + jb, nst), lds, red8);
      publish_fence();
      __syncthreads();
      if (threadIdx.x == 0) atomicAdd(&a.ready[a.dn_of_gu[c]], 1);
    } else {
      const int v = u - total_gu, ks = a.dn.ks, per = nbH2 * ks;
      const int w0 = a.dn.chunks[v / per].w, cg = v / per - (w0 & 0xffff), ng = w0 >> 16, r = v - cg * per;
      const int c = cg + r % ng, j2 = r / ng / ks, kp = r / ng % ks;
      const int4 ch = a.dn.chunks[c];
      const ChunkRows cr{ch.z, ch.y, a.dn.perm, a.dn.K};
      const ReadyWait ready{&a.ready[c], nbI, &meta[kMetaError]};
      const int nstp = a.dn.I / kMxStageK / ks;
      down_mx_batch(a.dn, ch.x, j2, kp, cr, mx_rotation(((ch.x + a.dn.ebase) * nbH2 + j2) * ks + kp, nstp), ready,
                    lds);
    }
    if (threadIdx.x == 0) slot = next;
    __syncthreads();
    u = slot;
  }
}

// =======================================================================================
// The MXFP4 form as one launch (megamoe_mx_layer_forward): the routing is an input, so the
// queue is the permute (unit 0), the units of k_experts_mx over its lists, and combine units
// of 2048 outputs (with one slot per token and no K split the down units write y, and the
// combine units only write NaN if something failed). The hand-overs and signals are the
// single-launch fp8 kernel's: device-coherent stores, counters raised after the stores
// completed, spread flags for the waits on a whole phase, the control words zeroed by the
// last workgroup out. The batch-shaped form (k_experts_mx_batch, the EP share) stays
// stream-ordered.
// =======================================================================================

struct LayerMxArgs {
  ExpertMxArgs ex;        // offset 0
  const int64_t* ids;     // topk_idx [T, K]
  int64_t base;           // id of local expert 0
  PermuteOut po;
  uint16_t* y;
  int* ctl;
  int T, H, K, E, ks;
  int direct;             // the down units write y
  int tile_waves;         // the permute's ranking form
  int force_timeout;      // test hook, as LayerArgs::force_timeout
};

// Combine unit c of the MXFP4 form: outputs [c * kCombineUnit, +kCombineUnit) of y, as
// k_combine without weights (applied in the gate/up epilogue) and without a shared expert.
__device__ __forceinline__ void layer_mx_combine(const LayerMxArgs& a, int c) {
  const DownMxArgs& dn = a.ex.dn;
  const int i = c * (kCombineUnit / 8) + threadIdx.x, per_row = a.H / 8;
  if (i >= a.T * per_row) return;
  if (load_count(&a.ctl[kCtlError]) || load_count(&a.po.meta[kMetaError])) {
    *reinterpret_cast<uint4*>(a.y + (size_t)i * 8) = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
    return;
  }
  if (a.direct) return;
  const int t = i / per_row, h0 = (i % per_row) * 8;
  float acc[8];
  if (a.ks > 1)
    combine8_parts(dn.pd, nullptr, a.ks, SlotMap{a.po.inv, nullptr, 0}, nullptr, a.T, a.T * a.K, a.H, a.K, 0, t, h0,
                   acc, SlotRows{}, false);
  else
    combine8(dn.d, nullptr, SlotMap{a.po.inv, nullptr, 0}, nullptr, a.H, a.K, 0, t, h0, acc, SlotRows{}, false);
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16_bits(acc[2 * j]) | (f32_to_bf16_bits(acc[2 * j + 1]) << 16);
  *reinterpret_cast<uint4*>(a.y + (size_t)i * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

__global__ __launch_bounds__(256, 2) void k_layer_mx(LayerMxArgs args) {
  typedef const __attribute__((address_space(4))) LayerMxArgs* ArgsPtr;
  typedef const __attribute__((address_space(4))) ExpertMxArgs* ExArgsPtr;
  __shared__ uint8_t red8[4][64];
  __shared__ __attribute__((aligned(16))) uint8_t rings[4 * kRingWave];  // weight rings; the permute's LDS
  __shared__ int slot, next, flags[2], units[3];
  static_assert(sizeof(LayerMxArgs) % 8 == 0 && offsetof(LayerMxArgs, ex) == 0, "argument segment layout");
  static_assert(kPermuteLdsInts * sizeof(int) <= sizeof(rings), "the permute's LDS in the rings");
  int* ctl = args.ctl;
  // Every unit after the first (the permute) waits for the lists, so the workgroups claim one
  // after another, ~27 ns apart by index, rather than all at once (as k_layer's past its
  // front-end units): claims arriving together queue at the one counter, and the permute's
  // own atomics wait behind them.
  if (threadIdx.x == 0) {
    for (int k = (int)blockIdx.x; k > 0; --k) __builtin_amdgcn_s_sleep(1);
    slot = atomicAdd(&ctl[kCtlQueue], 1);
  }
  __syncthreads();
  int u = slot;

  // Phase 1: unit 0, the permute of the given routing (ids less the base; bad ids set the
  // error word and leave no units).
  if (u == 0) {
    ArgsPtr ap = (ArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    LayerMxArgs a;
    __builtin_memcpy(&a, (const LayerMxArgs*)ap, sizeof(a));
    permute_block<true>(a.ids, a.base, a.T, a.K, a.E, 0, a.ex.gu.I / kBlock, a.H / kBlock, a.ks, kChunkRowsMx, 1,
                        a.po, reinterpret_cast<int*>(rings), flags, a.tile_waves);
    publish_fence();
    __syncthreads();
    raise_signal(ctl, kSigPermuted);
    __syncthreads();
    if (threadIdx.x == 0) slot = atomicAdd(&ctl[kCtlQueue], 1);
    __syncthreads();
    u = slot;
  }

  // Phase 2: the work lists (none if the wait gave up or the ids were bad). Every other
  // workgroup waits here while unit 0 permutes: polls back off to ~3.6 us apart, as in
  // k_layer (-1.1 us over four A/B runs).
  wait_ready(ReadyWait{my_signal_flag(ctl, kSigPermuted), 1, &ctl[kCtlError], kWaitTicks, true, 8});
  if (threadIdx.x == 0) {
    const bool lists = load_count(my_signal_flag(ctl, kSigPermuted)) != 0;
    units[0] = lists ? load_count(&args.po.meta[kMetaUnitsGU]) : 0;
    units[1] = lists ? load_count(&args.po.meta[kMetaUnitsDN]) : 0;
    units[2] = lists ? load_count(&args.po.meta[kMetaWide]) : 0;
  }
  __syncthreads();
  const int n_gu = units[0], n_dn = units[1], nwide = units[2];
  const int experts_end = 1 + n_gu + n_dn;
  const int total = experts_end + (args.T * args.H + kCombineUnit - 1) / kCombineUnit;

  // Phase 3: the expert units, as k_experts_mx runs them.
  int my_down = 0;
  while (u < experts_end) {
    ExArgsPtr ap = (ExArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();  // LayerMxArgs::ex is at offset 0
    asm volatile("" : "+s"(ap));
    ExpertMxArgs a;
    __builtin_memcpy(&a, (const ExpertMxArgs*)ap, sizeof(a));
    uint8_t* ring = rings + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * kRingWave;
    __syncthreads();
    if (threadIdx.x == 0) next = atomicAdd(&ctl[kCtlQueue], 1);
    if (u - 1 < n_gu) {
      const int c = gateup_mx_work<1>(a.gu, u - 1, nwide, red8, ring);
      publish_fence();
      __syncthreads();
      if (threadIdx.x == 0) atomicAdd(&a.ready[a.dn_of_gu[c]], 1);
    } else {
      down_mx_work<true>(a.dn, u - 1 - n_gu, nwide, a.ready, &ctl[kCtlError], ring);
      ++my_down;
    }
    __syncthreads();
    u = next;
  }
  if (my_down) publish_count(ctl, kCtlDown, my_down, n_dn, kSigDown, &units[0]);

  // Phase 4: the combine units, once every down unit is counted.
  if (u < total) {
    ArgsPtr ap = (ArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    LayerMxArgs a;
    __builtin_memcpy(&a, (const LayerMxArgs*)ap, sizeof(a));
    if (n_dn) wait_signal(ctl, kSigDown, 1 + a.force_timeout, a.force_timeout ? (uint64_t)2000 : kWaitTicks);
    while (u < total) {
      __syncthreads();
      if (threadIdx.x == 0) next = atomicAdd(&ctl[kCtlQueue], 1);
      layer_mx_combine(a, u - experts_end);
      __syncthreads();
      u = next;
    }
  }
  // Leaving: as k_layer (the status word keeps whether a wait gave up or the ids were bad).
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = atomicAdd(&ctl[kCtlExited], 1) == (int)gridDim.x - 1;
    if (last)
      __hip_atomic_store(&ctl[kCtlStatus], load_count(&ctl[kCtlError]) | load_count(&args.po.meta[kMetaError]),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    slot = last;
  }
  __syncthreads();
  if (slot) {
    constexpr int words[] = {kCtlQueue, kCtlDown, kCtlError, kCtlExited};
    constexpr int n_words = sizeof(words) / sizeof(words[0]);
    const int i = threadIdx.x;
    if (i < n_words)
      __hip_atomic_store(&ctl[words[i]], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else if (i < n_words + kSignals * kSigLines)
      __hip_atomic_store(signal_flag(ctl, (i - n_words) / kSigLines, (i - n_words) % kSigLines), 0,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------

constexpr int kStages = 5;  // router, select + x quantization, permute, experts, combine
constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Layout {
  size_t xn, partial, xq, xs, counts, offsets, meta, perm, inv, gu, dn, dn_of_gu, ready, ready_l, pairs, hq_r, hs_r,
      hq_s, hs_s, st_r, st_s, h16_r, h16_s, d_r, d_s, p_r, p_s, spare, ctl, total;
  int nsplit;
  int ks;  // K parts of each down unit
  int ready_stride;  // ints between two readiness counters
  int dense;         // dense_experts
  int rows_r;        // routed rows of h and d: T*K, or E*T in the dense schedule
  int n_ready_l;     // the single launch's own readiness counters (dense schedule), zeroed per call
};

// Upper bound of list entries: every hit expert has at most ceil(rows/64) chunks, so the
// routed chunks number at most min(E, T*K) + T*K/64; the shared expert adds ceil(T/64)
// per copy.
size_t max_chunks(const megamoe_desc& d, int copies, int chunk = kChunkRows) {
  const size_t T = d.tokens, TK = (size_t)d.tokens * d.topk, E = d.experts;
  return (E < TK ? E : TK) + TK / chunk + 1 + (size_t)copies * ((T + chunk - 1) / chunk);
}

// K parts of each down unit: when the routing can yield fewer than four down units per
// workgroup of a reference grid (2 per CU on 256 CUs), the down GEMMs are split along K
// into 2, 4 or 8 parts (dividing the K blocks), so the down phase keeps every workgroup
// busy and its last units, which set the kernel's tail, are short.
// Depends on the geometry only, so the numerics do not depend on the device.
int down_splits(const megamoe_desc& d) {
  const size_t nbH = d.hidden / kBlock, nkb = d.intermediate / kBlock;
  const size_t hit = (size_t)(d.experts < (int64_t)d.tokens * d.topk ? d.experts : (int64_t)d.tokens * d.topk);
  const size_t units = (hit + (d.shared_experts > 0 ? 1 : 0)) * nbH;
  const size_t target = 4 * 512;
  int ks = 1;
  while (ks < 8 && units * ks < target && nkb % (2 * ks) == 0) ks *= 2;
  return ks;
}

// Whether the expert kernel works gate and up of each 128-row block as separate units
// (k_experts<true>). Worth it only when the whole-block units cannot fill one round of a
// reference grid (2 per CU on 256 CUs) even if every expert is hit, and the rows are long
// enough (32 or more K blocks) for the hand-over between the halves to be cheap next to the
// stream. A Mixtral-shaped layer (8 experts of 112 blocks: 896 units, 1.75 rounds) streams
// its gate/up phase at 6.3-6.6 TB/s split and at 6.9-7.0 whole (per-unit timelines;
// 231 -> 224 us for the stream-ordered expert kernel, 286 -> 282 us for the single launch),
// and DeepSeek-V3, Kimi-K2 and Qwen3-30B-A3B measured 3-7% slower split. Depends on the
// geometry only; both forms give the same bits.
// Whether the expert units follow the dense schedule: every expert's gate/up and down units
// over all T tokens, in lists known from the geometry, so they start as soon as x is
// quantized instead of after the router, the routing and the permute (the single launch's
// front end: ~30 us with HBM idle), and only the combine waits for the routing. Taken when
// T <= 16, where any set of an expert's rows is one 16-column MFMA tile (all T tokens cost
// no more MFMA work or activation reads than the routed rows), and T*K >= E, where every
// expert can be hit (under uniform routing 1 - (1 - K/E)^T of them are: 99% for the
// Mixtral shape, 68% for Tiny). An expert the routing leaves unpicked has its units skipped
// from the moment the routing is known; those started before stream weights no combine
// reads, which the roofline's algorithmic bytes do not count. Each routed row's bits are the
// routed schedule's (each MFMA output column depends only on its own row); only the K
// rotation of a unit, keyed by its place in the lists, differs, and both forms (single
// launch and stream-ordered) take the same lists. Depends on the geometry only.
bool dense_experts(const megamoe_desc& d) {
  return d.tokens <= 16 && (int64_t)d.tokens * d.topk >= d.experts;
}

bool split_gate_up(const megamoe_desc& d) {
  if (dense_experts(d)) return false;  // the dense schedule's units are whole blocks
  const size_t hit = (size_t)(d.experts < (int64_t)d.tokens * d.topk ? d.experts : (int64_t)d.tokens * d.topk);
  const size_t units = (hit + (size_t)d.shared_experts) * (size_t)(d.intermediate / kBlock);
  return units < 512 && d.hidden / kBlock >= 32;
}

Layout make_layout(const megamoe_desc& d) {
  Layout L{};
  const size_t T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate, S = d.shared_experts;
  L.nsplit = router_splits((int)H);
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t o = at;
    at += align_up(bytes > 0 ? bytes : 1);
    return o;
  };
  L.xn = take(T * H * 2);  // normalized x of the block form
  L.partial = take((size_t)L.nsplit * T * E * sizeof(double));
  L.counts = take(E * sizeof(int));
  L.offsets = take((E + 1) * sizeof(int));
  L.meta = take(kMetaInts * sizeof(int));
  L.perm = take(T * K * sizeof(int));
  L.inv = take(T * K * sizeof(int));
  // The lists hold the chunks of either form (the W8A16 form's are smaller, so more).
  L.gu = take(max_chunks(d, (int)S, kChunkRowsA16) * sizeof(int4));
  L.dn = take(max_chunks(d, S > 0 ? 1 : 0, kChunkRowsA16) * sizeof(int4));
  L.dn_of_gu = take(max_chunks(d, (int)S, kChunkRowsA16) * sizeof(int));
  const size_t dn_chunks = max_chunks(d, S > 0 ? 1 : 0);
  L.ready_stride = dn_chunks <= kReadySpreadChunks ? kReadySpread : kReadyLine;
  L.ready = take(max_chunks(d, S > 0 ? 1 : 0, kChunkRowsA16) * L.ready_stride * sizeof(int));
  // The dense schedule's down chunks: the routed experts and the shared expert. The single
  // launch counts them in a region of its own (the stream-ordered form leaves `ready`
  // counted up, and the permute that zeroes it runs after the single launch's first units).
  L.dense = dense_experts(d) ? 1 : 0;
  L.n_ready_l = L.dense ? (int)(E + (S > 0 ? 1 : 0)) : 0;
  L.ready_l = take((size_t)L.n_ready_l * L.ready_stride * sizeof(int));
  L.pairs = take(max_chunks(d, (int)S, kChunkRowsA16) * (I / kBlock) * sizeof(int));
  const size_t R = L.dense ? E * T : T * K;  // routed rows: grouped, or e*T + t
  L.rows_r = (int)R;
  // The quantized x and h of the W8A8 form and the bf16 h of the W8A16 form (which
  // quantizes nothing) share one region. A call writes only one of the two: in the single
  // launch, a line written through from one XCD and again from another would leave the
  // first XCD's L2 with the older copy.
  {
    const size_t q[6] = {align_up(T * H), align_up(T * (H / kBlock) * sizeof(float)), align_up(R * I),
                         align_up(R * scale_ld((int)(I / kBlock)) * sizeof(float)), align_up(T * S * I),
                         align_up(T * scale_ld((int)(S * I / kBlock)) * sizeof(float))};
    const size_t fp8 = q[0] + q[1] + q[2] + q[3] + q[4] + q[5], a16 = align_up(R * I * 2) + align_up(T * S * I * 2);
    const size_t base = take(fp8 > a16 ? fp8 : a16);
    L.xq = base;
    L.xs = L.xq + q[0];
    L.hq_r = L.xs + q[1];
    L.hs_r = L.hq_r + q[2];
    L.hq_s = L.hs_r + q[3];
    L.hs_s = L.hq_s + q[4];
    L.h16_r = base;
    L.h16_s = base + align_up(R * I * 2);
  }
  const bool split = split_gate_up(d);  // staging of the separate gate and up units
  L.st_r = take(split ? 2 * T * K * I * 2 : 0);
  L.st_s = take(split ? 2 * T * S * I * 2 : 0);
  L.d_r = take(R * H * 2);
  L.d_s = take(T * H * 2);
  L.ks = down_splits(d);
  L.p_r = take(L.ks > 1 ? L.ks * R * H * sizeof(float) : 0);
  L.p_s = take(L.ks > 1 && S ? L.ks * T * H * sizeof(float) : 0);
  L.spare = take(16 * (H > I * (S > 1 ? S : 1) ? H : I * (S > 1 ? S : 1)));
  L.ctl = take(kCtlInts * sizeof(int));  // the single-launch kernel's control words
  L.total = at;
  return L;
}

int validate(const megamoe_desc* d) {
  if (!d) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (d->tokens < 0 || d->hidden <= 0 || d->experts <= 0 || d->topk <= 0 || d->intermediate <= 0 ||
      d->shared_experts < 0 || d->groups <= 0 || d->top_groups <= 0)
    return MEGAMOE_ERR_SHAPE;
  if (d->hidden % kBlock || d->intermediate % kBlock) return MEGAMOE_ERR_SHAPE;
  if (d->topk > d->experts || d->experts % d->groups || d->top_groups > d->groups) return MEGAMOE_ERR_SHAPE;
  if (d->gate != MEGAMOE_GATE_SOFTMAX && d->gate != MEGAMOE_GATE_SIGMOID) return MEGAMOE_ERR_SHAPE;
  if (d->groups > 1 && (size_t)d->top_groups * (d->experts / d->groups) < (size_t)d->topk) return MEGAMOE_ERR_SHAPE;
  if (d->experts > kMaxExperts || d->topk > kMaxTopK || d->groups > 64) return MEGAMOE_ERR_UNSUPPORTED;
  // The permute's LDS (bitmap form, or the tiled form for long token counts).
  if (permute_tile_waves(d->tokens, d->experts, 256, kPermuteLdsInts) < 0) return MEGAMOE_ERR_UNSUPPORTED;
  // The permute kernel's packed scan holds up to 2^21-1 rows and 2^15-1 chunks.
  if ((size_t)d->tokens * d->topk >= ((size_t)1 << 21) - kMaxExperts * 64) return MEGAMOE_ERR_UNSUPPORTED;
  return MEGAMOE_OK;
}

struct DeviceInfo {
  int cus = 0;
  int experts_per_cu = 0;     // resident k_experts workgroups per CU
  int experts_mx_per_cu = 0;  // resident k_experts_mx workgroups per CU
  int batch_mx_per_cu = 0;    // resident k_experts_mx_batch workgroups per CU
  int layer_per_cu = 0;       // resident k_layer workgroups per CU
  int layer_mx_per_cu = 0;    // resident k_layer_mx workgroups per CU
};

// The figures of the current device, queried on its first call and kept per device. The
// mutex covers the fill: two host threads making their first calls at once must not see a
// half-filled entry (a zero per-CU count would give a launch of no workgroups).
int device_info(DeviceInfo* out) {
  static std::mutex mutex;
  static DeviceInfo cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return MEGAMOE_ERR_HIP;
  std::lock_guard<std::mutex> lock(mutex);
  DeviceInfo& di = cache[dev];
  if (di.cus == 0) {
    DeviceInfo fill;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return MEGAMOE_ERR_HIP;
    int per_cu_split = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_experts<false>, 256, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_split, k_experts<true>, 256, 0) != hipSuccess)
      return MEGAMOE_ERR_HIP;
    per_cu = per_cu_split < per_cu ? per_cu_split : per_cu;
    fill.experts_per_cu = per_cu > 0 ? per_cu : 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_experts_mx, 256, 0) != hipSuccess)
      return MEGAMOE_ERR_HIP;
    fill.experts_mx_per_cu = per_cu > 0 ? per_cu : 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_experts_mx_batch, 256, 0) != hipSuccess)
      return MEGAMOE_ERR_HIP;
    fill.batch_mx_per_cu = per_cu > 0 ? per_cu : 1;
    int per_cu_split2 = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_layer<false>, 256, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_split2, k_layer<true>, 256, 0) != hipSuccess)
      return MEGAMOE_ERR_HIP;
    per_cu = per_cu_split2 < per_cu ? per_cu_split2 : per_cu;
    fill.layer_per_cu = per_cu > 0 ? per_cu : 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_layer_mx, 256, 0) != hipSuccess)
      return MEGAMOE_ERR_HIP;
    fill.layer_mx_per_cu = per_cu > 0 ? per_cu : 1;
    fill.cus = cus > 0 ? cus : 1;
    di = fill;
  }
  *out = di;
  return MEGAMOE_OK;
}

#define MEGAMOE_LAUNCH_CHECK()                                   \
  do {                                                           \
    if (hipGetLastError() != hipSuccess) return MEGAMOE_ERR_HIP; \
  } while (0)

// Router partials (and, with the extra expert tile, the quantized x) for all tokens.
int launch_router(const megamoe_desc& d, const Layout& L, const void* x, const float* router, char* ws,
                  hipStream_t st) {
  const int n_et = (d.experts + kRouterTile - 1) / kRouterTile, tiles = (d.tokens + kRouterTile - 1) / kRouterTile;
  const int ntt = tiles <= 1 ? 1 : (tiles <= 2 ? 2 : 4), passes = (tiles + ntt - 1) / ntt;
  const dim3 grid(n_et * L.nsplit * passes), block(kRouterWaves * 64);
#define MEGAMOE_ROUTER(NTT)                                                                                    \
  hipLaunchKernelGGL(k_router<NTT>, grid, block, 0, st, (const uint16_t*)x, router, (double*)(ws + L.partial),  \
                     d.tokens, d.hidden, d.experts, n_et, L.nsplit)
  if (tiles <= 1)
    MEGAMOE_ROUTER(1);
  else if (tiles <= 2)
    MEGAMOE_ROUTER(2);
  else
    MEGAMOE_ROUTER(4);
#undef MEGAMOE_ROUTER
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int launch_logits(const megamoe_desc& d, const Layout& L, const void* x, const float* router, char* ws,
                  float* logits, hipStream_t st) {
  int rc = launch_router(d, L, x, router, ws, st);
  if (rc) return rc;
  const size_t n = (size_t)d.tokens * d.experts;
  hipLaunchKernelGGL(k_logits, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const double*)(ws + L.partial),
                     L.nsplit, d.tokens, d.experts, logits);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int launch_quant(int rows, int cols, const void* x, uint8_t* q, float* s, int pow2, hipStream_t st) {
  const long blocks = ((long)rows * ((cols + kBlock - 1) / kBlock) + 3) / 4;
  const int grid = (int)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
  hipLaunchKernelGGL(k_quant_rows, dim3(grid), dim3(256), 0, st, (const uint16_t*)x, q, s, rows, cols, pow2);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

// Routing from fp32 logits, or (logits == NULL) from the router's fp64 split partials; with
// x != NULL, extra workgroups quantize x into xq / xs.
int launch_select(const megamoe_desc& d, const double* partial, int nsplit, const float* logits, const float* bias,
                  int64_t* ids, float* w, const void* x, uint8_t* xq, float* xs, hipStream_t st) {
  const int n_sel = (d.tokens + kSelectTokens - 1) / kSelectTokens;
  const dim3 grid(n_sel + (x ? router_quant_groups(d.tokens, d.hidden) : 0)), block(256);
#define MEGAMOE_SELECT(VPL)                                                                                   \
  hipLaunchKernelGGL(k_select<VPL>, grid, block, 0, st, partial, nsplit, logits, bias, d.tokens, d.experts,   \
                     d.topk, d.groups, d.top_groups, d.gate, d.renormalize, d.routed_scaling, ids, w, n_sel,   \
                     (const uint16_t*)x, xq, xs, d.hidden, d.pow2_scales)
  if (d.experts <= 64)
    MEGAMOE_SELECT(1);
  else if (d.experts <= 128)
    MEGAMOE_SELECT(2);
  else if (d.experts <= 256)
    MEGAMOE_SELECT(4);
  else if (d.experts <= 512)
    MEGAMOE_SELECT(8);
  else
    MEGAMOE_SELECT(16);
#undef MEGAMOE_SELECT
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int launch_norm(int rows, int cols, const void* x, const void* w, float eps, int weight_in_fp32, void* out,
                hipStream_t st) {
  hipLaunchKernelGGL(k_norm, dim3(rows), dim3(256), 0, st,
                     (const uint16_t*)x, (const uint16_t*)w, rows, cols, eps, weight_in_fp32, (uint16_t*)out);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

PermuteOut make_permute_out(const Layout& L, char* ws) {
  PermuteOut po{(int*)(ws + L.counts), (int*)(ws + L.offsets), (int*)(ws + L.meta), (int*)(ws + L.perm),
                (int*)(ws + L.inv),    (int4*)(ws + L.gu),     (int4*)(ws + L.dn),  (int*)(ws + L.dn_of_gu),
                (int*)(ws + L.ready),  (int*)(ws + L.pairs), L.ready_stride};
  // The dense schedule counts every expert's down chunk, hit or not (n_ready_l of them).
  po.ready_min = L.n_ready_l;
  return po;
}

// The expert kernels' arguments for a forward call over workspace `ws`.
void fill_expert_args(const megamoe_desc& d, const Layout& L, const megamoe_tensors* t, char* ws,
                      const PermuteOut& po, const megamoe_epilogue* epi, ExpertArgs& ea) {
  const int T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate, S = d.shared_experts;
  GateUpArgs& ga = ea.gu;
  ga.xq = (const uint8_t*)(ws + L.xq);
  ga.xs = (const float*)(ws + L.xs);
  ga.gate = t->gate; ga.gate_scale = t->gate_scale;
  ga.up = t->up; ga.up_scale = t->up_scale;
  ga.sgate = t->shared_gate; ga.sgate_scale = t->shared_gate_scale;
  ga.sup = t->shared_up; ga.sup_scale = t->shared_up_scale;
  ga.offsets = po.offsets; ga.perm = po.perm; ga.chunks = po.gu; ga.meta = po.meta;
  ga.hq_r = (uint8_t*)(ws + L.hq_r); ga.hs_r = (float*)(ws + L.hs_r);
  ga.hq_s = (uint8_t*)(ws + L.hq_s); ga.hs_s = (float*)(ws + L.hs_s);
  ga.st_r = (uint16_t*)(ws + L.st_r); ga.st_s = (uint16_t*)(ws + L.st_s);
  ga.pairs = po.pairs;
  ga.spare = (const uint8_t*)(ws + L.spare);
  ga.T = T; ga.H = H; ga.I = I; ga.K = K; ga.S = S; ga.E = E; ga.pow2 = d.pow2_scales;
  ga.swiglu = epi ? epi->swiglu : 0;
  ga.limit = epi ? epi->swiglu_limit : 0.0f;
  ga.dense = L.dense;
  ga.x16 = nullptr;  // set by the W8A16 form
  ga.h16_r = (uint16_t*)(ws + L.h16_r);
  ga.h16_s = (uint16_t*)(ws + L.h16_s);
  DownArgs& da = ea.dn;
  da.down = t->down; da.down_scale = t->down_scale;
  da.sdown = t->shared_down; da.sdown_scale = t->shared_down_scale;
  da.offsets = po.offsets; da.perm = po.perm; da.chunks = po.dn; da.meta = po.meta;
  da.hq_r = ga.hq_r; da.hs_r = ga.hs_r; da.hq_s = ga.hq_s; da.hs_s = ga.hs_s;
  da.d_r = (uint16_t*)(ws + L.d_r); da.d_s = (uint16_t*)(ws + L.d_s);
  da.spare = ga.spare;
  da.p_r = (float*)(ws + L.p_r);
  da.p_s = (float*)(ws + L.p_s);
  da.ks = L.ks;
  da.T = T; da.H = H; da.I = I; da.K = K; da.S = S; da.E = E;
  da.dense = L.dense;
  da.rows_r = L.rows_r;
  da.h16_r = ga.h16_r;
  da.h16_s = ga.h16_s;
  ea.dn_of_gu = po.dn_of_gu;
  ea.ready = po.ready;
  ea.ready_stride = po.ready_stride;
}

// The most gate/up and down units one call's lists can hold (the dense schedule's exactly).
size_t expert_units_max(const megamoe_desc& d, const Layout& L, bool split, int chunk = kChunkRows) {
  const size_t nbI = d.intermediate / kBlock, nbH = d.hidden / kBlock, S = d.shared_experts, E = d.experts;
  if (L.dense) return (S + E) * nbI + (E + (S > 0 ? 1 : 0)) * nbH * L.ks;
  return (split ? 2 : 1) * max_chunks(d, (int)S, chunk) * nbI + max_chunks(d, S > 0 ? 1 : 0, chunk) * nbH * L.ks;
}

// The layer; with `blk`, the block form: RMSNorm of x before the router (the layer then
// reads the normalized rows) and the residual add in the combine. With `a16`, the W8A16
// form: the experts read the bf16 rows (x is not quantized) and keep h in bf16.
int forward_impl(const megamoe_desc* desc, const megamoe_tensors* t, hipStream_t st, hipEvent_t* ev,
                 const megamoe_block* blk = nullptr, const megamoe_epilogue* epi = nullptr, bool a16 = false) {
  int rc = validate(desc);
  if (rc) return rc;
  if (!t) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const megamoe_desc& d = *desc;
  if (d.tokens == 0) {
    if (ev)
      for (int i = 0; i < kStages + 1; ++i)
        if (hipEventRecord(ev[i], st) != hipSuccess) return MEGAMOE_ERR_HIP;
    return MEGAMOE_OK;
  }
  if (!t->x || !t->router || !t->gate || !t->gate_scale || !t->up || !t->up_scale || !t->down ||
      !t->down_scale || !t->y || !t->expert_ids || !t->expert_weights || !t->workspace)
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (d.shared_experts > 0 && (!t->shared_gate || !t->shared_gate_scale || !t->shared_up ||
                               !t->shared_up_scale || !t->shared_down || !t->shared_down_scale))
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  const Layout L = make_layout(d);
  if (t->workspace_bytes < L.total) return MEGAMOE_ERR_WORKSPACE;
  DeviceInfo di;
  if ((rc = device_info(&di))) return rc;
  char* ws = (char*)t->workspace;
  auto mark = [&](int i) { return ev ? hipEventRecord(ev[i], st) : hipSuccess; };
  const int T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate, S = d.shared_experts;

  if (mark(0) != hipSuccess) return MEGAMOE_ERR_HIP;
  const void* x = t->x;  // the rows the layer reads
  if (blk && blk->norm_weight) {
    if ((rc = launch_norm(T, H, t->x, blk->norm_weight, blk->eps, blk->weight_in_fp32, ws + L.xn, st))) return rc;
    x = ws + L.xn;
  }
  if ((rc = launch_router(d, L, x, t->router, ws, st))) return rc;
  if (mark(1) != hipSuccess) return MEGAMOE_ERR_HIP;

  if ((rc = launch_select(d, (const double*)(ws + L.partial), L.nsplit, nullptr, t->router_bias, t->expert_ids,
                          t->expert_weights, a16 ? nullptr : x, (uint8_t*)(ws + L.xq), (float*)(ws + L.xs), st)))
    return rc;
  if (mark(2) != hipSuccess) return MEGAMOE_ERR_HIP;

  const PermuteOut po = make_permute_out(L, ws);
  const int nbI = I / kBlock, nbH = H / kBlock;
  const int chunk = a16 ? kChunkRowsA16 : kChunkRows;
  const uint8_t* shared_w[3] = {t->shared_gate, t->shared_up, t->shared_down};
  if ((rc = launch_permute(t->expert_ids, 0, T, K, E, S, nbI, nbH, L.ks, chunk, 0, po, st, S > 0 ? shared_w : nullptr,
                           (size_t)S * I * H)))
    return rc;
  if (mark(3) != hipSuccess) return MEGAMOE_ERR_HIP;

  ExpertArgs ea;
  fill_expert_args(d, L, t, ws, po, epi, ea);
  if (a16) ea.gu.x16 = (const uint16_t*)x;
  const GateUpArgs& ga = ea.gu;
  const DownArgs& da = ea.dn;
  // As many workgroups as fit on the device at once, and no more than the most units the
  // routing can produce.
  const bool split = !a16 && split_gate_up(d);
  const size_t units_max = expert_units_max(d, L, split, chunk);
  const size_t resident = (size_t)di.cus * di.experts_per_cu;
  const unsigned grid = (unsigned)(units_max < resident ? units_max : resident);
  if (a16)
    hipLaunchKernelGGL((k_experts<false, true>), dim3(grid), dim3(256), 0, st, ea);
  else if (split)
    hipLaunchKernelGGL(k_experts<true>, dim3(grid), dim3(256), 0, st, ea);
  else
    hipLaunchKernelGGL(k_experts<false>, dim3(grid), dim3(256), 0, st, ea);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(4) != hipSuccess) return MEGAMOE_ERR_HIP;

  const int rows8 = T * (H / 8);
  const SlotMap slots = L.dense ? SlotMap{nullptr, t->expert_ids, T} : SlotMap{po.inv, nullptr, 0};
  hipLaunchKernelGGL(k_combine, dim3((rows8 + 255) / 256), dim3(256), 0, st, (const uint16_t*)da.d_r,
                     (const uint16_t*)da.d_s, (const float*)da.p_r, (const float*)da.p_s, L.ks, slots, L.rows_r,
                     (const float*)t->expert_weights, T, H, K, S, (const int*)po.meta,
                     (const uint16_t*)(blk && blk->residual ? t->x : nullptr), (uint16_t*)t->y,
                     (int*)(ws + L.ctl) + kCtlStatus);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(5) != hipSuccess) return MEGAMOE_ERR_HIP;
  return MEGAMOE_OK;
}

// The layer (with `blk`, the block form) as one launch of k_layer; see the kernel for the
// unit queue. `ev` is NULL or two events, recorded before and after the launch.
int forward_layer_impl(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* blk,
                       const megamoe_epilogue* epi, hipStream_t st, hipEvent_t* ev, bool a16 = false) {
  int rc = validate(desc);
  if (rc) return rc;
  if (!t) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (blk && !(blk->eps >= 0.0f)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const megamoe_desc& d = *desc;
  auto mark = [&](int i) { return ev ? hipEventRecord(ev[i], st) : hipSuccess; };
  if (d.tokens == 0) return (mark(0) == hipSuccess && mark(1) == hipSuccess) ? MEGAMOE_OK : MEGAMOE_ERR_HIP;
  if (!t->x || !t->router || !t->gate || !t->gate_scale || !t->up || !t->up_scale || !t->down ||
      !t->down_scale || !t->y || !t->expert_ids || !t->expert_weights || !t->workspace)
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (d.shared_experts > 0 && (!t->shared_gate || !t->shared_gate_scale || !t->shared_up ||
                               !t->shared_up_scale || !t->shared_down || !t->shared_down_scale))
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  const Layout L = make_layout(d);
  if (t->workspace_bytes < L.total) return MEGAMOE_ERR_WORKSPACE;
  DeviceInfo di;
  if ((rc = device_info(&di))) return rc;
  char* ws = (char*)t->workspace;
  const int T = d.tokens, H = d.hidden, E = d.experts, I = d.intermediate, S = d.shared_experts;
  const int nbI = I / kBlock, nbH = H / kBlock;

  LayerArgs la{};
  la.po = make_permute_out(L, ws);
  fill_expert_args(d, L, t, ws, la.po, epi, la.ex);
  const bool norm = blk && blk->norm_weight;
  la.x_in = (const uint16_t*)t->x;
  la.xn = (uint16_t*)(ws + L.xn);
  la.x = norm ? la.xn : la.x_in;
  if (a16) la.ex.gu.x16 = la.x;  // the W8A16 experts read the bf16 rows the router reads
  la.norm_w = norm ? (const uint16_t*)blk->norm_weight : nullptr;
  la.eps = blk ? blk->eps : 0.0f;
  la.weight_in_fp32 = blk ? blk->weight_in_fp32 : 0;
  la.router = t->router;
  la.bias = t->router_bias;
  la.partial = (double*)(ws + L.partial);
  la.ids = t->expert_ids;
  la.wts = t->expert_weights;
  la.xq = (uint8_t*)(ws + L.xq);
  la.xs = (float*)(ws + L.xs);
  la.y = (uint16_t*)t->y;
  la.residual = blk && blk->residual ? (const uint16_t*)t->x : nullptr;
  la.ctl = (int*)(ws + L.ctl);
  la.scaling = d.routed_scaling;
  la.T = T; la.H = H; la.E = E; la.K = d.topk; la.S = S; la.G = d.groups; la.TG = d.top_groups;
  la.gate = d.gate; la.renorm = d.renormalize; la.pow2 = d.pow2_scales;
  la.nsplit = L.nsplit;
  la.n_et = (E + kRouterTile - 1) / kRouterTile;
  const int tiles = (T + kRouterTile - 1) / kRouterTile;
  // Token tiles per router unit: k_router's choice, halved while the units still fit in one
  // round of the grid (a shorter fp64 MFMA chain per unit: Qwen3-30B-A3B 139 -> 136 us).
  la.ntt = tiles <= 1 ? 1 : (tiles <= 2 ? 2 : 4);
  while (la.ntt > 1 && (size_t)la.n_et * L.nsplit * ((tiles + la.ntt / 2 - 1) / (la.ntt / 2)) <=
                           (size_t)di.cus * di.layer_per_cu)
    la.ntt /= 2;
  const int passes = (tiles + la.ntt - 1) / la.ntt;
  la.vpl = E <= 64 ? 1 : (E <= 128 ? 2 : (E <= 256 ? 4 : (E <= 512 ? 8 : 16)));
  la.ks = L.ks;
  la.n_norm = norm ? T : 0;
  la.n_router = la.n_et * la.nsplit * passes;
  const char* force = getenv("MEGAMOE_FORCE_WAIT_TIMEOUT");
  la.force_timeout = force && force[0] == '1' ? 1 : 0;

  // As many workgroups as fit on the device at once, and no more than the most units the
  // queue can hold.
  const bool split = !a16 && split_gate_up(d);
  const size_t units_max = (size_t)la.n_norm + la.n_router + T +
                           expert_units_max(d, L, split, a16 ? kChunkRowsA16 : kChunkRows) +
                           ((size_t)T * H + kCombineUnit - 1) / kCombineUnit;
  la.dense = L.dense;
  la.n_ready = L.n_ready_l;
  if (L.dense) la.ex.ready = (int*)(ws + L.ready_l);
  const size_t resident = (size_t)di.cus * di.layer_per_cu;
  const unsigned grid = (unsigned)(units_max < resident ? units_max : resident);
  // Router units taken by workgroup index: the first round of them, when there are 64 or more
  // (fewer are claimed from the queue in ~1 us: Mixtral's 8 measured 2 us slower by index);
  // none in the block form, whose first units are the norm rows.
  la.n_first = norm || la.n_router < 64 ? 0 : (int)grid < la.n_router ? (int)grid : la.n_router;
  if (la.n_first > kMaxStartUnits) la.n_first = kMaxStartUnits;
  const char* rescue = getenv("MEGAMOE_FORCE_RESCUE");
  la.force_rescue = rescue && rescue[0] == '1' ? 1 : 0;
  if (mark(0) != hipSuccess) return MEGAMOE_ERR_HIP;
  if (a16)
    hipLaunchKernelGGL((k_layer<false, true>), dim3(grid), dim3(256), 0, st, la);
  else if (split)
    hipLaunchKernelGGL(k_layer<true>, dim3(grid), dim3(256), 0, st, la);
  else
    hipLaunchKernelGGL(k_layer<false>, dim3(grid), dim3(256), 0, st, la);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(1) != hipSuccess) return MEGAMOE_ERR_HIP;
  return MEGAMOE_OK;
}

// -- The MXFP4 form ----------------------------------------------------------------------

// With the output written by the down units (one slot per token, no K split), this stands
// in for the combine: if the permute flagged bad ids, every element of y is NaN. `status`
// (NULL: none) keeps the call's outcome, as k_combine's does.
__global__ __launch_bounds__(256) void k_error_fill(const int* __restrict__ meta, size_t n8, uint16_t* __restrict__ y,
                                                    int* __restrict__ status) {
  if (status && blockIdx.x == 0 && threadIdx.x == 0) *status = meta[kMetaError];
  if (!meta[kMetaError]) return;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256)
    *reinterpret_cast<uint4*>(y + i * 8) = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
}

constexpr int kStagesMx = 3;  // permute, experts, combine

int validate_mx(const megamoe_desc* d) {
  if (!d) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (d->tokens < 0 || d->hidden <= 0 || d->experts <= 0 || d->topk <= 0 || d->intermediate <= 0 ||
      d->shared_experts != 0)
    return MEGAMOE_ERR_SHAPE;
  if (d->hidden % kMxStageK || d->intermediate % kMxStageK || d->topk > d->experts) return MEGAMOE_ERR_SHAPE;
  if (d->experts > kMaxExperts || d->topk > kMaxTopK) return MEGAMOE_ERR_UNSUPPORTED;
  if (permute_tile_waves(d->tokens, d->experts, 1024, kPermuteLdsInts) < 0) return MEGAMOE_ERR_UNSUPPORTED;
  if ((size_t)d->tokens * d->topk >= ((size_t)1 << 21) - kMaxExperts * 64) return MEGAMOE_ERR_UNSUPPORTED;
  return MEGAMOE_OK;
}

struct LayoutMx {
  size_t counts, offsets, meta, perm, inv, gu, dn, dn_of_gu, ready, hq, hs, d, p, spare, ctl, xcd, total;
  int ks, hs_ld;
};

// K parts of the down units, as down_splits for the fp8 form, over stages of 256.
int down_splits_mx(const megamoe_desc& d) {
  const size_t nbH = d.hidden / kBlock, nst = d.intermediate / kMxStageK;
  const size_t hit = (size_t)(d.experts < (int64_t)d.tokens * d.topk ? d.experts : (int64_t)d.tokens * d.topk);
  const size_t units = hit * nbH, target = 4 * 512;
  int ks = 1;
  while (ks < 8 && units * ks < target && nst % (2 * ks) == 0) ks *= 2;
  return ks;
}

LayoutMx make_layout_mx(const megamoe_desc& d) {
  LayoutMx L{};
  const size_t T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t o = at;
    at += align_up(bytes > 0 ? bytes : 1);
    return o;
  };
  const size_t chunks = max_chunks(d, 0, kBatchRows < kChunkRowsMx ? kBatchRows : kChunkRowsMx);
  L.counts = take(E * sizeof(int));
  L.offsets = take((E + 1) * sizeof(int));
  L.meta = take(kMetaInts * sizeof(int));
  L.perm = take(T * K * sizeof(int));
  L.inv = take(T * K * sizeof(int));
  L.gu = take(chunks * sizeof(int4));
  L.dn = take(chunks * sizeof(int4));
  L.dn_of_gu = take(chunks * sizeof(int));
  L.ready = take(chunks * sizeof(int));
  L.hq = take(T * K * I);
  L.hs_ld = (int)((I / 32 + 127) / 128 * 128);  // each row's scale bytes on lines of their own
  L.hs = take(T * K * (size_t)L.hs_ld);
  L.d = take(T * K * H * 2);
  L.ks = down_splits_mx(d);
  L.p = take(L.ks > 1 ? L.ks * T * K * H * sizeof(float) : 0);
  L.spare = take(16 * (H > I ? H : I) / 2);
  L.ctl = take(kCtlInts * sizeof(int));  // the single-launch kernel's control words
  L.xcd = take(kXcdInts * sizeof(int));  // the batch kernel's per-XCD queues
  L.total = at;
  return L;
}

// The MXFP4 expert kernels' arguments over workspace `ws`.
void fill_expert_mx_args(const megamoe_desc& d, const LayoutMx& L, const megamoe_mx_tensors* t, char* ws,
                         const PermuteOut& po, float limit, int64_t base, bool direct, ExpertMxArgs& ea) {
  const int T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate;
  GateUpMxArgs& ga = ea.gu;
  ga.x = t->x; ga.xs = t->x_scales; ga.wts = t->topk_weights;
  ga.l1 = t->l1_blocks; ga.l1s = t->l1_scales;
  ga.offsets = po.offsets; ga.perm = po.perm; ga.chunks = po.gu; ga.meta = po.meta;
  ga.hq = (uint8_t*)(ws + L.hq); ga.hs = (uint8_t*)(ws + L.hs);
  ga.spare = (const uint8_t*)(ws + L.spare);
  ga.T = T; ga.H = H; ga.I = I; ga.K = K; ga.E = E; ga.hs_ld = L.hs_ld; ga.limit = limit;
  ga.ebase = (int)base;
  DownMxArgs& da = ea.dn;
  da.l2 = t->l2_blocks; da.l2s = t->l2_scales;
  da.offsets = po.offsets; da.perm = po.perm; da.chunks = po.dn; da.meta = po.meta;
  da.hq = ga.hq; da.hs = ga.hs;
  da.d = (uint16_t*)(ws + L.d); da.pd = (float*)(ws + L.p);
  da.y = direct ? (uint16_t*)t->y : nullptr;
  da.spare = ga.spare;
  da.T = T; da.H = H; da.I = I; da.K = K; da.E = E; da.hs_ld = L.hs_ld; da.ks = L.ks;
  da.ebase = (int)base;
  ea.dn_of_gu = po.dn_of_gu;
  ea.ready = po.ready;
  ea.xcd = po.xcd;
}

// `status` (NULL: none) receives the call's outcome (1: bad expert ids, y is NaN) from the
// last kernel: the single-launch entry point passes its status word when it falls back here.
int forward_mx_impl(const megamoe_desc* desc, float limit, const megamoe_mx_tensors* t, hipStream_t st,
                    hipEvent_t* ev, int64_t base = 0, int* status = nullptr) {
  int rc = validate_mx(desc);
  if (rc) return rc;
  if (!t || !(limit > 0.0f)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const megamoe_desc& d = *desc;
  auto mark = [&](int i) { return ev ? hipEventRecord(ev[i], st) : hipSuccess; };
  if (d.tokens == 0) {
    for (int i = 0; i < kStagesMx + 1; ++i)
      if (mark(i) != hipSuccess) return MEGAMOE_ERR_HIP;
    return MEGAMOE_OK;
  }
  if (!t->x || !t->x_scales || !t->topk_idx || !t->topk_weights || !t->l1_blocks || !t->l1_scales ||
      !t->l2_blocks || !t->l2_scales || !t->y || !t->workspace)
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  const LayoutMx L = make_layout_mx(d);
  if (t->workspace_bytes < L.total) return MEGAMOE_ERR_WORKSPACE;
  DeviceInfo di;
  if ((rc = device_info(&di))) return rc;
  char* ws = (char*)t->workspace;
  const int T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate;
  const int nbI = I / kBlock, nbH = H / kBlock;

  if (mark(0) != hipSuccess) return MEGAMOE_ERR_HIP;
  PermuteOut po{(int*)(ws + L.counts), (int*)(ws + L.offsets), (int*)(ws + L.meta), (int*)(ws + L.perm),
                (int*)(ws + L.inv),    (int4*)(ws + L.gu),     (int4*)(ws + L.dn),  (int*)(ws + L.dn_of_gu),
                (int*)(ws + L.ready)};
  // Batch mode (k_experts_mx_batch) when the rows per expert average kBatchMinRows or more:
  // chunks of up to 64 rows, down units of 256 rows, no wide units; the lists in expert
  // order and the units claimed from per-XCD queues.
  const bool batch = (int64_t)T * K >= (int64_t)kBatchMinRows * E && (H / kMxStageK) % 2 == 0 &&
                     (I / kMxStageK / L.ks) % 2 == 0;
  if (batch) po.xcd = (int*)(ws + L.xcd);
  if ((rc = launch_permute(t->topk_idx, base, T, K, E, 0, nbI, batch ? nbH / 2 : nbH, L.ks,
                           batch ? kBatchRows : kChunkRowsMx, batch ? 2 : 1, po, st)))
    return rc;
  if (mark(1) != hipSuccess) return MEGAMOE_ERR_HIP;

  ExpertMxArgs ea;
  const bool direct = K == 1 && L.ks == 1;  // the down units write y; no combine
  fill_expert_mx_args(d, L, t, ws, po, limit, base, direct, ea);
  const DownMxArgs& da = ea.dn;
  if (batch) {
    const size_t chunks = max_chunks(d, 0, kBatchRows);
    const size_t units_max = chunks * (size_t)nbI + chunks * (size_t)(nbH / 2) * L.ks;
    const size_t resident = (size_t)di.cus * di.batch_mx_per_cu;
    hipLaunchKernelGGL(k_experts_mx_batch, dim3((unsigned)(units_max < resident ? units_max : resident)), dim3(256),
                       0, st, ea);
  } else {
    const size_t chunks = max_chunks(d, 0, kChunkRowsMx);
    const size_t units_max = chunks * 4 * (size_t)nbI + chunks * 2 * (size_t)nbH * L.ks;
    const size_t resident = (size_t)di.cus * di.experts_mx_per_cu;
    hipLaunchKernelGGL(k_experts_mx, dim3((unsigned)(units_max < resident ? units_max : resident)), dim3(256), 0,
                       st, ea);
  }
  MEGAMOE_LAUNCH_CHECK();
  if (mark(2) != hipSuccess) return MEGAMOE_ERR_HIP;

  const int rows8 = T * (H / 8);
  if (direct)
    hipLaunchKernelGGL(k_error_fill, dim3((unsigned)((rows8 + 255) / 256 < 1024 ? (rows8 + 255) / 256 : 1024)),
                       dim3(256), 0, st, (const int*)po.meta, (size_t)rows8, (uint16_t*)t->y, status);
  else
    hipLaunchKernelGGL(k_combine, dim3((rows8 + 255) / 256), dim3(256), 0, st, (const uint16_t*)da.d,
                       (const uint16_t*)nullptr, (const float*)da.pd, (const float*)nullptr, L.ks,
                       SlotMap{po.inv, nullptr, 0}, T * K, (const float*)nullptr, T, H, K, 0, (const int*)po.meta,
                       (const uint16_t*)nullptr, (uint16_t*)t->y, status);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(3) != hipSuccess) return MEGAMOE_ERR_HIP;
  return MEGAMOE_OK;
}

// The MXFP4 form as one launch of k_layer_mx (see the kernel). Batch-shaped rows (the
// batch kernel's geometry) and permutes beyond one workgroup's LDS take the stream-ordered
// kernels instead (forward_mx_impl). `ev`: NULL or two events, recorded around the call.
int forward_mx_layer_impl(const megamoe_desc* desc, float limit, const megamoe_mx_tensors* t, hipStream_t st,
                          hipEvent_t* ev, int64_t base = 0) {
  int rc = validate_mx(desc);
  if (rc) return rc;
  if (!t || !(limit > 0.0f)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const megamoe_desc& d = *desc;
  auto mark = [&](int i) { return ev ? hipEventRecord(ev[i], st) : hipSuccess; };
  if (d.tokens == 0) return (mark(0) == hipSuccess && mark(1) == hipSuccess) ? MEGAMOE_OK : MEGAMOE_ERR_HIP;
  if (!t->x || !t->x_scales || !t->topk_idx || !t->topk_weights || !t->l1_blocks || !t->l1_scales ||
      !t->l2_blocks || !t->l2_scales || !t->y || !t->workspace)
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  const LayoutMx L = make_layout_mx(d);
  if (t->workspace_bytes < L.total) return MEGAMOE_ERR_WORKSPACE;
  const int T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate;
  const int nbI = I / kBlock, nbH = H / kBlock;
  const bool batch = (int64_t)T * K >= (int64_t)kBatchMinRows * E && (H / kMxStageK) % 2 == 0 &&
                     (I / kMxStageK / L.ks) % 2 == 0;
  const int tile_waves = permute_tile_waves(T, E, 256, kPermuteLdsInts);
  if (batch || tile_waves < 0) {  // the stream-ordered kernels, between the caller's two events
    if (mark(0) != hipSuccess) return MEGAMOE_ERR_HIP;
    int* status = (int*)((char*)t->workspace + L.ctl) + kCtlStatus;  // megamoe_mx_layer_status reads it
    if ((rc = forward_mx_impl(desc, limit, t, st, nullptr, base, status))) return rc;
    return mark(1) == hipSuccess ? MEGAMOE_OK : MEGAMOE_ERR_HIP;
  }
  DeviceInfo di;
  if ((rc = device_info(&di))) return rc;
  char* ws = (char*)t->workspace;

  LayerMxArgs la{};
  la.po = PermuteOut{(int*)(ws + L.counts), (int*)(ws + L.offsets), (int*)(ws + L.meta), (int*)(ws + L.perm),
                     (int*)(ws + L.inv),    (int4*)(ws + L.gu),     (int4*)(ws + L.dn),  (int*)(ws + L.dn_of_gu),
                     (int*)(ws + L.ready)};
  const bool direct = K == 1 && L.ks == 1;
  fill_expert_mx_args(d, L, t, ws, la.po, limit, base, direct, la.ex);
  la.ids = t->topk_idx;
  la.base = base;
  la.y = (uint16_t*)t->y;
  la.ctl = (int*)(ws + L.ctl);
  la.T = T; la.H = H; la.K = K; la.E = E; la.ks = L.ks;
  la.direct = direct ? 1 : 0;
  la.tile_waves = tile_waves;
  const char* force = getenv("MEGAMOE_FORCE_WAIT_TIMEOUT");
  la.force_timeout = force && force[0] == '1' ? 1 : 0;
  // As many workgroups as fit on the device at once, and no more than the most units.
  const size_t chunks = max_chunks(d, 0, kChunkRowsMx);
  const size_t units_max = 1 + chunks * 4 * (size_t)nbI + chunks * 2 * (size_t)nbH * L.ks +
                           ((size_t)T * H + kCombineUnit - 1) / kCombineUnit;
  const size_t resident = (size_t)di.cus * di.layer_mx_per_cu;
  if (mark(0) != hipSuccess) return MEGAMOE_ERR_HIP;
  hipLaunchKernelGGL(k_layer_mx, dim3((unsigned)(units_max < resident ? units_max : resident)), dim3(256), 0, st, la);
  MEGAMOE_LAUNCH_CHECK();
  return mark(1) == hipSuccess ? MEGAMOE_OK : MEGAMOE_ERR_HIP;
}


// -- Expert parallelism: one rank's share ---------------------------------------------------
//
// Under EP (megamoe.py:153-182) expert e belongs to rank e / (E/ep). A rank sends each of its
// (token, slot) rows to the owner of the slot's expert, in a stable order by owner
// (megamoe.py:160-171; the per-destination counts are those of parallel.py:59-68), runs its
// local experts over the rows it receives (megamoe.py:131-150: the MXFP4 form with one slot
// per row) and, once the outputs have come back in send order, sums each token's slots in
// slot order (megamoe.py:176-182). The exchanges in between are collectives of the caller.

constexpr int kMaxRanks = 256;              // owner ranks are held as bytes
constexpr int kMaxDispatch = 48 * 1024;     // (token, slot) entries of one dispatch (LDS bytes)
constexpr int kDispatchList = 1024;         // entries one workgroup packs at most

// The dispatch in one kernel: a stable counting sort by owner rank and the payload gather.
// Workgroup (o, j) of ep x m: every workgroup reads all owners into LDS (coalesced; an id
// outside [0, E) makes every count and send row -1); each thread owns a contiguous run of
// entries; a reduction of the runs' counts below o and a scan of their counts of o give the
// send row of every entry of owner o (owner o's rows start after all rows of lower owners and
// keep (token, slot) order). Workgroup j packs the entries of owner o whose rank falls in
// its j-th share, the whole workgroup copying one row (E4M3 bytes and E8M0 scales) at a
// time; workgroup (o, 0) writes owner o's count.
__global__ __launch_bounds__(256) void k_ep_dispatch(const int64_t* __restrict__ ids, const uint8_t* __restrict__ x,
                                                     const uint8_t* __restrict__ xs, const float* __restrict__ wts,
                                                     int n, int K, int H, int E, int local, int m,
                                                     int64_t* __restrict__ counts, int32_t* __restrict__ slot_rows,
                                                     uint8_t* __restrict__ rows, uint8_t* __restrict__ row_scales,
                                                     int64_t* __restrict__ out_ids, float* __restrict__ out_wts) {
  extern __shared__ uint8_t owner[];  // n bytes
  __shared__ unsigned long long tmp[4];
  __shared__ int2 list[kDispatchList];
  __shared__ int bad, nlist, below;
  const int o = blockIdx.x / m, j = blockIdx.x % m, tid = threadIdx.x;
  if (tid == 0) {
    bad = 0;
    nlist = 0;
    below = 0;
  }
  __syncthreads();
  for (int i0 = tid; i0 < n; i0 += 256 * 8) {  // eight id loads in flight per thread
    int64_t e[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) e[u] = i0 + 256 * u < n ? ids[i0 + 256 * u] : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + 256 * u;
      if (i < n) {
        if (e[u] < 0 || e[u] >= E)
          bad = 1;
        else
          owner[i] = (uint8_t)((int)e[u] / local);
      }
    }
  }
  __syncthreads();
  if (bad) {
    for (int i = blockIdx.x * 256 + tid; i < n; i += gridDim.x * 256) slot_rows[i] = -1;
    if (j == 0 && tid == 0) counts[o] = -1;
    return;
  }
  const int per = (n + 255) / 256, lo = min(n, tid * per), hi = min(n, lo + per);
  int c_lt = 0, c_eq = 0;
  for (int i = lo; i < hi; ++i) {
    c_lt += owner[i] < o;
    c_eq += owner[i] == o;
  }
  {
    const int wave_lt = wave_sum_small(c_lt);
    if ((tid & 63) == 0 && wave_lt) atomicAdd(&below, wave_lt);
  }
  unsigned long long total;
  const int first = (int)block_exclusive_scan((unsigned long long)c_eq, tmp, &total);
  __syncthreads();  // `below` complete
  const int base = below, n_o = (int)total;
  if (j == 0 && tid == 0) counts[o] = n_o;
  const int r0 = (int)((int64_t)n_o * j / m), r1 = (int)((int64_t)n_o * (j + 1) / m);
  for (int i = lo, rank = first; i < hi; ++i) {
    if (owner[i] != o) continue;
    if (rank >= r0 && rank < r1) {
      const int at = atomicAdd(&nlist, 1);
      list[at] = make_int2(i, base + rank);
    }
    ++rank;
  }
  __syncthreads();
  // The rows as one flat list of 16-byte chunks, eight loads in flight per thread.
  const int cnt = nlist, nch = H / 16, total_ch = cnt * nch;
  for (int k0 = tid; k0 < total_ch; k0 += 256 * 8) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + 256 * u;
      if (k < total_ch) {
        const int q = k / nch;
        v[u] = reinterpret_cast<const uint4*>(x + (size_t)(list[q].x / K) * H)[k - q * nch];
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + 256 * u;
      if (k < total_ch) {
        const int q = k / nch;
        reinterpret_cast<uint4*>(rows + (size_t)list[q].y * H)[k - q * nch] = v[u];
      }
    }
  }
  const int nsc = H / 256;  // 8-byte scale words per row
  for (int k = tid; k < cnt * nsc; k += 256) {
    const int q = k / nsc;
    reinterpret_cast<uint2*>(row_scales + (size_t)list[q].y * (H / 32))[k - q * nsc] =
        reinterpret_cast<const uint2*>(xs + (size_t)(list[q].x / K) * (H / 32))[k - q * nsc];
  }
  for (int q = tid; q < cnt; q += 256) {
    const int i = list[q].x, pos = list[q].y;
    out_ids[pos] = ids[i];
    out_wts[pos] = wts[i];
    slot_rows[i] = pos;
  }
}

// y[t] = bf16 of the slot-order fp32 sum of the returned rows of token t's slots; a slot
// without a send row (bad ids at the dispatch) makes the token's row NaN.
__global__ __launch_bounds__(256) void k_ep_combine(const uint16_t* __restrict__ returned,
                                                    const int32_t* __restrict__ slot_rows, int T, int H, int K,
                                                    uint16_t* __restrict__ y) {
  const int i = blockIdx.x * 256 + threadIdx.x, per_row = H / 8;
  if (i >= T * per_row) return;
  const int t = i / per_row, h0 = (i % per_row) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  bool bad = false;
  for (int k = 0; k < K; ++k) {
    const int r = slot_rows[(size_t)t * K + k];
    if (r < 0) {
      bad = true;
      continue;
    }
    const uint4 v = *reinterpret_cast<const uint4*>(returned + (size_t)r * H + h0);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[2 * j] = __fadd_rn(acc[2 * j], bf16_bits_to_f32(q[j] & 0xffffu));
      acc[2 * j + 1] = __fadd_rn(acc[2 * j + 1], bf16_bits_to_f32(q[j] >> 16));
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = bad ? 0x7fc07fc0u : (f32_to_bf16_bits(acc[2 * j]) | (f32_to_bf16_bits(acc[2 * j + 1]) << 16));
  *reinterpret_cast<uint4*>(y + (size_t)t * H + h0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// GPT-OSS's combine (gptoss.py:112-124): a token's expert outputs accumulate in ascending
// expert id order, independent of the router's rank order, in bf16: o = bf16(o + bf16(p * e))
// from o = 0, with bf16 weights p; then y = bf16(x + o) with a residual x, else y = o.
__global__ __launch_bounds__(256) void k_combine_id_order(const uint16_t* __restrict__ out,
                                                          const int64_t* __restrict__ ids,
                                                          const uint16_t* __restrict__ wts,
                                                          const uint16_t* __restrict__ residual, int T, int H, int K,
                                                          uint16_t* __restrict__ y) {
  const int i = blockIdx.x * 256 + threadIdx.x, per_row = H / 8;
  if (i >= T * per_row) return;
  const int t = i / per_row, h0 = (i % per_row) * 8;
  const int64_t* row_ids = ids + (size_t)t * K;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t last = INT64_MIN;
  for (int n = 0; n < K; ++n) {
    // The slot with the smallest id above the previous one (ids of a token are distinct).
    int k = -1;
    int64_t best = INT64_MAX;
    for (int j = 0; j < K; ++j) {
      const int64_t e = row_ids[j];
      if (e > last && e <= best) {
        best = e;
        k = j;
      }
    }
    if (k < 0) break;
    last = best;
    const float p = bf16_bits_to_f32(wts[(size_t)t * K + k]);
    const uint4 v = *reinterpret_cast<const uint4*>(out + ((size_t)t * K + k) * H + h0);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = round_bf16(__fadd_rn(o[2 * j], round_bf16(__fmul_rn(p, bf16_bits_to_f32(q[j] & 0xffffu)))));
      o[2 * j + 1] = round_bf16(__fadd_rn(o[2 * j + 1], round_bf16(__fmul_rn(p, bf16_bits_to_f32(q[j] >> 16)))));
    }
  }
  uint32_t r[4];
  if (residual) {
    const uint4 v = *reinterpret_cast<const uint4*>(residual + (size_t)t * H + h0);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      r[j] = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(q[j] & 0xffffu), o[2 * j])) |
             (f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(q[j] >> 16), o[2 * j + 1])) << 16);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = f32_to_bf16_bits(o[2 * j]) | (f32_to_bf16_bits(o[2 * j + 1]) << 16);
  }
  *reinterpret_cast<uint4*>(y + (size_t)t * H + h0) = make_uint4(r[0], r[1], r[2], r[3]);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// ---------------------------------------------------------------------------------------
// Fixed device scratch of megamoe_forward_noalloc: the workspace of one layer call in a
// file-scope device array, which each GPU the library runs on holds (its own copy, at its
// own address) until the process ends. In host code `scratch` names a host-side stand-in,
// not device memory, so host code never passes it to a kernel or a copy: the device
// address comes from hipGetSymbolAddress, taken once per device with that device current,
// and is kept per device. The forward path initialises what it needs in the workspace
// itself (the permute kernel clears the queue, readiness and pair counters each call), so
// the array's contents from an earlier call do not matter; calls that overlap on one GPU
// share the array and race.
// ---------------------------------------------------------------------------------------

static __device__ __align__(256) uint8_t scratch[MEGAMOE_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

// The current device's copy of `scratch`.
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MEGAMOE_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_address[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return MEGAMOE_ERR_HIP;
    g_scratch_address[dev] = p;
  }
  *out = g_scratch_address[dev];
  return MEGAMOE_OK;
}

}  // namespace

extern "C" {

int megamoe_abi_version(void) { return 11; }

const char* megamoe_status_string(int status) {
  switch (status) {
    case MEGAMOE_OK: return "ok";
    case MEGAMOE_ERR_INVALID_ARGUMENT: return "invalid argument (a required pointer is NULL)";
    case MEGAMOE_ERR_SHAPE: return "invalid MoE geometry";
    case MEGAMOE_ERR_WORKSPACE: return "workspace smaller than megamoe_workspace_bytes()";
    case MEGAMOE_ERR_HIP: return "HIP runtime error";
    case MEGAMOE_ERR_UNSUPPORTED: return "geometry beyond this build's limits";
    case MEGAMOE_ERR_SCRATCH: return "the layer needs more workspace than the fixed device scratch (MEGAMOE_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

int megamoe_workspace_bytes(const megamoe_desc* desc, size_t* bytes) {
  if (!bytes) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const int rc = validate(desc);
  if (rc) return rc;
  *bytes = make_layout(*desc).total;
  return MEGAMOE_OK;
}

int megamoe_forward(const megamoe_desc* desc, const megamoe_tensors* t, void* stream) {
  return forward_impl(desc, t, (hipStream_t)stream, nullptr);
}

int megamoe_layer_forward(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                          const megamoe_epilogue* epilogue, void* stream, void* const* events) {
  if (epilogue && ((epilogue->swiglu != 0 && epilogue->swiglu != 1) || !(epilogue->swiglu_limit >= 0.0f)))
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[2];
  if (events) {
    if (!events[0] || !events[1]) return MEGAMOE_ERR_INVALID_ARGUMENT;
    ev[0] = (hipEvent_t)events[0];
    ev[1] = (hipEvent_t)events[1];
  }
  return forward_layer_impl(desc, t, block, epilogue, (hipStream_t)stream, events ? ev : nullptr);
}

int megamoe_layer_forward_w8a16(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                                const megamoe_epilogue* epilogue, void* stream, void* const* events) {
  if (epilogue && ((epilogue->swiglu != 0 && epilogue->swiglu != 1) || !(epilogue->swiglu_limit >= 0.0f)))
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[2];
  if (events) {
    if (!events[0] || !events[1]) return MEGAMOE_ERR_INVALID_ARGUMENT;
    ev[0] = (hipEvent_t)events[0];
    ev[1] = (hipEvent_t)events[1];
  }
  return forward_layer_impl(desc, t, block, epilogue, (hipStream_t)stream, events ? ev : nullptr, true);
}

int megamoe_layer_status(const megamoe_desc* desc, const void* workspace, size_t workspace_bytes, int32_t* gave_up,
                         void* stream) {
  const int rc = validate(desc);
  if (rc) return rc;
  if (!workspace || !gave_up) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const Layout L = make_layout(*desc);
  if (workspace_bytes < L.total) return MEGAMOE_ERR_WORKSPACE;
  int32_t v = 0;
  if (hipMemcpyAsync(&v, (const char*)workspace + L.ctl + kCtlStatus * sizeof(int), sizeof(v), hipMemcpyDeviceToHost,
                     (hipStream_t)stream) != hipSuccess ||
      hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
    return MEGAMOE_ERR_HIP;
  *gave_up = v;
  return MEGAMOE_OK;
}

int megamoe_forward_noalloc(const megamoe_desc* desc, const megamoe_tensors* t, void* stream) {
  int rc = validate(desc);
  if (rc) return rc;
  if (!t) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (make_layout(*desc).total > (size_t)MEGAMOE_SCRATCH_BYTES) return MEGAMOE_ERR_SCRATCH;
  void* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  megamoe_tensors with_scratch = *t;
  with_scratch.workspace = ws;
  with_scratch.workspace_bytes = MEGAMOE_SCRATCH_BYTES;
  return forward_impl(desc, &with_scratch, (hipStream_t)stream, nullptr);
}

int megamoe_forward_events(const megamoe_desc* desc, const megamoe_tensors* t, void* stream, void* const* events) {
  if (!events) return MEGAMOE_ERR_INVALID_ARGUMENT;
  for (int i = 0; i < kStages + 1; ++i)
    if (!events[i]) return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[kStages + 1];
  for (int i = 0; i < kStages + 1; ++i) ev[i] = (hipEvent_t)events[i];
  return forward_impl(desc, t, (hipStream_t)stream, ev);
}

int megamoe_forward_timed(const megamoe_desc* desc, const megamoe_tensors* t, void* stream, float* stage_ms) {
  if (!stage_ms) return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[kStages + 1];
  int made = 0, rc = MEGAMOE_OK;
  for (; made < kStages + 1; ++made)
    if (hipEventCreate(&ev[made]) != hipSuccess) {
      rc = MEGAMOE_ERR_HIP;
      break;
    }
  if (rc == MEGAMOE_OK) rc = forward_impl(desc, t, (hipStream_t)stream, ev);
  if (rc == MEGAMOE_OK && hipEventSynchronize(ev[kStages]) != hipSuccess) rc = MEGAMOE_ERR_HIP;
  for (int i = 0; rc == MEGAMOE_OK && i < kStages; ++i)
    if (hipEventElapsedTime(&stage_ms[i], ev[i], ev[i + 1]) != hipSuccess) rc = MEGAMOE_ERR_HIP;
  for (int i = 0; i < made; ++i) (void)hipEventDestroy(ev[i]);
  return rc;
}

int megamoe_router_logits(const megamoe_desc* desc, const void* x, const float* router, float* logits,
                          void* workspace, size_t workspace_bytes, void* stream) {
  int rc = validate(desc);
  if (rc) return rc;
  if (desc->tokens == 0) return MEGAMOE_OK;
  if (!x || !router || !logits || !workspace) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const Layout L = make_layout(*desc);
  if (workspace_bytes < L.total) return MEGAMOE_ERR_WORKSPACE;
  return launch_logits(*desc, L, x, router, (char*)workspace, logits, (hipStream_t)stream);
}

int megamoe_route(const megamoe_desc* desc, const float* logits, const float* bias, int64_t* expert_ids,
                  float* expert_weights, void* stream) {
  const int rc = validate(desc);
  if (rc) return rc;
  if (desc->tokens == 0) return MEGAMOE_OK;
  if (!logits || !expert_ids || !expert_weights) return MEGAMOE_ERR_INVALID_ARGUMENT;
  return launch_select(*desc, nullptr, 0, logits, bias, expert_ids, expert_weights, nullptr, nullptr, nullptr,
                       (hipStream_t)stream);
}

int megamoe_block_forward(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                          void* stream, void* const* events) {
  if (!block) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (!(block->eps >= 0.0f)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[kStages + 1];
  if (events) {
    for (int i = 0; i < kStages + 1; ++i) {
      if (!events[i]) return MEGAMOE_ERR_INVALID_ARGUMENT;
      ev[i] = (hipEvent_t)events[i];
    }
  }
  return forward_impl(desc, t, (hipStream_t)stream, events ? ev : nullptr, block);
}

int megamoe_forward_ex(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                       const megamoe_epilogue* epilogue, void* stream, void* const* events) {
  if (block && !(block->eps >= 0.0f)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (epilogue && ((epilogue->swiglu != 0 && epilogue->swiglu != 1) || !(epilogue->swiglu_limit >= 0.0f)))
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[kStages + 1];
  if (events) {
    for (int i = 0; i < kStages + 1; ++i) {
      if (!events[i]) return MEGAMOE_ERR_INVALID_ARGUMENT;
      ev[i] = (hipEvent_t)events[i];
    }
  }
  return forward_impl(desc, t, (hipStream_t)stream, events ? ev : nullptr, block, epilogue);
}

int megamoe_forward_w8a16(const megamoe_desc* desc, const megamoe_tensors* t, const megamoe_block* block,
                          const megamoe_epilogue* epilogue, void* stream, void* const* events) {
  if (block && !(block->eps >= 0.0f)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (epilogue && ((epilogue->swiglu != 0 && epilogue->swiglu != 1) || !(epilogue->swiglu_limit >= 0.0f)))
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[kStages + 1];
  if (events) {
    for (int i = 0; i < kStages + 1; ++i) {
      if (!events[i]) return MEGAMOE_ERR_INVALID_ARGUMENT;
      ev[i] = (hipEvent_t)events[i];
    }
  }
  return forward_impl(desc, t, (hipStream_t)stream, events ? ev : nullptr, block, epilogue, true);
}

int megamoe_combine_by_expert_id(int32_t tokens, int32_t hidden, int32_t topk, const void* expert_out,
                                 const int64_t* expert_ids, const void* weights, const void* residual, void* y,
                                 void* stream) {
  if (tokens < 0 || hidden <= 0 || topk <= 0 || hidden % 8) return MEGAMOE_ERR_SHAPE;
  if (topk > kMaxTopK) return MEGAMOE_ERR_UNSUPPORTED;
  if (tokens == 0) return MEGAMOE_OK;
  if (!expert_out || !expert_ids || !weights || !y) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (!aligned16(expert_out) || !aligned16(y) || (residual && !aligned16(residual))) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const int64_t work = (int64_t)tokens * (hidden / 8);
  if (work >= ((int64_t)1 << 31)) return MEGAMOE_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(k_combine_id_order, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)expert_out, expert_ids, (const uint16_t*)weights, (const uint16_t*)residual,
                     tokens, hidden, topk, (uint16_t*)y);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int megamoe_mx_workspace_bytes(const megamoe_desc* desc, size_t* bytes) {
  if (!bytes) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const int rc = validate_mx(desc);
  if (rc) return rc;
  *bytes = make_layout_mx(*desc).total;
  return MEGAMOE_OK;
}

int megamoe_mx_forward(const megamoe_desc* desc, float swiglu_limit, const megamoe_mx_tensors* t, void* stream,
                       void* const* events) {
  hipEvent_t ev[kStagesMx + 1];
  if (events) {
    for (int i = 0; i < kStagesMx + 1; ++i) {
      if (!events[i]) return MEGAMOE_ERR_INVALID_ARGUMENT;
      ev[i] = (hipEvent_t)events[i];
    }
  }
  return forward_mx_impl(desc, swiglu_limit, t, (hipStream_t)stream, events ? ev : nullptr);
}
int megamoe_mx_layer_forward(const megamoe_desc* desc, float swiglu_limit, const megamoe_mx_tensors* t,
                             void* stream, void* const* events) {
  hipEvent_t ev[2];
  if (events) {
    if (!events[0] || !events[1]) return MEGAMOE_ERR_INVALID_ARGUMENT;
    ev[0] = (hipEvent_t)events[0];
    ev[1] = (hipEvent_t)events[1];
  }
  return forward_mx_layer_impl(desc, swiglu_limit, t, (hipStream_t)stream, events ? ev : nullptr);
}
int megamoe_mx_layer_status(const megamoe_desc* desc, const void* workspace, size_t workspace_bytes, int32_t* failed,
                            void* stream) {
  const int rc = validate_mx(desc);
  if (rc) return rc;
  if (!workspace || !failed) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const LayoutMx L = make_layout_mx(*desc);
  if (workspace_bytes < L.total) return MEGAMOE_ERR_WORKSPACE;
  int32_t v = 0;
  if (hipMemcpyAsync(&v, (const char*)workspace + L.ctl + kCtlStatus * sizeof(int), sizeof(v), hipMemcpyDeviceToHost,
                     (hipStream_t)stream) != hipSuccess ||
      hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
    return MEGAMOE_ERR_HIP;
  *failed = v;
  return MEGAMOE_OK;
}

int megamoe_ep_dispatch(const megamoe_desc* desc, int32_t ep, const megamoe_mx_tensors* t,
                        const megamoe_ep_send* send, void* stream) {
  if (!desc || !t || !send) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const int64_t T = desc->tokens, H = desc->hidden, E = desc->experts, K = desc->topk;
  if (T < 0 || H <= 0 || E <= 0 || K <= 0 || K > E || H % kMxStageK || ep <= 0 || E % ep) return MEGAMOE_ERR_SHAPE;
  if (ep > kMaxRanks || T * K > kMaxDispatch) return MEGAMOE_ERR_UNSUPPORTED;
  if (!send->counts) return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipStream_t st = (hipStream_t)stream;
  const int n = (int)(T * K);
  // Workgroups per owner: about 512 in all, each packing at most kDispatchList entries.
  int m = 512 / ep;
  if (m < 1) m = 1;
  while ((int64_t)m * kDispatchList < n) ++m;
  if (n == 0) {  // zero counts, written by the kernel (no memset, so the call may be captured)
    hipLaunchKernelGGL(k_ep_dispatch, dim3((unsigned)ep), dim3(256), 16, st, (const int64_t*)nullptr,
                       (const uint8_t*)nullptr, (const uint8_t*)nullptr, (const float*)nullptr, 0, (int)K, (int)H,
                       (int)E, (int)(E / ep), 1, send->counts, (int32_t*)nullptr, (uint8_t*)nullptr,
                       (uint8_t*)nullptr, (int64_t*)nullptr, (float*)nullptr);
    MEGAMOE_LAUNCH_CHECK();
    return MEGAMOE_OK;
  }
  if (!t->x || !t->x_scales || !t->topk_idx || !t->topk_weights || !send->rows || !send->row_scales || !send->ids ||
      !send->weights || !send->slot_rows)
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (!aligned16(t->x) || !aligned16(send->rows) || ((uintptr_t)t->x_scales & 7) || ((uintptr_t)send->row_scales & 7))
    return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(k_ep_dispatch, dim3((unsigned)(ep * m)), dim3(256), (size_t)n, st, t->topk_idx, t->x,
                     t->x_scales, t->topk_weights, n, (int)K, (int)H, (int)E, (int)(E / ep), m, send->counts,
                     send->slot_rows, send->rows, send->row_scales, send->ids, send->weights);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int megamoe_ep_experts(const megamoe_desc* desc, float swiglu_limit, int64_t expert_base, const megamoe_mx_tensors* t,
                       void* stream, void* const* events) {
  if (!desc) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (desc->topk != 1) return MEGAMOE_ERR_SHAPE;
  if (expert_base < 0 || expert_base > ((int64_t)1 << 30)) return MEGAMOE_ERR_SHAPE;
  hipEvent_t ev[kStagesMx + 1];
  if (events) {
    for (int i = 0; i < kStagesMx + 1; ++i) {
      if (!events[i]) return MEGAMOE_ERR_INVALID_ARGUMENT;
      ev[i] = (hipEvent_t)events[i];
    }
  }
  return forward_mx_impl(desc, swiglu_limit, t, (hipStream_t)stream, events ? ev : nullptr, expert_base);
}

int megamoe_ep_combine(int32_t tokens, int32_t hidden, int32_t topk, const void* returned, const int32_t* slot_rows,
                       void* y, void* stream) {
  if (tokens < 0 || hidden <= 0 || topk <= 0 || hidden % 8) return MEGAMOE_ERR_SHAPE;
  if (tokens == 0) return MEGAMOE_OK;
  if (!returned || !slot_rows || !y) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (!aligned16(returned) || !aligned16(y)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const int64_t work = (int64_t)tokens * (hidden / 8);
  if (work >= ((int64_t)1 << 31)) return MEGAMOE_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(k_ep_combine, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)returned, slot_rows, tokens, hidden, topk, (uint16_t*)y);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int megamoe_rms_norm(int32_t rows, int32_t cols, const void* x, const void* weight, float eps,
                     int32_t weight_in_fp32, void* out, void* stream) {
  if (rows < 0 || cols < 0 || !(eps >= 0.0f)) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (cols % 8) return MEGAMOE_ERR_SHAPE;
  if (rows == 0 || cols == 0) return MEGAMOE_OK;
  if (!x || !weight || !out) return MEGAMOE_ERR_INVALID_ARGUMENT;
  return launch_norm(rows, cols, x, weight, eps, weight_in_fp32, out, (hipStream_t)stream);
}

int megamoe_quantize_rows(int32_t rows, int32_t cols, const void* x, uint8_t* q, float* scales, int32_t pow2,
                          void* stream) {
  if (rows < 0 || cols < 0) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (rows == 0 || cols == 0) return MEGAMOE_OK;
  if (!x || !q || !scales) return MEGAMOE_ERR_INVALID_ARGUMENT;
  return launch_quant(rows, cols, x, q, scales, pow2, (hipStream_t)stream);
}

int megamoe_e4m3_selftest(uint32_t first, uint32_t count, uint64_t* mismatches, void* stream) {
  if (!mismatches || (uint64_t)first + count > 0x80000000ull) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (count == 0) return MEGAMOE_OK;
  const uint32_t blocks = (count + 255u) / 256u;
  hipLaunchKernelGGL(k_e4m3_selftest, dim3(blocks < 8192u ? blocks : 8192u), dim3(256), 0, (hipStream_t)stream,
                     first, count, reinterpret_cast<unsigned long long*>(mismatches));
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

}  // extern "C"
