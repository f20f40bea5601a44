// megamoe.hip — FP8 (E4M3, 128x128 block-scaled) MoE decode layer for MI355X (gfx950).
//
// The layer, as six stream-ordered kernels (one process, one GPU):
//   k_router / k_quant_rows   router logits (fp64-accumulated GEMV over H splits) and the
//                             per-token-per-128 E4M3 quantization of x
//   k_select                  one wavefront per token: sigmoid/softmax gate, group-limited
//                             top-k with a (value desc, index asc) total order
//   k_permute                 one workgroup: expert histogram, exclusive scan, stable
//                             (token, slot)-ordered permutation, list of hit experts
//   k_gateup                  persistent grid over (hit expert, 128-row block of I) units:
//                             gate and up rows streamed from HBM into fp8 MFMA
//                             (16x16x128, weights as the M operand, tokens as N),
//                             128x128 block scales applied per K block, SwiGLU and the
//                             per-128 E4M3 requantization of h fused in the epilogue
//   k_down                    persistent grid over (hit expert, 128-row block of H) units
//   k_combine                 slot-order fp32 sum of bf16(d)*w plus the shared expert,
//                             rounded once to bf16
//
// Reference math (all eager PyTorch in the reference): megabench/tasks/frontier.py:180-186
// (linear), :229-242 (route), :335-354 (MoE block); megabench/tasks/quantization.py:57-131
// (FP8 formats); megabench/tasks/references/moe.py:66-78 and distributed.py:174-176
// (softmax routing); megabench/tasks/megamoe.py:131-150,161-168 (expert grouping order).

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "megamoe.h"

namespace {

constexpr int kBlock = 128;  // quantization block edge (weights 128x128, activations 1x128)

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------------------
// Router logits: partial[split][t][e] = sum over one H split of x[t,h] * W[e,h] in fp64.
// Products of a bf16 and an fp32 value are exact in fp64, so the only rounding that
// survives is the final fp64 -> fp32 one in k_select.
// ---------------------------------------------------------------------------------------

constexpr int kRouterE = 16;   // experts per workgroup
constexpr int kRouterT = 64;   // tokens per workgroup
constexpr int kRouterH = 256;  // hidden channels per split

__global__ __launch_bounds__(256) void k_router(const uint16_t* __restrict__ x, const float* __restrict__ w,
                                                double* __restrict__ partial, int T, int H, int E) {
  __shared__ float ws[kRouterE][kRouterH + 1];
  __shared__ uint16_t xs[kRouterT][kRouterH + 8];
  const int e0 = blockIdx.x * kRouterE, split = blockIdx.y, t0 = blockIdx.z * kRouterT;
  const int h0 = split * kRouterH;
  const int hc = min(kRouterH, H - h0);
  const int tid = threadIdx.x;

  for (int i = tid; i < kRouterE * (kRouterH / 4); i += 256) {
    const int r = i / (kRouterH / 4), c = (i % (kRouterH / 4)) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 + r < E && c < hc) v = *reinterpret_cast<const float4*>(w + (size_t)(e0 + r) * H + h0 + c);
    ws[r][c] = v.x;
    ws[r][c + 1] = v.y;
    ws[r][c + 2] = v.z;
    ws[r][c + 3] = v.w;
  }
  for (int i = tid; i < kRouterT * (kRouterH / 8); i += 256) {
    const int r = i / (kRouterH / 8), c = (i % (kRouterH / 8)) * 8;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (t0 + r < T && c < hc) v = *reinterpret_cast<const uint4*>(x + (size_t)(t0 + r) * H + h0 + c);
    *reinterpret_cast<uint4*>(&xs[r][c]) = v;
  }
  __syncthreads();

  const int el = tid % kRouterE, tg = tid / kRouterE;  // 16 experts x 16 token groups
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  for (int k = 0; k < hc; ++k) {
    const double wv = (double)ws[el][k];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = fma(wv, (double)bf16_bits_to_f32(xs[tg + 16 * j][k]), acc[j]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = t0 + tg + 16 * j, e = e0 + el;
    if (t < T && e < E) partial[((size_t)split * T + t) * E + e] = acc[j];
  }
}

// logits[t][e] = fp32(sum of the splits in split order)
__global__ __launch_bounds__(256) void k_logits(const double* __restrict__ partial, int nsplit, int T, int E,
                                                float* __restrict__ logits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)T * E) return;
  double s = 0.0;
  for (int p = 0; p < nsplit; ++p) s += partial[(size_t)p * T * E + i];
  logits[i] = (float)s;
}

// ---------------------------------------------------------------------------------------
// Dynamic E4M3 quantization, one wavefront per (row, 128-column block).
// ---------------------------------------------------------------------------------------

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
    if (c < cols) dst[c] = (uint8_t)f32_to_e4m3(clamp448(v0 / s));
    if (c + 1 < cols) dst[c + 1] = (uint8_t)f32_to_e4m3(clamp448(v1 / s));
    if (lane == 0) scales[(size_t)r * nb + cb] = s;
  }
}

// ---------------------------------------------------------------------------------------
// Routing, one wavefront per token. Lane l holds experts l, l+64, ...
// Selection order is (score descending, expert index ascending), the order a stable
// descending argsort produces (frontier.py:236,240; distributed.py:174).
// ---------------------------------------------------------------------------------------

constexpr int kMaxVPL = 16;  // experts per lane: E <= 1024
constexpr int kMaxTopK = 32;

__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

__global__ __launch_bounds__(64) void k_select(const double* __restrict__ partial, int nsplit,
                                               const float* __restrict__ logits_in, const float* __restrict__ bias,
                                               int T, int E, int K, int G, int TG, int gate, int renorm,
                                               float scaling, int64_t* __restrict__ ids_out,
                                               float* __restrict__ w_out) {
  const int t = blockIdx.x, lane = threadIdx.x;
  float logit[kMaxVPL], prob[kMaxVPL], choice[kMaxVPL];
#pragma unroll
  for (int j = 0; j < kMaxVPL; ++j) {
    const int e = lane + 64 * j;
    float v = -INFINITY;
    if (e < E) {
      if (logits_in) {
        v = logits_in[(size_t)t * E + e];
      } else {
        double s = 0.0;
        for (int p = 0; p < nsplit; ++p) s += partial[((size_t)p * T + t) * E + e];
        v = (float)s;
      }
    }
    logit[j] = v;
    if (gate == MEGAMOE_GATE_SIGMOID) {
      const float p = 1.0f / (1.0f + expf(-v));
      prob[j] = p;
      choice[j] = e < E ? p + (bias ? bias[e] : 0.0f) : -INFINITY;
    } else {
      prob[j] = v;
      choice[j] = v;
    }
  }

  if (G > 1) {
    // Group score: sum of the two largest choices in the group (frontier.py:234).
    const int gs = E / G;
    float my_group_score = -INFINITY;
    for (int g = 0; g < G; ++g) {
      float b1 = -INFINITY, b2 = -INFINITY;
#pragma unroll
      for (int j = 0; j < kMaxVPL; ++j) {
        const int e = lane + 64 * j;
        if (e < E && e / gs == g) {
          const float v = choice[j];
          if (v > b1) {
            b2 = b1;
            b1 = v;
          } else if (v > b2) {
            b2 = v;
          }
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float o1 = __shfl_xor(b1, o), o2 = __shfl_xor(b2, o);
        const float n2 = fmaxf(fminf(b1, o1), fmaxf(b2, o2));
        b1 = fmaxf(b1, o1);
        b2 = n2;
      }
      const float score = gs >= 2 ? b1 + b2 : b1;
      if (lane == g) my_group_score = score;
    }
    // Keep the top TG groups, ties to the lower group index (frontier.py:235).
    bool keep = false;
    for (int r = 0; r < TG; ++r) {
      float bv = (lane < G && !keep) ? my_group_score : -INFINITY;
      int bi = (lane < G && !keep) ? lane : 0x7fffffff;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ranks_before(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == bi) keep = true;
    }
    const unsigned long long kept = __ballot(keep);
#pragma unroll
    for (int j = 0; j < kMaxVPL; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !((kept >> (e / gs)) & 1ull)) choice[j] = -INFINITY;
    }
  }

  // Top-K, one expert per round.
  unsigned taken = 0u;
  int my_id = 0;
  float my_val = 0.0f;
  for (int r = 0; r < K; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kMaxVPL; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !((taken >> j) & 1u) && ranks_before(choice[j], e, bv, bi)) {
        bv = choice[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ranks_before(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    const int owner = bi & 63, slot = bi >> 6;
    float pv = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxVPL; ++j)
      if (j == slot) pv = prob[j];
    pv = __shfl(pv, owner);
    if (lane == owner) taken |= 1u << slot;
    if (lane == r) {
      my_id = bi;
      my_val = pv;
    }
  }

  // Weights, in slot order.
  float w = 0.0f;
  if (gate == MEGAMOE_GATE_SIGMOID) {
    if (renorm) {
      float s = 0.0f;
      for (int r = 0; r < K; ++r) s += __shfl(my_val, r);
      w = my_val / (s + 1e-20f) * scaling;
    } else {
      w = my_val * scaling;
    }
  } else if (renorm) {
    const float m = __shfl(my_val, 0);  // the first pick holds the largest logit
    const float ex = expf(my_val - m);
    float s = 0.0f;
    for (int r = 0; r < K; ++r) s += __shfl(ex, r);
    w = ex / s * scaling;
  } else {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMaxVPL; ++j) m = fmaxf(m, logit[j]);
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxVPL; ++j)
      if (lane + 64 * j < E) s += expf(logit[j] - m);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    w = expf(my_val - m) / s * scaling;
  }
  if (lane < K) {
    ids_out[(size_t)t * K + lane] = my_id;
    w_out[(size_t)t * K + lane] = w;
  }
}

// ---------------------------------------------------------------------------------------
// Histogram, scan and stable permutation in one workgroup (megamoe.py:138-149 order):
// rows of expert e are its (token, slot) entries in increasing token order, and each
// token picks an expert at most once, so an entry's rank is the number of earlier
// tokens that picked the same expert: a popcount over a per-expert token bitmap.
// ---------------------------------------------------------------------------------------

__device__ int block_exclusive_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wid] = x;
  __syncthreads();
  if (wid == 0) {
    int s = lane < nw ? tmp[lane] : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(s, o);
      if (lane >= o) s += y;
    }
    if (lane < nw) tmp[lane] = s;
  }
  __syncthreads();
  const int base = wid ? tmp[wid - 1] : 0;
  *total = tmp[nw - 1];
  __syncthreads();
  return base + x - v;
}

struct PermuteOut {
  int* counts;   // [E]
  int* offsets;  // [E+1]
  int* hit;      // [E] hit experts in increasing order
  int* meta;     // [0] hit count U, [1] gate/up units, [2] down units
  int* perm;     // [T*K] row -> flat (token*K + slot)
  int* inv;      // [T*K] flat -> row
};

__global__ __launch_bounds__(1024) void k_permute(const int64_t* __restrict__ ids, int T, int K, int E,
                                                  int units_shared_gu, int units_per_expert_gu,
                                                  int units_shared_dn, int units_per_expert_dn, PermuteOut out) {
  extern __shared__ int smem[];
  int* cnt = smem;             // E
  int* tmp = cnt + E;          // 16
  unsigned* bm = (unsigned*)(tmp + 16);  // E * words
  const int words = (T + 31) / 32;
  const int tid = threadIdx.x, n = T * K;
  for (int i = tid; i < E; i += blockDim.x) cnt[i] = 0;
  for (int i = tid; i < E * words; i += blockDim.x) bm[i] = 0u;
  __syncthreads();
  for (int i = tid; i < n; i += blockDim.x) {
    const int e = (int)ids[i], t = i / K;
    atomicAdd(&cnt[e], 1);
    atomicOr(&bm[e * words + (t >> 5)], 1u << (t & 31));
  }
  __syncthreads();
  // E <= 1024 = blockDim: one expert per thread for the scans.
  const int c = tid < E ? cnt[tid] : 0;
  int total = 0, nhit = 0;
  const int off = block_exclusive_scan(c, tmp, &total);
  const int hpos = block_exclusive_scan(c > 0 ? 1 : 0, tmp, &nhit);
  if (tid < E) {
    out.counts[tid] = c;
    out.offsets[tid] = off;
    if (c > 0) out.hit[hpos] = tid;
    cnt[tid] = off;  // reuse as offsets
  }
  if (tid == 0) {
    out.offsets[E] = total;
    out.meta[0] = nhit;
    out.meta[1] = units_shared_gu + nhit * units_per_expert_gu;
    out.meta[2] = units_shared_dn + nhit * units_per_expert_dn;
  }
  __syncthreads();
  for (int i = tid; i < n; i += blockDim.x) {
    const int e = (int)ids[i], t = i / K;
    const unsigned* row = bm + e * words;
    int rank = __popc(row[t >> 5] & ((1u << (t & 31)) - 1u));
    for (int q = 0; q < (t >> 5); ++q) rank += __popc(row[q]);
    const int pos = cnt[e] + rank;
    out.perm[pos] = i;
    out.inv[i] = pos;
  }
}

// ---------------------------------------------------------------------------------------
// Expert GEMM core. One wavefront multiplies RT row tiles (16 weight rows each) by NCT
// column tiles (16 activation rows each) over the whole reduction axis with
// v_mfma_scale_f32_16x16x128_f8f6f4 (E4M3 x E4M3, unit E8M0 scales): one MFMA per
// (row tile, column tile, 128-wide K block), so each 128x128 weight scale block and each
// 1x128 activation scale block meets exactly one MFMA result, which is scaled in fp32
// and added to the accumulator.
//
// Operand layout: lane l supplies row (l % 16) of its tile and the 32 K bytes
// [16*(l/16), +16) and [64 + 16*(l/16), +16) of the block, the same byte positions for
// the weight (A) and the activation (B) operand, so A and B agree on K. Each 16-byte
// load instruction of a wavefront covers 64 contiguous bytes of 16 rows. Result layout:
// lane l holds rows 4*(l/16) .. +3 of column (l % 16).
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ f32x4 mfma_e4m3(const i32x8& a, const i32x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

__device__ __forceinline__ i32x8 load_k32(const uint8_t* p) {
  const i32x4 lo = *reinterpret_cast<const i32x4*>(p);
  const i32x4 hi = *reinterpret_cast<const i32x4*>(p + 64);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <int RT, int NCT, int SG>
struct Stage {
  i32x8 a[RT];
  i32x8 b[NCT];
  float sw[SG];
  float sx[NCT];
};

template <int RT, int NCT, int SG>
struct Operands {
  const uint8_t* a[RT];    // lane's weight row at its K byte offset
  const float* sw[SG];     // per-K-block weight scales of scale group g (wave-uniform)
  const uint8_t* b[NCT];   // lane's activation row at its K byte offset
  const float* sx[NCT];    // lane's activation scale row
};

template <int RT, int NCT, int SG>
__device__ __forceinline__ void load_stage(Stage<RT, NCT, SG>& s, const Operands<RT, NCT, SG>& op, int kb) {
  const size_t o = (size_t)kb * kBlock;
#pragma unroll
  for (int r = 0; r < RT; ++r) s.a[r] = load_k32(op.a[r] + o);
#pragma unroll
  for (int c = 0; c < NCT; ++c) s.b[c] = load_k32(op.b[c] + o);
#pragma unroll
  for (int g = 0; g < SG; ++g) s.sw[g] = op.sw[g][kb];
#pragma unroll
  for (int c = 0; c < NCT; ++c) s.sx[c] = op.sx[c][kb];
}

template <int RT, int NCT, int SG>
__device__ __forceinline__ void compute_stage(const Stage<RT, NCT, SG>& s, f32x4 (&acc)[RT][NCT]) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RT; ++r) {
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      const f32x4 p = mfma_e4m3(s.a[r], s.b[c], zero);
      const float k = s.sw[r * SG / RT] * s.sx[c];
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[r][c][v] = __builtin_fmaf(p[v], k, acc[r][c][v]);
    }
  }
}

// Streams nkb K blocks with D stages of loads in flight per wavefront.
template <int RT, int NCT, int SG, int D>
__device__ __forceinline__ void stream_gemm(const Operands<RT, NCT, SG>& op, int nkb, f32x4 (&acc)[RT][NCT]) {
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int c = 0; c < NCT; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  Stage<RT, NCT, SG> st[D];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) load_stage(st[s], op, min(s, nkb - 1));
  for (int kb0 = 0; kb0 < nkb; kb0 += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int kb = kb0 + s;
      // The load index is clamped rather than skipped so the loop body stays
      // branch-free; the clamped tail re-reads the last block, which is in cache.
      load_stage(st[(s + D - 1) % D], op, min(kb + D - 1, nkb - 1));
      if (kb < nkb) compute_stage(st[s], acc);
    }
  }
}

// Work unit description shared by the two expert kernels.
struct ExpertRows {
  int n;            // rows (token, slot entries) of this expert
  int row0;         // first output row in the grouped buffers
  const int* perm;  // grouped row -> token*K + slot, or NULL for the shared expert (row = token)
  int K;
};

__device__ __forceinline__ int row_token(const ExpertRows& er, int r) {
  return er.perm ? er.perm[er.row0 + r] / er.K : r;
}

struct GateUpArgs {
  const uint8_t* xq;   // [T, H] e4m3
  const float* xs;     // [T, H/128]
  const uint8_t* gate; const float* gate_scale;
  const uint8_t* up; const float* up_scale;
  const uint8_t* sgate; const float* sgate_scale;
  const uint8_t* sup; const float* sup_scale;
  const int* counts; const int* offsets; const int* hit; const int* meta; const int* perm;
  uint8_t* hq_r; float* hs_r;   // routed rows [T*K, I], [T*K, I/128]
  uint8_t* hq_s; float* hs_s;   // shared rows [T, S*I], [T, S*I/128]
  int T, H, I, K, S, pow2;
};

// One gate/up unit: rows [j*128, j*128+128) of gate and of up against the activation
// rows c0 .. c0+16*NCT-1 of the expert. Wave w owns gate and up rows 32w .. 32w+31 of the
// block, so SwiGLU pairs matching registers; the per-row amax over the 128-block for the
// requantization of h is reduced across the four wavefronts through LDS.
template <int NCT>
__device__ void gateup_chunk(const GateUpArgs& a, const uint8_t* wg, const uint8_t* wu, const float* sg,
                             const float* su, const ExpertRows& er, int c0, int j, uint8_t* hq, float* hs,
                             int ldh, float (*red)[64]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kofs = 16 * (lane >> 4);
  const int H = a.H, nkb = H / kBlock, nbh = ldh / kBlock;
  Operands<4, NCT, 2> op;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const size_t row = (size_t)(32 * w + 16 * r + (lane & 15));
    op.a[r] = wg + row * H + kofs;
    op.a[r + 2] = wu + row * H + kofs;
  }
  op.sw[0] = sg;
  op.sw[1] = su;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = min(c0 + 16 * c + (lane & 15), er.n - 1);  // padding columns repeat a valid row
    const int tok = row_token(er, r);
    op.b[c] = a.xq + (size_t)tok * H + kofs;
    op.sx[c] = a.xs + (size_t)tok * nkb;
  }
  f32x4 acc[4][NCT];
  stream_gemm<4, NCT, 2, 3>(op, nkb, acc);

  // h = bf16(silu(fp32 bf16(g)) * fp32 bf16(u)) (frontier.py:184-186,337)
  float hv[NCT][2][4];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float g = round_bf16(acc[p][c][v]);
        const float u = round_bf16(acc[p + 2][c][v]);
        const float h = round_bf16(silu(g) * u);
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
    const int r = c0 + col;
    if (r < er.n) {
      uint8_t* dst = hq + (size_t)(er.row0 + r) * ldh + (size_t)j * kBlock + 32 * w + 4 * (lane >> 4);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        uint32_t packed = 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) packed |= f32_to_e4m3(clamp448(hv[c][p][v] / s)) << (8 * v);
        *reinterpret_cast<uint32_t*>(dst + 16 * p) = packed;
      }
      if (w == 0 && lane < 16) hs[(size_t)(er.row0 + r) * nbh + j] = s;
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(256) void k_gateup(GateUpArgs a) {
  __shared__ float red[4][64];
  const int nbI = a.I / kBlock, nkb = a.H / kBlock;
  const int nsh = a.S * nbI;  // shared expert: S*I rows of gate/up
  const int total = a.meta[1];
  for (int u = blockIdx.x; u < total; u += gridDim.x) {
    const uint8_t *wg, *wu;
    const float *sg, *su;
    ExpertRows er;
    uint8_t* hq;
    float* hs;
    int ldh, j;
    if (u < nsh) {
      j = u;
      wg = a.sgate + (size_t)j * kBlock * a.H;
      wu = a.sup + (size_t)j * kBlock * a.H;
      sg = a.sgate_scale + (size_t)j * nkb;
      su = a.sup_scale + (size_t)j * nkb;
      er = ExpertRows{a.T, 0, nullptr, a.K};
      hq = a.hq_s;
      hs = a.hs_s;
      ldh = a.S * a.I;
    } else {
      const int v = u - nsh, e = a.hit[v / nbI];
      j = v % nbI;
      const size_t rowblk = (size_t)e * nbI + j;
      wg = a.gate + rowblk * kBlock * a.H;
      wu = a.up + rowblk * kBlock * a.H;
      sg = a.gate_scale + rowblk * nkb;
      su = a.up_scale + rowblk * nkb;
      er = ExpertRows{a.counts[e], a.offsets[e], a.perm, a.K};
      hq = a.hq_r;
      hs = a.hs_r;
      ldh = a.I;
    }
    // Experts with more than 16 rows stream their unit once per 16 rows.
    for (int c0 = 0; c0 < er.n; c0 += 16) gateup_chunk<1>(a, wg, wu, sg, su, er, c0, j, hq, hs, ldh, red);
  }
}

struct DownArgs {
  const uint8_t* down; const float* down_scale;
  const uint8_t* sdown; const float* sdown_scale;
  const int* counts; const int* offsets; const int* hit; const int* meta; const int* perm;
  const uint8_t* hq_r; const float* hs_r;
  const uint8_t* hq_s; const float* hs_s;
  uint16_t* d_r;  // [T*K, H] bf16, grouped rows
  uint16_t* d_s;  // [T, H] bf16
  int T, H, I, K, S;
};

// One down unit: rows [j*128, j*128+128) of the down matrix [H, ldk] against the
// expert's requantized h rows. Wave w owns rows 32w .. 32w+31.
template <int NCT>
__device__ void down_chunk(const DownArgs& a, const uint8_t* wd, const float* sd, int ldk, const uint8_t* hq,
                           const float* hs, const ExpertRows& er, int c0, int j, uint16_t* d) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kofs = 16 * (lane >> 4);
  const int nkb = ldk / kBlock;
  Operands<2, NCT, 1> op;
#pragma unroll
  for (int r = 0; r < 2; ++r) op.a[r] = wd + (size_t)(32 * w + 16 * r + (lane & 15)) * ldk + kofs;
  op.sw[0] = sd;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = min(c0 + 16 * c + (lane & 15), er.n - 1);
    op.b[c] = hq + (size_t)(er.row0 + r) * ldk + kofs;
    op.sx[c] = hs + (size_t)(er.row0 + r) * nkb;
  }
  f32x4 acc[2][NCT];
  stream_gemm<2, NCT, 1, 4>(op, nkb, acc);
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int r = c0 + 16 * c + (lane & 15);
    if (r < er.n) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint32_t lo = f32_to_bf16_bits(acc[p][c][0]) | (f32_to_bf16_bits(acc[p][c][1]) << 16);
        const uint32_t hi = f32_to_bf16_bits(acc[p][c][2]) | (f32_to_bf16_bits(acc[p][c][3]) << 16);
        uint16_t* dst = d + (size_t)(er.row0 + r) * a.H + (size_t)j * kBlock + 32 * w + 16 * p + 4 * (lane >> 4);
        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
      }
    }
  }
}

__global__ __launch_bounds__(256) void k_down(DownArgs a) {
  const int nbH = a.H / kBlock, nbI = a.I / kBlock;
  const int nsh = a.S > 0 ? nbH : 0;
  const int total = a.meta[2];
  for (int u = blockIdx.x; u < total; u += gridDim.x) {
    const uint8_t* wd;
    const float* sd;
    const uint8_t* hq;
    const float* hs;
    uint16_t* d;
    int ldk, j;
    ExpertRows er;
    if (u < nsh) {
      j = u;
      ldk = a.S * a.I;
      wd = a.sdown + (size_t)j * kBlock * ldk;
      sd = a.sdown_scale + (size_t)j * (ldk / kBlock);
      hq = a.hq_s;
      hs = a.hs_s;
      d = a.d_s;
      er = ExpertRows{a.T, 0, nullptr, a.K};
    } else {
      const int v = u - nsh, e = a.hit[v / nbH];
      j = v % nbH;
      ldk = a.I;
      const size_t rowblk = (size_t)e * nbH + j;
      wd = a.down + rowblk * kBlock * ldk;
      sd = a.down_scale + rowblk * nbI;
      hq = a.hq_r;
      hs = a.hs_r;
      d = a.d_r;
      er = ExpertRows{a.counts[e], a.offsets[e], a.perm, a.K};
    }
    for (int c0 = 0; c0 < er.n; c0 += 16) down_chunk<1>(a, wd, sd, ldk, hq, hs, er, c0, j, d);
  }
}

// y[t] = bf16( sum_slot fp32(d[t,slot]) * w[t,slot]  (slot order, each product rounded)
//              + fp32(shared[t]) )                      frontier.py:349-354
__global__ __launch_bounds__(256) void k_combine(const uint16_t* __restrict__ d_r, const uint16_t* __restrict__ d_s,
                                                 const int* __restrict__ inv, const float* __restrict__ wts, int H,
                                                 int K, int S, uint16_t* __restrict__ y) {
  const int t = blockIdx.y;
  const int h0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (h0 >= H) return;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int s = 0; s < K; ++s) {
    const int pos = inv[t * K + s];
    const float wv = wts[t * K + s];
    const uint4 v = *reinterpret_cast<const uint4*>(d_r + (size_t)pos * H + h0);
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(bf16_bits_to_f32(q[i] & 0xffffu), wv));
      acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(bf16_bits_to_f32(q[i] >> 16), wv));
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
  uint4 o;
  o.x = f32_to_bf16_bits(acc[0]) | (f32_to_bf16_bits(acc[1]) << 16);
  o.y = f32_to_bf16_bits(acc[2]) | (f32_to_bf16_bits(acc[3]) << 16);
  o.z = f32_to_bf16_bits(acc[4]) | (f32_to_bf16_bits(acc[5]) << 16);
  o.w = f32_to_bf16_bits(acc[6]) | (f32_to_bf16_bits(acc[7]) << 16);
  *reinterpret_cast<uint4*>(y + (size_t)t * H + h0) = o;
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Layout {
  size_t partial, xq, xs, counts, offsets, hit, meta, perm, inv, hq_r, hs_r, hq_s, hs_s, d_r, d_s, total;
  int nsplit;
};

Layout make_layout(const megamoe_desc& d) {
  Layout L{};
  const size_t T = d.tokens, H = d.hidden, E = d.experts, K = d.topk, I = d.intermediate, S = d.shared_experts;
  L.nsplit = (int)((H + kRouterH - 1) / kRouterH);
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t o = at;
    at += align_up(bytes > 0 ? bytes : 1);
    return o;
  };
  L.partial = take((size_t)L.nsplit * T * E * sizeof(double));
  L.xq = take(T * H);
  L.xs = take(T * (H / kBlock) * sizeof(float));
  L.counts = take(E * sizeof(int));
  L.offsets = take((E + 1) * sizeof(int));
  L.hit = take(E * sizeof(int));
  L.meta = take(16 * sizeof(int));
  L.perm = take(T * K * sizeof(int));
  L.inv = take(T * K * sizeof(int));
  L.hq_r = take(T * K * I);
  L.hs_r = take(T * K * (I / kBlock) * sizeof(float));
  L.hq_s = take(T * S * I);
  L.hs_s = take(T * (S * I / kBlock) * sizeof(float));
  L.d_r = take(T * K * H * 2);
  L.d_s = take(T * H * 2);
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
  if (d->experts > 64 * kMaxVPL || d->topk > kMaxTopK || d->groups > 64) return MEGAMOE_ERR_UNSUPPORTED;
  // Permute bitmap in LDS: (E counts + 16 scan words + E*ceil(T/32) bitmap words) * 4 bytes.
  const size_t words = ((size_t)d->tokens + 31) / 32;
  if (((size_t)d->experts * (1 + words) + 16) * 4 > 64 * 1024) return MEGAMOE_ERR_UNSUPPORTED;
  if ((size_t)d->tokens * d->topk > (size_t)1 << 30) return MEGAMOE_ERR_UNSUPPORTED;
  return MEGAMOE_OK;
}

struct DeviceInfo {
  int cus = 0;
  int gateup_per_cu = 0;
  int down_per_cu = 0;
};

int device_info(DeviceInfo* out) {
  static DeviceInfo cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return MEGAMOE_ERR_HIP;
  DeviceInfo& di = cache[dev];
  if (di.cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return MEGAMOE_ERR_HIP;
    int g = 0, dn = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&g, k_gateup, 256, 0) != hipSuccess) return MEGAMOE_ERR_HIP;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&dn, k_down, 256, 0) != hipSuccess) return MEGAMOE_ERR_HIP;
    di.gateup_per_cu = g > 0 ? g : 1;
    di.down_per_cu = dn > 0 ? dn : 1;
    di.cus = cus > 0 ? cus : 1;
  }
  *out = di;
  return MEGAMOE_OK;
}

#define MEGAMOE_LAUNCH_CHECK()                              \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return MEGAMOE_ERR_HIP; \
  } while (0)

int launch_router(const megamoe_desc& d, const Layout& L, const void* x, const float* router, char* ws,
                  hipStream_t st) {
  const dim3 grid((d.experts + kRouterE - 1) / kRouterE, L.nsplit, (d.tokens + kRouterT - 1) / kRouterT);
  hipLaunchKernelGGL(k_router, grid, dim3(256), 0, st, (const uint16_t*)x, router, (double*)(ws + L.partial),
                     d.tokens, d.hidden, d.experts);
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

int forward_impl(const megamoe_desc* desc, const megamoe_tensors* t, hipStream_t st, hipEvent_t* ev) {
  int rc = validate(desc);
  if (rc) return rc;
  if (!t) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const megamoe_desc& d = *desc;
  if (d.tokens == 0) {
    if (ev)
      for (int i = 0; i < 7; ++i)
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
  if ((rc = launch_router(d, L, t->x, t->router, ws, st))) return rc;
  if ((rc = launch_quant(T, H, t->x, (uint8_t*)(ws + L.xq), (float*)(ws + L.xs), d.pow2_scales, st))) return rc;
  if (mark(1) != hipSuccess) return MEGAMOE_ERR_HIP;

  hipLaunchKernelGGL(k_select, dim3(T), dim3(64), 0, st, (const double*)(ws + L.partial), L.nsplit,
                     (const float*)nullptr, t->router_bias, T, E, K, d.groups, d.top_groups, d.gate, d.renormalize,
                     d.routed_scaling, t->expert_ids, t->expert_weights);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(2) != hipSuccess) return MEGAMOE_ERR_HIP;

  PermuteOut po{(int*)(ws + L.counts), (int*)(ws + L.offsets), (int*)(ws + L.hit),
                (int*)(ws + L.meta),   (int*)(ws + L.perm),    (int*)(ws + L.inv)};
  const int nbI = I / kBlock, nbH = H / kBlock;
  const size_t lds = ((size_t)E * (1 + (T + 31) / 32) + 16) * 4;
  hipLaunchKernelGGL(k_permute, dim3(1), dim3(1024), lds, st, t->expert_ids, T, K, E, S * nbI, nbI,
                     S > 0 ? nbH : 0, nbH, po);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(3) != hipSuccess) return MEGAMOE_ERR_HIP;

  GateUpArgs ga;
  ga.xq = (const uint8_t*)(ws + L.xq);
  ga.xs = (const float*)(ws + L.xs);
  ga.gate = t->gate; ga.gate_scale = t->gate_scale;
  ga.up = t->up; ga.up_scale = t->up_scale;
  ga.sgate = t->shared_gate; ga.sgate_scale = t->shared_gate_scale;
  ga.sup = t->shared_up; ga.sup_scale = t->shared_up_scale;
  ga.counts = po.counts; ga.offsets = po.offsets; ga.hit = po.hit; ga.meta = po.meta; ga.perm = po.perm;
  ga.hq_r = (uint8_t*)(ws + L.hq_r); ga.hs_r = (float*)(ws + L.hs_r);
  ga.hq_s = (uint8_t*)(ws + L.hq_s); ga.hs_s = (float*)(ws + L.hs_s);
  ga.T = T; ga.H = H; ga.I = I; ga.K = K; ga.S = S; ga.pow2 = d.pow2_scales;
  hipLaunchKernelGGL(k_gateup, dim3(di.cus * di.gateup_per_cu), dim3(256), 0, st, ga);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(4) != hipSuccess) return MEGAMOE_ERR_HIP;

  DownArgs da;
  da.down = t->down; da.down_scale = t->down_scale;
  da.sdown = t->shared_down; da.sdown_scale = t->shared_down_scale;
  da.counts = po.counts; da.offsets = po.offsets; da.hit = po.hit; da.meta = po.meta; da.perm = po.perm;
  da.hq_r = ga.hq_r; da.hs_r = ga.hs_r; da.hq_s = ga.hq_s; da.hs_s = ga.hs_s;
  da.d_r = (uint16_t*)(ws + L.d_r); da.d_s = (uint16_t*)(ws + L.d_s);
  da.T = T; da.H = H; da.I = I; da.K = K; da.S = S;
  hipLaunchKernelGGL(k_down, dim3(di.cus * di.down_per_cu), dim3(256), 0, st, da);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(5) != hipSuccess) return MEGAMOE_ERR_HIP;

  hipLaunchKernelGGL(k_combine, dim3((H / 8 + 255) / 256, T), dim3(256), 0, st, (const uint16_t*)da.d_r,
                     (const uint16_t*)da.d_s, (const int*)po.inv, (const float*)t->expert_weights, H, K, S,
                     (uint16_t*)t->y);
  MEGAMOE_LAUNCH_CHECK();
  if (mark(6) != hipSuccess) return MEGAMOE_ERR_HIP;
  return MEGAMOE_OK;
}

}  // namespace

extern "C" {

int megamoe_abi_version(void) { return 1; }

const char* megamoe_status_string(int status) {
  switch (status) {
    case MEGAMOE_OK: return "ok";
    case MEGAMOE_ERR_INVALID_ARGUMENT: return "invalid argument (a required pointer is NULL)";
    case MEGAMOE_ERR_SHAPE: return "invalid MoE geometry";
    case MEGAMOE_ERR_WORKSPACE: return "workspace smaller than megamoe_workspace_bytes()";
    case MEGAMOE_ERR_HIP: return "HIP runtime error";
    case MEGAMOE_ERR_UNSUPPORTED: return "geometry beyond this build's limits";
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

int megamoe_forward_timed(const megamoe_desc* desc, const megamoe_tensors* t, void* stream, float* stage_ms) {
  if (!stage_ms) return MEGAMOE_ERR_INVALID_ARGUMENT;
  hipEvent_t ev[7];
  int made = 0, rc = MEGAMOE_OK;
  for (; made < 7; ++made)
    if (hipEventCreate(&ev[made]) != hipSuccess) {
      rc = MEGAMOE_ERR_HIP;
      break;
    }
  if (rc == MEGAMOE_OK) rc = forward_impl(desc, t, (hipStream_t)stream, ev);
  if (rc == MEGAMOE_OK && hipEventSynchronize(ev[6]) != hipSuccess) rc = MEGAMOE_ERR_HIP;
  for (int i = 0; rc == MEGAMOE_OK && i < 6; ++i)
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
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  if ((rc = launch_router(*desc, L, x, router, ws, st))) return rc;
  const size_t n = (size_t)desc->tokens * desc->experts;
  hipLaunchKernelGGL(k_logits, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (const double*)(ws + L.partial),
                     L.nsplit, desc->tokens, desc->experts, logits);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int megamoe_route(const megamoe_desc* desc, const float* logits, const float* bias, int64_t* expert_ids,
                  float* expert_weights, void* stream) {
  const int rc = validate(desc);
  if (rc) return rc;
  if (desc->tokens == 0) return MEGAMOE_OK;
  if (!logits || !expert_ids || !expert_weights) return MEGAMOE_ERR_INVALID_ARGUMENT;
  const megamoe_desc& d = *desc;
  hipLaunchKernelGGL(k_select, dim3(d.tokens), dim3(64), 0, (hipStream_t)stream, (const double*)nullptr, 0, logits,
                     bias, d.tokens, d.experts, d.topk, d.groups, d.top_groups, d.gate, d.renormalize,
                     d.routed_scaling, expert_ids, expert_weights);
  MEGAMOE_LAUNCH_CHECK();
  return MEGAMOE_OK;
}

int megamoe_quantize_rows(int32_t rows, int32_t cols, const void* x, uint8_t* q, float* scales, int32_t pow2,
                          void* stream) {
  if (rows < 0 || cols < 0) return MEGAMOE_ERR_INVALID_ARGUMENT;
  if (rows == 0 || cols == 0) return MEGAMOE_OK;
  if (!x || !q || !scales) return MEGAMOE_ERR_INVALID_ARGUMENT;
  return launch_quant(rows, cols, x, q, scales, pow2, (hipStream_t)stream);
}

}  // extern "C"
