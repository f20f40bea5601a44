/*
 * codec.c — plain-C restatement of the byte and integer parts of the FP8 MoE layer.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (ctypes) as an independent checker.
 *
 * The rounding functions are written differently from the GPU kernels on purpose
 * (search over the code table and distance comparison, not bit arithmetic), so a
 * mistake in one is unlikely to be repeated in the other.
 *
 *   oc_e4m3_to_f32 / oc_f32_to_e4m3   E4M3FN decode / round-to-nearest-even encode with
 *                                     the +-448 clamp of megabench/tasks/quantization.py:106,125
 *   oc_f32_to_bf16                    round to nearest even (torch .to(torch.bfloat16))
 *   oc_select                         group-limited stable top-k on choice values
 *                                     (megabench/tasks/frontier.py:232-240)
 *   oc_permute                        histogram, exclusive scan, stable permutation
 *                                     (megabench/tasks/megamoe.py:138-149)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static uint32_t bits_of(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

static float float_of(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* Magnitude of a non-negative finite code 0x00..0x7e: (8+m)*2^(e-10), or m*2^-9 if e == 0. */
static double e4m3_magnitude(int code) {
  const int e = (code >> 3) & 15, m = code & 7;
  return e == 0 ? ldexp((double)m, -9) : ldexp((double)(8 + m), e - 10);
}

float oc_e4m3_to_f32(uint8_t code) {
  const int sign = code >> 7, mag = code & 0x7f;
  if (mag == 0x7f) return sign ? -NAN : NAN;
  const float v = (float)e4m3_magnitude(mag);
  return sign ? -v : v;
}

uint8_t oc_f32_to_e4m3(float x) {
  const uint8_t sign = (uint8_t)((bits_of(x) >> 31) << 7);
  if (isnan(x)) return (uint8_t)(sign | 0x7f);
  double a = fabs((double)x);
  if (a >= 448.0) return (uint8_t)(sign | 0x7e);
  int lo = 0, hi = 0x7e; /* magnitude(lo) <= a < magnitude(hi) */
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    if (e4m3_magnitude(mid) <= a)
      lo = mid;
    else
      hi = mid;
  }
  const double mid = 0.5 * (e4m3_magnitude(lo) + e4m3_magnitude(hi));
  int code;
  if (a < mid)
    code = lo;
  else if (a > mid)
    code = hi;
  else
    code = (lo & 1) ? hi : lo; /* tie: the even code */
  return (uint8_t)(sign | code);
}

void oc_f32_to_e4m3_array(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oc_f32_to_e4m3(x[i]);
}

uint16_t oc_f32_to_bf16(float x) {
  const uint32_t u = bits_of(x);
  if (isnan(x)) return 0x7fc0;
  const uint32_t down = u & 0xffff0000u; /* truncation toward zero */
  if (down == u) return (uint16_t)(u >> 16);
  const uint32_t up = down + 0x10000u;   /* next bf16 away from zero; may be infinity */
  const double vd = (double)float_of(down);
  /* Rounding to nearest treats the step past the largest finite value as 2^128. */
  const double vu = isinf(float_of(up)) ? copysign(ldexp(1.0, 128), (double)x) : (double)float_of(up);
  const double dd = fabs((double)x - vd), du = fabs(vu - (double)x);
  if (dd < du) return (uint16_t)(down >> 16);
  if (dd > du) return (uint16_t)(up >> 16);
  return (uint16_t)((((down >> 16) & 1u) ? up : down) >> 16); /* tie: even */
}

void oc_f32_to_bf16_array(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oc_f32_to_bf16(x[i]);
}

/* a ranks before b: larger value, then lower index (a stable descending sort). */
static int before(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

/* Insertion sort of idx[0..n) by (value desc, index asc). */
static void order(const float* v, int* idx, int n) {
  for (int i = 1; i < n; ++i) {
    const int k = idx[i];
    int j = i - 1;
    while (j >= 0 && before(v[k], k, v[idx[j]], idx[j])) {
      idx[j + 1] = idx[j];
      --j;
    }
    idx[j + 1] = k;
  }
}

/* Group-limited top-k of one token. choice[E]; groups G divide E; top_groups kept.
 * Returns 0, or -1 on bad arguments. ids[K] in selection order. */
int oc_select(const float* choice, int E, int K, int G, int top_groups, int64_t* ids) {
  if (E <= 0 || K <= 0 || K > E || G <= 0 || E % G || top_groups <= 0 || top_groups > G) return -1;
  float* c = (float*)malloc(sizeof(float) * (size_t)E);
  int* idx = (int*)malloc(sizeof(int) * (size_t)E);
  if (!c || !idx) {
    free(c);
    free(idx);
    return -1;
  }
  memcpy(c, choice, sizeof(float) * (size_t)E);
  if (G > 1) {
    const int gs = E / G;
    float* score = (float*)malloc(sizeof(float) * (size_t)G);
    int* gidx = (int*)malloc(sizeof(int) * (size_t)G);
    for (int g = 0; g < G; ++g) {
      for (int i = 0; i < gs; ++i) idx[i] = g * gs + i;
      order(c, idx, gs);
      score[g] = gs >= 2 ? c[idx[0]] + c[idx[1]] : c[idx[0]];
      gidx[g] = g;
    }
    order(score, gidx, G);
    for (int g = 0; g < G; ++g) {
      int kept = 0;
      for (int r = 0; r < top_groups; ++r) kept |= gidx[r] == g;
      if (!kept)
        for (int i = 0; i < gs; ++i) c[g * gs + i] = -INFINITY;
    }
    free(score);
    free(gidx);
  }
  for (int i = 0; i < E; ++i) idx[i] = i;
  order(c, idx, E);
  for (int r = 0; r < K; ++r) ids[r] = idx[r];
  free(c);
  free(idx);
  return 0;
}

/* Expert histogram, exclusive scan and the permutation that lists each expert's
 * (token, slot) entries in flat order. perm[row] = flat index, inv[flat] = row.
 * Returns the number of experts with at least one entry, or -1 on a bad id. */
int oc_permute(const int64_t* ids, int T, int K, int E, int32_t* counts, int32_t* offsets, int32_t* perm,
               int32_t* inv) {
  const int n = T * K;
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= E) return -1;
    counts[ids[i]]++;
  }
  int hit = 0, run = 0;
  for (int e = 0; e < E; ++e) {
    offsets[e] = run;
    run += counts[e];
    hit += counts[e] > 0;
  }
  offsets[E] = run;
  int32_t* next = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E > 0 ? E : 1));
  if (!next) return -1;
  for (int e = 0; e < E; ++e) next[e] = offsets[e];
  for (int i = 0; i < n; ++i) {
    const int row = next[ids[i]]++;
    perm[row] = i;
    inv[i] = row;
  }
  free(next);
  return hit;
}
