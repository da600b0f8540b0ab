/*
 * Oracle (test infrastructure only): bit-exact CPU specification of the
 * temperature + top-p sampler of the fused entropy/gate/sample kernel.
 *
 * The reference has no seeded sampler on the MENTAT path; its only
 * temperature/top-p sampling is HuggingFace generate() (baseline_rollout.py:56-66,
 * TemperatureLogitsWarper then TopPLogitsWarper, transformers
 * generation/logits_process.py:301-303 and :527-540): divide by T, keep the
 * smallest set of most-probable tokens whose probability mass reaches top_p
 * (at least one), renormalise, draw. This file fixes that procedure to one
 * bit-exact definition:
 *
 *   1. y_i   = fl(fl(x_i - m) * c), m = max_i x_i, c = fp32(log2(e) / T)
 *   2. q_i   = floor(det_exp2(y_i) * 2^40)  as uint64   (det_exp2 below; 0 for y < -64)
 *   3. order = x descending, index ascending (x are the logits as floats)
 *   4. Z = sum q_i; P = round(top_p * 2^32); need = ceil(Z * P / 2^32) (128-bit, >= 1)
 *      kept = the shortest prefix of `order` whose q-sum reaches `need`
 *   5. (u0, u1) = first two words of Philox4x32-10(counter = (row, step_lo,
 *      step_hi, 0), key = (seed_lo, seed_hi)); U = u0 << 32 | u1
 *      r = floor(U * S / 2^64), S = q-sum of the kept prefix
 *      sample = the first token of the kept prefix whose running q-sum exceeds r
 *
 * det_exp2(y): n = rint(y), f = y - n in [-1/2, 1/2], Horner evaluation of the
 * degree-7 Taylor polynomial of 2^f = e^(f ln 2) with fmaf (coefficients
 * (ln 2)^k / k! rounded to fp32), then ldexpf(p, n). Every step is an IEEE
 * operation with one rounding, so the device code reproduces it exactly.
 *
 * Philox4x32-10 is written from Salmon, Moraes, Dror, Shaw, "Parallel random
 * numbers: as easy as 1, 2, 3" (SC'11): round multipliers 0xD2511F53 and
 * 0xCD9E8D57, Weyl key increments 0x9E3779B9 and 0xBB67AE85.
 *
 * Build: oracle/build.py (gcc -O2 -ffp-contract=off -shared).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void oracle_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static const float kC[8] = {
    0x1.000000p+0f,  0x1.62e430p-1f, 0x1.ebfbe0p-3f, 0x1.c6b08ep-5f,
    0x1.3b2ab6p-7f,  0x1.5d87fep-10f, 0x1.430912p-13f, 0x1.ffcbfcp-17f,
};

float oracle_det_exp2(float y) {
  if (!(y >= -64.0f)) return 0.0f;
  const float n = rintf(y);
  const float f = y - n;
  float p = kC[7];
  for (int k = 6; k >= 0; --k) p = fmaf(p, f, kC[k]);
  return ldexpf(p, (int)n);
}

uint64_t oracle_det_q(float y) {
  const float e = oracle_det_exp2(y);
  return (uint64_t)(e * 0x1p40f);
}

typedef struct {
  float x;
  int32_t idx;
} item_t;

static int cmp_items(const void* a, const void* b) {
  const item_t* u = (const item_t*)a;
  const item_t* v = (const item_t*)b;
  if (u->x > v->x) return -1;
  if (u->x < v->x) return 1;
  return (u->idx > v->idx) - (u->idx < v->idx);
}

/* One row. x: V logits as floats (already penalised/rounded as the kernel
 * sees them). Returns the sampled index; *kept_out / *need_out / *z_out report
 * the nucleus size and masses (may be NULL). */
int32_t oracle_top_p_sample(const float* x, int32_t V, float c, float top_p, uint64_t seed,
                            uint64_t step, uint32_t row, int32_t* kept_out, uint64_t* z_out,
                            uint64_t* need_out) {
  float m = -INFINITY;
  for (int32_t i = 0; i < V; ++i)
    if (x[i] > m) m = x[i];
  item_t* it = (item_t*)malloc(sizeof(item_t) * (size_t)V);
  uint64_t* q = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
  uint64_t Z = 0;
  for (int32_t i = 0; i < V; ++i) {
    const float y = (x[i] - m) * c;
    q[i] = oracle_det_q(y);
    Z += q[i];
    it[i].x = x[i];
    it[i].idx = i;
  }
  qsort(it, (size_t)V, sizeof(item_t), cmp_items);
  const uint64_t P = (uint64_t)llrint((double)top_p * 4294967296.0);
  unsigned __int128 prod = (unsigned __int128)Z * P;
  uint64_t need = (uint64_t)((prod + 0xffffffffu) >> 32);
  if (need < 1) need = 1;
  uint64_t S = 0;
  int32_t kept = 0;
  while (kept < V) {
    S += q[it[kept].idx];
    ++kept;
    if (S >= need) break;
  }
  const uint32_t ctr[4] = {row, (uint32_t)step, (uint32_t)(step >> 32), 0u};
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t o[4];
  oracle_philox4x32_10(ctr, key, o);
  const uint64_t U = ((uint64_t)o[0] << 32) | o[1];
  const uint64_t r = (uint64_t)(((unsigned __int128)U * S) >> 64);
  uint64_t run = 0;
  int32_t pick = it[kept - 1].idx;
  for (int32_t j = 0; j < kept; ++j) {
    run += q[it[j].idx];
    if (run > r) {
      pick = it[j].idx;
      break;
    }
  }
  if (kept_out) *kept_out = kept;
  if (z_out) *z_out = Z;
  if (need_out) *need_out = need;
  free(it);
  free(q);
  return pick;
}
