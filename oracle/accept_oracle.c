/*
 * accept_oracle.c -- CPU restatement of the reference's acceptance / sampling path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product links or calls this file; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, as the checker.
 *
 * Follows (paths relative to the reference root):
 *   src/mlx_dspark/sampling.py:18-44   truncate_probs  (top-k then top-p, renormalise)
 *   src/mlx_dspark/sampling.py:47-49   sample_probs    (categorical draw)
 *   src/mlx_dspark/generate.py:659-688 _spec_sample_accept (min(1, p/q) test, residual)
 *   src/mlx_dspark/generate.py:910-921 fused greedy accept (argmax, cumprod of matches)
 *   src/mlx_dspark/generate.py:135-146 _sample_arr / _pick
 *
 * The reference computes these with MLX float32 reductions and MLX's threefry RNG, neither
 * of which is available here. The engine fixes one canonical definition, implemented twice
 * (here, with sorting and the reference's sequential truncation; on the GPU, with histograms
 * and a candidate select) and compared bit for bit:
 *   - exp is dsk_expf below (Cody-Waite reduction by ln 2, Taylor polynomial to r^7,
 *     explicit fmaf, inputs below -86 flush to 0 so no subnormal is ever formed);
 *   - a row's distribution is built on the unnormalised exponentials e_j = exp(y_j - max y)
 *     with fixed-point masses w_j = fx(e_j) = floor(e_j * 2^31) and Z = sum w_j (integer
 *     sums do not depend on summation order); softmax then truncation then renormalisation is
 *     the same as truncating e and dividing by the kept mass, so the final probability of a
 *     kept element is e_j / float(S * 2^-31) with S the kept mass;
 *   - top-k keeps e_j >= the k-th largest e; top-p keeps an element while the mass strictly
 *     before it (in descending order) is below TP = ceil(top_p * Z), an exact integer;
 *   - uniforms are Philox4x32-10 (Salmon et al., SC'11) words, u = (w >> 8) * 2^-24;
 *   - a categorical draw from weights w_j is the inverse CDF on the fixed-point masses:
 *     t = floor(u * sum fx(w)), pick the first j whose inclusive prefix exceeds t
 *     (uniform index floor(u * V) when every mass is zero); the residual draw uses the
 *     residual max(p - q, 0) itself (dividing it by its sum does not change the draw's law).
 * Compile with -ffp-contract=off: every fused multiply-add below is an explicit fmaf.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <string.h>

/* ------------------------------------------------------------------------ Philox4x32-10 */
static void philox4x32_10(uint32_t ctr[4], uint32_t k0, uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += W0;
      k1 += W1;
    }
    uint64_t p0 = (uint64_t)M0 * c0, p1 = (uint64_t)M1 * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  ctr[0] = c0;
  ctr[1] = c1;
  ctr[2] = c2;
  ctr[3] = c3;
}

void oracle_philox(const uint32_t ctr_in[4], uint32_t k0, uint32_t k1, uint32_t out[4]) {
  uint32_t c[4] = {ctr_in[0], ctr_in[1], ctr_in[2], ctr_in[3]};
  philox4x32_10(c, k0, k1);
  memcpy(out, c, sizeof(c));
}

/* Stream layout of the engine's uniforms (word 0 of one Philox block):
 *   accept test of draft position i in batch row b : ctr = {i, b, 0, offset}
 *   categorical draw for position i in batch row b : ctr = {i, b, 1, offset}
 *   dsk_sample_rows row r                          : ctr = {row, 0, 2, offset}        */
static uint32_t philox_word(uint64_t seed, uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3) {
  uint32_t c[4] = {c0, c1, c2, c3};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  return c[0];
}

static float u24_to_float(uint32_t w) { return (float)(w >> 8) * 0x1p-24f; }

/* ------------------------------------------------------------------------ exp */
float oracle_expf(float x) {
  if (x < -86.0f) return 0.0f;
  if (x != x) return x;
  if (x > 88.7f) return INFINITY;
  float t = x * 1.44269504f;
  float k = rintf(t);
  float r = fmaf(-k, 0.693145751953125f, x);
  r = fmaf(-k, 1.428606765330187e-06f, r);
  float p = 1.98412698e-4f;
  p = fmaf(p, r, 1.38888889e-3f);
  p = fmaf(p, r, 8.33333333e-3f);
  p = fmaf(p, r, 4.16666667e-2f);
  p = fmaf(p, r, 1.66666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ki = (int)k;
  if (ki > 127) {
    p = p * 0x1p127f;
    ki -= 127;
  }
  uint32_t eb = (uint32_t)(ki + 127) << 23;
  float sc;
  memcpy(&sc, &eb, 4);
  return p * sc;
}

/* every mass is in [0, 1] (e, final probabilities, residuals): p * 2^31 is exact and fits */
static uint64_t fx(float p) { return (uint64_t)(p * 0x1p31f); }
static float fx_to_float(uint64_t s) { return (float)((double)s * 0x1p-31); }

/* ------------------------------------------------------------------------ softmax + truncation */
typedef struct {
  float v;
  int64_t i;
} vi_t;

static int cmp_desc(const void* a, const void* b) {
  float x = ((const vi_t*)a)->v, y = ((const vi_t*)b)->v;
  if (x > y) return -1;
  if (x < y) return 1;
  int64_t i = ((const vi_t*)a)->i, j = ((const vi_t*)b)->i;
  return (i < j) ? -1 : (i > j);
}

/* TP = ceil(top_p * Z) exactly: top_p = M * 2^E with an integer M < 2^24, so the product is
 * an integer below 2^87 and the ceiling is a shift of a 128-bit sum. top_p <= 0 gives 0. */
uint64_t oracle_top_p_target(float top_p, uint64_t Z) {
  if (!(top_p > 0.0f)) return 0;
  uint32_t bits;
  memcpy(&bits, &top_p, 4);
  const uint32_t ex = (bits >> 23) & 0xFFu;
  uint64_t M = bits & 0x7FFFFFu;
  int E;
  if (ex == 0) {
    E = -149;
  } else {
    M |= 0x800000u;
    E = (int)ex - 150;
  }
  const unsigned __int128 P = (unsigned __int128)M * Z;
  if (E >= 0) return (uint64_t)(P << E); /* top_p >= 2^23: never reached for top_p < 1 */
  const int sh = -E;
  if (sh >= 128) return P ? 1 : 0;
  return (uint64_t)((P + (((unsigned __int128)1 << sh) - 1)) >> sh);
}

/* truncate(softmax(logits / T)) (or logits * (1/T) when mul_inv != 0) into out[V]: the final
 * probabilities the accept test and the draws read. Follows sampling.py:18-44 step by step on
 * the unnormalised exponentials: the k-th largest threshold, then the nucleus on the top-k
 * zeroed (not renormalised) values, then the division by the kept mass. */
void oracle_probs(const float* logits, int64_t V, float T, int mul_inv, float top_p, int top_k,
                  float* out) {
  const float inv_t = 1.0f / T;
  float m = -INFINITY;
  for (int64_t j = 0; j < V; ++j) {
    float y = mul_inv ? logits[j] * inv_t : logits[j] / T;
    out[j] = y;
    if (y > m) m = y;
  }
  uint64_t Z = 0;
  for (int64_t j = 0; j < V; ++j) {
    float e = oracle_expf(out[j] - m);
    out[j] = e;
    Z += fx(e);
  }
  const int do_k = (top_k > 0 && (int64_t)top_k < V);
  const int do_p = (top_p < 1.0f);
  if (do_k || do_p) {
    vi_t* s = (vi_t*)malloc(sizeof(vi_t) * (size_t)V);
    if (do_k) {
      for (int64_t j = 0; j < V; ++j) {
        s[j].v = out[j];
        s[j].i = j;
      }
      qsort(s, (size_t)V, sizeof(vi_t), cmp_desc);
      float kth = s[top_k - 1].v;
      for (int64_t j = 0; j < V; ++j)
        if (!(out[j] >= kth)) out[j] = 0.0f;
    }
    if (do_p) {
      const uint64_t TP = oracle_top_p_target(top_p, Z);
      for (int64_t j = 0; j < V; ++j) {
        s[j].v = out[j];
        s[j].i = j;
      }
      qsort(s, (size_t)V, sizeof(vi_t), cmp_desc);
      uint64_t before = 0;
      float cutoff = INFINITY;
      for (int64_t i = 0; i < V; ++i) {
        if (before < TP) cutoff = s[i].v; /* in the nucleus: mass strictly before it < top_p */
        else break;
        before += fx(s[i].v);
      }
      for (int64_t j = 0; j < V; ++j)
        if (!(out[j] >= cutoff)) out[j] = 0.0f;
    }
    free(s);
  }
  uint64_t S = 0;
  for (int64_t j = 0; j < V; ++j) S += fx(out[j]);
  if (S == 0) { /* an empty nucleus (top_p * Z rounds to 0): every probability is 0 */
    for (int64_t j = 0; j < V; ++j) out[j] = 0.0f;
    return;
  }
  const float Sf = fx_to_float(S);
  for (int64_t j = 0; j < V; ++j) out[j] = out[j] / Sf;
}

/* inverse-CDF categorical draw on fixed-point masses of w[0..V) */
int64_t oracle_categorical(const float* w, int64_t V, uint32_t word) {
  uint64_t W = 0;
  for (int64_t j = 0; j < V; ++j) W += fx(w[j]);
  const uint64_t u = word >> 8;
  if (W == 0) return (int64_t)((u * (uint64_t)V) >> 24);
  const uint64_t t = (W >> 24) * u + (((W & 0xFFFFFFull) * u) >> 24);
  uint64_t c = 0;
  for (int64_t j = 0; j < V; ++j) {
    c += fx(w[j]);
    if (c > t) return j;
  }
  return V - 1; /* unreachable: t < W */
}

/* ------------------------------------------------------------------------ accept (sampled) */
/* Every (row b, position i) item is independent (its p, q, residual and uniforms are keyed by
 * b and i), so the items run in parallel (OpenMP, each item in its own buffers); the accepted
 * prefix of each row is then read off in order. Results do not depend on the thread count. */
static void accept_item(const float* p_logits, const float* q_logits, int64_t V, int L, const int32_t* draft,
                        float T, float top_p, int top_k, int q_mul_inv_t, uint64_t seed, uint32_t offset, int b,
                        int i, float* p, float* q, float* r, uint8_t* acc_out, int32_t* samp_out) {
  const float* pl = p_logits + ((int64_t)b * (L + 1) + i) * V;
  oracle_probs(pl, V, T, 0, top_p, top_k, p);
  int acc = 0, samp;
  if (i < L) {
    const int32_t d = draft[(int64_t)b * L + i];
    const int dvalid = d >= 0 && (int64_t)d < V; /* an out-of-range id is rejected */
    float qd;
    if (q_logits) {
      oracle_probs(q_logits + ((int64_t)b * L + i) * V, V, T, q_mul_inv_t, top_p, top_k, q);
      qd = dvalid ? q[d] : 1.0f;
    } else {
      for (int64_t j = 0; j < V; ++j) q[j] = (j == d) ? 1.0f : 0.0f;
      qd = 1.0f;
    }
    const float pd = dvalid ? p[d] : 0.0f;
    const float u = u24_to_float(philox_word(seed, (uint32_t)i, (uint32_t)b, 0u, offset));
    float ratio = pd / (qd > 1e-9f ? qd : 1e-9f);
    if (ratio > 1.0f) ratio = 1.0f;
    acc = u < ratio;
    for (int64_t j = 0; j < V; ++j) {
      float t = p[j] - q[j];
      r[j] = t > 0.0f ? t : 0.0f;
    }
    samp = (int)oracle_categorical(r, V, philox_word(seed, (uint32_t)i, (uint32_t)b, 1u, offset));
  } else {
    samp = (int)oracle_categorical(p, V, philox_word(seed, (uint32_t)i, (uint32_t)b, 1u, offset));
  }
  *acc_out = (uint8_t)acc;
  *samp_out = samp;
}

int oracle_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

int oracle_accept_sample(const float* p_logits, const float* q_logits, int64_t V, int B, int L,
                         const int32_t* draft, float T, float top_p, int top_k, int q_mul_inv_t,
                         uint64_t seed, uint32_t offset, int32_t* n_out, int32_t* token_out,
                         int32_t* seq_lens, uint8_t* accept_out, int32_t* sample_out) {
  const int items = B * (L + 1);
  uint8_t* accv = (uint8_t*)malloc((size_t)items);
  int32_t* sampv = (int32_t*)malloc(sizeof(int32_t) * (size_t)items);
  if (!accv || !sampv) return -1;
  int fail = 0;
#pragma omp parallel for schedule(dynamic, 1)
  for (int it = 0; it < items; ++it) {
    float* p = (float*)malloc(sizeof(float) * (size_t)V);
    float* q = (float*)malloc(sizeof(float) * (size_t)V);
    float* r = (float*)malloc(sizeof(float) * (size_t)V);
    if (p && q && r)
      accept_item(p_logits, q_logits, V, L, draft, T, top_p, top_k, q_mul_inv_t, seed, offset, it / (L + 1),
                  it % (L + 1), p, q, r, accv + it, sampv + it);
    else {
#pragma omp atomic write
      fail = 1;
    }
    free(p);
    free(q);
    free(r);
  }
  if (fail) {
    free(accv);
    free(sampv);
    return -1;
  }
  for (int b = 0; b < B; ++b) {
    int n = 0, done = 0, token = -1;
    for (int i = 0; i <= L; ++i) {
      const int it = b * (L + 1) + i;
      if (accept_out && i < L) accept_out[(int64_t)b * L + i] = accv[it];
      if (sample_out) sample_out[(int64_t)b * (L + 1) + i] = sampv[it];
      if (!done) {
        if (i < L && accv[it]) {
          ++n;
        } else {
          done = 1;
          token = sampv[it];
        }
      }
    }
    n_out[b] = n;
    token_out[b] = token;
    if (seq_lens) seq_lens[b] += n + 1;
  }
  free(accv);
  free(sampv);
  return 0;
}

/* ------------------------------------------------------------------------ accept (greedy) */
static float bf16f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

int oracle_accept_greedy(const void* logits, int is_bf16, int64_t ldl, int B, int W, int64_t V,
                         const int32_t* draft, int32_t* tt, int32_t* n_out, int32_t* token_out,
                         int32_t* seq_lens) {
  for (int b = 0; b < B; ++b) {
    for (int i = 0; i < W; ++i) {
      int64_t row = (int64_t)b * W + i;
      float best = -INFINITY;
      int64_t bi = 0;
      for (int64_t j = 0; j < V; ++j) {
        float v = is_bf16 ? bf16f(((const uint16_t*)logits)[row * ldl + j])
                          : ((const float*)logits)[row * ldl + j];
        if (v > best) {
          best = v;
          bi = j;
        }
      }
      tt[row] = (int32_t)bi;
    }
    int n = 0;
    while (n < W - 1 && draft[(int64_t)b * (W - 1) + n] == tt[(int64_t)b * W + n]) ++n;
    n_out[b] = n;
    token_out[b] = tt[(int64_t)b * W + n];
    if (seq_lens) seq_lens[b] += n + 1;
  }
  return 0;
}

/* ------------------------------------------------------------------------ row sampling */
int oracle_sample_rows(const float* logits, int64_t V, int R, float T, float top_p, int top_k,
                       int mul_inv, uint64_t seed, uint32_t offset, int row0, int32_t* token_out,
                       float* probs_out) {
  float* p = (float*)malloc(sizeof(float) * (size_t)V);
  if (!p) return -1;
  for (int r = 0; r < R; ++r) {
    const float* l = logits + (int64_t)r * V;
    if (T <= 0.0f) {
      float best = -INFINITY;
      int64_t bi = 0;
      for (int64_t j = 0; j < V; ++j)
        if (l[j] > best) {
          best = l[j];
          bi = j;
        }
      token_out[r] = (int32_t)bi;
      continue;
    }
    oracle_probs(l, V, T, mul_inv, top_p, top_k, p);
    token_out[r] = (int32_t)oracle_categorical(p, V, philox_word(seed, (uint32_t)(row0 + r), 0u, 2u, offset));
    if (probs_out) memcpy(probs_out + (int64_t)r * V, p, sizeof(float) * (size_t)V);
  }
  free(p);
  return 0;
}
