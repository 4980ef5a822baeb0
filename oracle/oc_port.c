/*
 * CPU restatement ("port") of the reference's score -> mask -> compact ->
 * attend path, in C with OpenMP.  TEST INFRASTRUCTURE: it is the CPU
 * baseline bench.py times beside the GPU, and a second checker for tests.
 * It is never linked into the product library.
 *
 * It follows the reference's algorithm, not the GPU kernels' shortcuts:
 *   - scores materialise the full 512-point FWHT of every (block, head, dim)
 *     column with the nine radix-2 stages of src/orthocache/fwht.py:23-58 and
 *     the 1/sqrt(512) division of fwht.py:61, then sum squared coefficients
 *     over the natural-index bands (src/orthocache/spectral_energy.py:95-104),
 *     zeta = high / (low + 1e-6) (:138), E_AC over coefficients 1..511 and
 *     the bound q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d) (:159-177), max over
 *     queries (:195);
 *   - the mask is (tau_max >= tau) & (zeta <= zeta_max) in fp32 (:180-234);
 *   - compaction is the active-first stable partition (compaction.py:65-82);
 *   - attention is the fp32 online-softmax loop over the active blocks of
 *     src/orthocache/adaptive_attention.py:90-120 (m starts at -1e30).
 * fp32 arithmetic; bf16 inputs are widened on load.  Parallel over
 * (block, head) tiles for scores and over query heads for attention.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

int oc_port_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* keys: bf16 (nb*512, H, D); qf: fp32 folded queries (nq, H, D).
 * Outputs (nb, H): tau_max, zeta (either may be NULL). */
void oc_port_score(const uint16_t* keys, int nb, int H, int D, const float* qf, int nq, float* tau_max,
                   float* zeta) {
  const float sqrt512 = 22.627416997969522f;  /* fwht.py:61 */
  const float sqrt_d = sqrtf((float)D);
#pragma omp parallel
  {
    float* t = (float*)malloc(sizeof(float) * 512 * (size_t)D);
#pragma omp for schedule(static)
    for (long tile = 0; tile < (long)nb * H; ++tile) {
      const int b = (int)(tile / H), h = (int)(tile % H);
      for (int r = 0; r < 512; ++r) {
        const uint16_t* src = keys + (((size_t)b * 512 + r) * H + h) * D;
        float* dst = t + (size_t)r * D;
        for (int d = 0; d < D; ++d) dst[d] = bf16_to_f32(src[d]);
      }
      /* nine butterfly stages along the token axis, natural order */
      for (int hs = 1; hs < 512; hs <<= 1) {
        for (int i = 0; i < 512; i += 2 * hs) {
          for (int j = i; j < i + hs; ++j) {
            float* a = t + (size_t)j * D;
            float* c = t + (size_t)(j + hs) * D;
#pragma omp simd
            for (int d = 0; d < D; ++d) {
              const float u = a[d], v = c[d];
              a[d] = u + v;
              c[d] = u - v;
            }
          }
        }
      }
      for (size_t e = 0; e < 512 * (size_t)D; ++e) t[e] /= sqrt512;
      float lo = 0.f, mi = 0.f, hi = 0.f;
      for (int s = 1; s < 512; ++s) {
        const float* row = t + (size_t)s * D;
        float acc = 0.f;
#pragma omp simd reduction(+ : acc)
        for (int d = 0; d < D; ++d) acc += row[d] * row[d];
        if (s < 64) lo += acc;
        else if (s < 256) mi += acc;
        else hi += acc;
      }
      if (zeta) zeta[tile] = hi / (lo + 1e-6f);
      if (tau_max && nq > 0) {
        const float eac = lo + mi + hi;
        float best = -INFINITY;
        for (int qi = 0; qi < nq; ++qi) {
          const float* qv = qf + ((size_t)qi * H + h) * D;
          float dot = 0.f, nn = 0.f;
          for (int d = 0; d < D; ++d) {
            const float kbar = t[d] / sqrt512;  /* spectral_energy.py:166 */
            dot += qv[d] * kbar;
            nn += qv[d] * qv[d];
          }
          const float bound = dot / sqrt_d + (sqrtf(nn) * sqrtf(eac)) / sqrt_d;
          if (bound > best || bound != bound) best = bound;
        }
        tau_max[tile] = best;
      }
    }
    free(t);
  }
}

/* Two-gate mask, OR over heads, active-first stable permutation.  Returns num_active. */
int oc_port_compact(const float* tau_max, const float* zeta, int nb, int H, float tau, float zeta_max,
                    uint8_t* mask, int32_t* indices) {
  int n = 0;
  uint8_t* act = (uint8_t*)malloc((size_t)nb);
  for (int b = 0; b < nb; ++b) {
    int any = 0;
    for (int h = 0; h < H; ++h) {
      const size_t e = (size_t)b * H + h;
      const int k = (tau_max[e] >= tau) && (zeta == NULL || zeta[e] <= zeta_max);
      if (mask) mask[e] = (uint8_t)k;
      any |= k;
    }
    act[b] = (uint8_t)any;
    n += any;
  }
  int pa = 0, pi = n;
  for (int b = 0; b < nb; ++b) indices[act[b] ? pa++ : pi++] = b;
  free(act);
  return n;
}

/* q: fp32 (Sq, Hq, D); k, v: bf16 (S, Hkv, D); out: fp32 (Sq, Hq, D). */
void oc_port_attend(const float* q, const uint16_t* k, const uint16_t* v, int Sq, int Hq, int Hkv, int D,
                    const int32_t* indices, int num_active, float* out) {
  const int G = Hq / Hkv;
  const float scale = sqrtf((float)D);
#pragma omp parallel for collapse(2) schedule(static)
  for (int s = 0; s < Sq; ++s) {
    for (int hq = 0; hq < Hq; ++hq) {
      const int h = hq / G;
      const float* qv = q + ((size_t)s * Hq + hq) * D;
      float* o = out + ((size_t)s * Hq + hq) * D;
      float m = -1e30f, l = 0.f;
      float* acc = (float*)calloc((size_t)D, sizeof(float));
      float* logits = (float*)malloc(sizeof(float) * 512);
      for (int i = 0; i < num_active; ++i) {
        const size_t tok0 = (size_t)indices[i] * 512;
        float mb = -INFINITY;
        for (int r = 0; r < 512; ++r) {
          const uint16_t* kr = k + ((tok0 + r) * Hkv + h) * D;
          float dot = 0.f;
          for (int d = 0; d < D; ++d) dot += qv[d] * bf16_to_f32(kr[d]);
          logits[r] = dot / scale;
          if (logits[r] > mb) mb = logits[r];
        }
        const float mn = m > mb ? m : mb;
        const float ep = expf(m - mn);
        float ls = 0.f;
        for (int d = 0; d < D; ++d) acc[d] *= ep;
        for (int r = 0; r < 512; ++r) {
          const float p = expf(logits[r] - mn);
          ls += p;
          const uint16_t* vr = v + ((tok0 + r) * Hkv + h) * D;
          for (int d = 0; d < D; ++d) acc[d] += p * bf16_to_f32(vr[d]);
        }
        l = l * ep + ls;
        m = mn;
      }
      for (int d = 0; d < D; ++d) o[d] = num_active ? acc[d] / l : 0.f;
      free(logits);
      free(acc);
    }
  }
}
