// On-device token selection by one wave (generator.py:178-207 of the reference, with the
// Gumbel-max / Philox draw that replaces torch.multinomial).
#pragma once
#include "qtts_common.h"

namespace qtts {

struct SelParams {
  int do_sample;
  float temperature;
  int top_k;
  float top_p;
  uint64_t seed;
  int frame_step;
  int group;
};

// Keep the better of two (value, index) candidates: larger value, lower index on ties.
__device__ __forceinline__ void best_merge(float& bv, int& bi, float ov, int oi) {
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// Greedy argmax over lg[0..n) (lowest index on ties; all -inf -> index 0), run by one wave.
__device__ inline int wave_argmax(const float* lg, int n) {
  const int lane = threadIdx.x & 63;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = lane; i < n; i += 64) {
    const float v = lg[i];
    if (v > best || (v == best && i < bi)) { best = v; bi = i; }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  return bi == 0x7fffffff ? 0 : bi;
}

__device__ inline int wave_count_ge(const uint32_t* keys, int n, uint32_t t) {
  const int lane = threadIdx.x & 63;
  int c = 0;
  for (int i = lane; i < n; i += 64) c += keys[i] >= t;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) c += __shfl_xor(c, o, 64);
  return c;
}

// LDS scratch for one selection: scaled logits, their keys and (for top-p) probabilities.
struct SelScratch {
  float s[MAXV];
  uint32_t key[MAXV];
  double p[MAXV];
};

// Temperature / top-k / top-p / Gumbel-max over lg[0..n), n <= MAXV, one wave.
// lg holds the masked logits (bf16 values; suppressed ids = -inf). Returns the same id on
// every lane.
__device__ inline int wave_select(const float* lg, int n, const SelParams& sp, SelScratch* sc) {
  if (!sp.do_sample) return wave_argmax(lg, n);
  const int lane = threadIdx.x & 63;
  for (int i = lane; i < n; i += 64) {
    // logits / temperature on bf16 logits rounds to bf16 in the reference (generator.py:189)
    const float v = rbf(lg[i] / sp.temperature);
    sc->s[i] = v;
    sc->key[i] = fkey(v);
  }
  // top-k: the k-th largest key, found bit by bit; values >= it are kept (ties kept)
  uint32_t kth = 0u;
  if (sp.top_k > 0 && sp.top_k < n) {
    for (int b = 31; b >= 0; --b) {
      const uint32_t cand = kth | (1u << b);
      if (wave_count_ge(sc->key, n, cand) >= sp.top_k) kth = cand;
    }
  }
  // top-p: keep x when the probability mass of strictly larger kept values is <= top_p
  uint32_t pth = 0u;
  if (sp.top_p < 1.0f) {
    float m = -INFINITY;
    for (int i = lane; i < n; i += 64) if (sc->key[i] >= kth) m = fmaxf(m, sc->s[i]);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    double z = 0.0;
    for (int i = lane; i < n; i += 64) {
      const double pi = (sc->key[i] >= kth && sc->s[i] != -INFINITY) ? exp((double)sc->s[i] - (double)m) : 0.0;
      sc->p[i] = pi;
      z += pi;
    }
    z = wave_sum_d(z);
    // smallest t with sum_{key > t} p <= top_p * z  (non-increasing in t)
    uint32_t lo = 0u, hi = 0xffffffffu;
    while (lo < hi) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      double acc = 0.0;
      for (int i = lane; i < n; i += 64) acc += sc->key[i] > mid ? sc->p[i] : 0.0;
      acc = wave_sum_d(acc);
      if (acc <= (double)sp.top_p * z) hi = mid; else lo = mid + 1u;
    }
    pth = lo;
  }
  const uint32_t thr = kth > pth ? kth : pth;
  double best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = lane; i < n; i += 64) {
    if (sc->key[i] >= thr && sc->s[i] != -INFINITY) {
      const double u = sampler_uniform(sp.seed, sp.frame_step, sp.group, i);
      const double v = (double)sc->s[i] - log(-log(u));
      if (v > best || (v == best && i < bi)) { best = v; bi = i; }
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
  }
  return bi == 0x7fffffff ? wave_argmax(lg, n) : bi;
}

}  // namespace qtts
