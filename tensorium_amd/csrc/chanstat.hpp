// Final steps of the channel reductions taken inside the kernel that uses
// them: a workgroup forms the statistics of the channels it touches from the
// partial sums itself, in the fixed order of the separate final launch, so
// the results are the same bits with one launch fewer.
#pragma once
#include "common.hpp"

namespace tnh {

// The normalize step of the batch norm (TTensor.blockNormalize,
// ntensors.pas:8693-8718, with IEEE division): d = max(sqrt(var), 1e-6) for
// planes of more than one element (_snormblkvv, :4357), sqrt(max(var, 1e-6))
// for one element per channel (_snormvv, :4338); x_norm = (x - mean) / d.
// Shared by the forward pass and the backward passes that form x_norm again
// instead of reading it, so both give the same bits.
__device__ inline float bn_norm_d(float var, bool oneElem) {
  if (oneElem) return sqrtf(var > 1e-6f ? var : 1e-6f);
  const float d = sqrtf(var);
  return d > 1e-6f ? d : 1e-6f;
}
__device__ inline float bn_norm(float x, float mean, float d) {
  const float t = x - mean;
  return t / d;
}
// out = act(fl(scale * x_norm) + bias) (forwardScale, forwardBias, then the
// activation: leaky_array, nactivation.pas:234-268, or the logistic)
__device__ inline float bn_scale_add(float s, float b, float xn) {
  const float u = s * xn;
  return b + u;
}
__device__ inline float bn_act(float v, int act) {
  if (act == TNH_AC_LEAKY) return 0.f > v ? 0.1f * v : v;
  if (act == TNH_AC_LOGISTIC) return 1.f / (1.f + expf(-v));
  return v;
}

// The tree of the channel reductions' final step over one value per lane
// (lane i adds lane i + w for w = 32, 16, ..., 1).  Called by a whole wave;
// every lane gets lane 0's total.
__device__ inline float lane_total(float t) {
  for (int w = 32; w > 0; w >>= 1) t = t + __shfl_down(t, w, 64);
  return __shfl(t, 0, 64);
}

// Sum of v[0 .. n) in the fixed order of the channel reductions' final step:
// lane l adds v[l], v[l + 64], ... in turn from +0, then lane_total.
__device__ inline float wave_total(const float* v, int n) {
  const int lane = threadIdx.x & 63;
  float t = 0.f;
  for (int k = lane; k < n; k += 64) t = t + v[k];
  return lane_total(t);
}

// The partials of tnh_bn_statistics' two passes over [groups][C][block]
// (the channel sums, then the residual sums of squares about the fp32 mean),
// P per channel, and where its final step stores.
struct StatParts {
  const float* sumPart;  // [C][P]
  const float* rssPart;  // [C][P]
  int P;
  float S;  // groups * block
  float* means;
  float* vars;
  float* rollMean;  // NULL: no rolling statistics
  float* rollVar;
  float keep, bm;  // 1 - momentum, momentum
  // This lane's terms of channel f's two totals when P <= 64 (0 + the
  // partial, +0 past P): loads that can be issued before the arithmetic.
  __device__ void lanes(int64_t f, float& sum, float& rss) const {
    const int lane = threadIdx.x & 63;
    sum = rss = 0.f;
    if (lane < P) {
      sum = 0.f + sumPart[f * P + lane];
      rss = 0.f + rssPart[f * P + lane];
    }
  }
  // finish() from the terms lanes() loaded (P <= 64)
  __device__ void finish_lanes(int64_t f, bool store, float sum, float rss, float& m, float& v) const {
    m = lane_total(sum) / S;
    v = lane_total(rss) / (S - 1.f);
    store_stats(f, store, m, v);
  }
  __device__ void store_stats(int64_t f, bool store, float m, float v) const {
    if (store && (threadIdx.x & 63) == 0) {
      means[f] = m;
      vars[f] = v;
      if (rollMean) {  // Multiply(1 - momentum), then axpy(momentum, .) (nbaselayer.pas:352-355)
        rollMean[f] = fmaf(bm, m, keep * rollMean[f]);
        rollVar[f] = fmaf(bm, v, keep * rollVar[f]);
      }
    }
  }
  // Channel f's mean and variance as the final step forms them (called by
  // a whole wave).  With `store`, lane 0 also stores them and advances the
  // rolling statistics: exactly one wave per channel may pass it.
  __device__ void finish(int64_t f, bool store, float& m, float& v) const {
    m = wave_total(sumPart + f * P, P) / S;
    const float rss = wave_total(rssPart + f * P, P);
    v = rss / (S - 1.f);
    store_stats(f, store, m, v);
  }
};

// Launches tnh_bn_statistics' two partial passes over x [groups][C][block]
// on the context stream and describes their partials in sp (the final step
// is the caller's).  Returns a TNH status.
int bn_stat_partials(int64_t C, int64_t block, int64_t groups, const float* x, float* means, float* vars,
                     float* rollMean, float* rollVar, float momentum, StatParts& sp);
// The final step of those statistics in a launch of its own (a wave per
// channel), for callers that cannot take it.
int bn_stat_final(int64_t C, const StatParts& sp);

}  // namespace tnh
