// YOLO detections and non-maximum suppression on the device, so that what
// leaves the GPU after a forward pass is the detection list, not the three
// head tensors.
//
// tnh_yolo_detections restates TNNet.Detections (nnet.pas:584-680) over the
// yolo heads: TYoloLayer.getDetections (nyololayer.pas:399-450) with getBox
// (nyololayer.pas:105-122, new_coords = 0) and correctBoxes
// (nyololayer.pas:452-498).  Detections are numbered in the reference's
// order -- head by head, location (row-major) outer, anchor inner -- by a
// per-image scan (no atomics), so the list is deterministic.
//
// tnh_yolo_nms_sort restates TDetectionsHelper.doNMSSort (ntypes.pas:
// 1612-1649): per class, the detections with a non-zero probability in
// descending order of that probability, then greedy suppression of every
// later one whose IoU with a kept one exceeds the threshold (box_iou,
// ntypes.pas:1059-1107, in the same float operations).  The reference sorts
// with an unstable quicksort; here equal probabilities keep detection order.
#include "common.hpp"

namespace tnh {
namespace {

constexpr int kMaxHeads = 8;
constexpr int kMaxAnchors = 16;
constexpr int kDetThreads = 1024;
constexpr int kNmsThreads = 1024;
constexpr int kNmsMax = 8192;  // candidates one class's NMS sorts in LDS

struct DetArgs {
  const float* head[kMaxHeads];
  int h[kMaxHeads], w[kMaxHeads];
  int64_t headBase[kMaxHeads + 1];  // candidates before head hd (per image)
  float anchorW[kMaxHeads][kMaxAnchors], anchorH[kMaxHeads][kMaxAnchors];
  int nHeads, n, classes;
  int netW, netH, imgW, imgH;
  float thresh;
  float deltaW, deltaH, ratioW, ratioH;  // correctBoxes
  int relative;
  int64_t capacity;
  float* boxes;  // [batch][capacity][4]: x, y, w, h
  float* obj;    // [batch][capacity]
  float* prob;   // [batch][capacity][classes]
  int32_t* counts;
};

// One workgroup per image walks the candidates in the reference's order in
// chunks of kDetThreads; a wave ballot plus a prefix over the 16 waves gives
// each kept candidate its detection index.
__global__ __launch_bounds__(kDetThreads) void yolo_detect_kernel(DetArgs a) {
  __shared__ int waveSum[kDetThreads / 64];
  __shared__ int64_t base;
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t total = a.headBase[a.nHeads];
  if (threadIdx.x == 0) base = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < total; c0 += kDetThreads) {
    const int64_t c = c0 + threadIdx.x;
    bool keep = false;
    int hd = 0;
    int64_t loc = 0;
    int an = 0;
    float objv = 0.f;
    const float* out = nullptr;
    int hw = 1;
    if (c < total) {
      while (hd + 1 < a.nHeads && c >= a.headBase[hd + 1]) ++hd;
      const int64_t r = c - a.headBase[hd];
      loc = r / a.n;  // location outer, anchor inner (getDetections loop order)
      an = static_cast<int>(r - loc * a.n);
      hw = a.h[hd] * a.w[hd];
      // entryIndex: b*outputs + an*(classes+5)*hw + entry*hw + loc
      out = a.head[hd] + (static_cast<int64_t>(b) * a.n + an) * (a.classes + 5) * hw + loc;
      objv = out[4 * hw];
      keep = objv > a.thresh;
    }
    const uint64_t m = __ballot(keep);
    const int before = __popcll(m & ((uint64_t(1) << lane) - 1));
    if (lane == 0) waveSum[wave] = __popcll(m);
    __syncthreads();
    int64_t pos = base + before;
    for (int w = 0; w < wave; ++w) pos += waveSum[w];
    if (keep && pos < a.capacity) {
      const int W = a.w[hd], H = a.h[hd];
      const int row = static_cast<int>(loc / W), col = static_cast<int>(loc - static_cast<int64_t>(row) * W);
      // getBox
      float x = (static_cast<float>(col) + out[0]) / static_cast<float>(W);
      float y = (static_cast<float>(row) + out[hw]) / static_cast<float>(H);
      float bw = expf(out[2 * hw]) * a.anchorW[hd][an] / static_cast<float>(a.netW);
      float bh = expf(out[3 * hw]) * a.anchorH[hd][an] / static_cast<float>(a.netH);
      // correctBoxes
      x = (x - a.deltaW / 2.0f / static_cast<float>(a.netW)) / a.ratioW;
      y = (y - a.deltaH / 2.0f / static_cast<float>(a.netH)) / a.ratioH;
      bw = bw * (1.0f / a.ratioW);
      bh = bh * (1.0f / a.ratioH);
      if (!a.relative) {
        x = x * static_cast<float>(a.imgW);
        bw = bw * static_cast<float>(a.imgW);
        y = y * static_cast<float>(a.imgH);
        bh = bh * static_cast<float>(a.imgH);
      }
      float* bx = a.boxes + (static_cast<int64_t>(b) * a.capacity + pos) * 4;
      bx[0] = x;
      bx[1] = y;
      bx[2] = bw;
      bx[3] = bh;
      a.obj[static_cast<int64_t>(b) * a.capacity + pos] = objv;
      float* pr = a.prob + (static_cast<int64_t>(b) * a.capacity + pos) * a.classes;
      for (int j = 0; j < a.classes; ++j) {
        const float p = objv * out[(5 + j) * hw];
        pr[j] = p > a.thresh ? p : 0.f;
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int64_t t = 0;
      for (int w = 0; w < kDetThreads / 64; ++w) t += waveSum[w];
      base += t;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) a.counts[b] = static_cast<int32_t>(base);
}

// box_iou (ntypes.pas:1059-1107): overlap per axis, intersection 0 when
// either overlap is negative, union = a.w*a.h + b.w*b.h - I, IoU 0 when I or
// U is 0.
__device__ inline float overlap1(float x1, float w1, float x2, float w2) {
  const float l1 = x1 - w1 / 2.f, l2 = x2 - w2 / 2.f;
  const float left = l1 > l2 ? l1 : l2;
  const float r1 = x1 + w1 / 2.f, r2 = x2 + w2 / 2.f;
  const float right = r1 < r2 ? r1 : r2;
  return right - left;
}
__device__ inline float box_iou(float ax, float ay, float aw, float ah, float bx, float by, float bw, float bh) {
  const float w = overlap1(ax, aw, bx, bw), h = overlap1(ay, ah, by, bh);
  const float I = (w < 0.f || h < 0.f) ? 0.f : w * h;
  const float U = aw * ah + bw * bh - I;
  if (I == 0.f || U == 0.f) return 0.f;
  return I / U;
}

// One workgroup per (class, image): gather the detections with a non-zero
// probability for the class, bitonic-sort them by (probability descending,
// detection index ascending) in LDS, then greedy suppression in that order.
// Compacts the candidates of class k of image b (non-zero probability, in
// detection order) into score/idx and sorts them: higher score first, then
// lower detection index.  Returns the candidate count (every thread).
__device__ inline int nms_collect_sort(int64_t capacity, int classes, const float* pr, int64_t m, float* score,
                                       int* idx, int* waveSum, int& q) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) q = 0;
  __syncthreads();
  for (int64_t d0 = 0; d0 < m; d0 += kNmsThreads) {
    const int64_t d = d0 + threadIdx.x;
    const float p = d < m ? pr[d * classes] : 0.f;
    const bool keep = p != 0.f;
    const uint64_t bal = __ballot(keep);
    const int before = __popcll(bal & ((uint64_t(1) << lane) - 1));
    if (lane == 0) waveSum[wave] = __popcll(bal);
    __syncthreads();
    int pos = q + before;
    for (int w = 0; w < wave; ++w) pos += waveSum[w];
    if (keep) {
      score[pos] = p;
      idx[pos] = static_cast<int>(d);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int t = 0;
      for (int w = 0; w < kNmsThreads / 64; ++w) t += waveSum[w];
      q += t;
    }
    __syncthreads();
  }
  const int n = q;
  if (n <= 1) return n;
  int P = 2;
  while (P < n) P <<= 1;
  for (int i = n + threadIdx.x; i < P; i += kNmsThreads) {
    score[i] = -__builtin_inff();
    idx[i] = 0x7fffffff;
  }
  __syncthreads();
  // bitonic sort: "before" = higher score, then lower detection index
  for (int size = 2; size <= P; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < P; i += kNmsThreads) {
        const int j = i ^ stride;
        if (j > i) {
          const bool up = (i & size) == 0;  // this run ascends in "before" order
          const float si = score[i], sj = score[j];
          const int ii = idx[i], ij = idx[j];
          const bool jFirst = sj > si || (sj == si && ij < ii);
          if (jFirst == up) {
            score[i] = sj;
            score[j] = si;
            idx[i] = ij;
            idx[j] = ii;
          }
        }
      }
      __syncthreads();
    }
  return n;
}

__global__ __launch_bounds__(kNmsThreads) void yolo_nms_sort_kernel(int64_t capacity, int classes,
                                                                  const float* __restrict__ boxes, float* prob,
                                                                  const int32_t* counts, float thresh) {
  __shared__ float score[kNmsMax];
  __shared__ int idx[kNmsMax];
  __shared__ unsigned char alive[kNmsMax];
  __shared__ int waveSum[kNmsThreads / 64];
  __shared__ int q;
  constexpr int PER = kNmsMax / kNmsThreads;
  const int k = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m = min(static_cast<int64_t>(counts[b]), capacity);
  float* pr = prob + static_cast<int64_t>(b) * capacity * classes + k;
  const int n = nms_collect_sort(capacity, classes, pr, m, score, idx, waveSum, q);
  if (n <= 1) return;
  // Greedy suppression in chunks of 64 sorted candidates (thread t owns
  // sorted positions t + r * kNmsThreads and keeps their boxes in
  // registers).  Per chunk: wave 0 resolves the chunk by itself -- lane l
  // builds the 64-bit mask of later chunk members its box suppresses, then a
  // 64-step scan keeps l if no kept earlier member suppresses it -- and then
  // every thread drops its later candidates that a kept chunk member
  // suppresses.  A candidate is dropped iff a kept earlier one overlaps it
  // by more than thresh: the greedy result, with two barriers per chunk.
  float bxr[PER][4];
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int j = threadIdx.x + r * kNmsThreads;
    if (j < n) {
      const float* bp = boxes + (static_cast<int64_t>(b) * capacity + idx[j]) * 4;
      bxr[r][0] = bp[0];
      bxr[r][1] = bp[1];
      bxr[r][2] = bp[2];
      bxr[r][3] = bp[3];
      alive[j] = 1;
    }
  }
  __shared__ float cb[64][4];
  __shared__ uint64_t keptBits;
  for (int c0 = 0; c0 < n; c0 += 64) {
    // chunk boxes to LDS (owners of positions c0 .. c0+63)
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int j = threadIdx.x + r * kNmsThreads;
      if (j >= c0 && j < c0 + 64 && j < n) {
        cb[j - c0][0] = bxr[r][0];
        cb[j - c0][1] = bxr[r][1];
        cb[j - c0][2] = bxr[r][2];
        cb[j - c0][3] = bxr[r][3];
      }
    }
    __syncthreads();
    if (wave == 0) {
      const int l = lane;
      const bool in = c0 + l < n;
      uint64_t mask = 0;
      if (in) {
        const float ax = cb[l][0], ay = cb[l][1], aw = cb[l][2], ah = cb[l][3];
        for (int m = l + 1; m < 64 && c0 + m < n; ++m)
          if (box_iou(ax, ay, aw, ah, cb[m][0], cb[m][1], cb[m][2], cb[m][3]) > thresh) mask |= uint64_t(1) << m;
      }
      uint64_t keep = __ballot(in && alive[c0 + l]);
      const uint32_t mlo = static_cast<uint32_t>(mask), mhi = static_cast<uint32_t>(mask >> 32);
      for (int i = 0; i < 64; ++i)
        if ((keep >> i) & 1) {
          // readlane returns a signed int: widen through uint32_t so the low
          // word does not sign-extend into the high one
          const uint64_t mi = (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(mhi, i))) << 32) |
                              static_cast<uint32_t>(__builtin_amdgcn_readlane(mlo, i));
          keep &= ~mi;
        }
      if (in) alive[c0 + l] = static_cast<unsigned char>((keep >> l) & 1);
      if (lane == 0) keptBits = keep;
    }
    __syncthreads();
    const uint64_t kept = keptBits;
    if (kept) {
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        const int j = threadIdx.x + r * kNmsThreads;
        if (j >= c0 + 64 && j < n && alive[j]) {
          bool drop = false;
          for (uint64_t k2 = kept; k2 && !drop; k2 &= k2 - 1) {
            const int l = __builtin_ctzll(k2);
            drop = box_iou(cb[l][0], cb[l][1], cb[l][2], cb[l][3], bxr[r][0], bxr[r][1], bxr[r][2], bxr[r][3]) >
                   thresh;
          }
          if (drop) alive[j] = 0;
        }
      }
    }
    __syncthreads();
  }
  for (int j = threadIdx.x; j < n; j += kNmsThreads)
    if (!alive[j]) pr[static_cast<int64_t>(idx[j]) * classes] = 0.f;
}

// Overlap bits of one image's detections (D = min(count, capacity)): bit t
// of word w of row i is box_iou(box i, box j) > thresh for j = 64w + t < D,
// j != i.  box_iou is symmetric bit for bit (max, min, products and the sum
// of the two areas commute), so row i also answers "does i suppress j".
// One thread per (row, word); the word's 64 column boxes are staged in LDS.
__global__ __launch_bounds__(256) void nms_overlap_bits_kernel(int64_t capacity, int64_t words,
                                                               const float* __restrict__ boxes,
                                                               const int32_t* counts, float thresh, uint64_t* bits) {
  __shared__ float cb[64][4];
  const int64_t b = blockIdx.z, w = blockIdx.y;
  const int64_t D = min(static_cast<int64_t>(counts[b]), capacity);
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256;
  if (i0 >= D || 64 * w >= D) return;  // uniform
  const float* bb = boxes + b * capacity * 4;
  const int64_t jn = min(static_cast<int64_t>(64), D - 64 * w);
  if (threadIdx.x < jn) {
    const float* p = bb + (64 * w + threadIdx.x) * 4;
    cb[threadIdx.x][0] = p[0];
    cb[threadIdx.x][1] = p[1];
    cb[threadIdx.x][2] = p[2];
    cb[threadIdx.x][3] = p[3];
  }
  __syncthreads();
  const int64_t i = i0 + threadIdx.x;
  if (i >= D) return;
  const float ax = bb[i * 4], ay = bb[i * 4 + 1], aw = bb[i * 4 + 2], ah = bb[i * 4 + 3];
  uint64_t m = 0;
  for (int t = 0; t < jn; ++t)
    if (64 * w + t != i && box_iou(ax, ay, aw, ah, cb[t][0], cb[t][1], cb[t][2], cb[t][3]) > thresh)
      m |= uint64_t(1) << t;
  bits[(b * capacity + i) * words + w] = m;
}

// doNMSSort of class k of image b over the overlap bits: the sorted
// candidates go in chunks of 64.  Wave 0 resolves a chunk (a member is alive
// unless an earlier kept candidate removed it; lane l reads the bits of the
// later chunk members it suppresses; a 64-step scan keeps l if no kept
// earlier member suppresses it), then the kept members' bit rows are OR-ed
// into `removed` (a bitset over detection indices).  A kept candidate's bit
// is never set (an earlier kept box overlapping it would have removed it),
// so at the end a candidate survives iff its bit is clear: the greedy
// result, without recomputing an overlap per class.
__global__ __launch_bounds__(kNmsThreads) void yolo_nms_bits_kernel(int64_t capacity, int64_t words, int classes,
                                                                  float* prob, const int32_t* counts,
                                                                  const uint64_t* __restrict__ bits) {
  __shared__ float score[kNmsMax];
  __shared__ int idx[kNmsMax + 64];
  __shared__ uint64_t removed[kNmsMax / 64];
  __shared__ int waveSum[kNmsThreads / 64];
  __shared__ int q;
  __shared__ uint64_t keptBits;
  const int k = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m = min(static_cast<int64_t>(counts[b]), capacity);
  float* pr = prob + static_cast<int64_t>(b) * capacity * classes + k;
  const int n = nms_collect_sort(capacity, classes, pr, m, score, idx, waveSum, q);
  if (n <= 1) return;
  const int W = static_cast<int>((m + 63) / 64);
  for (int w = threadIdx.x; w < W; w += kNmsThreads) removed[w] = 0;
  // positions past the last candidate name candidate 0, so every lookup
  // below reads a valid row and word and needs no condition
  for (int j = n + threadIdx.x; j < n + 64; j += kNmsThreads) idx[j] = idx[0];
  __syncthreads();
  const uint64_t* rows = bits + static_cast<int64_t>(b) * capacity * words;
  constexpr int kPairs = 64 * (kNmsMax / 64) / kNmsThreads;  // (member, word) pairs per thread at most
  for (int c0 = 0; c0 < n; c0 += 64) {
    // removed |= row of every kept member, over (member, word) pairs spread
    // over the threads: the rows of all 64 members are loaded first, before
    // the chunk is resolved (the loads depend only on the sorted order), so
    // their latency passes while wave 0 resolves it; the kept ones are
    // selected afterwards
    uint64_t r[kPairs];
#pragma unroll
    for (int u = 0; u < kPairs; ++u) {
      const int p = threadIdx.x + u * kNmsThreads;
      const int l = p / W, w = p - (p / W) * W;
      r[u] = rows[static_cast<int64_t>(idx[c0 + (l & 63)]) * words + w];
    }
    if (wave == 0) {
      const int l = lane;
      const bool in = c0 + l < n;
      const int di = idx[c0 + l];
      const bool alive = in && !((removed[di >> 6] >> (di & 63)) & 1);
      // the later chunk members l suppresses: 64 independent loads with no
      // condition around them (a load inside a lane-dependent branch waits
      // for every outstanding load at the branch's join), masked afterwards;
      // each reads the 32-bit half of the word that holds the member's bit
      uint64_t mask = 0;
      const uint32_t* row = reinterpret_cast<const uint32_t*>(rows + static_cast<int64_t>(idx[c0 + l]) * words);
#pragma unroll
      for (int g = 0; g < 64; g += 16) {  // 16 loads in flight, then their bits
        int dt[16];
        uint32_t wv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) dt[u] = idx[c0 + g + u];
#pragma unroll
        for (int u = 0; u < 16; ++u) wv[u] = row[dt[u] >> 5];
#pragma unroll
        for (int u = 0; u < 16; ++u) mask |= static_cast<uint64_t>((wv[u] >> (dt[u] & 31)) & 1u) << (g + u);
      }
      const int rest = n - c0;  // chunk members present
      const uint64_t present = rest >= 64 ? ~uint64_t(0) : (uint64_t(1) << rest) - 1;
      mask &= present & (l == 63 ? 0 : ~uint64_t(0) << (l + 1));
      uint64_t keep = __ballot(alive);
      const uint32_t mlo = static_cast<uint32_t>(mask), mhi = static_cast<uint32_t>(mask >> 32);
      for (int i = 0; i < 64; ++i)
        if ((keep >> i) & 1) {
          // readlane returns a signed int: widen through uint32_t so the low
          // word does not sign-extend into the high one
          const uint64_t mi = (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(mhi, i))) << 32) |
                              static_cast<uint32_t>(__builtin_amdgcn_readlane(mlo, i));
          keep &= ~mi;
        }
      if (lane == 0) keptBits = keep;
    }
    __syncthreads();
    const uint64_t kept = keptBits;
#pragma unroll
    for (int u = 0; u < kPairs; ++u) {
      const int p = threadIdx.x + u * kNmsThreads;
      const int l = p / W;
      const bool use = p < 64 * W && ((kept >> l) & 1);  // kept members are < n
      if (use && r[u])
        atomicOr(reinterpret_cast<unsigned long long*>(&removed[p % W]), static_cast<unsigned long long>(r[u]));
    }
    __syncthreads();
  }
  for (int j = threadIdx.x; j < n; j += kNmsThreads) {
    const int dj = idx[j];
    if ((removed[dj >> 6] >> (dj & 63)) & 1) pr[static_cast<int64_t>(dj) * classes] = 0.f;
  }
}

}  // namespace
}  // namespace tnh

using namespace tnh;

extern "C" int32_t tnh_yolo_detections(int64_t batch, int32_t nHeads, const float* const* heads, const int64_t* hw,
                                       int64_t n, int64_t classes, const float* anchors, int64_t netW, int64_t netH,
                                       int64_t imgW, int64_t imgH, float thresh, int32_t relative, int32_t letter,
                                       int64_t capacity, float* boxes, float* objectness, float* prob,
                                       int32_t* counts) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch > 0 && nHeads > 0 && nHeads <= kMaxHeads, "yolo_detections: batch %lld, %d heads (1..%d)",
          (long long)batch, nHeads, kMaxHeads);
  TNH_ARG(n > 0 && n <= kMaxAnchors && classes > 0, "yolo_detections: n %lld (1..%d), classes %lld", (long long)n,
          kMaxAnchors, (long long)classes);
  TNH_ARG(heads && hw && anchors && boxes && objectness && prob && counts, "yolo_detections: NULL argument");
  TNH_ARG(netW > 0 && netH > 0 && imgW > 0 && imgH > 0 && capacity > 0, "yolo_detections: bad sizes");
  TNH_ARG(batch <= 65535, "yolo_detections: batch too large");
  DetArgs a{};
  a.nHeads = nHeads;
  a.n = static_cast<int>(n);
  a.classes = static_cast<int>(classes);
  a.headBase[0] = 0;
  for (int hd = 0; hd < nHeads; ++hd) {
    TNH_ARG(heads[hd] && hw[2 * hd] > 0 && hw[2 * hd + 1] > 0, "yolo_detections: head %d", hd);
    a.head[hd] = heads[hd];
    a.h[hd] = static_cast<int>(hw[2 * hd]);
    a.w[hd] = static_cast<int>(hw[2 * hd + 1]);
    a.headBase[hd + 1] = a.headBase[hd] + hw[2 * hd] * hw[2 * hd + 1] * n;
    for (int an = 0; an < n; ++an) {
      a.anchorW[hd][an] = anchors[(hd * n + an) * 2];
      a.anchorH[hd][an] = anchors[(hd * n + an) * 2 + 1];
    }
  }
  TNH_ARG(a.headBase[nHeads] < (int64_t(1) << 31), "yolo_detections: too many candidates");
  a.netW = static_cast<int>(netW);
  a.netH = static_cast<int>(netH);
  a.imgW = static_cast<int>(imgW);
  a.imgH = static_cast<int>(imgH);
  a.thresh = thresh;
  a.relative = relative != 0;
  // correctBoxes (nyololayer.pas:452-476): letterbox size, then the float
  // shifts and ratios (integer / integer is a floating division, rounded to
  // single on assignment)
  int64_t newW = netW, newH = netH;
  if (letter) {
    if (static_cast<double>(netW) / imgW < static_cast<double>(netH) / imgH) {
      newW = netW;
      newH = (imgH * netW) / imgW;
    } else {
      newH = netH;
      newW = (imgW * netH) / imgH;
    }
  }
  a.deltaW = static_cast<float>(netW - newW);
  a.deltaH = static_cast<float>(netH - newH);
  a.ratioW = static_cast<float>(static_cast<double>(newW) / netW);
  a.ratioH = static_cast<float>(static_cast<double>(newH) / netH);
  a.capacity = capacity;
  a.boxes = boxes;
  a.obj = objectness;
  a.prob = prob;
  a.counts = counts;
  hipLaunchKernelGGL(yolo_detect_kernel, dim3(static_cast<unsigned>(batch)), dim3(kDetThreads), 0, cx->stream, a);
  return launch_status("yolo_detect_kernel");
}

extern "C" int32_t tnh_yolo_nms_sort(int64_t batch, int64_t classes, int64_t capacity, const float* boxes, float* prob,
                                     const int32_t* counts, float thresh) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch > 0 && batch <= 65535 && classes > 0 && classes <= 65535, "yolo_nms_sort: bad batch/classes");
  TNH_ARG(capacity > 0 && capacity <= kNmsMax, "yolo_nms_sort: capacity %lld (1..%d detections per image)",
          (long long)capacity, kNmsMax);
  TNH_ARG(boxes && prob && counts, "yolo_nms_sort: NULL argument");
  // Overlap bits of every image in the context scratch (batch x capacity x
  // capacity/64 words), computed once and shared by the classes; without the
  // scratch (no memory, or a stream under capture that would need it grown)
  // each class computes its overlaps itself.
  const int64_t words = (capacity + 63) / 64;
  uint64_t* bits =
      static_cast<uint64_t*>(workspace(cx, static_cast<size_t>(batch * capacity * words) * sizeof(uint64_t)));
  const dim3 grid(static_cast<unsigned>(classes), static_cast<unsigned>(batch));
  if (!bits) {
    hipLaunchKernelGGL(yolo_nms_sort_kernel, grid, dim3(kNmsThreads), 0, cx->stream, capacity,
                       static_cast<int>(classes), boxes, prob, counts, thresh);
    return launch_status("yolo_nms_sort_kernel");
  }
  hipLaunchKernelGGL(nms_overlap_bits_kernel,
                     dim3(static_cast<unsigned>((capacity + 255) / 256), static_cast<unsigned>(words),
                          static_cast<unsigned>(batch)),
                     dim3(256), 0, cx->stream, capacity, words, boxes, counts, thresh, bits);
  if (int st = launch_status("nms_overlap_bits_kernel")) return st;
  hipLaunchKernelGGL(yolo_nms_bits_kernel, grid, dim3(kNmsThreads), 0, cx->stream, capacity, words,
                     static_cast<int>(classes), prob, counts, bits);
  return launch_status("yolo_nms_bits_kernel");
}
