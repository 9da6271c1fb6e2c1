/*
 * refcpu.c -- CPU restatement of Tensorium's fp32 convolution hot path.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle + "port" CPU baseline).  The
 * product library never links or calls this file.
 *
 * Build: oracle/build.sh (gcc -O3 -mavx2 -mfma -ffp-contract=off, pthreads).
 * -ffp-contract=off matters: the reference's SSE/AVX code issues separate
 * mul/add except where it uses vfmadd explicitly, and every FMA here is an
 * explicit intrinsic or fmaf().
 *
 * How each routine is pinned (tests/test_oracle.py, tests/golden/):
 *   ref_sgemm NN/TN   exact-integer fixture (any order exact), numpy fp64
 *                     bound, FMA-vs-mul+add discriminating case, K=1/alpha/beta
 *                     closed forms.
 *   ref_sgemm NT      same + a hand-derived case that only an 8-lane
 *                     accumulator with the (t0+t1)+(t2+t3) reduction yields.
 *   ref_sgemm TT      same (scalar chain, FMA contraction left as mul+add).
 *   im2col            literal hand-written 2x3x3 fixture + torch.nn.functional
 *                     .unfold (library) bit-exact.
 *   col2im            adjoint identity <im2col x, y> = <x, col2im y> on small
 *                     integers (exact), torch fold (library) on integers, and
 *                     a hand-derived accumulation-order case.
 *   bias/scale/leaky  closed forms, bit-exact (single fp32 op per element).
 *   maxpool           torch max_pool2d (library) values + indices, tie rule,
 *                     all-(-inf) window case (-MaxSingle, index -1).
 *   upsample          torch interpolate(nearest) (library), backward on
 *                     integers vs a brute-force sum.
 *   bn normalize      closed form vs numpy fp64 within 1 ulp; fuse_bn vs
 *                     unfused forward within tolerance.
 *   conv_forward      torch conv2d fp64 (library) per-tensor bound.
 *   logistic          exact mode vs fp64 sigmoid within 2e-3 (the reference
 *                     polynomial's own error).
 */
#define _GNU_SOURCE
#include "refcpu.h"

#include <float.h>
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------
 * steroids-equivalent worker pool (steroids.pas:281-296, 606-641, 716-749)
 * ---------------------------------------------------------------------- */
static int g_threads = 0;

void ref_set_threads(int p) { g_threads = p; }

int ref_get_threads(void) {
  if (g_threads > 0) return g_threads;
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 4 ? (int)n : 4; /* GetSystemThreadCount = max(ProcessorCount,4) */
}

typedef void (*range_fn)(int64_t from, int64_t to, void *ctx); /* inclusive */

typedef struct {
  range_fn fn;
  void *ctx;
  int64_t from, to;
} range_job;

static void *range_thread(void *p) {
  range_job *j = (range_job *)p;
  j->fn(j->from, j->to, j->ctx);
  return NULL;
}

/* TOPool.&For chunked dispatch (steroids.pas:606-641): worker i gets
 * ceil((N+1)/P) - (i > N mod P) consecutive indices, N = to - from. */
static void par_for_chunked(range_fn fn, int64_t from, int64_t to, void *ctx) {
  if (to < from) return;
  int P = ref_get_threads();
  int64_t N = to - from;
  int64_t group_t = (N + 1 + P - 1) / P;
  int64_t group_m = N % P;
  range_job jobs[1024];
  pthread_t th[1024];
  int nj = 0;
  int64_t ii = 0;
  if (P > 1024) P = 1024;
  for (int i = 0; i < P; ++i) {
    int64_t start = ii;
    ii += group_t - (i > group_m ? 1 : 0);
    if (ii <= start) break;
    jobs[nj].fn = fn;
    jobs[nj].ctx = ctx;
    jobs[nj].from = from + start;
    jobs[nj].to = from + ii - 1;
    ++nj;
  }
  if (nj == 1) {
    fn(jobs[0].from, jobs[0].to, ctx);
    return;
  }
  for (int i = 0; i < nj; ++i) pthread_create(&th[i], NULL, range_thread, &jobs[i]);
  for (int i = 0; i < nj; ++i) pthread_join(th[i], NULL);
}

typedef void (*idx_fn)(int64_t idx, void *ctx);
typedef struct {
  idx_fn fn;
  void *ctx;
  int64_t start, count, span;
} strided_job;

static void *strided_thread(void *p) {
  strided_job *j = (strided_job *)p;
  for (int64_t i = j->start; i < j->count; i += j->span) j->fn(i, j->ctx);
  return NULL;
}

/* TOPool.&for strided dispatch (steroids.pas:716-749, loop :492-499). */
static void par_for_strided(idx_fn fn, int64_t count, void *ctx) {
  int P = ref_get_threads();
  if (P > 1024) P = 1024;
  strided_job jobs[1024];
  pthread_t th[1024];
  int nj = 0;
  for (int i = 0; i < P && i < count; ++i) {
    jobs[nj].fn = fn;
    jobs[nj].ctx = ctx;
    jobs[nj].start = i;
    jobs[nj].count = count;
    jobs[nj].span = P;
    ++nj;
  }
  if (nj <= 1) {
    for (int64_t i = 0; i < count; ++i) fn(i, ctx);
    return;
  }
  for (int i = 0; i < nj; ++i) pthread_create(&th[i], NULL, strided_thread, &jobs[i]);
  for (int i = 0; i < nj; ++i) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------
 * BLAS-1 kernels
 * ---------------------------------------------------------------------- */

/* saxpy_avx2 (ntensors.pas:1308-1436), SIMD_REGS = 8: y[j] = fma(a, x[j], y[j])
 * in 32-, 8- and 1-wide steps; every element is one fused multiply-add. */
static void saxpy8(int64_t n, float a, const float *x, float *y) {
  __m256 va = _mm256_set1_ps(a);
  int64_t j = 0;
  for (; j + 32 <= n; j += 32) {
    __m256 y0 = _mm256_loadu_ps(y + j), y1 = _mm256_loadu_ps(y + j + 8);
    __m256 y2 = _mm256_loadu_ps(y + j + 16), y3 = _mm256_loadu_ps(y + j + 24);
    y0 = _mm256_fmadd_ps(va, _mm256_loadu_ps(x + j), y0);
    y1 = _mm256_fmadd_ps(va, _mm256_loadu_ps(x + j + 8), y1);
    y2 = _mm256_fmadd_ps(va, _mm256_loadu_ps(x + j + 16), y2);
    y3 = _mm256_fmadd_ps(va, _mm256_loadu_ps(x + j + 24), y3);
    _mm256_storeu_ps(y + j, y0);
    _mm256_storeu_ps(y + j + 8, y1);
    _mm256_storeu_ps(y + j + 16, y2);
    _mm256_storeu_ps(y + j + 24, y3);
  }
  for (; j + 8 <= n; j += 8)
    _mm256_storeu_ps(y + j, _mm256_fmadd_ps(va, _mm256_loadu_ps(x + j), _mm256_loadu_ps(y + j)));
  for (; j < n; ++j) y[j] = fmaf(a, x[j], y[j]);
}

/* sdot_avx2 (ntensors.pas:1233-1306), SIMD_REGS = 8:
 * acc[l] = fma chain over k = 8q + l; masked tail lanes add fma(0,0,acc);
 * reduce t[l] = acc[l] + acc[l+4] (vextractf128/vaddps), then two vhaddps:
 * s = (t0 + t1) + (t2 + t3). */
static float sdot8(int64_t n, const float *a, const float *b) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t q = n >> 3, j = 0;
  for (int64_t i = 0; i < q; ++i, j += 8)
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[j + l], b[j + l], acc[l]);
  int64_t r = n & 7;
  if (r) {
    for (int l = 0; l < 8; ++l) {
      float av = l < r ? a[j + l] : 0.0f;
      float bv = l < r ? b[j + l] : 0.0f;
      acc[l] = fmaf(av, bv, acc[l]);
    }
  }
  float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5];
  float t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
  return (t0 + t1) + (t2 + t3);
}

/* ------------------------------------------------------------------------
 * cblas_sgemm (ntensors.pas:2231-2286) and its row workers
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t M, N, K, lda, ldb, ldc;
  float alpha;
  const float *A, *B;
  float *C;
} gemm_ctx;

/* s_nn (ntensors.pas:2061-2134): for i, for kk: saxpy(N, alpha*A[i,kk], B[kk,:], C[i,:]) */
static void s_nn(int64_t f, int64_t t, void *p) {
  gemm_ctx *g = (gemm_ctx *)p;
  for (int64_t i = f; i <= t; ++i) {
    const float *a = g->A + i * g->lda;
    float *c = g->C + i * g->ldc;
    for (int64_t kk = 0; kk < g->K; ++kk)
      saxpy8(g->N, g->alpha * a[kk], g->B + kk * g->ldb, c);
  }
}

/* s_tn (ntensors.pas:2007-2032): A_PART = alpha*A[kk*lda + i] */
static void s_tn(int64_t f, int64_t t, void *p) {
  gemm_ctx *g = (gemm_ctx *)p;
  for (int64_t i = f; i <= t; ++i) {
    float *c = g->C + i * g->ldc;
    for (int64_t kk = 0; kk < g->K; ++kk)
      saxpy8(g->N, g->alpha * g->A[kk * g->lda + i], g->B + kk * g->ldb, c);
  }
}

/* s_nt (ntensors.pas:1957-1983): sum = alpha*sdot(K, A[i,:], B[j,:]); C += sum */
static void s_nt(int64_t f, int64_t t, void *p) {
  gemm_ctx *g = (gemm_ctx *)p;
  for (int64_t i = f; i <= t; ++i)
    for (int64_t j = 0; j < g->N; ++j) {
      float sum = g->alpha * sdot8(g->K, g->A + i * g->lda, g->B + j * g->ldb);
      float *c = g->C + i * g->ldc + j;
      *c = *c + sum;
    }
}

/* s_tt (ntensors.pas:2159-2184): scalar; sum := sum + ALPHA*A*B evaluated as
 * separate single-precision mul, mul, add (no contraction, left to right). */
static void s_tt(int64_t f, int64_t t, void *p) {
  gemm_ctx *g = (gemm_ctx *)p;
  for (int64_t i = f; i <= t; ++i)
    for (int64_t j = 0; j < g->N; ++j) {
      float sum = 0.0f;
      for (int64_t kk = 0; kk < g->K; ++kk) {
        float prod = g->alpha * g->A[i + kk * g->lda];
        prod = prod * g->B[kk + j * g->ldb];
        sum = sum + prod;
      }
      float *c = g->C + i * g->ldc + j;
      *c = *c + sum;
    }
}

/* sscal (ntensors.pas:1439-1464) via cblas_sscal (:1566): x = alpha*x */
static void sscal_row(int64_t n, float a, float *x) {
  for (int64_t j = 0; j < n; ++j) x[j] = a * x[j];
}

/* cblas_saxpy (bound at ntensors.pas:12691) -> saxpy_avx2: y = fma(a, x, y) */
void ref_axpy(int64_t n, float a, const float *x, float *y) { saxpy8(n, a, x, y); }

void ref_sgemm(int transA, int transB, int64_t M, int64_t N, int64_t K,
               float alpha, const float *A, int64_t lda, const float *B,
               int64_t ldb, float beta, float *C, int64_t ldc) {
  /* if beta <> 1 then C[i,:] *= beta (ntensors.pas:2259-2261) */
  if (beta != 1.0f)
    for (int64_t i = 0; i < M; ++i) sscal_row(N, beta, C + i * ldc);
  gemm_ctx g = {M, N, K, lda, ldb, ldc, alpha, A, B, C};
  range_fn fn = !transA ? (!transB ? s_nn : s_nt) : (!transB ? s_tn : s_tt);
  par_for_chunked(fn, 0, M - 1, &g);
}

void ref_sgemm_strided_batched(int transA, int transB, int64_t M, int64_t N,
                               int64_t K, float alpha, const float *A,
                               int64_t lda, int64_t strideA, const float *B,
                               int64_t ldb, int64_t strideB, float beta,
                               float *C, int64_t ldc, int64_t strideC,
                               int64_t batch) {
  for (int64_t i = 0; i < batch; ++i)
    ref_sgemm(transA, transB, M, N, K, alpha, A + i * strideA, lda,
              B + i * strideB, ldb, beta, C + i * strideC, ldc);
}

/* ------------------------------------------------------------------------
 * im2col / col2im
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t C, H, W, kh, kw, pH, pW, sY, sX, dY, dX, OH, OW;
  const float *src;
  float *dst;
  int64_t srcStride, dstStride;
} conv_geom;

static int64_t out_dim(int64_t in, int64_t k, int64_t p, int64_t s, int64_t d) {
  return (in + 2 * p - (d * (k - 1) + 1)) / s + 1;
}

/* i2c_ext body of sim2Col (ntensors.pas:11425-11463) for one channel */
static void i2c_channel(const conv_geom *g, const float *im, float *col, int64_t ch) {
  const float *d_im = im + g->H * g->W * ch;
  float *d_col = col + g->kh * g->kw * g->OH * g->OW * ch;
  for (int64_t ky = 0; ky < g->kh; ++ky)
    for (int64_t kx = 0; kx < g->kw; ++kx) {
      int64_t iy = -g->pH + ky * g->dY;
      for (int64_t oy = 0; oy < g->OH; ++oy) {
        if ((uint64_t)iy < (uint64_t)g->H) {
          int64_t ix = -g->pW + kx * g->dX;
          for (int64_t ox = 0; ox < g->OW; ++ox, ix += g->sX)
            d_col[ox] = (uint64_t)ix < (uint64_t)g->W ? d_im[iy * g->W + ix] : 0.0f;
        } else {
          for (int64_t ox = 0; ox < g->OW; ++ox) d_col[ox] = 0.0f;
        }
        d_col += g->OW;
        iy += g->sY;
      }
    }
}

static void i2c_image(int64_t b, void *p) {
  conv_geom *g = (conv_geom *)p;
  for (int64_t ch = 0; ch < g->C; ++ch)
    i2c_channel(g, g->src + b * g->srcStride, g->dst + b * g->dstStride, ch);
}


static void i2c_chan_job(int64_t ch, void *p) {
  conv_geom *g = (conv_geom *)p;
  i2c_channel(g, g->src, g->dst, ch);
}

void ref_im2col_batched(int64_t C, int64_t H, int64_t W, int64_t kh,
                        int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                        int64_t sX, int64_t dY, int64_t dX, const float *im,
                        int64_t imStride, float *col, int64_t colStride,
                        int64_t batch) {
  conv_geom g = {C, H, W, kh, kw, pH, pW, sY, sX, dY, dX,
                 out_dim(H, kh, pH, sY, dY), out_dim(W, kw, pW, sX, dX),
                 im, col, imStride, colStride};

  if (batch == 1)
    par_for_strided(i2c_chan_job, C, &g); /* mp2 over channels (:11482) */
  else
    par_for_strided(i2c_image, batch, &g); /* mp over images (:11521) */
}

/* c2i (ntensors.pas:11650-11715) for row i = c*k*k + ky*kw + kx of col,
 * accumulating into the channel plane of im. */
static void c2i_row(const conv_geom *g, const float *col, float *im, int64_t i) {
  int64_t ksz = g->kh * g->kw;
  int64_t chan = i / ksz, index = i % ksz;
  int64_t krow = index / g->kw, kcol = index % g->kw;
  const float *d_col = col + i * g->OH * g->OW;
  float *d_im = im + g->H * g->W * chan;
  int64_t iy = (krow - g->pH) * g->dY;
  for (int64_t oy = 0; oy < g->OH; ++oy, iy += g->sY) {
    if ((uint64_t)iy >= (uint64_t)g->H) {
      d_col += g->OW;
      continue;
    }
    int64_t ix = (kcol - g->pW) * g->dX;
    for (int64_t ox = 0; ox < g->OW; ++ox, ++d_col, ix += g->sX)
      if ((uint64_t)ix < (uint64_t)g->W) {
        float *t = d_im + iy * g->W + ix;
        *t = *t + d_col[0];
      }
  }
}

static void c2i_image(int64_t b, void *p) {
  conv_geom *g = (conv_geom *)p;
  for (int64_t i = 0; i < g->C * g->kh * g->kw; ++i)
    c2i_row(g, g->src + b * g->srcStride, g->dst + b * g->dstStride, i);
}

void ref_col2im_batched(int64_t C, int64_t H, int64_t W, int64_t kh,
                        int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                        int64_t sX, int64_t dY, int64_t dX, const float *col,
                        int64_t colStride, float *im, int64_t imStride,
                        int64_t batch) {
  conv_geom g = {C, H, W, kh, kw, pH, pW, sY, sX, dY, dX,
                 out_dim(H, kh, pH, sY, dY), out_dim(W, kw, pW, sX, dX),
                 col, im, colStride, imStride};
  /* The reference spreads rows i over workers at batch = 1 (:11754), which
   * races on shared channel planes; the parity target is the serial order. */
  if (batch == 1)
    c2i_image(0, &g);
  else
    par_for_strided(c2i_image, batch, &g); /* mp over images (:11867) */
}

/* ------------------------------------------------------------------------
 * bias / scale / activation
 * ---------------------------------------------------------------------- */
void ref_forward_bias(float *x, int64_t nb, int64_t blockSize,
                      const float *bias, int64_t batch) {
  for (int64_t k = 0; k < batch; ++k)
    for (int64_t i = 0; i < nb; ++i) {
      float *c = x + (k * nb + i) * blockSize;
      float bb = bias[i];
      for (int64_t j = 0; j < blockSize; ++j) c[j] = bb + c[j];
    }
}

void ref_forward_scale(float *x, int64_t nb, int64_t blockSize,
                       const float *scale, int64_t batch) {
  for (int64_t k = 0; k < batch; ++k)
    for (int64_t i = 0; i < nb; ++i) {
      float *c = x + (k * nb + i) * blockSize;
      float bb = scale[i];
      for (int64_t j = 0; j < blockSize; ++j) c[j] = bb * c[j];
    }
}

/* logistic_array (nactivation.pas:36-127): exp(-x) = 2^i * p(f) with a
 * degree-2 polynomial, then 1/(1+e) by vrcpps (exact=0) or IEEE (exact=1). */
static float logistic_ref(float x, int exact) {
  const float l2e = 1.442695041f, c0 = 1.00172476f, c1 = 0.657636276f,
              c2 = 0.3371894346f, mx = 8.872283E+001f, mn = -8.733654E+001f;
  float t = 0.0f - x;
  if (t >= mx) t = mx;
  if (t <= mn) t = mn;
  t = l2e * t;
  float fi = floorf(t);
  float f = t - fi;
  int32_t i = (int32_t)lrintf(fi);
  float p = fmaf(f, c2, c1);
  p = fmaf(p, f, c0);
  int32_t bits;
  memcpy(&bits, &p, 4);
  bits += (int32_t)((uint32_t)i << 23);
  float e;
  memcpy(&e, &bits, 4);
  float d = e + 1.0f;
  if (exact) return 1.0f / d;
  return _mm_cvtss_f32(_mm_rcp_ss(_mm_set_ss(d)));
}

void ref_activate(float *x, int64_t n, int act, int exact) {
  switch (act) {
    case REF_AC_LEAKY: /* leaky_array (nactivation.pas:234-268) */
      for (int64_t i = 0; i < n; ++i)
        if (0.0f > x[i]) x[i] = 0.1f * x[i];
      break;
    case REF_AC_LOGISTIC:
      for (int64_t i = 0; i < n; ++i) x[i] = logistic_ref(x[i], exact);
      break;
    default: /* acLINEAR: no-op */
      break;
  }
}

void ref_derive(const float *x, int64_t n, int act, float *delta) {
  if (act == REF_AC_LEAKY) /* leaky_gradient (nactivation.pas:472-476) */
    for (int64_t i = 0; i < n; ++i) delta[i] = delta[i] * (x[i] > 0.0f ? 1.0f : 0.1f);
}

void ref_yolo_fwd(int64_t batch, int64_t n, int64_t classes, int64_t h,
                  int64_t w, const float *in, float *out, int exact) {
  int64_t hw = h * w, per = (classes + 5) * hw;
  memcpy(out, in, sizeof(float) * batch * n * per); /* state.input.copyTo(output) */
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t a = 0; a < n; ++a) {
      float *o = out + (b * n + a) * per;
      ref_activate(o, 2 * hw, REF_AC_LOGISTIC, exact);                    /* x, y */
      ref_activate(o + 4 * hw, (1 + classes) * hw, REF_AC_LOGISTIC, exact); /* obj, classes */
    }
}

/* ------------------------------------------------------------------------
 * maxpool
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t b, C, H, W, OH, OW, size, sX, sY, off;
  const float *in;
  float *out;
  int64_t *idx;
} pool_ctx;

/* maxpoolMP (nMaxPoolLayer.pas:265-324), channel range [f..t] of image b */
static void maxpool_chan(int64_t f, int64_t t, void *p) {
  pool_ctx *g = (pool_ctx *)p;
  for (int64_t k = f; k <= t; ++k)
    for (int64_t i = 0; i < g->OH; ++i)
      for (int64_t j = 0; j < g->OW; ++j) {
        int64_t out_index = j + g->OW * (i + g->OH * (k + g->C * g->b));
        float mx = -FLT_MAX;
        int64_t max_i = -1;
        for (int64_t n = 0; n < g->size; ++n)
          for (int64_t m = 0; m < g->size; ++m) {
            int64_t cur_h = g->off + i * g->sY + n;
            int64_t cur_w = g->off + j * g->sX + m;
            int64_t index = cur_w + g->W * (cur_h + g->H * (k + g->b * g->C));
            float val = (cur_h >= 0 && cur_h < g->H && cur_w >= 0 && cur_w < g->W)
                            ? g->in[index] : -FLT_MAX;
            if (val > mx) {
              max_i = index;
              mx = val;
            }
          }
        g->out[out_index] = mx;
        if (g->idx) g->idx[out_index] = max_i;
      }
}

void ref_maxpool_fwd(int64_t batch, int64_t C, int64_t H, int64_t W,
                     int64_t size, int64_t strideX, int64_t strideY,
                     int64_t pad, const float *in, float *out, int64_t *idx) {
  pool_ctx g;
  g.C = C; g.H = H; g.W = W; g.size = size; g.sX = strideX; g.sY = strideY;
  g.OH = (H + pad - size) / strideY + 1; /* TMaxPoolLayer.Create :107-108 */
  g.OW = (W + pad - size) / strideX + 1;
  g.off = -pad / 2;                      /* w_offset := -Padding div 2 */
  g.in = in; g.out = out; g.idx = idx;
  for (int64_t b = 0; b < batch; ++b) {
    g.b = b;
    par_for_chunked(maxpool_chan, 0, C - 1, &g);
  }
}

void ref_maxpool_bwd(int64_t nOut, const int64_t *idx, const float *dOut, float *dIn) {
  for (int64_t i = 0; i < nOut; ++i) {
    int64_t index = idx[i];
    /* index -1 marks a window with no tap above -MaxSingle (all -inf or
     * outside the image); the reference's serial loop would add into
     * dIn[-1], outside the tensor.  Skipped here, as on the device. */
    if (index < 0) continue;
    dIn[index] = dIn[index] + dOut[i];
  }
}

/* ------------------------------------------------------------------------
 * upsample, shortcut
 * ---------------------------------------------------------------------- */
void ref_upsample(float *in, int64_t w, int64_t h, int64_t C, int64_t batch,
                  int64_t stride, int forward, float scale, float *out) {
  for (int64_t c = 0; c < batch * C; ++c)
    for (int64_t y = 0; y < h * stride; ++y)
      for (int64_t x = 0; x < w * stride; ++x) {
        int64_t in_index = (c * h + y / stride) * w + x / stride;
        int64_t out_index = (c * h * stride + y) * stride * w + x;
        if (forward)
          out[out_index] = scale * in[in_index];
        else {
          float t = scale * out[out_index];
          in[in_index] = in[in_index] + t;
        }
      }
}

void ref_addvv(int64_t n, const float *a, const float *b, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* ------------------------------------------------------------------------
 * batch norm (inference) and folding
 * ---------------------------------------------------------------------- */
void ref_bn_normalize(float *x, int64_t nb, int64_t blockSize,
                      const float *mean, const float *var, int64_t batch,
                      int exact) {
  /* TTensor.blockNormalize (ntensors.pas:8693-8718): one element per channel
   * goes through normvv = _snormvv (:4338), which clamps the variance,
   * (x - m) / sqrt(max(v, 1e-6)), exact division; longer blocks through
   * normblkvv = _snormblkvv (:4357), which clamps the standard deviation,
   * max(sqrt(v), 1e-6), and on AVX2 hosts multiplies by rcpss of it. */
  if (blockSize == 1) {
    for (int64_t g = 0; g < batch; ++g)
      for (int64_t i = 0; i < nb; ++i) {
        float v = var[i] > 1e-6f ? var[i] : 1e-6f; /* Max(v, sEPSILON) */
        float d = sqrtf(v);
        float t = x[g * nb + i] - mean[i];
        x[g * nb + i] = t / d;
      }
    return;
  }
  for (int64_t g = 0; g < batch; ++g)
    for (int64_t i = 0; i < nb; ++i) {
      float *o = x + (g * nb + i) * blockSize;
      float d = sqrtf(var[i]);
      if (!(d > 1e-6f)) d = 1e-6f; /* math.Max(d, sEPSILON) = d > eps ? d : eps, sEPSILON = 1e-6 */
      float m = mean[i];
      if (exact) {
        for (int64_t j = 0; j < blockSize; ++j) o[j] = (o[j] - m) / d;
      } else {
        float r = _mm_cvtss_f32(_mm_rcp_ss(_mm_set_ss(d)));
        float nm = 0.0f - m;
        for (int64_t j = 0; j < blockSize; ++j) o[j] = r * (nm + o[j]);
      }
    }
}

void ref_fuse_bn(int64_t F, int64_t filterSize, float *W, float *bias,
                 const float *scales, const float *mean, const float *var) {
  for (int64_t f = 0; f < F; ++f) {
    float v = var[f] > 1e-6f ? var[f] : 1e-6f;
    float pre = scales[f] / sqrtf(v);
    float mp = mean[f] * pre;
    bias[f] = bias[f] - mp;
    for (int64_t i = 0; i < filterSize; ++i) W[f * filterSize + i] = W[f * filterSize + i] * pre;
  }
}

/* ------------------------------------------------------------------------
 * training-mode batch norm: channel statistics and their deltas, addDots,
 * softmax.  Two coherent configurations of the reference are restated:
 *   avx2 = 1  the Makefile build on an AVX2 host (AVX2Support true): the
 *             assembler routines vssum_avx2, srss, sVarinceDelta_avx, sdot;
 *   avx2 = 0  the same build on a host without AVX2: the Pascal loops.
 * srss and sVarinceDelta_avx drop the upper four lanes of their eight-lane
 * accumulator when N % 8 == 0 (they fold lanes 4..7 into 0..3 only on the
 * path that handles a remainder, ntensors.pas:1508-1513, 8738-8743, and
 * reduce xmm0 alone otherwise), so on an AVX2 host the variances and
 * variance deltas of blocks whose length is a multiple of 8 sum only the
 * elements k with k % 8 < 4.  The parity target is the avx2 = 0 form (the
 * definition the Pascal loops and TNNCuda's kernels compute).
 * ---------------------------------------------------------------------- */

/* vssum_avx2 (ntensors.pas:3530-3560): lane l sums a[8q + l]; the lanes
 * fold t[l] = acc[l] + acc[l + 4], two haddps give (t0 + t1) + (t2 + t3),
 * then the n % 8 tail is added in order. */
static float vssum8(int64_t n, const float *a) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t q = n >> 3, j = 0;
  for (int64_t i = 0; i < q; ++i, j += 8)
    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + a[j + l];
  float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5], t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
  float s = (t0 + t1) + (t2 + t3);
  for (; j < n; ++j) s = s + a[j];
  return s;
}

/* vsSumI's Pascal loop (ntensors.pas:3631-3633) */
static float sum_scalar(int64_t n, const float *a) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s = s + a[i];
  return s;
}

/* The common tail of srss / sVarinceDelta_avx: with a remainder the upper
 * lanes fold into the lower ones and the remainder terms add to lane 0 in
 * order; with none lanes 4..7 are dropped; then two haddps. */
static float lane_tail(float acc[8], const float *terms, int64_t r) {
  float t0 = acc[0], t1 = acc[1], t2 = acc[2], t3 = acc[3];
  if (r) {
    t0 = t0 + acc[4];
    t1 = t1 + acc[5];
    t2 = t2 + acc[6];
    t3 = t3 + acc[7];
    for (int64_t i = 0; i < r; ++i) t0 = t0 + terms[i];
  }
  return (t0 + t1) + (t2 + t3);
}

/* srss (ntensors.pas:1493-1525): acc[l] += (mean - a)^2 (vsubps, vmulps,
 * vaddps: separate roundings). */
static float srss8(int64_t n, float mean, const float *a) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, tail[8];
  int64_t q = n >> 3, j = 0, r = n & 7;
  for (int64_t i = 0; i < q; ++i, j += 8)
    for (int l = 0; l < 8; ++l) {
      float d = mean - a[j + l];
      acc[l] = acc[l] + d * d;
    }
  for (int64_t i = 0; i < r; ++i) {
    float d = mean - a[j + i];
    tail[i] = d * d;
  }
  return lane_tail(acc, tail, r);
}

/* vsRSS's Pascal loop (ntensors.pas:1655-1657): sqr(a - mean) in order */
static float rss_scalar(int64_t n, float mean, const float *a) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float d = a[i] - mean;
    s = s + d * d;
  }
  return s;
}

/* sVarinceDelta_avx (ntensors.pas:8721-8756): acc[l] += (x - mean) * delta */
static float var_delta8(int64_t n, float mean, const float *delta, const float *x) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, tail[8];
  int64_t q = n >> 3, j = 0, r = n & 7;
  for (int64_t i = 0; i < q; ++i, j += 8)
    for (int l = 0; l < 8; ++l) {
      float d = x[j + l] - mean;
      acc[l] = acc[l] + d * delta[j + l];
    }
  for (int64_t i = 0; i < r; ++i) {
    float d = x[j + i] - mean;
    tail[i] = d * delta[j + i];
  }
  return lane_tail(acc, tail, r);
}

typedef struct {
  const float *src, *delta, *x, *mean, *var;
  float *o1, *o2;
  int64_t nch, block, groups;
  int avx2;
} bn_ctx;

/* MnV of TTensor.MeansAndVars (ntensors.pas:9119-9136) for channels [f, t] */
static void mnv_range(int64_t f, int64_t t, void *p) {
  const bn_ctx *c = (const bn_ctx *)p;
  const float S = (float)(c->groups * c->block), S2 = (float)(c->groups * c->block - 1);
  for (int64_t i = f; i <= t; ++i) {
    float m = 0.0f, v = 0.0f;
    for (int64_t b = 0; b < c->groups; ++b) {
      const float *d = c->src + (i + b * c->nch) * c->block;
      m = m + (c->avx2 ? vssum8(c->block, d) : sum_scalar(c->block, d));
    }
    m = m / S;
    c->o1[i] = m;
    for (int64_t b = 0; b < c->groups; ++b) {
      const float *d = c->src + (i + b * c->nch) * c->block;
      v = v + (c->avx2 ? srss8(c->block, m, d) : rss_scalar(c->block, m, d));
    }
    c->o2[i] = v / S2;
  }
}

void ref_means_vars(const float *src, int64_t nch, int64_t block, int64_t groups, float *means, float *vars,
                    int avx2) {
  bn_ctx c = {src, NULL, NULL, NULL, NULL, means, vars, nch, block, groups, avx2};
  par_for_chunked(mnv_range, 0, nch - 1, &c); /* mp.&For(MnV, 0, N) */
}

/* MnVD of sMeanAndVarianceDelta (ntensors.pas:8838-8865) for channels [f, t]:
 * m sums the deltas (vsSumI); v sums delta * (x - mean) per block through
 * sVarinceDelta_avx on AVX2 hosts, else in one Pascal loop over every block;
 * mean_delta = m * (-1 / sqrt(max(var, eps))) in single precision,
 * variance_delta = v * -0.5 * Power(max(var, eps), -1.5) with Power in double. */
static void mnvd_range(int64_t f, int64_t t, void *p) {
  const bn_ctx *c = (const bn_ctx *)p;
  for (int64_t i = f; i <= t; ++i) {
    float m = 0.0f, v = 0.0f;
    const float mu = c->mean[i];
    for (int64_t j = 0; j < c->groups; ++j) {
      const int64_t idx = (i + j * c->nch) * c->block;
      m = m + (c->avx2 ? vssum8(c->block, c->delta + idx) : sum_scalar(c->block, c->delta + idx));
      if (c->avx2) {
        v = v + var_delta8(c->block, mu, c->delta + idx, c->x + idx);
      } else {
        for (int64_t k = 0; k < c->block; ++k) {
          float d = c->x[idx + k] - mu;
          v = v + c->delta[idx + k] * d;
        }
      }
    }
    float vc = c->var[i] > 1e-6f ? c->var[i] : 1e-6f;
    float r = -1.0f / sqrtf(vc);
    c->o1[i] = m * r;
    c->o2[i] = (float)((double)(v * -0.5f) * pow((double)vc, -1.5));
  }
}

void ref_means_vars_delta(const float *delta, const float *x, const float *mean, const float *var, int64_t nch,
                          int64_t block, int64_t groups, float *mean_delta, float *variance_delta, int avx2) {
  bn_ctx c = {NULL, delta, x, mean, var, mean_delta, variance_delta, nch, block, groups, avx2};
  par_for_chunked(mnvd_range, 0, nch - 1, &c);
}

/* TTensor.addDots (ntensors.pas:7783-7830): dst[i] += sum over groups of
 * cblas_sdot of the channel's block (sdot_avx2 on AVX2 hosts, ntensors.pas:
 * 12731, else the Pascal loop); one element per channel: one strided dot
 * over the groups (cblas_sdot's loop, :2217-2219). */
void ref_add_dots(float *dst, const float *a, const float *b, int64_t nch, int64_t block, int64_t groups,
                  int avx2) {
  for (int64_t i = 0; i < nch; ++i) {
    if (block == 1) {
      float s = 0.0f;
      for (int64_t g = 0; g < groups; ++g) s = s + a[i + g * nch] * b[i + g * nch];
      dst[i] = dst[i] + s;
      continue;
    }
    float sum = 0.0f;
    for (int64_t g = 0; g < groups; ++g) {
      const int64_t idx = (i + g * nch) * block;
      float d;
      if (avx2) {
        d = sdot8(block, a + idx, b + idx);
      } else {
        d = 0.0f;
        for (int64_t k = 0; k < block; ++k) d = d + a[idx + k] * b[idx + k];
      }
      sum = sum + d;
    }
    dst[i] = dst[i] + sum;
  }
}

/* softmax (nsoftmaxlayer.pas:81-105) over `rows` rows of n values:
 * e = exp((x - largest) / temp) with exp in double and e stored as single,
 * sum accumulated in order in single, out = e / sum. */
void ref_softmax_rows(const float *x, int64_t rows, int64_t n, float temp, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *in = x + r * n;
    float *o = out + r * n;
    float largest = in[0], sum = 0.0f;
    for (int64_t i = 1; i < n; ++i)
      if (in[i] > largest) largest = in[i];
    for (int64_t i = 0; i < n; ++i) {
      float e = (float)exp((double)((in[i] - largest) / temp));
      sum = sum + e;
      o[i] = e;
    }
    for (int64_t i = 0; i < n; ++i) o[i] = o[i] / sum;
  }
}

/* ------------------------------------------------------------------------
 * convolutional layer forward (BN folded)
 * ---------------------------------------------------------------------- */
void ref_conv_forward(int64_t batch, int64_t C, int64_t H, int64_t W,
                      int64_t F, int64_t k, int64_t stride, int64_t pad,
                      const float *x, const float *Wt, const float *bias,
                      int act, float *out, float *workspace) {
  int64_t OH = (H + 2 * pad - k) / stride + 1;
  int64_t OW = (W + 2 * pad - k) / stride + 1;
  int64_t N = OH * OW, K = C * k * k;
  const float *Bm;
  int64_t strideB;
  if (k != 1 || stride != 1) {
    ref_im2col_batched(C, H, W, k, k, pad, pad, stride, stride, 1, 1, x,
                       C * H * W, workspace, K * N, batch);
    Bm = workspace;
    strideB = K * N;
  } else {
    Bm = x;
    strideB = C * H * W;
  }
  for (int64_t b = 0; b < batch; ++b)
    ref_sgemm(0, 0, F, N, K, 1.0f, Wt, K, Bm + b * strideB, N, 0.0f,
              out + b * F * N, N);
  ref_forward_bias(out, F, N, bias, batch);
  ref_activate(out, batch * F * N, act, 1);
}
