/*
 * CPU oracle (test infrastructure only; see oracle.h). Plain C11 + OpenMP.
 * Each function restates the reference semantics it cites; nothing here is
 * shipped or called by the product library.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int valid_quant(int group, int bits) {
  return (group == 32 || group == 64 || group == 128) &&
         (bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8);
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

uint16_t orc_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t x) {
  uint32_t u = (uint32_t)x << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* native/projection_reference.h:16: bit = col*bits, word = bit/32, shift = bit%32,
 * the next word supplies the high bits when shift+bits > 32. */
unsigned orc_code(const uint32_t* row, size_t col, int bits) {
  size_t bit = col * (size_t)bits, word = bit / 32;
  unsigned shift = (unsigned)(bit % 32);
  uint64_t value = row[word];
  if (shift + (unsigned)bits > 32) value |= (uint64_t)row[word + 1] << 32;
  return (unsigned)((value >> shift) & ((1u << bits) - 1u));
}

static int all_finite(const float* v, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(v[i])) return 0;
  return 1;
}

int orc_qmm(const float* x, size_t rows, const uint32_t* packed, const float* scales,
            const float* biases, size_t outputs, size_t width, int group, int bits, double* y,
            int threads) {
  if (!x || !packed || !scales || !biases || !y || rows == 0 || outputs == 0 || width == 0 ||
      !valid_quant(group, bits) || width % (size_t)group || (width * bits) % 32)
    return -1;
  const size_t words = width * bits / 32, groups = width / group;
  if (!all_finite(x, rows * width) || !all_finite(scales, outputs * groups) ||
      !all_finite(biases, outputs * groups))
    return -1;
  if (threads <= 0) threads = orc_max_threads();
  (void)threads;
  long o;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (o = 0; o < (long)outputs; ++o) {
    const uint32_t* row = packed + (size_t)o * words;
    for (size_t r = 0; r < rows; ++r) {
      double sum = 0;
      for (size_t c = 0; c < width; ++c) {
        size_t g = (size_t)o * groups + c / group;
        unsigned q = orc_code(row, c, bits);
        sum += (double)x[r * width + c] * ((double)scales[g] * q + (double)biases[g]);
      }
      y[r * outputs + (size_t)o] = sum;
    }
  }
  return 0;
}

/* One output row's contribution: for each group of 64 columns the weights
 * s*q + b in f32, then every listed token row's dot product with them. */
static void qmm4_row_f32(const float* x, size_t width, const uint32_t* row, const float* s, const float* b,
                         const int32_t* tok, size_t ntok, float* acc) {
  float w[64];
  for (size_t t = 0; t < ntok; ++t) acc[t] = 0.f;
  for (size_t g = 0; g < width / 64; ++g) {
    for (int j = 0; j < 8; ++j) {
      const uint32_t word = row[g * 8 + j];
      for (int k = 0; k < 8; ++k) w[8 * j + k] = s[g] * (float)((word >> (4 * k)) & 15u) + b[g];
    }
    for (size_t t = 0; t < ntok; ++t) {
      const float* xr = x + (size_t)(tok ? tok[t] : (int32_t)t) * width + g * 64;
      /* eight running sums (lane c % 8), added in a fixed tree: a vectorisable order */
      float p[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int c = 0; c < 64; c += 8)
        for (int k = 0; k < 8; ++k) p[k] += xr[c + k] * w[c + k];
      acc[t] += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
  }
}

int orc_qmm4_f32(const float* x, size_t rows, const uint32_t* packed, const float* scales,
                 const float* biases, size_t outputs, size_t width, float* y, int threads) {
  if (!x || !packed || !scales || !biases || !y || rows == 0 || outputs == 0 || width == 0 || width % 64)
    return -1;
  if (threads <= 0) threads = orc_max_threads();
  (void)threads;
  const size_t words = width / 8, groups = width / 64;
  long o;
#pragma omp parallel num_threads(threads)
  {
    float* acc = (float*)malloc(sizeof(float) * rows);
#pragma omp for schedule(static)
    for (o = 0; o < (long)outputs; ++o) {
      qmm4_row_f32(x, width, packed + (size_t)o * words, scales + (size_t)o * groups, biases + (size_t)o * groups,
                   NULL, rows, acc);
      for (size_t r = 0; r < rows; ++r) y[r * outputs + (size_t)o] = acc[r];
    }
    free(acc);
  }
  return 0;
}

int orc_gather_qmm4_f32(const float* x, int rows, const uint32_t* packed, const float* scales,
                        const float* biases, int experts, int outputs, int width, const int32_t* idx,
                        int top, float* y, int threads) {
  if (!x || !packed || !scales || !biases || !idx || !y || rows <= 0 || experts <= 0 || outputs <= 0 ||
      width <= 0 || width % 64 || top <= 0)
    return -1;
  const int pairs = rows * top;
  for (int i = 0; i < pairs; ++i)
    if (idx[i] < 0 || idx[i] >= experts) return -1;
  if (threads <= 0) threads = orc_max_threads();
  (void)threads;
  /* the pairs of every expert, in pair order (a counting sort) */
  int32_t* start = (int32_t*)calloc((size_t)experts + 1, sizeof(int32_t));
  int32_t* pair = (int32_t*)malloc(sizeof(int32_t) * (size_t)pairs);
  int32_t* tok = (int32_t*)malloc(sizeof(int32_t) * (size_t)pairs);
  if (!start || !pair || !tok) {
    free(start);
    free(pair);
    free(tok);
    return -1;
  }
  for (int i = 0; i < pairs; ++i) start[idx[i] + 1]++;
  for (int e = 0; e < experts; ++e) start[e + 1] += start[e];
  {
    int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * (size_t)experts);
    if (!fill) {
      free(start);
      free(pair);
      free(tok);
      return -1;
    }
    memcpy(fill, start, sizeof(int32_t) * (size_t)experts);
    for (int i = 0; i < pairs; ++i) {
      const int at = fill[idx[i]]++;
      pair[at] = i;
      tok[at] = i / top;
    }
    free(fill);
  }
  const size_t words = (size_t)width / 8, groups = (size_t)width / 64;
  const long units = (long)experts * outputs;
  long u;
#pragma omp parallel num_threads(threads)
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)pairs);
#pragma omp for schedule(dynamic, 64)
    for (u = 0; u < units; ++u) {
      const int e = (int)(u / outputs), o = (int)(u % outputs);
      const int n = start[e + 1] - start[e];
      if (n == 0) continue;
      const size_t r = (size_t)e * outputs + (size_t)o;
      qmm4_row_f32(x, (size_t)width, packed + r * words, scales + r * groups, biases + r * groups,
                   tok + start[e], (size_t)n, acc);
      for (int t = 0; t < n; ++t) y[(size_t)pair[start[e] + t] * outputs + (size_t)o] = acc[t];
    }
    free(acc);
  }
  free(start);
  free(pair);
  free(tok);
  return 0;
}

int orc_dequant(const uint32_t* packed, const float* scales, const float* biases, size_t rows,
                size_t width, int group, int bits, double* out) {
  if (!packed || !scales || !biases || !out || rows == 0 || width == 0 ||
      !valid_quant(group, bits) || width % (size_t)group || (width * bits) % 32)
    return -1;
  const size_t words = width * bits / 32, groups = width / group;
  if (!all_finite(scales, rows * groups) || !all_finite(biases, rows * groups)) return -1;
  for (size_t r = 0; r < rows; ++r)
    for (size_t c = 0; c < width; ++c) {
      size_t g = r * groups + c / group;
      out[r * width + c] =
          (double)scales[g] * orc_code(packed + r * words, c, bits) + (double)biases[g];
    }
  return 0;
}

/* native/operator_reference.h:9 — branch on sign so exp never overflows. */
double orc_sigmoid(double x) {
  if (x >= 0) return 1. / (1. + exp(-x));
  double e = exp(x);
  return e / (1. + e);
}

int orc_silu(const float* x, size_t n, double* y) {
  if (!x || !y || !all_finite(x, n)) return -1;
  for (size_t i = 0; i < n; ++i) y[i] = (double)x[i] * orc_sigmoid(x[i]);
  return 0;
}

int orc_rms(const float* x, const float* weight, size_t rows, size_t width, double eps,
            double* y) {
  if (!x || !y || rows == 0 || width == 0 || !isfinite(eps) || eps <= 0) return -1;
  if (!all_finite(x, rows * width) || (weight && !all_finite(weight, width))) return -1;
  for (size_t r = 0; r < rows; ++r) {
    double square = 0;
    for (size_t c = 0; c < width; ++c) {
      double v = x[r * width + c];
      square += v * v;
    }
    double inverse = 1. / sqrt(square / (double)width + eps);
    for (size_t c = 0; c < width; ++c)
      y[r * width + c] = (double)x[r * width + c] * inverse * (weight ? (double)weight[c] : 1.);
  }
  return 0;
}

int orc_rope(const float* x, int tokens, int heads, int dim, int rotary, const int32_t* positions,
             double theta, double* y) {
  if (!x || !y || !positions || tokens <= 0 || heads <= 0 || dim <= 0 || rotary <= 0 ||
      rotary > dim || rotary % 2 || !isfinite(theta) || theta <= 1)
    return -1;
  size_t n = (size_t)tokens * heads * dim;
  if (!all_finite(x, n)) return -1;
  for (size_t i = 0; i < n; ++i) y[i] = x[i];
  const int half = rotary / 2;
  for (int t = 0; t < tokens; ++t) {
    if (positions[t] < 0) return -1;
    for (int h = 0; h < heads; ++h)
      for (int j = 0; j < half; ++j) {
        size_t first = ((size_t)t * heads + h) * dim + j, second = first + half;
        double angle = (double)positions[t] * pow(theta, -2. * j / rotary);
        double c = cos(angle), s = sin(angle);
        y[first] = (double)x[first] * c - (double)x[second] * s;
        y[second] = (double)x[first] * s + (double)x[second] * c;
      }
  }
  return 0;
}

int orc_paged_attention(const float* q, const float* kcache, const float* vcache,
                        const int32_t* block_table, int max_pages, const int32_t* cu_seqlens,
                        const int32_t* context, int rows, int hq, int hkv, int dim, int page,
                        double scale, const float* gate, double* out) {
  if (!q || !kcache || !vcache || !block_table || !cu_seqlens || !context || !out || rows <= 0 ||
      hq <= 0 || hkv <= 0 || hq % hkv || dim <= 0 || page <= 0 || max_pages <= 0 ||
      !isfinite(scale) || scale <= 0 || cu_seqlens[0] != 0)
    return -1;
  const int group = hq / hkv;
  int longest = 1;
  for (int r = 0; r < rows; ++r) {
    int n = cu_seqlens[r + 1] - cu_seqlens[r];
    if (n < 0 || context[r] < n || context[r] > max_pages * page) return -1;
    if (context[r] > longest) longest = context[r];
  }
  /* one (packed token, q head) item at a time; items are independent */
  const long items = (long)cu_seqlens[rows] * hq;
  int failed = 0;
#pragma omp parallel reduction(| : failed)
  {
    double* scores = (double*)malloc(sizeof(double) * (size_t)longest);
    if (!scores) failed = 1;
#pragma omp for schedule(dynamic, 4)
    for (long it = 0; it < items; ++it) {
      if (!scores) continue;
      const int i = (int)(it / hq), h = (int)(it % hq);
      int r = 0;
      while (cu_seqlens[r + 1] <= i) ++r; /* the row holding packed token i */
      const int t = i - cu_seqlens[r], n = cu_seqlens[r + 1] - cu_seqlens[r];
      const int offset = context[r] - n; /* length before the new tokens */
      const int kh = h / group;
      const float* qv = q + ((size_t)i * hq + h) * dim;
      const int visible = offset + t + 1; /* native/attention_reference.h:15 */
      double peak = -INFINITY;
      for (int j = 0; j < visible; ++j) {
        int pg = block_table[(size_t)r * max_pages + j / page];
        const float* kv = kcache + (((size_t)pg * hkv + kh) * page + j % page) * dim;
        double dot = 0;
        for (int z = 0; z < dim; ++z) dot += (double)qv[z] * kv[z];
        scores[j] = dot * scale;
        if (scores[j] > peak) peak = scores[j];
      }
      double total = 0;
      for (int j = 0; j < visible; ++j) {
        scores[j] = exp(scores[j] - peak);
        total += scores[j];
      }
      double* o = out + ((size_t)i * hq + h) * dim;
      for (int z = 0; z < dim; ++z) o[z] = 0;
      for (int j = 0; j < visible; ++j) {
        int pg = block_table[(size_t)r * max_pages + j / page];
        const float* vv = vcache + (((size_t)pg * hkv + kh) * page + j % page) * dim;
        double p = scores[j] / total;
        for (int z = 0; z < dim; ++z) o[z] += p * vv[z];
      }
      if (gate) {
        const float* gv = gate + ((size_t)i * hq + h) * dim;
        for (int z = 0; z < dim; ++z) o[z] *= orc_sigmoid(gv[z]);
      }
    }
    free(scores);
  }
  return failed ? -1 : 0;
}

int orc_gated_delta(const float* q, const float* k, const float* v, const float* decay,
                    const float* beta, const float* state, int b, int t, int hk, int hv, int dk,
                    int dv, double* out, double* state_out) {
  if (!q || !k || !v || !decay || !beta || !state || !out || !state_out || b <= 0 || t <= 0 ||
      hk <= 0 || hv <= 0 || hv % hk || dk <= 0 || dv <= 0)
    return -1;
  const int repeats = hv / hk;
  const size_t per = (size_t)hv * dv * dk;
  for (size_t i = 0; i < (size_t)b * per; ++i) state_out[i] = state[i];
  for (int bi = 0; bi < b; ++bi)
    for (int ti = 0; ti < t; ++ti)
      for (int h = 0; h < hv; ++h) {
        const int kh = h / repeats; /* mx::repeat along the head axis */
        const float* qv = q + (((size_t)bi * t + ti) * hk + kh) * dk;
        const float* kv = k + (((size_t)bi * t + ti) * hk + kh) * dk;
        const float* vv = v + (((size_t)bi * t + ti) * hv + h) * dv;
        const double g = decay[((size_t)bi * t + ti) * hv + h];
        const double be = beta[((size_t)bi * t + ti) * hv + h];
        double* s = state_out + (size_t)bi * per + (size_t)h * dv * dk;
        for (int i = 0; i < dv; ++i) {
          double* srow = s + (size_t)i * dk;
          double memory = 0;
          for (int j = 0; j < dk; ++j) {
            srow[j] *= g;
            memory += srow[j] * kv[j];
          }
          double change = ((double)vv[i] - memory) * be, read = 0;
          for (int j = 0; j < dk; ++j) {
            srow[j] += change * kv[j];
            read += srow[j] * qv[j];
          }
          out[(((size_t)bi * t + ti) * hv + h) * dv + i] = read;
        }
      }
  return 0;
}

int orc_gdn(const float* qkv, const float* history, const float* conv_w, const float* a,
            const float* b, const float* alog, const float* dt, const float* state, int t, int hk,
            int hv, int dk, int dv, int kernel, double* activated, double* history_out,
            double* out, double* state_out) {
  if (!qkv || !history || !conv_w || !a || !b || !alog || !dt || !state || !out || !state_out ||
      t <= 0 || hk <= 0 || hv <= 0 || hv % hk || dk <= 0 || dv <= 0 || kernel < 2)
    return -1;
  const size_t kd = (size_t)hk * dk, vd = (size_t)hv * dv, channels = 2 * kd + vd;
  const size_t hist = (size_t)(kernel - 1);
  double* stream = (double*)malloc(sizeof(double) * (hist + (size_t)t) * channels);
  double* act = (double*)malloc(sizeof(double) * (size_t)t * channels);
  double* q = (double*)malloc(sizeof(double) * dk);
  double* k = (double*)malloc(sizeof(double) * dk);
  if (!stream || !act || !q || !k) {
    free(stream); free(act); free(q); free(k);
    return -1;
  }
  for (size_t i = 0; i < hist * channels; ++i) stream[i] = history[i];
  for (size_t i = 0; i < (size_t)t * channels; ++i) stream[hist * channels + i] = qkv[i];
  if (history_out)
    for (size_t i = 0; i < hist * channels; ++i) history_out[i] = stream[(size_t)t * channels + i];
  const size_t per = (size_t)hv * dv * dk;
  for (size_t i = 0; i < per; ++i) state_out[i] = state[i];
  for (int ti = 0; ti < t; ++ti) {
    for (size_t ch = 0; ch < channels; ++ch) {
      double value = 0;
      for (int tap = 0; tap < kernel; ++tap)
        value += stream[((size_t)ti + tap) * channels + ch] * conv_w[ch * kernel + tap];
      act[(size_t)ti * channels + ch] = value * orc_sigmoid(value);
    }
    for (int h = 0; h < hv; ++h) {
      const int kh = h / (hv / hk);
      double qs = 0, ks = 0;
      for (int j = 0; j < dk; ++j) {
        q[j] = act[(size_t)ti * channels + (size_t)kh * dk + j];
        k[j] = act[(size_t)ti * channels + kd + (size_t)kh * dk + j];
        qs += q[j] * q[j];
        ks += k[j] * k[j];
      }
      /* native/operator_reference.h:32: q/(rms*dk), k/(rms*sqrt(dk)), eps 1e-6. */
      double qi = 1. / (sqrt(qs / dk + 1e-6) * dk), ki = 1. / (sqrt(ks / dk + 1e-6) * sqrt((double)dk));
      for (int j = 0; j < dk; ++j) {
        q[j] *= qi;
        k[j] *= ki;
      }
      double logit = (double)a[(size_t)ti * hv + h] + dt[h];
      double softplus = (logit > 0 ? logit : 0.) + log1p(exp(-fabs(logit)));
      double decay = exp(-exp((double)alog[h]) * softplus);
      double beta = orc_sigmoid(b[(size_t)ti * hv + h]);
      for (int i = 0; i < dv; ++i) {
        double* srow = state_out + ((size_t)h * dv + i) * dk;
        double memory = 0;
        for (int j = 0; j < dk; ++j) {
          srow[j] *= decay;
          memory += srow[j] * k[j];
        }
        double change = (act[(size_t)ti * channels + 2 * kd + (size_t)h * dv + i] - memory) * beta;
        double read = 0;
        for (int j = 0; j < dk; ++j) {
          srow[j] += change * k[j];
          read += srow[j] * q[j];
        }
        out[(size_t)ti * vd + (size_t)h * dv + i] = read;
      }
    }
  }
  if (activated)
    for (size_t i = 0; i < (size_t)t * channels; ++i) activated[i] = act[i];
  free(stream); free(act); free(q); free(k);
  return 0;
}

/* f32 total order key (Rust f32::total_cmp; native/selection.h:8-11). */
static uint32_t total_key(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return (u & 0x80000000u) ? ~u : (u ^ 0x80000000u);
}

int orc_route_topk(const float* logits, int rows, int experts, int top, int32_t* idx,
                   double* weights) {
  if (!logits || !idx || !weights || rows <= 0 || experts <= 0 || top <= 0 || top > experts)
    return -1;
  if (!all_finite(logits, (size_t)rows * experts)) return -1;
  unsigned char* taken = (unsigned char*)malloc((size_t)experts);
  if (!taken) return -1;
  for (int r = 0; r < rows; ++r) {
    const float* l = logits + (size_t)r * experts;
    memset(taken, 0, (size_t)experts);
    double peak = -INFINITY;
    for (int e = 0; e < experts; ++e)
      if (l[e] > peak) peak = l[e];
    double total = 0;
    for (int j = 0; j < top; ++j) {
      int best = -1;
      for (int e = 0; e < experts; ++e) {
        if (taken[e]) continue;
        if (best < 0 || total_key(l[e]) > total_key(l[best])) best = e;
      }
      taken[best] = 1;
      idx[(size_t)r * top + j] = best;
      total += exp((double)l[best] - peak);
    }
    for (int j = 0; j < top; ++j)
      weights[(size_t)r * top + j] = exp((double)l[idx[(size_t)r * top + j]] - peak) / total;
  }
  free(taken);
  return 0;
}

int orc_expert_permute(const int32_t* idx, int tokens, int top, int experts, int32_t* order,
                       int32_t* inverse, int32_t* offsets) {
  if (!idx || !order || !inverse || !offsets || tokens < 0 || top <= 0 || experts <= 0) return -1;
  const int pairs = tokens * top;
  for (int e = 0; e <= experts; ++e) offsets[e] = 0;
  for (int p = 0; p < pairs; ++p) {
    if (idx[p] < 0 || idx[p] >= experts) return -1;
    offsets[idx[p] + 1]++;
  }
  for (int e = 0; e < experts; ++e) offsets[e + 1] += offsets[e];
  int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)(experts > 0 ? experts : 1));
  if (!cursor) return -1;
  for (int e = 0; e < experts; ++e) cursor[e] = offsets[e];
  for (int p = 0; p < pairs; ++p) {
    int dst = cursor[idx[p]]++;
    order[dst] = p;
    inverse[p] = dst;
  }
  free(cursor);
  return 0;
}

int orc_gather_qmm(const float* x, int rows, const uint32_t* packed, const float* scales,
                   const float* biases, int experts, int outputs, int width, int group, int bits,
                   const int32_t* idx, int top, double* y, int threads) {
  if (!x || !packed || !scales || !biases || !idx || !y || rows <= 0 || experts <= 0 ||
      outputs <= 0 || width <= 0 || top <= 0 || !valid_quant(group, bits) || width % group)
    return -1;
  const size_t words = (size_t)width * bits / 32, groups = (size_t)width / group;
  for (int i = 0; i < rows * top; ++i)
    if (idx[i] < 0 || idx[i] >= experts) return -1;
  for (int r = 0; r < rows; ++r)
    for (int j = 0; j < top; ++j) {
      const int e = idx[r * top + j];
      int rc = orc_qmm(x + (size_t)r * width, 1, packed + (size_t)e * outputs * words,
                       scales + (size_t)e * outputs * groups, biases + (size_t)e * outputs * groups,
                       (size_t)outputs, (size_t)width, group, bits,
                       y + ((size_t)r * top + j) * outputs, threads);
      if (rc) return rc;
    }
  return 0;
}

int orc_mix(const float* experts, const float* scores, int rows, int top, int width, double* y) {
  if (!experts || !scores || !y || rows <= 0 || top <= 0 || width <= 0) return -1;
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < width; ++c) {
      double sum = 0;
      for (int j = 0; j < top; ++j)
        sum += (double)experts[((size_t)r * top + j) * width + c] * scores[(size_t)r * top + j];
      y[(size_t)r * width + c] = sum;
    }
  return 0;
}

/* src/serving/native_speculative.rs:49-73: strict total_cmp replacement keeps the
 * lowest index among equal keys; margin is an f32 subtraction. */
int orc_winner(const float* logits, size_t n, uint32_t* token, float* margin) {
  if (!logits || n == 0 || n > 300000 || !isfinite(logits[0])) return -1;
  size_t best = 0;
  float best_val = logits[0], second_val = -INFINITY;
  for (size_t i = 1; i < n; ++i) {
    float v = logits[i];
    if (!isfinite(v)) return -1;
    if (total_key(v) > total_key(best_val)) {
      second_val = best_val;
      best = i;
      best_val = v;
    } else if (total_key(v) > total_key(second_val)) {
      second_val = v;
    }
  }
  if (token) *token = (uint32_t)best;
  if (margin) *margin = isfinite(second_val) ? best_val - second_val : INFINITY;
  return 0;
}

static int contains(const uint32_t* v, size_t n, uint32_t t) {
  for (size_t i = 0; i < n; ++i)
    if (v[i] == t) return 1;
  return 0;
}

int orc_plan(const float* initial, size_t vocab, const uint32_t* draft, size_t n_draft,
             const float* rows, const uint32_t* eos, size_t n_eos, size_t remaining,
             uint32_t* emitted, size_t* n_emitted, size_t* accepted, int* terminal) {
  if (!initial || !emitted || !n_emitted || !accepted || !terminal) return -1;
  uint32_t initial_winner;
  if (orc_winner(initial, vocab, &initial_winner, NULL)) return -1;
  if (n_draft > 8 || n_draft > remaining || remaining == 0) return -1;
  if (n_draft && (!draft || !rows)) return -1;
  if (n_eos && !eos) return -1;
  for (size_t i = 0; i < n_draft; ++i)
    if (draft[i] >= vocab) return -1;
  for (size_t i = 0; i < n_eos; ++i)
    if (eos[i] >= vocab) return -1;
  uint32_t row_winners[8];
  for (size_t i = 0; i < n_draft; ++i)
    if (orc_winner(rows + i * vocab, vocab, &row_winners[i], NULL)) return -1;
  size_t n = 0, acc = 0;
  int term = 0;
  for (size_t i = 0; i < n_draft; ++i) {
    uint32_t target = i == 0 ? initial_winner : row_winners[i - 1];
    emitted[n++] = target;
    term = contains(eos, n_eos, target);
    if (draft[i] != target || term) {
      acc += draft[i] == target;
      *n_emitted = n;
      *accepted = acc;
      *terminal = term;
      return 0;
    }
    acc += 1;
  }
  if (n < remaining) {
    uint32_t bonus = n_draft ? row_winners[n_draft - 1] : initial_winner;
    emitted[n++] = bonus;
    term = contains(eos, n_eos, bonus);
  }
  *n_emitted = n;
  *accepted = acc;
  *terminal = term;
  return 0;
}

int orc_pack_tables(const int32_t* row_tokens, const int32_t* positions,
                    const int32_t* block_table, int max_pages, int rows, int page,
                    int32_t* cu_seqlens, int32_t* token_row, int32_t* token_pos,
                    int32_t* kv_slot, int32_t* context) {
  if (!row_tokens || !positions || !block_table || !cu_seqlens || rows < 0 || page <= 0 ||
      max_pages <= 0)
    return -1;
  cu_seqlens[0] = 0;
  for (int r = 0; r < rows; ++r) {
    if (row_tokens[r] < 0 || positions[r] < 0 ||
        (int64_t)positions[r] + row_tokens[r] > (int64_t)max_pages * page)
      return -1;
    cu_seqlens[r + 1] = cu_seqlens[r] + row_tokens[r];
    if (context) context[r] = positions[r] + row_tokens[r];
    for (int j = 0; j < row_tokens[r]; ++j) {
      int i = cu_seqlens[r] + j, pos = positions[r] + j;
      if (token_row) token_row[i] = r;
      if (token_pos) token_pos[i] = pos;
      if (kv_slot) kv_slot[i] = block_table[(size_t)r * max_pages + pos / page] * page + pos % page;
    }
  }
  return 0;
}
