/*
 * CPU ORACLE -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the numerics of MetalFish's reference CPU backend,
 * NN::Cpu::CpuNetwork::RunBatch (reference src/nn/cpu/cpu_network.cpp:580-1491
 * and helpers 302-460).  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker: the product path
 * (metalfish_amd) never calls into this file.
 *
 * The step list (which buffer feeds which step, residual parents, epsilon,
 * residual scale, activations) is resolved by oracle/plan.py, which restates
 * the reference's execution-plan rules; this file executes the steps with the
 * reference's loop order.  Build with -O3 -ffp-contract=off and without
 * -ffast-math so fp32 rounding follows the reference's default build
 * (reference CMakeLists.txt:17-21).
 *
 * Parity pinning of each routine is listed in oracle/plan.py's header.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum {
  OR_DENSE = 1,
  OR_LAYERNORM = 2,
  OR_GATE = 3,
  OR_FFN = 4,
  OR_ATTENTION = 5,
  OR_POLICY_MAP = 6,
  OR_DYNAMIC_PE = 7,
  OR_STATIC_PE = 8,
};

enum {
  OR_ACT_LINEAR = -1,
  OR_ACT_RELU = 0,
  OR_ACT_RELU2 = 1,
  OR_ACT_TANH = 2,
  OR_ACT_SIGMOID = 3,
  OR_ACT_SWISH = 4,
  OR_ACT_MISH = 5,
  OR_ACT_SELU = 6,
  OR_ACT_SOFTMAX = 7,
};

#define OR_MAX_TENSORS 24

typedef struct {
  int kind;
  int src;    /* input buffer id (0 = packed plane values, width 112) */
  int dst;    /* output buffer id */
  int parent; /* LAYERNORM residual parent buffer id, -1 for none */
  int act;    /* activation of DENSE / FFN hidden / smolgen */
  float alpha;
  float eps;
  int heads;  /* ATTENTION head count */
  int aux0;   /* POLICY_MAP: query buffer; GATE: number of gate tensors */
  int aux1;   /* POLICY_MAP: key buffer */
  int n_tensors;
  const float *t[OR_MAX_TENSORS];
  int d0[OR_MAX_TENSORS]; /* rows ([out] for matrices) */
  int d1[OR_MAX_TENSORS]; /* cols ([in] for matrices), 0 for vectors */
  int tag[OR_MAX_TENSORS]; /* GATE: 1 = multiply, 2 = add */
} or_step;

typedef struct {
  float *v;
  int rows;
  int width;
} or_buf;

static float act_value(float value, int kind) {
  switch (kind) {
  case OR_ACT_RELU:
    return value > 0.0f ? value : 0.0f; /* std::max(value, 0.0f) */
  case OR_ACT_RELU2: {
    const float relu = value > 0.0f ? value : 0.0f;
    return relu * relu;
  }
  case OR_ACT_TANH:
    return tanhf(value);
  case OR_ACT_SIGMOID:
    return 1.0f / (1.0f + expf(-value));
  case OR_ACT_SWISH:
    return value / (1.0f + expf(-value));
  case OR_ACT_MISH:
    return value * tanhf(log1pf(expf(value)));
  case OR_ACT_SELU:
    return 1.05070098f *
           (value > 0.0f ? value : 1.67326324f * (expf(value) - 1.0f));
  default:
    return value;
  }
}

/* ApplySoftmaxRows / softmax mode of ApplyDenseActivation
 * (cpu_network.cpp:336-351, 405-422). */
static void softmax_rows(float *values, int rows, int width) {
  for (int row = 0; row < rows; ++row) {
    float *base = values + (size_t)row * width;
    float max_value = -INFINITY;
    for (int col = 0; col < width; ++col)
      max_value = base[col] > max_value ? base[col] : max_value;
    float sum = 0.0f;
    for (int col = 0; col < width; ++col) {
      base[col] = expf(base[col] - max_value);
      sum += base[col];
    }
    if (sum == 0.0f)
      continue;
    const float inv_sum = 1.0f / sum;
    for (int col = 0; col < width; ++col)
      base[col] *= inv_sum;
  }
}

/* ApplyDenseActivation (cpu_network.cpp:325-352). */
static void apply_activation(float *values, int rows, int width, int act) {
  if (act == OR_ACT_LINEAR)
    return;
  if (act == OR_ACT_SOFTMAX) {
    softmax_rows(values, rows, width);
    return;
  }
  const size_t n = (size_t)rows * width;
  for (size_t i = 0; i < n; ++i)
    values[i] = act_value(values[i], act);
}

/* DenseAffine (cpu_network.cpp:382-403): bias is the initial sum. */
static void dense_affine(const float *input, int rows, int in_w,
                         const float *w, const float *bias, int out_w,
                         float *output) {
  for (int row = 0; row < rows; ++row) {
    const float *in_row = input + (size_t)row * in_w;
    float *out_row = output + (size_t)row * out_w;
    for (int out = 0; out < out_w; ++out) {
      const float *w_row = w + (size_t)out * in_w;
      float sum = bias ? bias[out] : 0.0f;
      for (int in = 0; in < in_w; ++in)
        sum += in_row[in] * w_row[in];
      out_row[out] = sum;
    }
  }
}

/* ApplyLayerNorm (cpu_network.cpp:424-460): E[x^2] - mean^2 variance. */
static void layer_norm(const float *input, const float *parent, float rscale,
                       const float *scale, const float *bias, float *output,
                       int rows, int width, float eps) {
  for (int row = 0; row < rows; ++row) {
    const float *in_row = input + (size_t)row * width;
    const float *p_row = parent ? parent + (size_t)row * width : NULL;
    float *out_row = output + (size_t)row * width;
    float sum = 0.0f, sq = 0.0f;
    for (int col = 0; col < width; ++col) {
      const float value = p_row ? p_row[col] + in_row[col] * rscale : in_row[col];
      sum += value;
      sq += value * value;
    }
    const float mean = sum / (float)width;
    float variance = sq / (float)width - mean * mean;
    if (variance < 0.0f)
      variance = 0.0f;
    const float inv_std = 1.0f / sqrtf(variance + eps);
    for (int col = 0; col < width; ++col) {
      const float value = p_row ? p_row[col] + in_row[col] * rscale : in_row[col];
      out_row[col] = (value - mean) * inv_std * scale[col] + bias[col];
    }
  }
}

static int set_buf(or_buf *b, int rows, int width) {
  free(b->v);
  b->v = (float *)calloc((size_t)rows * width > 0 ? (size_t)rows * width : 1,
                         sizeof(float));
  b->rows = rows;
  b->width = width;
  return b->v ? 0 : -1;
}

/* body.input_embedding_preprocess (cpu_network.cpp:691-800). */
static int run_dynamic_pe(const or_step *s, int batch, const uint64_t *masks,
                          const float *values, or_buf *out) {
  const int kPositionPlanes = 12, squares = 64, input_planes = 112;
  const float *w = s->t[0], *b = s->t[1];
  const int out_w = s->d0[0], in_w = s->d1[0];
  if (in_w != squares * kPositionPlanes || out_w % squares)
    return -10;
  float *pos_in = (float *)calloc((size_t)batch * in_w, sizeof(float));
  float *pos_out = (float *)calloc((size_t)batch * out_w, sizeof(float));
  if (!pos_in || !pos_out)
    return -1;
  for (int bi = 0; bi < batch; ++bi)
    for (int sq = 0; sq < squares; ++sq) {
      const uint64_t bit = 1ULL << sq;
      for (int p = 0; p < kPositionPlanes; ++p) {
        const size_t pi = (size_t)bi * input_planes + p;
        pos_in[(size_t)bi * in_w + (size_t)sq * kPositionPlanes + p] =
            (masks[pi] & bit) ? values[pi] : 0.0f;
      }
    }
  for (int bi = 0; bi < batch; ++bi) {
    const float *in_row = pos_in + (size_t)bi * in_w;
    float *out_row = pos_out + (size_t)bi * out_w;
    for (int o = 0; o < out_w; ++o) {
      const float *w_row = w + (size_t)o * in_w;
      float sum = b[o];
      for (int i = 0; i < in_w; ++i)
        sum += in_row[i] * w_row[i];
      out_row[o] = sum;
    }
  }
  const int pe_w = out_w / squares;
  if (set_buf(out, batch * squares, input_planes + pe_w))
    return -1;
  for (int bi = 0; bi < batch; ++bi)
    for (int sq = 0; sq < squares; ++sq) {
      const uint64_t bit = 1ULL << sq;
      float *row = out->v + ((size_t)bi * squares + sq) * out->width;
      for (int p = 0; p < input_planes; ++p) {
        const size_t pi = (size_t)bi * input_planes + p;
        row[p] = (masks[pi] & bit) ? values[pi] : 0.0f;
      }
      const float *pe = pos_out + (size_t)bi * out_w + (size_t)sq * pe_w;
      for (int c = 0; c < pe_w; ++c)
        row[input_planes + c] = pe[c];
    }
  free(pos_in);
  free(pos_out);
  return 0;
}

/* Static position encoding of PE_MAP nets: per square, the 112 planes then
 * the table row of that square (t[0] = [64][pe_w], d1[0] = pe_w).  The
 * reference CPU backend has no PE_MAP path; this restates the CUDA backend's
 * StaticPositionEncodingConcatKernel (cuda/cuda_kernels.cu:1016-1040),
 * which feeds body.input_embedding (cuda_stage_executor.cpp:487-492). */
static int run_static_pe(const or_step *s, int batch, const uint64_t *masks,
                         const float *values, or_buf *out) {
  const int squares = 64, input_planes = 112;
  const float *table = s->t[0];
  const int pe_w = s->d1[0];
  if (s->d0[0] != squares || pe_w <= 0)
    return -11;
  if (set_buf(out, batch * squares, input_planes + pe_w))
    return -1;
  for (int bi = 0; bi < batch; ++bi)
    for (int sq = 0; sq < squares; ++sq) {
      const uint64_t bit = 1ULL << sq;
      float *row = out->v + ((size_t)bi * squares + sq) * out->width;
      for (int p = 0; p < input_planes; ++p) {
        const size_t pi = (size_t)bi * input_planes + p;
        row[p] = (masks[pi] & bit) ? values[pi] : 0.0f;
      }
      for (int c = 0; c < pe_w; ++c)
        row[input_planes + c] = table[(size_t)sq * pe_w + c];
    }
  return 0;
}

/* Dense stage (cpu_network.cpp:822-890), with the flatten of square rows
 * into one row per position when the weight expects it (841-851). */
static int run_dense(const or_step *s, int batch, const or_buf *src,
                     or_buf *out) {
  const float *w = s->t[0], *b = s->t[1];
  const int out_w = s->d0[0], in_w = s->d1[0];
  int rows = src->rows;
  if (in_w != src->width) {
    if (batch <= 0 || rows % batch || in_w != (rows / batch) * src->width)
      return -11;
    rows = batch;
  }
  if (set_buf(out, rows, out_w))
    return -1;
  for (int row = 0; row < rows; ++row) {
    const float *in_row = src->v + (size_t)row * in_w;
    float *out_row = out->v + (size_t)row * out_w;
    for (int o = 0; o < out_w; ++o) {
      const float *w_row = w + (size_t)o * in_w;
      float sum = b[o];
      for (int i = 0; i < in_w; ++i)
        sum += in_row[i] * w_row[i];
      out_row[o] = sum;
    }
  }
  apply_activation(out->v, rows, out_w, s->act);
  return 0;
}

/* Gate stage (cpu_network.cpp:1268-1316): tensors applied in plan order. */
static int run_gate(const or_step *s, const or_buf *src, or_buf *out) {
  const int rows = src->rows, width = src->width;
  if (set_buf(out, rows, width))
    return -1;
  memcpy(out->v, src->v, sizeof(float) * (size_t)rows * width);
  float *next = (float *)malloc(sizeof(float) * (size_t)rows * width + 1);
  if (!next)
    return -1;
  for (int t = 0; t < s->n_tensors; ++t) {
    const size_t n = (size_t)s->d0[t] * (s->d1[t] ? (size_t)s->d1[t] : 1);
    int gate_rows = 0;
    if (n == (size_t)width)
      gate_rows = 1;
    else if (n % (size_t)width == 0)
      gate_rows = (int)(n / (size_t)width);
    if (gate_rows <= 0 || rows % gate_rows) {
      free(next);
      return -12;
    }
    const float *g = s->t[t];
    for (int row = 0; row < rows; ++row) {
      const int gr = gate_rows == 1 ? 0 : row % gate_rows;
      for (int col = 0; col < width; ++col) {
        const float gate = gate_rows == 1 ? g[col] : g[(size_t)col * gate_rows + gr];
        const size_t idx = (size_t)row * width + col;
        next[idx] = s->tag[t] == 1 ? out->v[idx] * gate : out->v[idx] + gate;
      }
    }
    memcpy(out->v, next, sizeof(float) * (size_t)rows * width);
  }
  free(next);
  return 0;
}

/* Feed-forward stage (cpu_network.cpp:1318-1397). */
static int run_ffn(const or_step *s, const or_buf *src, or_buf *out) {
  const float *w1 = s->t[0], *b1 = s->t[1], *w2 = s->t[2], *b2 = s->t[3];
  const int hidden_w = s->d0[0], in_w = s->d1[0], out_w = s->d0[2];
  const int rows = src->rows;
  if (in_w != src->width || s->d1[2] != hidden_w)
    return -13;
  float *hidden = (float *)calloc((size_t)rows * hidden_w + 1, sizeof(float));
  if (!hidden || set_buf(out, rows, out_w))
    return -1;
  for (int row = 0; row < rows; ++row) {
    const float *in_row = src->v + (size_t)row * in_w;
    float *h_row = hidden + (size_t)row * hidden_w;
    for (int o = 0; o < hidden_w; ++o) {
      const float *w_row = w1 + (size_t)o * in_w;
      float sum = b1[o];
      for (int i = 0; i < in_w; ++i)
        sum += in_row[i] * w_row[i];
      h_row[o] = sum;
    }
  }
  apply_activation(hidden, rows, hidden_w, s->act);
  for (int row = 0; row < rows; ++row) {
    const float *h_row = hidden + (size_t)row * hidden_w;
    float *out_row = out->v + (size_t)row * out_w;
    for (int o = 0; o < out_w; ++o) {
      const float *w_row = w2 + (size_t)o * hidden_w;
      float sum = b2[o];
      for (int i = 0; i < hidden_w; ++i)
        sum += h_row[i] * w_row[i];
      out_row[o] = sum;
    }
  }
  free(hidden);
  return 0;
}

/* Multi-head attention with optional smolgen bias
 * (cpu_network.cpp:1027-1266).  Tensor order: q_w q_b k_w k_b v_w v_b
 * dense_w dense_b [compress dense1_w dense1_b dense2_w dense2_b ln1_g ln1_b
 * ln2_g ln2_b global]. */
static int run_attention(const or_step *s, int batch, const or_buf *src,
                         or_buf *out) {
  const int squares = 64;
  const int heads = s->heads;
  const int in_w = s->d1[0], qkv_w = s->d0[0], out_w = s->d0[6];
  const int rows = src->rows;
  if (src->width != in_w || rows != batch * squares || heads <= 0 ||
      qkv_w % heads)
    return -14;
  const int depth = qkv_w / heads;
  float *q = (float *)malloc(sizeof(float) * (size_t)rows * qkv_w);
  float *k = (float *)malloc(sizeof(float) * (size_t)rows * qkv_w);
  float *v = (float *)malloc(sizeof(float) * (size_t)rows * qkv_w);
  if (!q || !k || !v)
    return -1;
  dense_affine(src->v, rows, in_w, s->t[0], s->t[1], qkv_w, q);
  dense_affine(src->v, rows, in_w, s->t[2], s->t[3], qkv_w, k);
  dense_affine(src->v, rows, in_w, s->t[4], s->t[5], qkv_w, v);

  float *bias = NULL;
  if (s->n_tensors >= 18) {
    const int c = s->d0[8];           /* compressed channels */
    const int d1w = s->d0[9];         /* dense1 width */
    const int d2w = s->d0[11];        /* dense2 width */
    const int per_head = d2w / heads; /* global projection input */
    const int flat = squares * c;
    if (s->d1[8] != in_w || s->d1[9] != flat || s->d1[11] != d1w ||
        d2w % heads || s->d0[17] != squares * squares || s->d1[17] != per_head)
      return -15;
    float *compressed = (float *)malloc(sizeof(float) * (size_t)rows * c);
    float *dense1 = (float *)malloc(sizeof(float) * (size_t)batch * d1w);
    float *norm1 = (float *)calloc((size_t)batch * d1w, sizeof(float));
    float *dense2 = (float *)malloc(sizeof(float) * (size_t)batch * d2w);
    float *norm2 = (float *)calloc((size_t)batch * d2w, sizeof(float));
    bias = (float *)malloc(sizeof(float) * (size_t)batch * heads * squares * squares);
    if (!compressed || !dense1 || !norm1 || !dense2 || !norm2 || !bias)
      return -1;
    dense_affine(src->v, rows, in_w, s->t[8], NULL, c, compressed);
    dense_affine(compressed, batch, flat, s->t[9], NULL, d1w, dense1);
    for (int r = 0; r < batch; ++r)
      for (int col = 0; col < d1w; ++col)
        dense1[(size_t)r * d1w + col] += s->t[10][col];
    apply_activation(dense1, batch, d1w, s->act);
    layer_norm(dense1, NULL, 1.0f, s->t[13], s->t[14], norm1, batch, d1w, 1e-3f);
    dense_affine(norm1, batch, d1w, s->t[11], NULL, d2w, dense2);
    for (int r = 0; r < batch; ++r)
      for (int col = 0; col < d2w; ++col)
        dense2[(size_t)r * d2w + col] += s->t[12][col];
    apply_activation(dense2, batch, d2w, s->act);
    layer_norm(dense2, NULL, 1.0f, s->t[15], s->t[16], norm2, batch, d2w, 1e-3f);
    dense_affine(norm2, batch * heads, per_head, s->t[17], NULL,
                 squares * squares, bias);
    free(compressed);
    free(dense1);
    free(norm1);
    free(dense2);
    free(norm2);
  }

  const int score_rows = batch * heads * squares;
  float *scores = (float *)calloc((size_t)score_rows * squares, sizeof(float));
  float *context = (float *)calloc((size_t)rows * qkv_w, sizeof(float));
  if (!scores || !context)
    return -1;
  const float scale = 1.0f / sqrtf((float)depth);
  for (int b = 0; b < batch; ++b)
    for (int h = 0; h < heads; ++h)
      for (int qs = 0; qs < squares; ++qs) {
        const int score_row = (b * heads + h) * squares + qs;
        for (int ks = 0; ks < squares; ++ks) {
          float sum = 0.0f;
          for (int d = 0; d < depth; ++d) {
            const int ch = h * depth + d;
            sum += q[((size_t)b * squares + qs) * qkv_w + ch] *
                   k[((size_t)b * squares + ks) * qkv_w + ch];
          }
          sum *= scale;
          if (bias)
            sum += bias[((size_t)b * heads + h) * squares * squares +
                        (size_t)qs * squares + ks];
          scores[(size_t)score_row * squares + ks] = sum;
        }
      }
  softmax_rows(scores, score_rows, squares);
  for (int b = 0; b < batch; ++b)
    for (int qs = 0; qs < squares; ++qs) {
      float *c_row = context + ((size_t)b * squares + qs) * qkv_w;
      for (int h = 0; h < heads; ++h) {
        const float *p_row =
            scores + (size_t)((b * heads + h) * squares + qs) * squares;
        for (int d = 0; d < depth; ++d) {
          const int ch = h * depth + d;
          float sum = 0.0f;
          for (int ks = 0; ks < squares; ++ks)
            sum += p_row[ks] * v[((size_t)b * squares + ks) * qkv_w + ch];
          c_row[ch] = sum;
        }
      }
    }
  if (set_buf(out, rows, out_w))
    return -1;
  dense_affine(context, rows, qkv_w, s->t[6], s->t[7], out_w, out->v);
  free(q);
  free(k);
  free(v);
  free(bias);
  free(scores);
  free(context);
  return 0;
}

/* Attention policy map (cpu_network.cpp:892-1025).  t[0] = promotion
 * offsets [4][Dp]; t[1] = gather table as floats (policy index -> raw
 * index or -1), 1858 entries. */
static int run_policy_map(const or_step *s, int batch, const or_buf *query,
                          const or_buf *key, or_buf *out) {
  const int squares = 64, raw_n = 64 * 64 + 192, outputs = 1858;
  const int dp = query->width;
  if (dp <= 0 || key->width != dp || query->rows != batch * squares ||
      key->rows != batch * squares || s->d0[0] * (s->d1[0] ? s->d1[0] : 1) != 4 * dp)
    return -16;
  const float *promo = s->t[0];
  const float *gather = s->t[1];
  float *raw = (float *)calloc((size_t)batch * raw_n, sizeof(float));
  if (!raw || set_buf(out, batch, outputs))
    return -1;
  const float scale = 1.0f / sqrtf((float)dp);
  for (int b = 0; b < batch; ++b)
    for (int qs = 0; qs < squares; ++qs) {
      const float *q_row = query->v + ((size_t)b * squares + qs) * dp;
      for (int ks = 0; ks < squares; ++ks) {
        const float *k_row = key->v + ((size_t)b * squares + ks) * dp;
        float sum = 0.0f;
        for (int c = 0; c < dp; ++c)
          sum += q_row[c] * k_row[c];
        raw[(size_t)b * raw_n + (size_t)qs * squares + ks] = sum * scale;
      }
    }
  for (int b = 0; b < batch; ++b)
    for (int p = 0; p < 192; ++p) {
      /* The QK term reads the 3x64 view while the learned offset keeps the
       * 8x8x3 order (cpu_network.cpp:959-1001). */
      const int prow = p % 3;
      const int pkey = 56 + (p % 24) / 3;
      const int pair = p % squares;
      const int qs = 48 + pair / 8;
      const int ks = 56 + pair % 8;
      const float *q_row = query->v + ((size_t)b * squares + qs) * dp;
      const float *k_row = key->v + ((size_t)b * squares + ks) * dp;
      const float *pk_row = key->v + ((size_t)b * squares + pkey) * dp;
      float value = 0.0f;
      for (int c = 0; c < dp; ++c) {
        value += q_row[c] * k_row[c] * scale;
        value += pk_row[c] * (promo[(size_t)prow * dp + c] + promo[(size_t)3 * dp + c]);
      }
      raw[(size_t)b * raw_n + squares * squares + p] = value;
    }
  for (int b = 0; b < batch; ++b)
    for (int i = 0; i < outputs; ++i) {
      const int r = (int)gather[i];
      out->v[(size_t)b * outputs + i] = r >= 0 ? raw[(size_t)b * raw_n + r] : 0.0f;
    }
  free(raw);
  return 0;
}

/* Runs the resolved step list for one batch.  Buffer 0 holds the packed
 * plane values ([batch, 112]); results are copied out of `policy_buf`,
 * `value_buf` and (if >= 0) `moves_buf`.  Returns 0 or a negative error. */
int or_run(int batch, const uint64_t *masks, const float *values,
           const or_step *steps, int n_steps, int n_buffers, int policy_buf,
           float *policy_out, int policy_width, int value_buf,
           float *value_out, int value_width, int moves_buf, float *moves_out) {
  if (batch <= 0 || n_buffers <= 0)
    return -2;
  or_buf *bufs = (or_buf *)calloc((size_t)n_buffers, sizeof(or_buf));
  if (!bufs)
    return -1;
  int rc = set_buf(&bufs[0], batch, 112);
  if (!rc)
    memcpy(bufs[0].v, values, sizeof(float) * (size_t)batch * 112);
  for (int i = 0; rc == 0 && i < n_steps; ++i) {
    const or_step *s = &steps[i];
    if (s->dst <= 0 || s->dst >= n_buffers || s->src < 0 || s->src >= n_buffers) {
      rc = -3;
      break;
    }
    or_buf *dst = &bufs[s->dst];
    const or_buf *src = &bufs[s->src];
    switch (s->kind) {
    case OR_DYNAMIC_PE:
      rc = run_dynamic_pe(s, batch, masks, values, dst);
      break;
    case OR_STATIC_PE:
      rc = run_static_pe(s, batch, masks, values, dst);
      break;
    case OR_DENSE:
      rc = run_dense(s, batch, src, dst);
      break;
    case OR_LAYERNORM: {
      const or_buf *parent = s->parent >= 0 ? &bufs[s->parent] : NULL;
      if (parent && (parent->width != src->width || parent->rows != src->rows))
        parent = NULL;
      if (set_buf(dst, src->rows, src->width)) {
        rc = -1;
        break;
      }
      layer_norm(src->v, parent ? parent->v : NULL, parent ? s->alpha : 1.0f,
                 s->t[0], s->t[1], dst->v, src->rows, src->width, s->eps);
      break;
    }
    case OR_GATE:
      rc = run_gate(s, src, dst);
      break;
    case OR_FFN:
      rc = run_ffn(s, src, dst);
      break;
    case OR_ATTENTION:
      rc = run_attention(s, batch, src, dst);
      break;
    case OR_POLICY_MAP:
      rc = run_policy_map(s, batch, &bufs[s->aux0], &bufs[s->aux1], dst);
      break;
    default:
      rc = -4;
    }
  }
  if (rc == 0) {
    const or_buf *p = &bufs[policy_buf];
    const or_buf *v = &bufs[value_buf];
    if ((size_t)p->rows * p->width != (size_t)batch * policy_width ||
        (size_t)v->rows * v->width != (size_t)batch * value_width)
      rc = -5;
    else {
      memcpy(policy_out, p->v, sizeof(float) * (size_t)batch * policy_width);
      memcpy(value_out, v->v, sizeof(float) * (size_t)batch * value_width);
      if (moves_buf >= 0 && moves_out) {
        const or_buf *m = &bufs[moves_buf];
        memcpy(moves_out, m->v, sizeof(float) * (size_t)batch);
      }
    }
  }
  for (int i = 0; i < n_buffers; ++i)
    free(bufs[i].v);
  free(bufs);
  return rc;
}

/* PackInputPlanesRaw (reference src/nn/input_plane_packing.h:30-83). */
void or_pack_planes(const float *planes, int batch, uint64_t *masks,
                    float *values) {
  for (int b = 0; b < batch; ++b)
    for (int p = 0; p < 112; ++p) {
      const float *plane = planes + ((size_t)b * 112 + p) * 64;
      const size_t idx = (size_t)b * 112 + p;
      const int uniform = (p < 104 && p % 13 == 12) || p == 106 || p == 107 ||
                          p >= 109;
      if (uniform) {
        values[idx] = plane[0];
        masks[idx] = plane[0] != 0.0f ? ~0ULL : 0ULL;
        continue;
      }
      uint64_t mask = 0;
      float value = 0.0f;
      for (int sq = 0; sq < 64; ++sq) {
        const float v = plane[sq];
        if (v != 0.0f) {
          if (mask == 0)
            value = v;
          mask |= 1ULL << sq;
        }
      }
      masks[idx] = mask;
      values[idx] = value;
    }
}
