/*
 * CPU oracle for the ProteinMPNN v_48_020 design path (test infrastructure).
 *
 * Plain-C restatement of the reference's scalar path; see pmpnn_oracle.h for
 * the pinning of each function. Citations are relative to the reference
 * repository root. Build with -ffp-contract=off (oracle/Makefile): the
 * reference's default build forbids FMA contraction (meson.build:34).
 *
 * Linear layers: the reference's default "fast" GEMM
 * (cpp/primitives/linalg/gemm_scalar_fast.cpp:249-314) accumulates every
 * output element as one sequential float sum over k (K-blocks carry the
 * partial sum through the output buffer), then adds the bias
 * (cpp/include/hikoboshi/modules/mpnn/detail/mpnn_inner_inline.hpp:319-339).
 * linear_rows() below keeps exactly that per-element order while iterating
 * over a transposed weight copy so that the output loop vectorises.
 */
#include "pmpnn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { ST_OK = 0, ST_INVALID = 1, ST_PRECONDITION = 2 };

#define H PMO_H
#define V PMO_V
#define FF PMO_FF
#define DEC_IN (4 * PMO_H) /* [h_t, h_E, h_S, h_V] */

typedef struct {
  float* wt; /* [in][out] transposed copy */
  const float* b;
  int in, out;
} lin_t;

typedef struct {
  const float* g;
  const float* b;
} norm_t;

typedef struct {
  lin_t W1, W2, W3, W11, W12, W13, Win, Wout;
  norm_t n1, n2, n3;
} enc_layer_t;

typedef struct {
  lin_t W1, W2, W3, Win, Wout;
  norm_t n1, n2;
} dec_layer_t;

struct pmo_model {
  const float* pos_w; /* [16,66] */
  const float* pos_b; /* [16] */
  lin_t edge;         /* 416 -> 128, no bias */
  norm_t norm_edges;
  lin_t We;
  const float* Ws; /* [21,128] */
  enc_layer_t enc[PMO_LAYERS];
  dec_layer_t dec[PMO_LAYERS];
  lin_t Wout;
};

static lin_t make_lin(const float* w, const float* b, int out, int in) {
  lin_t l;
  l.wt = (float*)malloc(sizeof(float) * (size_t)in * (size_t)out);
  for (int o = 0; o < out; ++o)
    for (int p = 0; p < in; ++p) l.wt[(size_t)p * out + o] = w[(size_t)o * in + p];
  l.b = b;
  l.in = in;
  l.out = out;
  return l;
}

pmo_model* pmo_model_create(const float* const* t) {
  pmo_model* m = (pmo_model*)calloc(1, sizeof(pmo_model));
  m->pos_w = t[0];
  m->pos_b = t[1];
  m->edge = make_lin(t[2], NULL, H, PMO_EDGE_IN);
  m->norm_edges.g = t[3];
  m->norm_edges.b = t[4];
  m->We = make_lin(t[5], t[6], H, H);
  m->Ws = t[7];
  for (int l = 0; l < PMO_LAYERS; ++l) {
    const float* const* e = t + 8 + 22 * l;
    enc_layer_t* L = &m->enc[l];
    L->W1 = make_lin(e[0], e[1], H, 3 * H);
    L->W2 = make_lin(e[2], e[3], H, H);
    L->W3 = make_lin(e[4], e[5], H, H);
    L->W11 = make_lin(e[6], e[7], H, 3 * H);
    L->W12 = make_lin(e[8], e[9], H, H);
    L->W13 = make_lin(e[10], e[11], H, H);
    L->n1.g = e[12]; L->n1.b = e[13];
    L->n2.g = e[14]; L->n2.b = e[15];
    L->n3.g = e[16]; L->n3.b = e[17];
    L->Win = make_lin(e[18], e[19], FF, H);
    L->Wout = make_lin(e[20], e[21], H, FF);
  }
  for (int l = 0; l < PMO_LAYERS; ++l) {
    const float* const* d = t + 74 + 14 * l;
    dec_layer_t* L = &m->dec[l];
    L->W1 = make_lin(d[0], d[1], H, DEC_IN);
    L->W2 = make_lin(d[2], d[3], H, H);
    L->W3 = make_lin(d[4], d[5], H, H);
    L->n1.g = d[6]; L->n1.b = d[7];
    L->n2.g = d[8]; L->n2.b = d[9];
    L->Win = make_lin(d[10], d[11], FF, H);
    L->Wout = make_lin(d[12], d[13], H, FF);
  }
  m->Wout = make_lin(t[116], t[117], V, H);
  return m;
}

static void free_lin(lin_t* l) { free(l->wt); }

void pmo_model_destroy(pmo_model* m) {
  if (!m) return;
  free_lin(&m->edge);
  free_lin(&m->We);
  for (int l = 0; l < PMO_LAYERS; ++l) {
    enc_layer_t* e = &m->enc[l];
    free_lin(&e->W1); free_lin(&e->W2); free_lin(&e->W3);
    free_lin(&e->W11); free_lin(&e->W12); free_lin(&e->W13);
    free_lin(&e->Win); free_lin(&e->Wout);
    dec_layer_t* d = &m->dec[l];
    free_lin(&d->W1); free_lin(&d->W2); free_lin(&d->W3);
    free_lin(&d->Win); free_lin(&d->Wout);
  }
  free_lin(&m->Wout);
  free(m);
}

/* ---- elementwise numerics --------------------------------------------- */

/* cpp/include/hikoboshi/primitives/detail/fast_exp_neg.hpp:12-55 */
float pmo_fast_exp_neg(float x) {
  static const float table[17] = {
      1.0F,
      0.36787944117144232F,
      0.13533528323661270F,
      0.04978706836786394F,
      0.01831563888873418F,
      0.00673794699908547F,
      0.00247875217666636F,
      0.00091188196555452F,
      0.00033546262790251F,
      0.00012340980408668F,
      0.00004539992976248F,
      0.00001670170079024F,
      0.00000614421235333F,
      0.00000226032940698F,
      0.00000083152871910F,
      0.00000030590232050F,
      0.00000011253517471F,
  };
  if (x != x) return x;
  float neg_x = -x;
  if (neg_x > 16.0F) return 0.0F;
  if (neg_x < 0.0F) neg_x = 0.0F;
  int n = (int)(neg_x + 0.5F);
  if (n > 16) n = 16;
  const float r = -(neg_x - (float)n);
  const float e =
      1.0F +
      r * (1.0F +
           r * (0.5F +
                r * (1.0F / 6.0F +
                     r * (1.0F / 24.0F + r * (1.0F / 120.0F + r * (1.0F / 720.0F))))));
  return table[n] * e;
}

/* cpp/include/hikoboshi/primitives/compute/gelu.hpp:22-51 (A&S 7.1.26 erf) */
static float fast_erf(float v) {
  float sign = 1.0F;
  if (v < 0.0F) {
    sign = -1.0F;
    v = -v;
  }
  if (v > 4.0F) return sign;
  const float a1 = 0.254829592F, a2 = -0.284496736F, a3 = 1.421413741F;
  const float a4 = -1.453152027F, a5 = 1.061405429F, p = 0.3275911F;
  const float t = 1.0F / (1.0F + p * v);
  const float poly = (((((a5 * t + a4) * t) + a3) * t + a2) * t + a1) * t;
  return sign * (1.0F - poly * pmo_fast_exp_neg(-(v * v)));
}

float pmo_gelu(float x) { return 0.5F * x * (1.0F + fast_erf(x * 0.7071067811865475F)); }

static void gelu_inplace(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = pmo_gelu(x[i]);
}

/* cpp/primitives/compute/layer_norm_scalar.cpp:8-40 (Welford, eps 1e-5) */
static void layer_norm_row(const float* in, norm_t n, float* out) {
  float mean = 0.0F, m2 = 0.0F;
  for (int d = 0; d < H; ++d) {
    const float x = in[d];
    const float count = (float)(d + 1);
    const float delta = x - mean;
    mean += delta / count;
    const float delta2 = x - mean;
    m2 += delta * delta2;
  }
  const float var = m2 / (float)H;
  const float inv_std = 1.0F / sqrtf(var + 1.0e-5F);
  for (int d = 0; d < H; ++d) {
    const float normalized = (in[d] - mean) * inv_std;
    out[d] = normalized * n.g[d] + n.b[d];
  }
}

/* mpnn_inner_inline.hpp:410-419: input += 1*residual, then LayerNorm. */
static void ln_residual_row(float* in, const float* residual, norm_t n, float* out) {
  for (int d = 0; d < H; ++d) in[d] = 1.0F * residual[d] + in[d];
  layer_norm_row(in, n, out);
}

/* Sequential-k linear layer; see file header. */
static void linear_rows(const float* x, size_t rows, const lin_t* l, float* y) {
  const int in = l->in, out = l->out;
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * (size_t)in;
    float* yr = y + r * (size_t)out;
    for (int o = 0; o < out; ++o) yr[o] = 0.0F;
    for (int p = 0; p < in; ++p) {
      const float xp = xr[p];
      const float* w = l->wt + (size_t)p * out;
      for (int o = 0; o < out; ++o) yr[o] += xp * w[o];
    }
    if (l->b)
      for (int o = 0; o < out; ++o) yr[o] = yr[o] + l->b[o];
  }
}

/* ---- featurisation ------------------------------------------------------ */

static int atom_present(const uint8_t* src, int32_t r, int a) { return src[(size_t)r * 5 + a] != 0; }

/* inverse_fold_scalar.cpp:82-88,181-193: residue present iff N, CA, C, O. */
static void residue_mask(const uint8_t* src, int32_t L, float* mask, uint8_t* valid) {
  for (int32_t r = 0; r < L; ++r) {
    const int ok = atom_present(src, r, 0) && atom_present(src, r, 1) &&
                   atom_present(src, r, 2) && atom_present(src, r, 3);
    mask[r] = ok ? 1.0F : 0.0F;
    valid[r] = ok ? 1 : 0;
  }
}

/* cpp/primitives/compute/knn_scalar.cpp:46-51 */
static float knn_d2(const float* a, const float* b) {
  const float dx = a[0] - b[0];
  const float dy = a[1] - b[1];
  const float dz = a[2] - b[2];
  return dx * dx + dy * dy + dz * dz + 1.0e-6F;
}

/* cpp/primitives/compute/knn_scalar.cpp:72-168 with include_self = true,
 * query = target = CA buffer, validity masks given
 * (inverse_fold_scalar.cpp:211-234). */
void pmo_knn(const float* ca, const uint8_t* valid, int32_t L, int32_t K, int32_t* idx, float* d2) {
  if (K == 0 || L == 0) return;
  for (int32_t q = 0; q < L; ++q) {
    int32_t* ind = idx + (size_t)q * K;
    float* dist = d2 + (size_t)q * K;
    for (int32_t s = 0; s < K; ++s) {
      ind[s] = -1;
      dist[s] = INFINITY;
    }
    const float* qx = ca + (size_t)q * 3;
    const int qvalid = valid[q] != 0;
    float row_max = 1.0e-6F;
    if (qvalid) {
      for (int32_t t = 0; t < L; ++t) {
        if (!valid[t]) continue;
        const float c = knn_d2(qx, ca + (size_t)t * 3);
        if (c > row_max) row_max = c;
      }
    }
    for (int32_t t = 0; t < L; ++t) {
      float d;
      if (!qvalid || !valid[t])
        d = row_max;
      else
        d = knn_d2(qx, ca + (size_t)t * 3);
      int32_t at = K;
      for (int32_t s = 0; s < K; ++s) {
        if (d < dist[s]) {
          at = s;
          break;
        }
      }
      if (at == K) continue;
      for (int32_t s = K - 1; s > at; --s) {
        dist[s] = dist[s - 1];
        ind[s] = ind[s - 1];
      }
      dist[at] = d;
      ind[at] = t;
    }
    for (int32_t s = 0; s < K; ++s)
      if (dist[s] == INFINITY) dist[s] = row_max;
  }
}

/* cpp/primitives/compute/atom_pair_distance_scalar.cpp:21-72 (query, neighbour) */
static const int kPairs[PMO_PAIRS][2] = {
    {1, 1}, {0, 0}, {2, 2}, {3, 3}, {4, 4}, {1, 0}, {1, 2}, {1, 3}, {1, 4},
    {0, 2}, {0, 3}, {0, 4}, {4, 2}, {4, 3}, {3, 2}, {0, 1}, {2, 1}, {3, 1},
    {4, 1}, {2, 0}, {3, 0}, {4, 0}, {2, 4}, {3, 4}, {2, 3}};

static int32_t effective_k(int32_t L) { return L < PMO_KMAX ? L : PMO_KMAX; }

/* cpp/modules/mpnn/edge_rbf_features_scalar.cpp:117-152 with
 * atom_pair_distance_scalar.cpp:103-164, rbf_scalar.cpp:10-35 and the
 * positional one-hot linear edge_rbf_features_scalar.cpp:45-76. */
static void edge_features_from_idx(const pmo_model* m, const float* coords, const uint8_t* src,
                                   const int32_t* resid, const int32_t* chain, int32_t L,
                                   int32_t K, const int32_t* idx, float* feat) {
  const float center_step = (22.0F - 2.0F) / (float)(PMO_RBF - 1);
  const float sigma = (22.0F - 2.0F) / ((float)PMO_RBF / 0.7071067811865475F);
  const float two_sigma_sq = 2.0F * sigma * sigma;
  for (int32_t r = 0; r < L; ++r) {
    for (int32_t k = 0; k < K; ++k) {
      const size_t slot = (size_t)r * K + k;
      float* row = feat + slot * PMO_EDGE_IN;
      const int32_t j = idx[slot];
      if (j < 0 || j >= L) {
        memset(row, 0, sizeof(float) * PMO_EDGE_IN);
        continue;
      }
      /* positional features */
      int cls;
      const int32_t ci = chain ? chain[r] : 0, cj = chain ? chain[j] : 0;
      if (ci != cj) {
        cls = PMO_POS_CLASSES - 1;
      } else {
        int32_t off = (resid ? resid[r] : r) - (resid ? resid[j] : j);
        if (off < -32) off = -32;
        if (off > 32) off = 32;
        cls = off + 32;
      }
      for (int d = 0; d < PMO_POS; ++d)
        row[d] = m->pos_w[d * PMO_POS_CLASSES + cls] + m->pos_b[d];
      /* atom-pair distances + RBF */
      for (int p = 0; p < PMO_PAIRS; ++p) {
        float* rbf = row + PMO_POS + p * PMO_RBF;
        const int qa = kPairs[p][0], na = kPairs[p][1];
        if (!atom_present(src, r, qa) || !atom_present(src, j, na)) {
          for (int f = 0; f < PMO_RBF; ++f) rbf[f] = 0.0F;
          continue;
        }
        float sq = 0.0F;
        for (int ax = 0; ax < 3; ++ax) {
          const float qv = coords[((size_t)r * 5 + qa) * 3 + ax];
          const float nv = coords[((size_t)j * 5 + na) * 3 + ax];
          const float delta = nv - qv;
          sq += delta * delta;
        }
        sq = sq + 1.0e-6F;
        const float dist = sqrtf(sq);
        for (int f = 0; f < PMO_RBF; ++f) {
          const float center = 2.0F + (float)f * center_step;
          const float delta = dist - center;
          rbf[f] = pmo_fast_exp_neg(-(delta * delta) / two_sigma_sq);
        }
      }
    }
  }
}

static void ca_coords(const float* coords, const uint8_t* src, int32_t L, float* ca) {
  for (int32_t r = 0; r < L; ++r)
    for (int ax = 0; ax < 3; ++ax)
      ca[(size_t)r * 3 + ax] = atom_present(src, r, 1) ? coords[((size_t)r * 5 + 1) * 3 + ax] : 0.0F;
}

int pmo_edge_features(const pmo_model* m, const float* coords, const uint8_t* src,
                      const int32_t* resid, const int32_t* chain, int32_t L, int32_t* idx,
                      float* features) {
  if (L <= 0) return ST_OK;
  const int32_t K = effective_k(L);
  float* mask = (float*)malloc(sizeof(float) * L);
  uint8_t* valid = (uint8_t*)malloc(L);
  float* ca = (float*)malloc(sizeof(float) * 3 * L);
  float* d2 = (float*)malloc(sizeof(float) * (size_t)L * K);
  residue_mask(src, L, mask, valid);
  ca_coords(coords, src, L, ca);
  pmo_knn(ca, valid, L, K, idx, d2);
  edge_features_from_idx(m, coords, src, resid, chain, L, K, idx, features);
  free(mask); free(valid); free(ca); free(d2);
  return ST_OK;
}

/* ---- encoder ------------------------------------------------------------ */

/* cpp/modules/mpnn/proteinmpnn_encoder_scalar.cpp:169-189: rows [h_i, e_ij, h_j]
 * with the gather zero-filling invalid neighbours (gather_scalar.cpp:8-29). */
static void enc_message_inputs(const float* hv, const float* he, const int32_t* idx, int32_t L,
                               int32_t K, float* x) {
  for (int32_t r = 0; r < L; ++r)
    for (int32_t k = 0; k < K; ++k) {
      const size_t slot = (size_t)r * K + k;
      float* row = x + slot * 3 * H;
      memcpy(row, hv + (size_t)r * H, sizeof(float) * H);
      memcpy(row + H, he + slot * H, sizeof(float) * H);
      const int32_t j = idx[slot];
      if (j >= 0 && j < L)
        memcpy(row + 2 * H, hv + (size_t)j * H, sizeof(float) * H);
      else
        memset(row + 2 * H, 0, sizeof(float) * H);
    }
}

/* inverse_fold_scalar.cpp:300-352 (encode_backbone) and
 * proteinmpnn_encoder_scalar.cpp:323-333 (three layers). */
int pmo_encode(const pmo_model* m, const float* coords, const uint8_t* src, const int32_t* resid,
               const int32_t* chain, int32_t L, float* mask, int32_t* idx, float* hv, float* he) {
  if (L <= 0) return ST_OK;
  const int32_t K = effective_k(L);
  const size_t S = (size_t)L * K;
  uint8_t* valid = (uint8_t*)malloc(L);
  float* ca = (float*)malloc(sizeof(float) * 3 * L);
  float* d2 = (float*)malloc(sizeof(float) * S);
  residue_mask(src, L, mask, valid);
  ca_coords(coords, src, L, ca);
  pmo_knn(ca, valid, L, K, idx, d2);

  float* big = (float*)malloc(sizeof(float) * S * PMO_EDGE_IN); /* features / message inputs */
  float* t1 = (float*)malloc(sizeof(float) * S * H);
  float* t2 = (float*)malloc(sizeof(float) * S * H);
  float* mask_attend = (float*)calloc(S, sizeof(float));
  float* scratch = (float*)malloc(sizeof(float) * (size_t)L * H);
  float* ffn = (float*)malloc(sizeof(float) * (size_t)L * FF);

  /* edge embedding: inverse_fold_scalar.cpp:236-279 */
  edge_features_from_idx(m, coords, src, resid, chain, L, K, idx, big);
  linear_rows(big, S, &m->edge, t1);
  for (size_t s = 0; s < S; ++s) layer_norm_row(t1 + s * H, m->norm_edges, t2 + s * H);
  linear_rows(t2, S, &m->We, he);

  /* mask_attend: inverse_fold_scalar.cpp:281-298 */
  for (int32_t r = 0; r < L; ++r)
    for (int32_t k = 0; k < K; ++k) {
      const int32_t j = idx[(size_t)r * K + k];
      if (j >= 0 && j < L) mask_attend[(size_t)r * K + k] = mask[r] * mask[j];
    }

  memset(hv, 0, sizeof(float) * (size_t)L * H);
  const float scale = 1.0F / 30.0F;
  for (int l = 0; l < PMO_LAYERS; ++l) {
    const enc_layer_t* E = &m->enc[l];
    /* message MLP: proteinmpnn_encoder_scalar.cpp:191-213 */
    enc_message_inputs(hv, he, idx, L, K, big);
    linear_rows(big, S, &E->W1, t1);
    gelu_inplace(t1, S * H);
    linear_rows(t1, S, &E->W2, t2);
    gelu_inplace(t2, S * H);
    linear_rows(t2, S, &E->W3, t1);
    /* aggregate + LN1: proteinmpnn_encoder_scalar.cpp:215-249 */
    memset(scratch, 0, sizeof(float) * (size_t)L * H);
    for (int32_t r = 0; r < L; ++r) {
      float* upd = scratch + (size_t)r * H;
      for (int32_t k = 0; k < K; ++k) {
        const size_t slot = (size_t)r * K + k;
        const int32_t j = idx[slot];
        if (!(j >= 0 && j < L)) continue;
        float alpha = scale;
        alpha *= mask_attend[slot];
        if (alpha == 0.0F) continue;
        const float* msg = t1 + slot * H;
        for (int d = 0; d < H; ++d) upd[d] = alpha * msg[d] + upd[d];
      }
      ln_residual_row(upd, hv + (size_t)r * H, E->n1, hv + (size_t)r * H);
    }
    /* FFN + LN2: proteinmpnn_encoder_scalar.cpp:251-272 */
    linear_rows(hv, L, &E->Win, ffn);
    gelu_inplace(ffn, (size_t)L * FF);
    linear_rows(ffn, L, &E->Wout, scratch);
    for (int32_t r = 0; r < L; ++r)
      ln_residual_row(scratch + (size_t)r * H, hv + (size_t)r * H, E->n2, hv + (size_t)r * H);
    /* mask_v: proteinmpnn_encoder_scalar.cpp:274-287 */
    for (int32_t r = 0; r < L; ++r)
      for (int d = 0; d < H; ++d) hv[(size_t)r * H + d] *= mask[r];
    /* edge update: proteinmpnn_encoder_scalar.cpp:289-321 */
    enc_message_inputs(hv, he, idx, L, K, big);
    linear_rows(big, S, &E->W11, t1);
    gelu_inplace(t1, S * H);
    linear_rows(t1, S, &E->W12, t2);
    gelu_inplace(t2, S * H);
    linear_rows(t2, S, &E->W13, t1);
    for (size_t s = 0; s < S; ++s) {
      const int32_t j = idx[s];
      if (!(j >= 0 && j < L)) continue;
      ln_residual_row(t1 + s * H, he + s * H, E->n3, he + s * H);
    }
  }
  free(valid); free(ca); free(d2); free(big); free(t1); free(t2);
  free(mask_attend); free(scratch); free(ffn);
  return ST_OK;
}

/* ---- decode order + RNG --------------------------------------------------- */

/* cpp/modules/mpnn/decode_order_scalar.cpp:21-27, sampler_scalar.cpp:19-25 */
static uint64_t splitmix64(uint64_t* state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double uniform01(uint64_t* state) {
  return (double)(splitmix64(state) >> 11) * (1.0 / 9007199254740992.0);
}

/* decode_order_scalar.cpp:34-42 */
static float normal_abs(uint64_t* state) {
  double u1 = uniform01(state);
  if (u1 <= 0.0) u1 = 1.0 / 9007199254740992.0;
  const double u2 = uniform01(state);
  const double radius = sqrt(-2.0 * log(u1));
  return (float)fabs(radius * cos(6.283185307179586476925286766559 * u2));
}

static const float* g_sort_scores;
static int cmp_order(const void* a, const void* b) {
  const int32_t l = *(const int32_t*)a, r = *(const int32_t*)b;
  const float ls = g_sort_scores[l], rs = g_sort_scores[r];
  if (ls == rs) return (l > r) - (l < r);
  return ls < rs ? -1 : 1;
}

/* decode_order_scalar.cpp:61-116. The comparator is a total order (ties
 * broken by index), so any sort reproduces std::stable_sort's result. */
int pmo_decode_order(const float* chain_mask, const float* residue_mask_v, int32_t L,
                     uint64_t seed, const int32_t* input_order, int use_input_order,
                     int32_t* order) {
  if (use_input_order) {
    unsigned char* seen = (unsigned char*)calloc(L > 0 ? L : 1, 1);
    for (int32_t p = 0; p < L; ++p) {
      const int32_t r = input_order ? input_order[p] : p;
      if (r < 0 || r >= L || seen[r]) {
        free(seen);
        return ST_INVALID;
      }
      seen[r] = 1;
      order[p] = r;
    }
    free(seen);
    return ST_OK;
  }
  float* scores = (float*)malloc(sizeof(float) * (L > 0 ? L : 1));
  uint64_t state = seed;
  for (int32_t r = 0; r < L; ++r) {
    const float c = chain_mask ? chain_mask[r] : 1.0F;
    const float mk = residue_mask_v ? residue_mask_v[r] : 1.0F;
    order[r] = r;
    scores[r] = (c * mk + 0.0001F) * normal_abs(&state);
  }
  g_sort_scores = scores;
  qsort(order, (size_t)L, sizeof(int32_t), cmp_order);
  free(scores);
  return ST_OK;
}

/* decode_order_scalar.cpp:118-164 */
static int causal_masks(const int32_t* order, const int32_t* idx, const float* mask, int32_t L,
                        int32_t K, float* bw, float* fw) {
  int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * L);
  for (int32_t r = 0; r < L; ++r) pos[r] = -1;
  for (int32_t p = 0; p < L; ++p) {
    const int32_t r = order[p];
    if (r < 0 || r >= L || pos[r] >= 0) {
      free(pos);
      return ST_INVALID;
    }
    pos[r] = p;
  }
  for (int32_t r = 0; r < L; ++r)
    for (int32_t k = 0; k < K; ++k) {
      const size_t slot = (size_t)r * K + k;
      const int32_t j = idx[slot];
      float b = 0.0F, f = 0.0F;
      if (j >= 0 && j < L) {
        if (pos[j] < pos[r])
          b = mask[r];
        else
          f = mask[r];
      }
      bw[slot] = b;
      fw[slot] = f;
    }
  free(pos);
  return ST_OK;
}

/* ---- decoder ------------------------------------------------------------- */

typedef struct {
  float* msg_in; /* [K, 512] */
  float* m1;     /* [K, 128] */
  float* m2;     /* [K, 128] */
  float* upd;    /* [128] */
  float* ffn;    /* [512] */
} dec_ws_t;

static void dec_ws_init(dec_ws_t* w, int32_t K) {
  w->msg_in = (float*)malloc(sizeof(float) * (size_t)K * DEC_IN);
  w->m1 = (float*)malloc(sizeof(float) * (size_t)K * H);
  w->m2 = (float*)malloc(sizeof(float) * (size_t)K * H);
  w->upd = (float*)malloc(sizeof(float) * H);
  w->ffn = (float*)malloc(sizeof(float) * FF);
}

static void dec_ws_free(dec_ws_t* w) {
  free(w->msg_in); free(w->m1); free(w->m2); free(w->upd); free(w->ffn);
}

/* One residue row of proteinmpnn_decoder_layer_scalar
 * (cpp/modules/mpnn/decoder_layer_scalar.cpp:26-151) with no attention mask.
 * ctx is [K, 384]; out may not alias node. */
static void dec_layer_row(const dec_layer_t* D, const float* node, const float* ctx, int32_t K,
                          float row_mask, dec_ws_t* w, float* out) {
  for (int32_t k = 0; k < K; ++k) {
    memcpy(w->msg_in + (size_t)k * DEC_IN, node, sizeof(float) * H);
    memcpy(w->msg_in + (size_t)k * DEC_IN + H, ctx + (size_t)k * 3 * H, sizeof(float) * 3 * H);
  }
  linear_rows(w->msg_in, K, &D->W1, w->m1);
  gelu_inplace(w->m1, (size_t)K * H);
  linear_rows(w->m1, K, &D->W2, w->m2);
  gelu_inplace(w->m2, (size_t)K * H);
  linear_rows(w->m2, K, &D->W3, w->m1);
  const float scale = 1.0F / 30.0F;
  for (int d = 0; d < H; ++d) w->upd[d] = 0.0F;
  for (int32_t k = 0; k < K; ++k) {
    const float alpha = 1.0F * scale;
    const float* msg = w->m1 + (size_t)k * H;
    for (int d = 0; d < H; ++d) w->upd[d] = alpha * msg[d] + w->upd[d];
  }
  ln_residual_row(w->upd, node, D->n1, out);
  linear_rows(out, 1, &D->Win, w->ffn);
  gelu_inplace(w->ffn, FF);
  linear_rows(w->ffn, 1, &D->Wout, w->upd);
  ln_residual_row(w->upd, out, D->n2, out);
  if (row_mask != 1.0F)
    for (int d = 0; d < H; ++d) out[d] *= row_mask;
}

/* decoder_layer_scalar.cpp:153-175 */
static void logits_row(const pmo_model* m, const float* h, float* logits) { linear_rows(h, 1, &m->Wout, logits); }

static int valid_token(int32_t t) { return t >= 0 && t < V; }

static int32_t fallback_token(const int32_t* true_tokens, int32_t r) {
  if (true_tokens && valid_token(true_tokens[r])) return true_tokens[r];
  return V - 1;
}

/* inverse_fold_scalar.cpp:471-493 */
static float average_nll(const int32_t* tokens, const float* lp, const float* chain_mask,
                         const float* mask, int32_t L) {
  double loss = 0.0, msum = 0.0;
  for (int32_t r = 0; r < L; ++r) {
    const float active = (chain_mask ? chain_mask[r] : 1.0F) * mask[r];
    if (active == 0.0F) continue;
    const int32_t t = tokens[r];
    if (!valid_token(t)) continue;
    loss -= (double)lp[(size_t)r * V + t];
    msum += (double)active;
  }
  return msum > 0.0 ? (float)(loss / msum) : 0.0F;
}

/* cpp/modules/mpnn/sampler_scalar.cpp:27-131. Returns the token; writes the
 * temperature-scaled log-probs. When gap != NULL and a draw is made, *gap is
 * the distance between the draw and the nearest CDF boundary. */
static int32_t sample_row(const float* logits, float temperature, int greedy, uint64_t* rng,
                          float* log_probs, double* gap) {
  const float T = (temperature > 0.0F && isfinite(temperature)) ? temperature : 1.0F;
  float z[V], p[V];
  float row_max = -INFINITY;
  for (int i = 0; i < V; ++i) {
    z[i] = logits[i] / T;
    row_max = (row_max < z[i]) ? z[i] : row_max; /* std::max */
  }
  float row_sum = 0.0F;
  for (int i = 0; i < V; ++i) {
    const float e = expf(z[i] - row_max);
    p[i] = e;
    row_sum += e;
  }
  const float log_sum = logf(row_sum);
  const float inv_sum = 1.0F / row_sum;
  for (int i = 0; i < V; ++i) {
    p[i] *= inv_sum;
    log_probs[i] = (z[i] - row_max) - log_sum;
  }
  if (greedy || temperature <= 0.0F) {
    int32_t best = 0;
    float bv = z[0];
    for (int i = 1; i < V; ++i)
      if (z[i] > bv) {
        best = i;
        bv = z[i];
      }
    if (gap) *gap = INFINITY;
    return best;
  }
  const double u = uniform01(rng);
  double cum = 0.0;
  double best_gap = INFINITY;
  int32_t chosen = -1;
  for (int i = 0; i < V; ++i) {
    cum += (double)p[i];
    const double g = fabs(u - cum);
    if (g < best_gap) best_gap = g;
    if (chosen < 0 && u < cum) chosen = i;
  }
  if (chosen < 0) chosen = V - 1;
  if (gap) *gap = best_gap;
  return chosen;
}

/* Autoregressive decoder: inverse_fold_scalar.cpp:752-888. forced_tokens,
 * when given, replaces the sampled token written back into the sequence
 * state (the RNG still advances as in the reference), which replays a
 * foreign token trajectory through the reference arithmetic; `sampled`
 * then receives the oracle's own choice at each position. */
int pmo_decode(const pmo_model* m, const float* mask, const int32_t* idx, const float* hv,
               const float* he, int32_t L, const float* chain_mask, const int32_t* true_tokens,
               const int32_t* order, uint64_t seed, float temperature, int greedy,
               const int32_t* forced_tokens, int32_t* tokens, float* log_probs, float* score,
               int32_t* sampled, double* cdf_gap) {
  if (L <= 0) return ST_OK;
  const int32_t K = effective_k(L);
  const size_t S = (size_t)L * K;
  float* bw = (float*)malloc(sizeof(float) * S);
  float* fw = (float*)malloc(sizeof(float) * S);
  int st = causal_masks(order, idx, mask, L, K, bw, fw);
  if (st != ST_OK) {
    free(bw); free(fw);
    return st;
  }
  /* encoder context fw * [h_E, 0, h_V_enc_j]: inverse_fold_scalar.cpp:377-398,443-456 */
  float* enc_fw = (float*)malloc(sizeof(float) * S * 3 * H);
  for (size_t s = 0; s < S; ++s) {
    float row[3 * H];
    memcpy(row, he + s * H, sizeof(float) * H);
    memset(row + H, 0, sizeof(float) * H);
    const int32_t j = idx[s];
    if (j >= 0 && j < L)
      memcpy(row + 2 * H, hv + (size_t)j * H, sizeof(float) * H);
    else
      memset(row + 2 * H, 0, sizeof(float) * H);
    const float f = fw[s];
    for (int d = 0; d < 3 * H; ++d) enc_fw[s * 3 * H + d] = f * row[d];
  }
  float* hs = (float*)calloc((size_t)L * H, sizeof(float));
  float* stack = (float*)calloc((size_t)(PMO_LAYERS + 1) * L * H, sizeof(float));
  memcpy(stack, hv, sizeof(float) * (size_t)L * H);
  float* es_row = (float*)malloc(sizeof(float) * (size_t)K * 2 * H);
  float* ctx = (float*)malloc(sizeof(float) * (size_t)K * 3 * H);
  float node_in[H], logits[V], lp_row[V];
  dec_ws_t w;
  dec_ws_init(&w, K);
  uint64_t rng = seed;

  for (int32_t oi = 0; oi < L; ++oi) {
    const int32_t r = order[oi];
    const float active = mask[r];
    if (active == 0.0F) {
      const int32_t t = fallback_token(true_tokens, r);
      tokens[r] = t;
      memset(log_probs + (size_t)r * V, 0, sizeof(float) * V);
      memcpy(hs + (size_t)r * H, m->Ws + (size_t)t * H, sizeof(float) * H);
      if (sampled) sampled[r] = t;
      if (cdf_gap) cdf_gap[r] = INFINITY;
      continue;
    }
    /* build_h_es_row: inverse_fold_scalar.cpp:665-685 */
    for (int32_t k = 0; k < K; ++k) {
      const size_t slot = (size_t)r * K + k;
      memcpy(es_row + (size_t)k * 2 * H, he + slot * H, sizeof(float) * H);
      const int32_t j = idx[slot];
      if (j >= 0 && j < L)
        memcpy(es_row + (size_t)k * 2 * H + H, hs + (size_t)j * H, sizeof(float) * H);
      else
        memset(es_row + (size_t)k * 2 * H + H, 0, sizeof(float) * H);
    }
    for (int l = 0; l < PMO_LAYERS; ++l) {
      const float* layer_state = stack + (size_t)l * L * H;
      /* build_h_esv_row + combine_context_row: inverse_fold_scalar.cpp:687-728 */
      for (int32_t k = 0; k < K; ++k) {
        const size_t slot = (size_t)r * K + k;
        float dec[3 * H];
        memcpy(dec, es_row + (size_t)k * 2 * H, sizeof(float) * 2 * H);
        const int32_t j = idx[slot];
        if (j >= 0 && j < L)
          memcpy(dec + 2 * H, layer_state + (size_t)j * H, sizeof(float) * H);
        else
          memset(dec + 2 * H, 0, sizeof(float) * H);
        const float b = bw[slot];
        const float* e = enc_fw + slot * 3 * H;
        float* out = ctx + (size_t)k * 3 * H;
        for (int d = 0; d < 3 * H; ++d) out[d] = b * dec[d] + e[d];
      }
      memcpy(node_in, layer_state + (size_t)r * H, sizeof(float) * H);
      dec_layer_row(&m->dec[l], node_in, ctx, K, active, &w,
                    stack + (size_t)(l + 1) * L * H + (size_t)r * H);
    }
    logits_row(m, stack + (size_t)PMO_LAYERS * L * H + (size_t)r * H, logits);
    double gap = INFINITY;
    const int32_t s_tok = sample_row(logits, temperature, greedy, &rng, lp_row, &gap);
    const float design = (chain_mask ? chain_mask[r] : 1.0F) * mask[r];
    int32_t t = design != 0.0F ? s_tok : fallback_token(true_tokens, r);
    if (sampled) sampled[r] = t;
    if (cdf_gap) cdf_gap[r] = gap;
    if (forced_tokens) t = forced_tokens[r];
    tokens[r] = t;
    memcpy(log_probs + (size_t)r * V, lp_row, sizeof(float) * V);
    memcpy(hs + (size_t)r * H, m->Ws + (size_t)t * H, sizeof(float) * H);
  }
  if (score) *score = average_nll(tokens, log_probs, chain_mask, mask, L);
  dec_ws_free(&w);
  free(bw); free(fw); free(enc_fw); free(hs); free(stack); free(es_row); free(ctx);
  return ST_OK;
}

/* Teacher-forced decoder: inverse_fold_scalar.cpp:575-663 (plain log_softmax,
 * cpp/primitives/compute/log_softmax_scalar.cpp:8-37). Rows are independent,
 * so the full-sequence layer is evaluated row by row. */
int pmo_teacher_forced_decode(const pmo_model* m, const float* mask, const int32_t* idx,
                              const float* hv, const float* he, int32_t L,
                              const float* chain_mask, const int32_t* tokens,
                              const int32_t* order, float* log_probs, float* score) {
  if (L <= 0) return ST_OK;
  for (int32_t r = 0; r < L; ++r)
    if (!valid_token(tokens[r])) return ST_INVALID;
  const int32_t K = effective_k(L);
  const size_t S = (size_t)L * K;
  float* bw = (float*)malloc(sizeof(float) * S);
  float* fw = (float*)malloc(sizeof(float) * S);
  int st = causal_masks(order, idx, mask, L, K, bw, fw);
  if (st != ST_OK) {
    free(bw); free(fw);
    return st;
  }
  float* cur = (float*)malloc(sizeof(float) * (size_t)L * H);
  float* nxt = (float*)malloc(sizeof(float) * (size_t)L * H);
  memcpy(cur, hv, sizeof(float) * (size_t)L * H);
  float* ctx = (float*)malloc(sizeof(float) * (size_t)K * 3 * H);
  dec_ws_t w;
  dec_ws_init(&w, K);
  for (int l = 0; l < PMO_LAYERS; ++l) {
    for (int32_t r = 0; r < L; ++r) {
      for (int32_t k = 0; k < K; ++k) {
        const size_t slot = (size_t)r * K + k;
        const int32_t j = idx[slot];
        const int jv = j >= 0 && j < L;
        float esv[3 * H], exv[3 * H];
        memcpy(esv, he + slot * H, sizeof(float) * H);
        memcpy(exv, he + slot * H, sizeof(float) * H);
        memset(exv + H, 0, sizeof(float) * H);
        if (jv) {
          memcpy(esv + H, m->Ws + (size_t)tokens[j] * H, sizeof(float) * H);
          memcpy(esv + 2 * H, cur + (size_t)j * H, sizeof(float) * H);
          memcpy(exv + 2 * H, hv + (size_t)j * H, sizeof(float) * H);
        } else {
          memset(esv + H, 0, sizeof(float) * 2 * H);
          memset(exv + 2 * H, 0, sizeof(float) * H);
        }
        const float b = bw[slot], f = fw[slot];
        float* out = ctx + (size_t)k * 3 * H;
        for (int d = 0; d < 3 * H; ++d) out[d] = b * esv[d] + f * exv[d];
      }
      dec_layer_row(&m->dec[l], cur + (size_t)r * H, ctx, K, mask[r], &w, nxt + (size_t)r * H);
    }
    float* tmp = cur;
    cur = nxt;
    nxt = tmp;
  }
  for (int32_t r = 0; r < L; ++r) {
    float logits[V];
    logits_row(m, cur + (size_t)r * H, logits);
    float row_max = -INFINITY;
    for (int d = 0; d < V; ++d)
      if (logits[d] > row_max) row_max = logits[d];
    float row_sum = 0.0F;
    for (int d = 0; d < V; ++d) row_sum += expf(logits[d] - row_max);
    const float lrs = logf(row_sum);
    for (int d = 0; d < V; ++d) log_probs[(size_t)r * V + d] = (logits[d] - row_max) - lrs;
  }
  if (score) *score = average_nll(tokens, log_probs, chain_mask, mask, L);
  dec_ws_free(&w);
  free(bw); free(fw); free(cur); free(nxt); free(ctx);
  return ST_OK;
}

/* ---- module and algorithm level -------------------------------------------- */

/* inverse_fold_scalar.cpp:954-1000 */
int pmo_inverse_fold(const pmo_model* m, const float* coords, const uint8_t* src, int32_t L,
                     const int32_t* resid, const int32_t* chain, const float* chain_mask,
                     const int32_t* input_order, const int32_t* true_tokens, uint64_t seed,
                     uint64_t order_seed, float temperature, int greedy, int use_input_order,
                     int32_t* tokens, float* log_probs, int32_t* order_out, float* score) {
  if (L <= 0) return ST_OK;
  const int32_t K = effective_k(L);
  const size_t S = (size_t)L * K;
  float* mask = (float*)malloc(sizeof(float) * L);
  int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * S);
  float* hv = (float*)malloc(sizeof(float) * (size_t)L * H);
  float* he = (float*)malloc(sizeof(float) * S * H);
  int st = pmo_encode(m, coords, src, resid, chain, L, mask, idx, hv, he);
  if (st == ST_OK) st = pmo_decode_order(chain_mask, mask, L, order_seed, input_order, use_input_order, order_out);
  if (st == ST_OK)
    st = pmo_decode(m, mask, idx, hv, he, L, chain_mask, true_tokens, order_out, seed, temperature,
                    greedy, NULL, tokens, log_probs, score, NULL, NULL);
  free(mask); free(idx); free(hv); free(he);
  return st;
}

/* inverse_fold_scalar.cpp:905-952 */
int pmo_teacher_forced(const pmo_model* m, const float* coords, const uint8_t* src, int32_t L,
                       const int32_t* resid, const int32_t* chain, const float* chain_mask,
                       const int32_t* tokens, const int32_t* input_order, float* log_probs,
                       float* score) {
  if (L <= 0) return ST_OK;
  const int32_t K = effective_k(L);
  const size_t S = (size_t)L * K;
  float* mask = (float*)malloc(sizeof(float) * L);
  int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * S);
  int32_t* order = (int32_t*)malloc(sizeof(int32_t) * L);
  float* hv = (float*)malloc(sizeof(float) * (size_t)L * H);
  float* he = (float*)malloc(sizeof(float) * S * H);
  int st = pmo_encode(m, coords, src, resid, chain, L, mask, idx, hv, he);
  if (st == ST_OK) st = pmo_decode_order(chain_mask, mask, L, 0, input_order, 1, order);
  if (st == ST_OK)
    st = pmo_teacher_forced_decode(m, mask, idx, hv, he, L, chain_mask, tokens, order, log_probs, score);
  free(mask); free(idx); free(order); free(hv); free(he);
  return st;
}

/* cpp/algorithms/inverse_fold.cpp:221-356 with backbone_noise = 0: one
 * module call per sample, seed + i for both the order and the sampler, the
 * whole backbone re-encoded every sample exactly as the reference does. */
int pmo_algorithm_inverse_fold(const pmo_model* m, const float* coords, const uint8_t* src,
                               int32_t L, int32_t num_seqs, uint64_t seed, float temperature,
                               int n_to_c, int32_t* tokens, float* log_probs, float* scores) {
  if (L <= 0 || num_seqs <= 0) return ST_INVALID;
  if (!isfinite(temperature) || temperature < 0.0F) return ST_INVALID;
  int32_t* order = (int32_t*)malloc(sizeof(int32_t) * L);
  int st = ST_OK;
  for (int32_t i = 0; i < num_seqs && st == ST_OK; ++i) {
    const uint64_t s = seed + (uint64_t)i;
    st = pmo_inverse_fold(m, coords, src, L, NULL, NULL, NULL, NULL, NULL, s, s, temperature,
                          temperature <= 0.0F, n_to_c, tokens + (size_t)i * L,
                          log_probs + (size_t)i * L * V, order, scores + i);
  }
  free(order);
  return st;
}
