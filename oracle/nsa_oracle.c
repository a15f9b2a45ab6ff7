/*
 * CPU oracle for the NSA selection path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker.  The product path (omnimem_amd) never calls it.
 *
 * Restates, in plain C:
 *   - block scores with a fixed fp32 arithmetic: acc = fmaf(q[d], k[d], acc) for d ascending
 *     from acc = 0, then acc * scale (the reference computes q.k * scale in fp32,
 *     cuda_backend/csrc/topk.cu:179-291 and :389; nsa/ops/index_topk.py:99);
 *   - the top-k visibility rule of cuda_backend/csrc/topk.cu:36-97 (chunk-causal, non-causal
 *     with q_chunk_offset, teacher-forcing four-case, AWE sink/window, progressive gating);
 *   - the ordering (score desc, id asc; -0 == +0) and -1 padding of topk.cu:3,100-102 and
 *     ops.h:11-12, by a plain comparison sort of each row's visible candidates.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int32_t block_size, group_size, chunk_q, chunk_k, blocks_per_chunk, q_chunk_offset;
  int32_t q_half, k_half, ex_win, ex_sink, causal, tf_mask, prog_excl;
} orc_mask;

/* q: [B, MG, H, D] f32, k: [B, NC, H, D] f32 (exact images of the input elements), contiguous.
 * scores: [B, MG, H, NC]. */
void orc_scores(const float* q, const float* k, int64_t B, int64_t MG, int64_t H, int64_t NC,
                int64_t D, float scale, float* scores) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t g = 0; g < MG; ++g)
      for (int64_t h = 0; h < H; ++h) {
        const float* qr = q + ((b * MG + g) * H + h) * D;
        float* out = scores + ((b * MG + g) * H + h) * NC;
        for (int64_t c = 0; c < NC; ++c) {
          const float* kr = k + ((b * NC + c) * H + h) * D;
          float acc = 0.0f;
          for (int64_t d = 0; d < D; ++d) acc = fmaf(qr[d], kr[d], acc);
          out[c] = acc * scale;
        }
      }
}

static int orc_visible(const orc_mask* m, int64_t g, int64_t c) {
  const int q_cid = (int)((g * (int64_t)m->group_size) / m->chunk_q) + m->q_chunk_offset;
  int q_clean = 1, q_rel = q_cid;
  if (m->tf_mask) {
    q_clean = q_cid < m->q_half;
    q_rel = q_clean ? q_cid : q_cid - m->q_half;
  }
  const int do_excl = m->prog_excl ? (q_rel >= m->ex_sink + m->ex_win) : 1;
  const int k_cid = m->blocks_per_chunk > 0 ? (int)(c / m->blocks_per_chunk)
                                            : (int)((c * (int64_t)m->block_size) / m->chunk_k);
  const int k_clean = m->tf_mask ? (k_cid < m->k_half) : 1;
  const int k_rel = (m->tf_mask && !k_clean) ? k_cid - m->k_half : k_cid;
  int ok;
  if (m->tf_mask) {
    ok = (q_clean && k_clean && k_rel <= q_rel) || (!q_clean && k_clean && k_rel < q_rel) ||
         (!q_clean && !k_clean && k_rel == q_rel);
  } else {
    ok = m->causal ? (k_cid <= q_cid) : 1;
  }
  if (m->ex_sink > 0) ok = ok && ((!k_clean || k_rel >= m->ex_sink) || !do_excl);
  if (m->ex_win > 0) {
    int in_win;
    if (m->tf_mask) {
      in_win = k_clean && k_rel >= q_rel - m->ex_win + 1;
    } else {
      in_win = k_cid >= q_cid - m->ex_win + 1;
      if (!m->causal) in_win = in_win && k_cid <= q_cid + m->ex_win - 1;
    }
    ok = ok && (!in_win || !do_excl);
  }
  return ok;
}

/* visible: [MG, NC] uint8 for one (b, h) -- the rule does not depend on b or h. */
void orc_visible_matrix(const orc_mask* m, int64_t MG, int64_t NC, uint8_t* out) {
  for (int64_t g = 0; g < MG; ++g)
    for (int64_t c = 0; c < NC; ++c) out[g * NC + c] = (uint8_t)orc_visible(m, g, c);
}

typedef struct {
  float s;
  int32_t id;
} cand;

static int cand_cmp(const void* a, const void* b) {
  const cand* x = (const cand*)a;
  const cand* y = (const cand*)b;
  if (x->s > y->s) return -1; /* -0.0f == +0.0f under these comparisons */
  if (x->s < y->s) return 1;
  return (x->id < y->id) ? -1 : (x->id > y->id);
}

/* scores: [B, MG, H, NC] (already scaled); out: [B, MG, H, topk]. */
void orc_topk(const float* scores, int64_t B, int64_t MG, int64_t H, int64_t NC, int32_t topk,
              const orc_mask* m, int32_t* out) {
  cand* buf = (cand*)malloc(sizeof(cand) * (size_t)(NC > 0 ? NC : 1));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t g = 0; g < MG; ++g)
      for (int64_t h = 0; h < H; ++h) {
        const float* row = scores + ((b * MG + g) * H + h) * NC;
        int32_t* o = out + ((b * MG + g) * H + h) * topk;
        int64_t n = 0;
        for (int64_t c = 0; c < NC; ++c) {
          const float s = row[c];
          if (!(s > -INFINITY)) continue; /* -inf and NaN are never selected */
          if (!orc_visible(m, g, c)) continue;
          buf[n].s = s;
          buf[n].id = (int32_t)c;
          ++n;
        }
        qsort(buf, (size_t)n, sizeof(cand), cand_cmp);
        for (int32_t i = 0; i < topk; ++i) o[i] = (i < n) ? buf[i].id : -1;
      }
  free(buf);
}
