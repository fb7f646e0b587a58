/*
 * Scalar float64 restatement of the KDA token recurrence — TEST
 * INFRASTRUCTURE ONLY (a second, independent implementation used to pin the
 * PyTorch oracle in oracle/kda_oracle.py; never linked into the product).
 *
 * Follows src/kda/recurrent.py:62-74 of pablo-reyes8/kimi-k3-pytorch:
 *   S <- diag(exp g_t) S ; e = v_t - S^T k_t ; S <- S + beta_t k_t e^T ; o_t = S^T q_t
 * Layouts: q,k,g [B,T,H,K]; v,out [B,T,H,V]; beta [B,T,H]; states [B,H,K,V].
 * `valid` (optional, [B]) gives the number of real tokens per row; padded
 * tokens output 0 and leave the state untouched (src/kda/utils.py:82-94).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

void kda_recurrent_ref(const double* q, const double* k, const double* v, const double* g, const double* beta,
                       const double* s0, const long* valid, double* out, double* s_final, long B, long T, long H,
                       long K, long V) {
  double* S = (double*)malloc(sizeof(double) * (size_t)(K * V));
  double* e = (double*)malloc(sizeof(double) * (size_t)V);
  for (long b = 0; b < B; ++b) {
    for (long h = 0; h < H; ++h) {
      const long sbase = (b * H + h) * K * V;
      for (long i = 0; i < K * V; ++i) S[i] = s0 ? s0[sbase + i] : 0.0;
      const long nvalid = valid ? valid[b] : T;
      for (long t = 0; t < T; ++t) {
        const long kb = ((b * T + t) * H + h) * K;
        const long vb = ((b * T + t) * H + h) * V;
        if (t >= nvalid) {
          for (long c = 0; c < V; ++c) out[vb + c] = 0.0;
          continue;
        }
        const double bt = beta[(b * T + t) * H + h];
        for (long r = 0; r < K; ++r) {
          const double a = exp(g[kb + r]);
          for (long c = 0; c < V; ++c) S[r * V + c] *= a;
        }
        for (long c = 0; c < V; ++c) {
          double rec = 0.0;
          for (long r = 0; r < K; ++r) rec += S[r * V + c] * k[kb + r];
          e[c] = v[vb + c] - rec;
        }
        for (long r = 0; r < K; ++r)
          for (long c = 0; c < V; ++c) S[r * V + c] += bt * k[kb + r] * e[c];
        for (long c = 0; c < V; ++c) {
          double o = 0.0;
          for (long r = 0; r < K; ++r) o += S[r * V + c] * q[kb + r];
          out[vb + c] = o;
        }
      }
      if (s_final) memcpy(s_final + sbase, S, sizeof(double) * (size_t)(K * V));
    }
  }
  free(S);
  free(e);
}
