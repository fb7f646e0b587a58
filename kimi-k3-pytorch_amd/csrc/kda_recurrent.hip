// Exact token-by-token KDA recurrence on gfx950 (decode step and
// mode="recurrent").  Reference semantics: src/kda/recurrent.py:62-74
//   S <- diag(exp g_t) S ; r = S^T k_t ; e = v_t - r ; S <- S + beta_t k_t e^T ; o_t = S^T q_t
//
// One workgroup owns one (sequence, head, V-tile) state tile in registers for
// the whole sequence: the state is read from HBM once and written once, so a
// T = 1 decode step moves the algorithmic minimum of 2 * 4*K*V bytes per
// (sequence, head).  The output uses o = S'^T q = (decayed S)^T q + beta (k.q) e,
// so q, k and the decayed state are consumed in the same pass as the recall.
//
// Thread layout: tid = tk * TV + tv.  Thread (tk, tv) holds rows
// [tk*KPT, tk*KPT+KPT) and columns [tv*VPT, tv*VPT+VPT) of the tile.  With
// K = V = 128, KPT = 16, VPT = 4, TV = 32: a wave's 64 lanes read two 512-byte
// state rows per 128-bit load.  The reductions over K (S^T k, S^T q, k.q) go
// through LDS, double-buffered by token parity so one barrier per token
// suffices.
#include "kda_common.h"

namespace kda {

template <class IT, class ST>
struct RecArgs {
  const IT* q;
  const IT* k;
  const IT* v;
  const IT* g;
  const IT* beta;
  IT* out;
  const ST* s_in;
  ST* s_out;
  ST* s_hist;  // [T, N, H, K, V] or nullptr
  SeqDesc seq;
  int64_t N, H, K, V;
};

template <int N, class T>
struct alignas(sizeof(T) * N) VecN {
  T x[N];
};

template <class ST, int VPT, bool NT>
__device__ __forceinline__ void load_state_row(const ST* p, ST (&dst)[VPT]) {
  if constexpr (VPT * sizeof(ST) == 16 && NT) {
    typedef ST v_t __attribute__((ext_vector_type(VPT)));
    v_t x = __builtin_nontemporal_load(reinterpret_cast<const v_t*>(p));
#pragma unroll
    for (int j = 0; j < VPT; ++j) dst[j] = x[j];
  } else if constexpr (VPT * sizeof(ST) == 16) {
    VecN<VPT, ST> x = *reinterpret_cast<const VecN<VPT, ST>*>(p);
#pragma unroll
    for (int j = 0; j < VPT; ++j) dst[j] = x.x[j];
  } else {
#pragma unroll
    for (int j = 0; j < VPT; ++j) dst[j] = p[j];
  }
}

template <class ST, int VPT, bool NT>
__device__ __forceinline__ void store_state_row(ST* p, const ST (&src)[VPT]) {
  if constexpr (VPT * sizeof(ST) == 16 && NT) {
    typedef ST v_t __attribute__((ext_vector_type(VPT)));
    v_t x;
#pragma unroll
    for (int j = 0; j < VPT; ++j) x[j] = src[j];
    __builtin_nontemporal_store(x, reinterpret_cast<v_t*>(p));
  } else if constexpr (VPT * sizeof(ST) == 16) {
    VecN<VPT, ST> x;
#pragma unroll
    for (int j = 0; j < VPT; ++j) x.x[j] = src[j];
    *reinterpret_cast<VecN<VPT, ST>*>(p) = x;
  } else {
#pragma unroll
    for (int j = 0; j < VPT; ++j) p[j] = src[j];
  }
}

// FULL: K == TK*KPT and V % (TV*VPT) == 0, all accesses in range without checks.
template <class IT, class ST, int TK, int KPT, int TV, int VPT, bool FULL, bool NT>
__global__ __launch_bounds__(TK* TV) void recurrent_kernel(const RecArgs<IT, ST> a) {
  constexpr int VT = TV * VPT;
  __shared__ ST red_r[2][TK][VT];
  __shared__ ST red_o[2][TK][VT];
  __shared__ ST red_kq[2][TK];

  const int tid = threadIdx.x;
  const int tv = tid % TV;
  const int tk = tid / TV;
  const int64_t nvt = (a.V + VT - 1) / VT;
  const int64_t bid = blockIdx.x;
  const int64_t vt = bid % nvt;
  const int64_t h = (bid / nvt) % a.H;
  const int64_t s = bid / (nvt * a.H);
  const SeqRange sr = seq_range(a.seq, s);

  const int k0 = tk * KPT;
  const int64_t vcol0 = vt * VT + tv * VPT;
  const int64_t state_base = (s * a.H + h) * a.K * a.V;

  auto row_ok = [&](int i) -> bool { return FULL || (k0 + i) < a.K; };
  auto col_ok = [&](int j) -> bool { return FULL || (vcol0 + j) < a.V; };

  ST st[KPT][VPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    if (a.s_in != nullptr && row_ok(i)) {
      const ST* p = a.s_in + state_base + static_cast<int64_t>(k0 + i) * a.V + vcol0;
      if (FULL) {
        load_state_row<ST, VPT, NT>(p, st[i]);
      } else {
#pragma unroll
        for (int j = 0; j < VPT; ++j) st[i][j] = col_ok(j) ? p[j] : ST(0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VPT; ++j) st[i][j] = ST(0);
    }
  }

  for (int64_t t = 0; t < sr.span; ++t) {
    const int64_t tok = sr.start + t;
    const int64_t out_base = (tok * a.H + h) * a.V + vcol0;
    if (t < sr.valid) {
      const int buf = static_cast<int>(t & 1);
      const int64_t kbase = (tok * a.H + h) * a.K + k0;
      ST kk[KPT], qq[KPT], alpha[KPT];
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        if (row_ok(i)) {
          kk[i] = to_compute<ST>(a.k[kbase + i]);
          qq[i] = to_compute<ST>(a.q[kbase + i]);
          alpha[i] = fast_exp(to_compute<ST>(a.g[kbase + i]));
        } else {
          kk[i] = ST(0);
          qq[i] = ST(0);
          alpha[i] = ST(1);
        }
      }
      const ST bt = to_compute<ST>(a.beta[tok * a.H + h]);
      ST vv[VPT];
#pragma unroll
      for (int j = 0; j < VPT; ++j) vv[j] = col_ok(j) ? to_compute<ST>(a.v[out_base + j]) : ST(0);

      // decay, then partial recall S^T k and partial read S^T q over my rows
      ST pr[VPT], po[VPT];
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        pr[j] = ST(0);
        po[j] = ST(0);
      }
      ST kq = ST(0);
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        kq += kk[i] * qq[i];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
          st[i][j] *= alpha[i];
          pr[j] += st[i][j] * kk[i];
          po[j] += st[i][j] * qq[i];
        }
      }
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        red_r[buf][tk][tv * VPT + j] = pr[j];
        red_o[buf][tk][tv * VPT + j] = po[j];
      }
      if (tv == 0) red_kq[buf][tk] = kq;
      __syncthreads();
      ST r[VPT], o1[VPT];
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        r[j] = ST(0);
        o1[j] = ST(0);
      }
      ST kqs = ST(0);
#pragma unroll
      for (int u = 0; u < TK; ++u) {
        kqs += red_kq[buf][u];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
          r[j] += red_r[buf][u][tv * VPT + j];
          o1[j] += red_o[buf][u][tv * VPT + j];
        }
      }
      ST e[VPT];
#pragma unroll
      for (int j = 0; j < VPT; ++j) e[j] = vv[j] - r[j];
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const ST bk = bt * kk[i];
#pragma unroll
        for (int j = 0; j < VPT; ++j) st[i][j] += bk * e[j];
      }
      if (tk == 0) {
#pragma unroll
        for (int j = 0; j < VPT; ++j)
          if (col_ok(j)) a.out[out_base + j] = from_compute<IT>(o1[j] + bt * kqs * e[j]);
      }
    } else if (tk == 0) {
#pragma unroll
      for (int j = 0; j < VPT; ++j)
        if (col_ok(j)) a.out[out_base + j] = from_compute<IT>(ST(0));
    }
    if (a.s_hist != nullptr) {
      const int64_t hbase = ((t * a.N + s) * a.H + h) * a.K * a.V;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        if (!row_ok(i)) continue;
        ST* p = a.s_hist + hbase + static_cast<int64_t>(k0 + i) * a.V + vcol0;
#pragma unroll
        for (int j = 0; j < VPT; ++j)
          if (col_ok(j)) p[j] = st[i][j];
      }
    }
  }

  if (a.s_out != nullptr) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      if (!row_ok(i)) continue;
      ST* p = a.s_out + state_base + static_cast<int64_t>(k0 + i) * a.V + vcol0;
      if (FULL) {
        store_state_row<ST, VPT, NT>(p, st[i]);
      } else {
#pragma unroll
        for (int j = 0; j < VPT; ++j)
          if (col_ok(j)) p[j] = st[i][j];
      }
    }
  }
}

template <class IT, class ST, int TK, int KPT, int TV, int VPT, bool FULL, bool NT>
static int launch_cfg(const RecArgs<IT, ST>& a, hipStream_t stream) {
  constexpr int VT = TV * VPT;
  const int64_t nvt = (a.V + VT - 1) / VT;
  const int64_t blocks = a.N * a.H * nvt;
  if (blocks <= 0) return KDA_OK;
  if (blocks > 0x7fffffffLL) {
    kda_host::set_detail("recurrent: grid of %lld workgroups is too large", (long long)blocks);
    return KDA_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((recurrent_kernel<IT, ST, TK, KPT, TV, VPT, FULL, NT>), dim3(static_cast<unsigned>(blocks)),
                     dim3(TK * TV), 0, stream, a);
  return kda_host::check_launch("recurrent_kernel");
}

template <class IT, class ST>
static int dispatch(const RecArgs<IT, ST>& a, hipStream_t stream, bool streaming_state) {
  if constexpr (sizeof(ST) == 4) {
    if (a.K == 128 && a.V % 128 == 0) {
      if (streaming_state) return launch_cfg<IT, ST, 8, 16, 32, 4, true, true>(a, stream);
      return launch_cfg<IT, ST, 8, 16, 32, 4, true, false>(a, stream);
    }
  }
  if (a.K <= 32) return launch_cfg<IT, ST, 16, 2, 16, 1, false, false>(a, stream);
  if (a.K <= 128) return launch_cfg<IT, ST, 16, 8, 16, 1, false, false>(a, stream);
  if (a.K <= 256) return launch_cfg<IT, ST, 16, 16, 16, 1, false, false>(a, stream);
  kda_host::set_detail("recurrent: key_dim %lld > 256 is not supported", (long long)a.K);
  return KDA_ERR_UNSUPPORTED;
}

template <class IT, class ST>
static int run_typed(const void* q, const void* k, const void* v, const void* g, const void* beta,
                     const void* s_in, void* s_out, void* out, void* s_hist, const SeqDesc& seq,
                     int64_t N, int64_t H, int64_t K, int64_t V, hipStream_t stream, bool streaming_state) {
  RecArgs<IT, ST> a;
  a.q = static_cast<const IT*>(q);
  a.k = static_cast<const IT*>(k);
  a.v = static_cast<const IT*>(v);
  a.g = static_cast<const IT*>(g);
  a.beta = static_cast<const IT*>(beta);
  a.out = static_cast<IT*>(out);
  a.s_in = static_cast<const ST*>(s_in);
  a.s_out = static_cast<ST*>(s_out);
  a.s_hist = static_cast<ST*>(s_hist);
  a.seq = seq;
  a.N = N;
  a.H = H;
  a.K = K;
  a.V = V;
  return dispatch<IT, ST>(a, stream, streaming_state);
}

}  // namespace kda

namespace kda_host {

int launch_recurrent(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                     const void* s_in, void* s_out, int state_dtype, void* out, void* s_hist,
                     const kda::SeqDesc& seq, int64_t N, int64_t H, int64_t K, int64_t V, hipStream_t stream,
                     bool streaming_state) {
  using namespace kda;
  if (state_dtype == KDA_DTYPE_F64) {
    if (in_dtype != KDA_DTYPE_F64) {
      set_detail("f64 state requires f64 inputs");
      return KDA_ERR_INVALID_ARGUMENT;
    }
    return run_typed<double, double>(q, k, v, g, beta, s_in, s_out, out, s_hist, seq, N, H, K, V, stream, false);
  }
  if (state_dtype != KDA_DTYPE_F32) {
    set_detail("state dtype must be f32 or f64");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  switch (in_dtype) {
    case KDA_DTYPE_BF16:
      return run_typed<bf16, float>(q, k, v, g, beta, s_in, s_out, out, s_hist, seq, N, H, K, V, stream,
                                    streaming_state);
    case KDA_DTYPE_F16:
      return run_typed<f16, float>(q, k, v, g, beta, s_in, s_out, out, s_hist, seq, N, H, K, V, stream,
                                   streaming_state);
    case KDA_DTYPE_F32:
      return run_typed<float, float>(q, k, v, g, beta, s_in, s_out, out, s_hist, seq, N, H, K, V, stream,
                                     streaming_state);
    default:
      set_detail("f32 state requires bf16, f16 or f32 inputs");
      return KDA_ERR_INVALID_ARGUMENT;
  }
}

}  // namespace kda_host
