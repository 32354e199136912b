// Exact recompute of the MFMA backward's non-finite units (gfx950).
//
// The MFMA backward kernels (block-sparse and band-gathered, dQ and dK / dV)
// stage whole key blocks, bands or row slots: a pair (row, key) that the
// row's entries do not list still meets the staged operands with a zero
// coefficient, and 0 * Inf is NaN.  So an Inf or NaN in K, V, Q or dO can
// reach outputs that the reference's gather never lets it reach
// (elastic_sparse_attention.py:189-228 reads only the listed K / V rows and
// adds dK / dV only at listed keys, :211-213, :226-228).  Each MFMA kernel
// writes a flag per unit it stores (a 16-row dQ group, a 16-key dK / dV
// block): 1 when the unit holds a non-finite value.  bwd_fix_kernel scans
// the flags (one wave per 64, leaving at once when none is set) and
// recomputes each flagged unit in float32 on the reference's pairs:
//
//   dQ row r:  per entry j (lane j) with key k_j listed (k_j <= r):
//              s = q . k_j * scale, p = exp(s - lse), dp = dO . v_j,
//              dS = p (dp - delta) * scale; dQ = sum_j dS_j k_j.  A row
//              with a non-finite delta and an entry that is not listed gets
//              NaN throughout: the reference scores that entry against zero
//              K / V rows and adds (0 * (0 - delta)) * 0 (:202-221).
//   dK, dV of key u: per query head of u's kv group and entry j, the rows
//              whose entry j is u form one range (entry j's key never
//              decreases along the rows), found by binary search from row
//              u; each row adds dV += p dO, dK += dS q.
//
// Finite units stay as the MFMA kernels stored them; a flagged unit's
// non-finite positions and kinds are those of the per-row gather backward.
#include "esa_gather.hpp"
#include "esa_tile.hpp"

namespace esa {

namespace {

constexpr int kFixWaves = 4;

template <Elem E>
__device__ void fix_dq_group(const BwdArgs& A, int D, int unit, float* qs, float* dos,
                             float* dsl, int* ksl, int lane) {
  using T = uint16_t;
  const int bh = unit / A.ng, gq = unit % A.ng;
  const int h = bh % A.H, b = bh / A.H;
  const int kvh = h / A.groups;
  IndexSource S{};
  S.w = A.pc.w;
  S.kv_len = A.kv_len;
  S.pc = A.pc;
  const T* kbase = A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh;
  const T* vbase = A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh;
  const int w = S.w;
  const int r1 = min(gq * 16 + 16, A.q_len);
  for (int r = gq * 16; r < r1; ++r) {
    const T* qrow = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
    const T* dorow = A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + (int64_t)r * A.doss;
    for (int d = lane; d < D; d += 64) {
      qs[d] = ElemT<E>::load(qrow + d);
      dos[d] = ElemT<E>::load(dorow + d);
    }
    wave_sync_lds();
    const float delta = A.delta[((int64_t)b * A.H + h) * A.qpad + r];
    const float lse = A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r];
    RowEntries row;
    row.init<true>(S, h, r);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    bool dead = false;
    for (int c0 = 0; c0 < w; c0 += 64) {
      const int j = c0 + lane;
      bool valid = false;
      int64_t key = 0;
      if (j < w) row.entry<true>(S, h, r, j, valid, key);
      dead |= j < w && !valid;
      float dsc = 0.f;
      if (valid) {
        const float s = row_dot<E>(qs, kbase + key * A.kss, D) * A.sm_scale;
        const float dp = row_dot<E>(dos, vbase + key * A.vss, D);
        dsc = expf(s - lse) * (dp - delta) * A.sm_scale;
      }
      dsl[lane] = dsc;
      ksl[lane] = valid ? (int)key : -1;
      wave_sync_lds();
      const int nj = min(64, w - c0);
      for (int jj = 0; jj < nj; ++jj) {
        const int kj = ksl[jj];
        if (kj < 0) continue;
        const float g = dsl[jj];
        const T* kr = kbase + (int64_t)kj * A.kss;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = lane + 64 * e;
          if (d < D) acc[e] += g * ElemT<E>::load(kr + d);
        }
      }
      wave_sync_lds();
    }
    const bool all_nan = wave_any(dead) && !__builtin_isfinite(delta);
    T* dqrow = A.dq + (int64_t)b * A.dqsb + (int64_t)h * A.dqsh + (int64_t)r * A.dqss;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = lane + 64 * e;
      if (d < D) ElemT<E>::store(dqrow + d, all_nan ? __builtin_nanf("") : acc[e]);
    }
  }
}

// key of entry j of row i for heads with weights hw (a listed entry's key
// never exceeds the row; rows here are >= the key sought)
__device__ __forceinline__ int entry_key(const PatternConsts& pc, const HeadWeights& hw, int i,
                                         int j, int kv_len) {
  const RowParams rp = row_params(pc, i);
  const int idx = interp_index(oversized(rp, j), oversized(rp, j + 1), hw);
  return idx > kv_len - 1 ? kv_len - 1 : idx;
}

template <Elem E>
__device__ void fix_dkdv_block(const BwdArgs& A, int D, int unit, int* ra, int* rc, int lane) {
  using T = uint16_t;
  const int bkv = unit / A.nkb16, kb = unit % A.nkb16;
  const int kvh = bkv % A.Hkv, b = bkv / A.Hkv;
  const int w = A.pc.w;
  const int u1 = min(kb * 16 + 16, A.kv_len);
  for (int u = kb * 16; u < u1; ++u) {
    const T* krow = A.k + (int64_t)b * A.ksb + (int64_t)kvh * A.ksh + (int64_t)u * A.kss;
    const T* vrow = A.v + (int64_t)b * A.vsb + (int64_t)kvh * A.vsh + (int64_t)u * A.vss;
    float kv[4], vv[4], dk[4] = {0.f, 0.f, 0.f, 0.f}, dv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = lane + 64 * e;
      kv[e] = d < D ? ElemT<E>::load(krow + d) : 0.f;
      vv[e] = d < D ? ElemT<E>::load(vrow + d) : 0.f;
    }
    for (int hg = 0; hg < A.groups; ++hg) {
      const int h = kvh * A.groups + hg;
      const HeadWeights hw = head_weights(A.pc, h);
      for (int c0 = 0; c0 < w; c0 += 64) {
        const int j = c0 + lane;
        int a0 = u, c = u;
        if (j < w) {
          int a1 = A.q_len;  // first row >= u whose key of entry j is >= u
          while (a0 < a1) {
            const int mid = (a0 + a1) >> 1;
            if (entry_key(A.pc, hw, mid, j, A.kv_len) >= u) a1 = mid; else a0 = mid + 1;
          }
          c = a0;
          int c1 = A.q_len;  // first row whose key of entry j is > u
          while (c < c1) {
            const int mid = (c + c1) >> 1;
            if (entry_key(A.pc, hw, mid, j, A.kv_len) > u) c1 = mid; else c = mid + 1;
          }
        }
        ra[lane] = a0;
        rc[lane] = c;
        wave_sync_lds();
        const int nj = min(64, w - c0);
        for (int jj = 0; jj < nj; ++jj) {
          const int re = rc[jj];
          for (int r = ra[jj]; r < re; ++r) {
            const T* qrow = A.q + (int64_t)b * A.qsb + (int64_t)h * A.qsh + (int64_t)r * A.qss;
            const T* dorow =
                A.dout + (int64_t)b * A.dosb + (int64_t)h * A.dosh + (int64_t)r * A.doss;
            float qv[4], gv[4], sp = 0.f, dpp = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int d = lane + 64 * e;
              qv[e] = d < D ? ElemT<E>::load(qrow + d) : 0.f;
              gv[e] = d < D ? ElemT<E>::load(dorow + d) : 0.f;
              if (d < D) {
                sp += qv[e] * kv[e];
                dpp += gv[e] * vv[e];
              }
            }
            const float s = wave_sum(sp) * A.sm_scale;
            const float dp = wave_sum(dpp);
            const float lse = A.lse[(int64_t)b * A.lsb + (int64_t)h * A.lsh + r];
            const float delta = A.delta[((int64_t)b * A.H + h) * A.qpad + r];
            const float p = expf(s - lse);
            const float ds = p * (dp - delta) * A.sm_scale;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              dv[e] += p * gv[e];
              dk[e] += ds * qv[e];
            }
          }
        }
        wave_sync_lds();
      }
    }
    T* dkrow = A.dk + (int64_t)b * A.dksb + (int64_t)kvh * A.dksh + (int64_t)u * A.dkss;
    T* dvrow = A.dv + (int64_t)b * A.dvsb + (int64_t)kvh * A.dvsh + (int64_t)u * A.dvss;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = lane + 64 * e;
      if (d < D) {
        ElemT<E>::store(dkrow + d, dk[e]);
        ElemT<E>::store(dvrow + d, dv[e]);
      }
    }
  }
}

// One wave per 64 flags; the flagged units of the wave's 64, in order.
template <Elem E>
__global__ __launch_bounds__(64 * kFixWaves) void bwd_fix_kernel(BwdArgs A, int D) {
  __shared__ float qs_all[kFixWaves][256];
  __shared__ float dos_all[kFixWaves][256];
  __shared__ float ds_all[kFixWaves][64];
  __shared__ int ks_all[kFixWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t total = (int64_t)A.n_qflags + A.n_kvflags;
  const int64_t f0 = ((int64_t)blockIdx.x * kFixWaves + wave) * 64;
  const bool set = f0 + lane < total && A.flags[f0 + lane] != 0;
  uint64_t todo = __builtin_amdgcn_ballot_w64(set);
  while (todo) {
    const int t = __builtin_ctzll(todo);
    todo &= todo - 1;
    const int64_t unit = f0 + t;
    if (unit < A.n_qflags)
      fix_dq_group<E>(A, D, (int)unit, qs_all[wave], dos_all[wave], ds_all[wave], ks_all[wave],
                      lane);
    else
      fix_dkdv_block<E>(A, D, (int)(unit - A.n_qflags), (int*)ds_all[wave], ks_all[wave], lane);
  }
}

}  // namespace

hipError_t launch_bwd_fix(const BwdArgs& a, int head_dim, hipStream_t stream) {
  const int64_t total = (int64_t)a.n_qflags + a.n_kvflags;
  if (total <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((total + 64 * kFixWaves - 1) / (64 * kFixWaves));
  if (a.elem == (int)Elem::f16)
    bwd_fix_kernel<Elem::f16><<<grid, 64 * kFixWaves, 0, stream>>>(a, head_dim);
  else
    bwd_fix_kernel<Elem::bf16><<<grid, 64 * kFixWaves, 0, stream>>>(a, head_dim);
  return hipGetLastError();
}

}  // namespace esa
