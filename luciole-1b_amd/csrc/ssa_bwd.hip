// SSA attention backward for gfx950: Delta preprocess, dK/dV (+ dn/db
// partials), dQ, and the fixed-order dn/db reduction.
//
// Replaces _ssa_attn_bwd_preprocess, _ssa_attn_bwd_dkdv, _ssa_attn_bwd_dq and
// _ssa_attn_bwd (training/train/train_ssa_triton/SSA/ssa_triton_kernel.py:
// 267-298, 305-401, 408-481, 488-719) and the dn_partial/db_partial sums
// (:894-895).  As in the reference, dQ is produced by its own pass with the
// scores recomputed, so no floating-point atomics are needed anywhere and the
// results are bitwise reproducible.
//
// Per valid (query i, key j), with s = scale * q_i.k_j, u = b|s|,
// sL = sign(s) log2(1+u) and M_i the base-2 normaliser saved by the forward:
//   P   = exp2(n sL - M_i)
//   dT  = P (dP - Delta_i)              dP = dO_i . v_j
//   dS' = dT / (1 + u)                  (dS = n b dS')
//   dV_j += P dO_i,  dK_j += scale n b dS' q_i,  dQ_i += scale n b dS' k_j
//   dn  += ln2 * dT sL,  db += n scale dS' (q_i.k_j)
// The constant factors (scale n b, ln2, n scale) are applied once at the end.
#include "ssa_common.hpp"
#include "ssa_launch.hpp"

namespace ssa {

// ---------------------------------------------------------------------------
// Delta_i = sum_d O_id dO_id (fp32).  HBM-bound: one 16-byte load of O and dO
// per lane, D/8 lanes per row, butterfly reduction inside the row group.
template <typename T, int D>
__global__ __launch_bounds__(256) void ssa_bwd_preprocess_kernel(BwdParams p) {
  constexpr int LPR = D / 8;         // lanes per row
  constexpr int RPB = 256 / LPR;     // rows per block
  typedef typename Vec8<T>::type v8;
  const int tid = threadIdx.x;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + tid / LPR;
  const int sub = tid % LPR;
  const int64_t total = static_cast<int64_t>(p.B) * p.Hq * p.N;
  float acc = 0.f;
  if (row < total) {
    const int s = static_cast<int>(row % p.N);
    const int64_t bh = row / p.N;
    const int h = static_cast<int>(bh % p.Hq), b = static_cast<int>(bh / p.Hq);
    const T* o = static_cast<const T*>(p.o.ptr) + b * p.o.sb + h * p.o.sh + s * p.o.ss + sub * 8;
    const T* g = static_cast<const T*>(p.dout.ptr) + b * p.dout.sb + h * p.dout.sh + s * p.dout.ss + sub * 8;
    const v8 ov = load16<v8>(o), gv = load16<v8>(g);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(static_cast<float>(ov[e]), static_cast<float>(gv[e]), acc);
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < total && sub == 0) p.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// dK, dV for a block of 128 keys (32 per wave) of one (batch, kv-head), looping
// over every q-head of the GQA group and every 32-query tile at or after the
// keys (causal).  S = Q K^T is computed with the keys on the lane axis, so
// P^T and dS'^T come out of the accumulators already in A-operand order for
// dV += P^T dO and dK += dS'^T Q.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void ssa_bwd_dkdv_kernel(BwdParams p) {
  constexpr int BN = 128, BMQ = 32, LDSD = D + 8;
  constexpr int ND16 = D / 16, ND32 = D / 32;
  constexpr int CH_PER_ROW = D / 8;
  constexpr int CH = BMQ * CH_PER_ROW;
  typedef typename Vec8<T>::type v8;

  __shared__ __attribute__((aligned(16))) T q_lds[BMQ * LDSD];
  __shared__ __attribute__((aligned(16))) T do_lds[BMQ * LDSD];
  __shared__ float m_lds[BMQ], dl_lds[BMQ];
  __shared__ float red[2][4];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hh = lane >> 5;
  const int N = p.N;
  const int nkb = dkdv_key_blocks(N);
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int bhk = L / nkb;
  const int kb = L % nkb;  // ascending = heaviest first under causal
  const int b = bhk / p.Hkv, hk = bhk % p.Hkv;
  const int G = p.Hq / p.Hkv;

  const float n = *p.n_ptr;
  const float c = p.scale * *p.b_ptr;

  const int k0w = kb * BN + wave * 32;
  const int key = k0w + l32;
  const T* kg = static_cast<const T*>(p.k.ptr) + b * p.k.sb + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + b * p.v.sb + hk * p.v.sh;

  v8 kf[ND16], vf[ND16];
#pragma unroll
  for (int ds = 0; ds < ND16; ++ds) {
    kf[ds] = key < N ? load16<v8>(kg + key * p.k.ss + ds * 16 + 8 * hh) : zero8<v8>();
    vf[ds] = key < N ? load16<v8>(vg + key * p.v.ss + ds * 16 + 8 * hh) : zero8<v8>();
  }

  f32x16 dk[ND32], dv[ND32];
#pragma unroll
  for (int i = 0; i < ND32; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }
  float dn_acc = 0.f, dn_c = 0.f, db_acc = 0.f, db_c = 0.f;

  for (int g = 0; g < G; ++g) {
    const int hq = hk * G + g;
    const T* qg = static_cast<const T*>(p.q.ptr) + b * p.q.sb + hq * p.q.sh;
    const T* dog = static_cast<const T*>(p.dout.ptr) + b * p.dout.sb + hq * p.dout.sh;
    const float* mg = p.m + (static_cast<int64_t>(b) * p.Hq + hq) * N;
    const float* dlg = p.delta + (static_cast<int64_t>(b) * p.Hq + hq) * N;
    const int qstart = CAUSAL ? kb * BN : 0;
    for (int q0 = qstart; q0 < N; q0 += BMQ) {
      __syncthreads();
      for (int ch = tid; ch < CH; ch += 256) {
        const int row = ch / CH_PER_ROW, col = (ch % CH_PER_ROW) * 8;
        const int qi = q0 + row;
        u32x4 a = u32x4{0u, 0u, 0u, 0u}, d = u32x4{0u, 0u, 0u, 0u};
        if (qi < N) {
          a = *reinterpret_cast<const u32x4*>(qg + qi * p.q.ss + col);
          d = *reinterpret_cast<const u32x4*>(dog + qi * p.dout.ss + col);
        }
        *reinterpret_cast<u32x4*>(&q_lds[row * LDSD + col]) = a;
        *reinterpret_cast<u32x4*>(&do_lds[row * LDSD + col]) = d;
      }
      if (tid < BMQ) {
        const int qi = q0 + tid;
        m_lds[tid] = qi < N ? mg[qi] : 0.f;
        dl_lds[tid] = qi < N ? dlg[qi] : 0.f;
      }
      __syncthreads();
      if (k0w >= N) continue;
      if (CAUSAL && q0 + BMQ - 1 < k0w) continue;

      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int ds = 0; ds < ND16; ++ds) {
        const v8 qa = load16<v8>(&q_lds[l32 * LDSD + ds * 16 + 8 * hh]);
        const v8 da = load16<v8>(&do_lds[l32 * LDSD + ds * 16 + 8 * hh]);
        s = mfma32(qa, kf[ds], s);
        dp = mfma32(da, vf[ds], dp);
      }

      v8 pa[2], sa[2];
      float tdn = 0.f, tdb = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qo = crow(r, hh);
        const int qi = q0 + qo;
        const bool valid = qi < N && key < N && (!CAUSAL || key <= qi);
        const float x = s[r];
        const float u1 = fmaf(c, fabsf(x), 1.f);
        const float sl = copysignf(fast_log2(u1), x);
        const float pv = valid ? fast_exp2(fmaf(n, sl, -m_lds[qo])) : 0.f;
        const float dt = pv * (dp[r] - dl_lds[qo]);
        const float dsp = dt * fast_rcp(u1);
        tdn = fmaf(dt, sl, tdn);
        tdb = fmaf(dsp, x, tdb);
        pa[r >> 3][r & 7] = static_cast<T>(pv);
        sa[r >> 3][r & 7] = static_cast<T>(dsp);
      }
      {  // Kahan accumulation of the per-tile sums
        const float y = tdn - dn_c, t = dn_acc + y;
        dn_c = (t - dn_acc) - y;
        dn_acc = t;
        const float y2 = tdb - db_c, t2 = db_acc + y2;
        db_c = (t2 - db_acc) - y2;
        db_acc = t2;
      }

#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int db = 0; db < ND32; ++db) {
          v8 dob, qbv;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int qrow = ks * 16 + crow(e, hh);
            dob[e] = do_lds[qrow * LDSD + db * 32 + l32];
            qbv[e] = q_lds[qrow * LDSD + db * 32 + l32];
          }
          dv[db] = mfma32(pa[ks], dob, dv[db]);
          dk[db] = mfma32(sa[ks], qbv, dk[db]);
        }
      }
    }
  }

  // Store dK (scaled by scale * n * b) and dV: lane holds d = 32*db + l32,
  // key rows crow(r, hh) of this wave's 32 keys.
  const float kscale = p.scale * n * *p.b_ptr;
  T* dkg = static_cast<T*>(const_cast<void*>(p.dk.ptr)) + b * p.dk.sb + hk * p.dk.sh;
  T* dvg = static_cast<T*>(const_cast<void*>(p.dv.ptr)) + b * p.dv.sb + hk * p.dv.sh;
#pragma unroll
  for (int db = 0; db < ND32; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = k0w + crow(r, hh);
      if (kr < N) {
        dkg[kr * p.dk.ss + db * 32 + l32] = static_cast<T>(dk[db][r] * kscale);
        dvg[kr * p.dv.ss + db * 32 + l32] = static_cast<T>(dv[db][r]);
      }
    }
  }

  // dn / db partial of this workgroup: lane butterfly, then waves in order.
  float pdn = dn_acc - dn_c, pdb = db_acc - db_c;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    pdn += __shfl_xor(pdn, off, 64);
    pdb += __shfl_xor(pdb, off, 64);
  }
  if (lane == 0) {
    red[0][wave] = pdn;
    red[1][wave] = pdb;
  }
  __syncthreads();
  if (tid == 0) {
    const int64_t P = static_cast<int64_t>(p.B) * p.Hkv * nkb;
    const float sdn = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    const float sdb = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    p.partials[static_cast<int64_t>(bhk) * nkb + kb] = kLn2 * sdn;
    p.partials[P + static_cast<int64_t>(bhk) * nkb + kb] = n * p.scale * sdb;
  }
}

// ---------------------------------------------------------------------------
// dQ for 128 query rows (32 per wave) of one (batch, q-head): the forward's
// transposed layout (query on the lane axis), K/V tiles of 64 keys in LDS,
// dQ^T += K^T dS'^T with K^T gathered from the K tile.
template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(256) void ssa_bwd_dq_kernel(BwdParams p) {
  constexpr int BM = 128, BN = 64, LDSD = D + 8;
  constexpr int ND16 = D / 16, ND32 = D / 32;
  constexpr int CH_PER_ROW = D / 8;
  constexpr int CH_PER_T = BN * CH_PER_ROW / 256;
  typedef typename Vec8<T>::type v8;

  __shared__ __attribute__((aligned(16))) T k_lds[BN * LDSD];
  __shared__ __attribute__((aligned(16))) T v_lds[BN * LDSD];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hh = lane >> 5;
  const int N = p.N;
  const int nqb = (N + BM - 1) / BM;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = L / nqb;
  const int qb = nqb - 1 - (L % nqb);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / (p.Hq / p.Hkv);

  const T* qg = static_cast<const T*>(p.q.ptr) + b * p.q.sb + h * p.q.sh;
  const T* dog = static_cast<const T*>(p.dout.ptr) + b * p.dout.sb + h * p.dout.sh;
  const T* kg = static_cast<const T*>(p.k.ptr) + b * p.k.sb + hk * p.k.sh;
  const T* vg = static_cast<const T*>(p.v.ptr) + b * p.v.sb + hk * p.v.sh;

  const float n = *p.n_ptr;
  const float c = p.scale * *p.b_ptr;
  const int q0 = qb * BM;
  const int wq0 = q0 + wave * 32;
  const int qrow = wq0 + l32;

  v8 qf[ND16], dof[ND16];
#pragma unroll
  for (int ds = 0; ds < ND16; ++ds) {
    qf[ds] = qrow < N ? load16<v8>(qg + qrow * p.q.ss + ds * 16 + 8 * hh) : zero8<v8>();
    dof[ds] = qrow < N ? load16<v8>(dog + qrow * p.dout.ss + ds * 16 + 8 * hh) : zero8<v8>();
  }
  const int64_t rowbase = static_cast<int64_t>(bh) * N;
  const float mq = qrow < N ? p.m[rowbase + qrow] : 0.f;
  const float dlq = qrow < N ? p.delta[rowbase + qrow] : 0.f;

  f32x16 dq[ND32];
#pragma unroll
  for (int i = 0; i < ND32; ++i) dq[i] = f32x16{};

  const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
  const int ntiles = (kv_end + BN - 1) / BN;

  u32x4 kreg[CH_PER_T], vreg[CH_PER_T];
  auto gload = [&](int tile) {
#pragma unroll
    for (int i = 0; i < CH_PER_T; ++i) {
      const int ch = tid + i * 256;
      const int row = ch / CH_PER_ROW, col = (ch % CH_PER_ROW) * 8;
      const int kk = tile * BN + row;
      if (kk < N) {
        kreg[i] = *reinterpret_cast<const u32x4*>(kg + kk * p.k.ss + col);
        vreg[i] = *reinterpret_cast<const u32x4*>(vg + kk * p.v.ss + col);
      } else {
        kreg[i] = u32x4{0u, 0u, 0u, 0u};
        vreg[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  gload(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CH_PER_T; ++i) {
      const int ch = tid + i * 256;
      const int row = ch / CH_PER_ROW, col = (ch % CH_PER_ROW) * 8;
      *reinterpret_cast<u32x4*>(&k_lds[row * LDSD + col]) = kreg[i];
      *reinterpret_cast<u32x4*>(&v_lds[row * LDSD + col]) = vreg[i];
    }
    __syncthreads();
    if (t + 1 < ntiles) gload(t + 1);

    const int kbase = t * BN;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kstart = kbase + kb * 32;
      if (kstart >= N || (CAUSAL && kstart > wq0 + 31)) continue;
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int ds = 0; ds < ND16; ++ds) {
        const v8 ka = load16<v8>(&k_lds[(kb * 32 + l32) * LDSD + ds * 16 + 8 * hh]);
        const v8 va = load16<v8>(&v_lds[(kb * 32 + l32) * LDSD + ds * 16 + 8 * hh]);
        s = mfma32(ka, qf[ds], s);
        dp = mfma32(va, dof[ds], dp);
      }
      v8 sb[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = kstart + crow(r, hh);
        const bool valid = qrow < N && kk < N && (!CAUSAL || kk <= qrow);
        const float x = s[r];
        const float u1 = fmaf(c, fabsf(x), 1.f);
        const float sl = copysignf(fast_log2(u1), x);
        const float pv = valid ? fast_exp2(fmaf(n, sl, -mq)) : 0.f;
        const float dsp = pv * (dp[r] - dlq) * fast_rcp(u1);
        sb[r >> 3][r & 7] = static_cast<T>(dsp);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int db = 0; db < ND32; ++db) {
          v8 ka;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int krow = kb * 32 + ks * 16 + crow(e, hh);
            ka[e] = k_lds[krow * LDSD + db * 32 + l32];
          }
          dq[db] = mfma32(ka, sb[ks], dq[db]);
        }
      }
    }
  }

  const float qscale = p.scale * n * *p.b_ptr;
  if (qrow < N) {
    T* dqg = static_cast<T*>(const_cast<void*>(p.dq.ptr)) + b * p.dq.sb + h * p.dq.sh + qrow * p.dq.ss;
#pragma unroll
    for (int db = 0; db < ND32; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = static_cast<T>(dq[db][4 * g + e] * qscale);
        *reinterpret_cast<t4*>(dqg + db * 32 + g * 8 + 4 * hh) = o4;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dn, db = fixed-order sums of the per-workgroup partials (one workgroup).
__global__ __launch_bounds__(256) void ssa_reduce_partials_kernel(const float* partials, int64_t count,
                                                                  float* dn, float* db) {
  __shared__ float sh[2][256];
  const int tid = threadIdx.x;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const float* src = partials + w * count;
    float acc = 0.f, comp = 0.f;
    for (int64_t i = tid; i < count; i += 256) {
      const float y = src[i] - comp, t = acc + y;
      comp = (t - acc) - y;
      acc = t;
    }
    sh[w][tid] = acc;
  }
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (tid < stride) {
      sh[0][tid] += sh[0][tid + stride];
      sh[1][tid] += sh[1][tid + stride];
    }
    __syncthreads();
  }
  if (tid == 0) {
    *dn = sh[0][0];
    *db = sh[1][0];
  }
}

// ---------------------------------------------------------------------------
template <typename T>
static hipError_t pre_dt(const BwdParams& p, int D, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.N;
  const int rpb = 256 / (D / 8);
  const int grid = static_cast<int>((rows + rpb - 1) / rpb);
  switch (D) {
    case 32: hipLaunchKernelGGL((ssa_bwd_preprocess_kernel<T, 32>), dim3(grid), dim3(256), 0, s, p); break;
    case 64: hipLaunchKernelGGL((ssa_bwd_preprocess_kernel<T, 64>), dim3(grid), dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL((ssa_bwd_preprocess_kernel<T, 128>), dim3(grid), dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_preprocess(const BwdParams& p, int dtype, int D, hipStream_t s) {
  return dtype == 0 ? pre_dt<__bf16>(p, D, s) : pre_dt<_Float16>(p, D, s);
}

template <typename T, int D, bool CAUSAL>
static hipError_t dkdv_t(const BwdParams& p, hipStream_t s) {
  const int grid = dkdv_key_blocks(p.N) * p.B * p.Hkv;
  hipLaunchKernelGGL((ssa_bwd_dkdv_kernel<T, D, CAUSAL>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int D, bool CAUSAL>
static hipError_t dq_t(const BwdParams& p, hipStream_t s) {
  const int grid = ((p.N + 127) / 128) * p.B * p.Hq;
  hipLaunchKernelGGL((ssa_bwd_dq_kernel<T, D, CAUSAL>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

#define SSA_DISPATCH(FN, T, D, CAUSAL, P, S)                        \
  switch (D) {                                                      \
    case 32: return CAUSAL ? FN<T, 32, true>(P, S) : FN<T, 32, false>(P, S);    \
    case 64: return CAUSAL ? FN<T, 64, true>(P, S) : FN<T, 64, false>(P, S);    \
    case 128: return CAUSAL ? FN<T, 128, true>(P, S) : FN<T, 128, false>(P, S); \
    default: return hipErrorInvalidValue;                           \
  }

hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  if (dtype == 0) {
    SSA_DISPATCH(dkdv_t, __bf16, D, causal, p, s)
  }
  SSA_DISPATCH(dkdv_t, _Float16, D, causal, p, s)
}

hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int D, bool causal, hipStream_t s) {
  if (dtype == 0) {
    SSA_DISPATCH(dq_t, __bf16, D, causal, p, s)
  }
  SSA_DISPATCH(dq_t, _Float16, D, causal, p, s)
}

hipError_t launch_reduce_partials(const BwdParams& p, hipStream_t s) {
  const int64_t count = static_cast<int64_t>(p.B) * p.Hkv * dkdv_key_blocks(p.N);
  hipLaunchKernelGGL(ssa_reduce_partials_kernel, dim3(1), dim3(256), 0, s,
                     static_cast<const float*>(p.partials), count, p.dn, p.db);
  return hipGetLastError();
}

}  // namespace ssa
