// SIMT (no MFMA) masked-attention kernels: the forward and the three backward
// stages in float32 arithmetic, for
//   * float32 inputs, whose 1e-5 tolerance rules out 16-bit operands, at head
//     dimensions 64, 128 and 256;
//   * 16-bit inputs at head dimensions 256 and 512 (any d in (128, 512],
//     zero-padded by the host), which the MFMA kernels' register and LDS
//     tiling does not hold.
//   * 16-bit inputs at D = 64 and 128 under MATTN_PRECISE (callers whose
//     kernels are too sharp for float16 operands).
// Same maths and tile walk as the MFMA path (/root/reference/jaxmodules/
// attention.py:52-105 forward, :266-342 backward): per 32-key (or 32-query)
// sub-block an online softmax, P = exp2(scale_log2 S - lse) in the backward,
// dS = P (dP - delta), dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO.
// dP - delta is formed as dO . (V_k - O) (delta = dO . O): where one key
// dominates a row, V_k - O is small and exact to float32 rounding, while
// dO . V_k and dO . O are two large dot products whose roundings (2^-24 of
// |dO| |V|) would be all that is left of their difference.
// TPR threads share a row (query or key), each holding D / TPR head dims; a
// workgroup of 512 threads owns 512 / TPR rows of a 128-row map tile, so a
// tile takes 128 TPR / 512 workgroups (one for TPR = 4, two for TPR = 8 at
// D = 256, four for TPR = 16 at D = 512).
#include <type_traits>

#include "common.hpp"

namespace mattn {
namespace {

// float element access to tensors of float32 or a 16-bit Tag
template <class T>
struct Mem {
  static __device__ __forceinline__ float get(const void* p, int64_t i) { return ((const float*)p)[i]; }
  // 4 consecutive values (i a multiple of 4: 16-byte aligned)
  static __device__ __forceinline__ void get4(const void* p, int64_t i, float* x) {
    const f32x4 y = *(const f32x4*)((const float*)p + i);
    x[0] = y[0]; x[1] = y[1]; x[2] = y[2]; x[3] = y[3];
  }
  static __device__ __forceinline__ void put(void* p, int64_t i, float x) { ((float*)p)[i] = x; }
};
template <class Tag>
struct Mem16 {
  using E = Elt<Tag>;
  static __device__ __forceinline__ float get(const void* p, int64_t i) {
    return E::to_f32(((const uint16_t*)p)[i]);
  }
  // 4 consecutive values (i a multiple of 4: 8-byte aligned)
  static __device__ __forceinline__ void get4(const void* p, int64_t i, float* x) {
    const u32x2 y = *(const u32x2*)((const uint16_t*)p + i);
    x[0] = E::to_f32(y[0] & 0xffffu); x[1] = E::to_f32(y[0] >> 16);
    x[2] = E::to_f32(y[1] & 0xffffu); x[3] = E::to_f32(y[1] >> 16);
  }
  static __device__ __forceinline__ void put(void* p, int64_t i, float x) {
    ((uint16_t*)p)[i] = (uint16_t)(E::pack2(x, 0.f) & 0xffffu);  // round to nearest even
  }
};
template <>
struct Mem<bf16_tag> : Mem16<bf16_tag> {};
template <>
struct Mem<f16_tag> : Mem16<f16_tag> {};

// keys (forward, dQ) or queries (dK/dV) per sub-block: 32, or 16 at D = 512,
// where four [SB, D] float32 LDS tiles (the dK/dV kernel's Q, dO, O and O's
// low parts) must fit 160 KiB
template <int D>
constexpr int sub_block() { return D > 256 ? 16 : 32; }

// mask bits of sub-block sb (SB keys or queries) of a partial tile's 128-bit
// row (or column) at `row`, one bit per element (words [mask][64-half][row])
template <int SB>
__device__ __forceinline__ uint32_t sub_bits(const uint64_t* bits, int mask, int sb, int row) {
  const int first = sb * SB;
  return (uint32_t)(bits[((int64_t)mask * 2 + (first >> 6)) * TILE + row] >> (first & 63));
}

// sum over the TPR lanes of a row (consecutive lanes)
template <int TPR>
__device__ __forceinline__ float row_sum(float x) {
#pragma unroll
  for (int o = 1; o < TPR; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

// a + b = s + e exactly (Knuth's TwoSum)
__device__ __forceinline__ void two_sum(float a, float b, float& s, float& e) {
  s = a + b;
  const float z = s - a;
  e = (a - (s - z)) + (b - z);
}

// Score of a row pair, q . y over the TPR lanes of the row (DP elements each),
// as hi + lo.  With `comp` (MATTN_PRECISE) it is the compensated dot product
// Dot2 of Ogita, Rump and Oishi (SIAM J. Sci. Comput. 26(6), 2005): every
// product's rounding error (an FMA gives it exactly) and every addition's
// (TwoSum) are summed apart, so hi + lo carries the dot product to about twice
// float32's precision.  The scores of a kernel sharper than 1/sqrt(d) reach
// tens of units (base 2 after scaling), where float32's 2^-24 relative
// rounding alone moves the weights exp2(S - lse) by 1e-5; otherwise lo = 0.
template <int DP, int TPR>
__device__ __forceinline__ void score(const float* qv, const float* y, bool comp, float& hi, float& lo) {
  if (!comp) {
    float p = 0.f;
#pragma unroll
    for (int i = 0; i < DP; ++i) p = fmaf(qv[i], y[i], p);
    hi = row_sum<TPR>(p);
    lo = 0.f;
    return;
  }
  float s = 0.f, c = 0.f;
#pragma unroll
  for (int i = 0; i < DP; ++i) {
    const float pr = qv[i] * y[i];
    const float ep = fmaf(qv[i], y[i], -pr);
    float e;
    two_sum(s, pr, s, e);
    c += ep + e;
  }
#pragma unroll
  for (int o = 1; o < TPR; o <<= 1) {
    const float so = __shfl_xor(s, o), co = __shfl_xor(c, o);
    float e;
    two_sum(s, so, s, e);
    c += co + e;
  }
  hi = s;
  lo = c;
}

// rows [r0, r0 + SB) of a [rows, D] tensor slice (row stride rs) as floats in
// LDS; rows past n - 1 re-read row n - 1 (their scores are masked)
template <int D, class T, int SB = sub_block<D>()>
__device__ __forceinline__ void stage_rows(float* dst, const void* base, int64_t rs, int r0, int n) {
  for (int c = threadIdx.x; c < SB * D / 4; c += 512) {
    const int r = c / (D / 4), col = 4 * (c % (D / 4));
    Mem<T>::get4(base, (int64_t)min(r0 + r, n - 1) * rs + col, dst + r * D + col);
  }
}

// PREC (MATTN_PRECISE): compensated scores, O and the row sum accumulated in
// float64 (v_fma_f64 issues at the rate of the scalar float32 FMA on these
// CUs), and the residual keeps what the stored lse and O round off: the
// backward's dP - delta = dO . (V_k - O) then sees O to float64 accuracy,
// which a row dominated by one key needs (V_k - O is then a small fraction of
// |V|, and O's own float32 rounding a large part of it).
template <int D, int TPR, class IT, class OT, bool PREC>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void fwd_simt(KArgs a) {
  using acc_t = typename std::conditional<PREC, double, float>::type;
  constexpr int DP = D / TPR, RPW = 512 / TPR, SPLIT = TILE / RPW, SB = sub_block<D>();
  constexpr int ES = std::is_same<IT, float>::value ? 4 : 2;
  __shared__ __attribute__((aligned(16))) float Ks[SB * D];
  __shared__ __attribute__((aligned(16))) float Vs[SB * D];

  const int item = a.q_order[blockIdx.x / SPLIT];
  if (item < 0 || item >= a.B * a.Hq * a.nqt) return;  // idle slot (or an entry out of range)
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  const int tid = threadIdx.x, part = tid % TPR;
  const int row = (blockIdx.x % SPLIT) * RPW + tid / TPR;  // row within the tile
  const int q = qt * TILE + row;
  const int qc = min(q, a.Lq - 1);

  float qv[DP];
  acc_t ov[DP];
  const int64_t qo = (int64_t)b * a.qs[0] + (int64_t)qc * a.qs[1] + (int64_t)h * a.qs[2] + part * DP;
#pragma unroll
  for (int i = 0; i < DP; i += 4) {
    Mem<IT>::get4(a.q, qo + i, qv + i);
    ov[i] = ov[i + 1] = ov[i + 2] = ov[i + 3] = 0;
  }
  const char* kb = (const char*)a.k + ES * ((int64_t)b * a.ks[0] + (int64_t)hk * a.ks[2]);
  const char* vb = (const char*)a.v + ES * ((int64_t)b * a.vs[0] + (int64_t)hk * a.vs[2]);
  float m = NEG_INF;
  acc_t l = 0;

  for (int e = e0; e < e1; ++e) {
    const int kt = a.row_ent[2 * e], mask = a.row_ent[2 * e + 1];
    for (int sb = 0; sb < TILE / SB; ++sb) {
      const int key0 = kt * TILE + sb * SB;
      if (key0 >= a.Lk) break;
      __syncthreads();
      stage_rows<D, IT>(Ks, kb, a.ks[1], key0, a.Lk);
      stage_rows<D, IT>(Vs, vb, a.vs[1], key0, a.Lk);
      __syncthreads();
      uint32_t bits = 0xffffffffu;
      if (mask >= 0)
        bits = sub_bits<SB>(a.row_bits, mask, sb, row);
      float sc[SB], sl[SB];  // scores s (scaled: s * scale_log2 = sc + sl)
      float mx = NEG_INF;
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        float hi, lo;
        score<DP, TPR>(qv, Ks + j * D + part * DP, PREC, hi, lo);
        float x = hi * a.scale_log2;
        sl[j] = fmaf(hi, a.scale_log2, -x) + lo * a.scale_log2;  // rounding of x, and the low part
        if (!((bits >> j) & 1u)) x = NEG_INF;
        sc[j] = x;
        mx = fmaxf(mx, x);
      }
      const float mn = fmaxf(m, mx);
      const float mu = (mn == NEG_INF) ? 0.f : mn;
      const acc_t alpha = exp2f(m - mu);   // a power of two's neighbourhood: exact enough in float
      m = mn;
      l *= alpha;
#pragma unroll
      for (int i = 0; i < DP; ++i) ov[i] *= alpha;
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const acc_t p = exp2f((sc[j] - mu) + sl[j]);  // -inf + finite: 0 for masked keys
        l += p;
#pragma unroll
        for (int i = 0; i < DP; ++i) ov[i] = p * (acc_t)Vs[j * D + part * DP + i] + ov[i];
      }
    }
  }
  if (q >= a.Lq) return;
  const acc_t inv = l > 0 ? 1 / l : 0;
  const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + q;
  if (part == 0) {
    float lse = NEG_INF, lo = 0.f;
    if (l > 0) {
      if constexpr (PREC) {
        const double full = (double)m + log2((double)l);
        lse = (float)full;
        lo = (float)(full - (double)lse);
      } else {
        two_sum(m, log2f(l), lse, lo);
      }
    }
    a.lse[rs] = lse;
    if constexpr (PREC) a.lse_lo[rs] = lo;  // lse + lse_lo = m + log2 l (to ~2^-48)
  }
  const int64_t oo = (int64_t)b * a.os[0] + (int64_t)q * a.os[1] + (int64_t)h * a.os[2] + part * DP;
#pragma unroll
  for (int i = 0; i < DP; ++i) {
    const acc_t o = ov[i] * inv;
    Mem<OT>::put(a.out, oo + i, (float)o);
    if constexpr (PREC)  // what the stored O (in OT) leaves off
      a.o_lo[rs * D + part * DP + i] = (float)(o - (acc_t)Mem<OT>::get(a.out, oo + i));
  }
}

template <int D, int TPR, class IT, class OT, bool PREC>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void bwd_dq_simt(KArgs a) {
  constexpr int DP = D / TPR, RPW = 512 / TPR, SPLIT = TILE / RPW, SB = sub_block<D>();
  constexpr int ES = std::is_same<IT, float>::value ? 4 : 2;
  __shared__ __attribute__((aligned(16))) float Ks[SB * D];
  __shared__ __attribute__((aligned(16))) float Vs[SB * D];

  const int item = a.q_order[blockIdx.x / SPLIT];
  if (item < 0 || item >= a.B * a.Hq * a.nqt) return;  // idle slot (or an entry out of range)
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  const int tid = threadIdx.x, part = tid % TPR;
  const int row = (blockIdx.x % SPLIT) * RPW + tid / TPR;
  const int q = qt * TILE + row;
  const int qc = min(q, a.Lq - 1);

  float qv[DP], gv[DP], ov[DP], ol[DP], dq[DP];
  const int64_t qo = (int64_t)b * a.qs[0] + (int64_t)qc * a.qs[1] + (int64_t)h * a.qs[2] + part * DP;
  const int64_t go = (int64_t)b * a.dos[0] + (int64_t)qc * a.dos[1] + (int64_t)h * a.dos[2] + part * DP;
  const int64_t oo = (int64_t)b * a.os[0] + (int64_t)qc * a.os[1] + (int64_t)h * a.os[2] + part * DP;
  const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + qc;
#pragma unroll
  for (int i = 0; i < DP; i += 4) {
    Mem<IT>::get4(a.q, qo + i, qv + i);
    Mem<OT>::get4(a.dO, go + i, gv + i);
    Mem<OT>::get4(a.o, oo + i, ov + i);
    if constexpr (PREC) Mem<float>::get4(a.o_lo, rs * D + part * DP + i, ol + i);
    else ol[i] = ol[i + 1] = ol[i + 2] = ol[i + 3] = 0.f;
    dq[i] = dq[i + 1] = dq[i + 2] = dq[i + 3] = 0.f;
  }
  const float lse = a.lse[rs], lse_lo = PREC ? a.lse_lo[rs] : 0.f;
  const char* kb = (const char*)a.k + ES * ((int64_t)b * a.ks[0] + (int64_t)hk * a.ks[2]);
  const char* vb = (const char*)a.v + ES * ((int64_t)b * a.vs[0] + (int64_t)hk * a.vs[2]);

  for (int e = e0; e < e1; ++e) {
    const int kt = a.row_ent[2 * e], mask = a.row_ent[2 * e + 1];
    for (int sb = 0; sb < TILE / SB; ++sb) {
      const int key0 = kt * TILE + sb * SB;
      if (key0 >= a.Lk) break;
      __syncthreads();
      stage_rows<D, IT>(Ks, kb, a.ks[1], key0, a.Lk);
      stage_rows<D, IT>(Vs, vb, a.vs[1], key0, a.Lk);
      __syncthreads();
      uint32_t bits = 0xffffffffu;
      if (mask >= 0)
        bits = sub_bits<SB>(a.row_bits, mask, sb, row);
      for (int j = 0; j < SB; ++j) {
        float g = 0.f;
#pragma unroll
        for (int i = 0; i < DP; ++i) g = fmaf(gv[i], (Vs[j * D + part * DP + i] - ov[i]) - ol[i], g);  // dP - delta
        g = row_sum<TPR>(g);
        float hi, lo;
        score<DP, TPR>(qv, Ks + j * D + part * DP, PREC, hi, lo);
        float p = exp2f(fmaf(hi, a.scale_log2, -lse) + fmaf(lo, a.scale_log2, -lse_lo));
        if (!((bits >> j) & 1u)) p = 0.f;
        const float ds = p * g;
#pragma unroll
        for (int i = 0; i < DP; ++i) dq[i] = fmaf(ds, Ks[j * D + part * DP + i], dq[i]);
      }
    }
  }
  if (q >= a.Lq) return;
  const int64_t qo2 = (int64_t)b * a.dqs[0] + (int64_t)q * a.dqs[1] + (int64_t)h * a.dqs[2] + part * DP;
#pragma unroll
  for (int i = 0; i < DP; ++i) Mem<IT>::put(a.dq, qo2 + i, dq[i] * a.scale);
}

template <int D, int TPR, class IT, class OT, bool PREC>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void bwd_dkdv_simt(KArgs a) {
  constexpr int DP = D / TPR, RPW = 512 / TPR, SPLIT = TILE / RPW, SB = sub_block<D>();
  constexpr int ES = std::is_same<IT, float>::value ? 4 : 2;
  constexpr int EO = std::is_same<OT, float>::value ? 4 : 2;
  __shared__ __attribute__((aligned(16))) float Qs[SB * D];
  __shared__ __attribute__((aligned(16))) float Gs[SB * D];
  __shared__ __attribute__((aligned(16))) float Os[SB * D];
  __shared__ __attribute__((aligned(16))) float Ol[PREC ? SB * D : 4];   // O's low parts (PREC)
  __shared__ float Ls[SB], Llo[SB];

  const int item = a.kv_order[blockIdx.x / SPLIT];
  if (item < 0 || item >= a.B * a.Hkv * a.nkt) return;  // idle slot (or an entry out of range)
  const int kt = item % a.nkt;
  const int bh = item / a.nkt;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  const int tid = threadIdx.x, part = tid % TPR;
  const int row = (blockIdx.x % SPLIT) * RPW + tid / TPR;  // key within the tile
  const int key = kt * TILE + row;
  const int kcl = min(key, a.Lk - 1);

  float kv[DP], vv[DP], dk[DP], dv[DP];
  const int64_t ko = (int64_t)b * a.ks[0] + (int64_t)kcl * a.ks[1] + (int64_t)hk * a.ks[2] + part * DP;
  const int64_t vo = (int64_t)b * a.vs[0] + (int64_t)kcl * a.vs[1] + (int64_t)hk * a.vs[2] + part * DP;
#pragma unroll
  for (int i = 0; i < DP; i += 4) {
    Mem<IT>::get4(a.k, ko + i, kv + i);
    Mem<IT>::get4(a.v, vo + i, vv + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) dk[i + j] = dv[i + j] = 0.f;
  }
  for (int g = 0; g < a.G; ++g) {
    const int h = hk * a.G + g;
    const int mc = map_row(a, b, h, a.nkt, kt);
    const int e0 = a.col_ptr[mc], e1 = a.col_ptr[mc + 1];
    const char* qb = (const char*)a.q + ES * ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[2]);
    const char* gb = (const char*)a.dO + EO * ((int64_t)b * a.dos[0] + (int64_t)h * a.dos[2]);
    const char* ob = (const char*)a.o + EO * ((int64_t)b * a.os[0] + (int64_t)h * a.os[2]);
    for (int e = e0; e < e1; ++e) {
      const int qt = a.col_ent[2 * e], mask = a.col_ent[2 * e + 1];
      for (int sb = 0; sb < TILE / SB; ++sb) {
        const int q0 = qt * TILE + sb * SB;
        if (q0 >= a.Lq) break;
        __syncthreads();
        stage_rows<D, IT>(Qs, qb, a.qs[1], q0, a.Lq);
        stage_rows<D, OT>(Gs, gb, a.dos[1], q0, a.Lq);
        stage_rows<D, OT>(Os, ob, a.os[1], q0, a.Lq);
        if constexpr (PREC) stage_rows<D, float>(Ol, a.o_lo + ((int64_t)b * a.Hq + h) * a.Lq * D, D, q0, a.Lq);
        if (tid < SB) {
          const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + min(q0 + tid, a.Lq - 1);
          Ls[tid] = a.lse[rs];
          Llo[tid] = PREC ? a.lse_lo[rs] : 0.f;
        }
        __syncthreads();
        uint32_t bits = 0xffffffffu;
        if (mask >= 0)
          bits = sub_bits<SB>(a.col_bits, mask, sb, row);
        for (int j = 0; j < SB; ++j) {
          float gd = 0.f;
#pragma unroll
          for (int i = 0; i < DP; ++i) {
            float dvo = vv[i] - Os[j * D + part * DP + i];  // V_k - O, then O's low part
            if constexpr (PREC) dvo -= Ol[j * D + part * DP + i];
            gd = fmaf(dvo, Gs[j * D + part * DP + i], gd);  // dP - delta
          }
          gd = row_sum<TPR>(gd);
          float hi, lo;
          score<DP, TPR>(kv, Qs + j * D + part * DP, PREC, hi, lo);
          float p = exp2f(fmaf(hi, a.scale_log2, -Ls[j]) + fmaf(lo, a.scale_log2, -Llo[j]));
          if (!((bits >> j) & 1u)) p = 0.f;
          const float ds = p * gd;
#pragma unroll
          for (int i = 0; i < DP; ++i) {
            dv[i] = fmaf(p, Gs[j * D + part * DP + i], dv[i]);
            dk[i] = fmaf(ds, Qs[j * D + part * DP + i], dk[i]);
          }
        }
      }
    }
  }
  if (key >= a.Lk) return;
  const int64_t dko = (int64_t)b * a.dks[0] + (int64_t)key * a.dks[1] + (int64_t)hk * a.dks[2] + part * DP;
  const int64_t dvo = (int64_t)b * a.dvs[0] + (int64_t)key * a.dvs[1] + (int64_t)hk * a.dvs[2] + part * DP;
#pragma unroll
  for (int i = 0; i < DP; ++i) {
    Mem<IT>::put(a.dk, dko + i, dk[i] * a.scale);
    Mem<IT>::put(a.dv, dvo + i, dv[i]);
  }
}

// the stages of one (D, TPR, input, output) combination
template <int D, int TPR, class IT, class OT>
struct Simt {
  static constexpr int SPLIT = TILE * TPR / 512;
  static void fwd(const KArgs& a, int grid, hipStream_t st) {
    if (a.precise) hipLaunchKernelGGL((fwd_simt<D, TPR, IT, OT, true>), dim3(grid * SPLIT), dim3(512), 0, st, a);
    else hipLaunchKernelGGL((fwd_simt<D, TPR, IT, OT, false>), dim3(grid * SPLIT), dim3(512), 0, st, a);
  }
  static void bwd(const KArgs& a, int stage, int q_grid, int kv_grid, hipStream_t st) {
    if (stage == MATTN_BWD_PRE) {
      // nothing: the SIMT kernels form dP - delta per pair from O
    } else if (stage == MATTN_BWD_DKDV) {
      if (a.precise)
        hipLaunchKernelGGL((bwd_dkdv_simt<D, TPR, IT, OT, true>), dim3(kv_grid * SPLIT), dim3(512), 0, st, a);
      else
        hipLaunchKernelGGL((bwd_dkdv_simt<D, TPR, IT, OT, false>), dim3(kv_grid * SPLIT), dim3(512), 0, st, a);
    } else {
      if (a.precise)
        hipLaunchKernelGGL((bwd_dq_simt<D, TPR, IT, OT, true>), dim3(q_grid * SPLIT), dim3(512), 0, st, a);
      else
        hipLaunchKernelGGL((bwd_dq_simt<D, TPR, IT, OT, false>), dim3(q_grid * SPLIT), dim3(512), 0, st, a);
    }
  }
};

// f(Simt<...>{}) for the problem's combination: D = 64, 128 (4 threads per
// row) or 256 (8); float32 inputs, or 16-bit inputs with a float32 or
// same-dtype output
template <class Tag, class F>
void dispatch16(int D, bool of32, F&& f) {
  if (D == 64) { if (of32) f(Simt<64, 4, Tag, float>{}); else f(Simt<64, 4, Tag, Tag>{}); }
  else if (D == 128) { if (of32) f(Simt<128, 4, Tag, float>{}); else f(Simt<128, 4, Tag, Tag>{}); }
  else if (D == 256) { if (of32) f(Simt<256, 8, Tag, float>{}); else f(Simt<256, 8, Tag, Tag>{}); }
  else { if (of32) f(Simt<512, 16, Tag, float>{}); else f(Simt<512, 16, Tag, Tag>{}); }
}
template <class F>
hipError_t dispatch(int D, int dtype, int o_dtype, F&& f) {
  const bool of32 = o_dtype == MATTN_F32;
  if (dtype == MATTN_F32) {
    if (D == 64) f(Simt<64, 4, float, float>{});
    else if (D == 128) f(Simt<128, 4, float, float>{});
    else if (D == 256) f(Simt<256, 8, float, float>{});
    else f(Simt<512, 16, float, float>{});
  } else if (dtype == MATTN_BF16) {
    dispatch16<bf16_tag>(D, of32, f);
  } else {
    dispatch16<f16_tag>(D, of32, f);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_simt(const KArgs& a, int D, int dtype, int o_dtype, int grid, hipStream_t st) {
  return dispatch(D, dtype, o_dtype, [&](auto s) { decltype(s)::fwd(a, grid, st); });
}

hipError_t launch_bwd_simt(const KArgs& a, int D, int dtype, int o_dtype, int stage, int q_grid, int kv_grid,
                           hipStream_t st) {
  return dispatch(D, dtype, o_dtype, [&](auto s) { decltype(s)::bwd(a, stage, q_grid, kv_grid, st); });
}

}  // namespace mattn
