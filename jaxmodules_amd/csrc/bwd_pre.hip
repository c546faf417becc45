// Backward pass of the masked attention (the custom_vjp bwd rule,
// /root/reference/jaxmodules/attention.py:266-342).
//
// The reference recomputes each query block's key scan and back-propagates
// through it, adding full-size dK/dV contributions per query block.  Here the
// gradient is computed from the saved base-2 log-sum-exp in three kernels:
//   bwd_pre  : delta = rowsum(dO * O) per query row; dO converted to the MFMA
//              dtypes (this file, with the float32 SIMT kernels);
//   bwd_dkdv : one workgroup per 128-key map column of (b, kv head); it walks
//              the column's present query tiles for every query head of the
//              GQA group and accumulates dK, dV in registers -- each element
//              written exactly once, no atomics;
//   bwd_dq   : one workgroup per 128-query map row; dQ accumulated in registers.
// With P = exp2(scale_log2 * S - lse) and dS = P * (dO V^T - delta):
//   dV = P^T dO,  dK = scale * dS^T Q,  dQ = scale * dS K.
#include <type_traits>

#include "common.hpp"

namespace mattn {


// ---------------------------------------------------------------------------
// preprocess
// ---------------------------------------------------------------------------
// The dV product P^T dO runs on float16 MFMA: P lies in [0, 1] and float16
// keeps 11 significant bits against bfloat16's 8, which matters because dO
// arrives in float32 (the reference's output dtype).  dO is scaled by a power
// of two s so that max |dO * s| < 2^14 (the scale is exact and undone on the
// float32 result).  s comes from a deterministic two-pass max: bwd_absmax
// writes NPART partial maxima, bwd_pre reduces them.

// Element loads of one 16-lane row group: PER = D / 16 consecutive values.
template <int D, class Tag, bool O_F32>
__device__ __forceinline__ void load_row(const void* base, int64_t off, int sub, float* g) {
  using E = Elt<Tag>;
  constexpr int PER = D / 16;
  if constexpr (O_F32) {
    const float* p = (const float*)base + off + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4) {
      const f32x4 y = *(const f32x4*)(p + i);
      g[i] = y[0]; g[i + 1] = y[1]; g[i + 2] = y[2]; g[i + 3] = y[3];
    }
  } else {
    const uint16_t* p = (const uint16_t*)base + off + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4) {
      const u32x2 y = *(const u32x2*)(p + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) g[i + j] = E::to_f32((y[j >> 1] >> (16 * (j & 1))) & 0xffffu);
    }
  }
}

__device__ __forceinline__ float block_max256(float x, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// NPART workgroups; grid-stride over (b, q, h) rows, 16 lanes per row, four
// rows in flight per lane group.
template <int D, class Tag, bool O_F32>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void bwd_absmax(KArgs a) {
  constexpr int PER = D / 16;
  constexpr int UNR = 4;
  __shared__ float red[4];
  const uint32_t nrows = (uint32_t)a.B * a.Lq * a.Hq;  // < 2^31 (checked by the C ABI)
  const int sub = threadIdx.x & 15;
  const uint32_t step = gridDim.x * 16;
  float mx = 0.f;
  for (uint32_t r0 = blockIdx.x * 16 + (threadIdx.x >> 4); r0 < nrows; r0 += UNR * step) {
    float g[UNR][PER];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const uint32_t row = min(r0 + u * step, nrows - 1);  // a repeated row leaves the max unchanged
      const int h = (int)(row % (uint32_t)a.Hq);
      const uint32_t bq = row / (uint32_t)a.Hq;
      const int q = (int)(bq % (uint32_t)a.Lq), b = (int)(bq / (uint32_t)a.Lq);
      load_row<D, Tag, O_F32>(a.dO, (int64_t)b * a.dos[0] + (int64_t)q * a.dos[1] + (int64_t)h * a.dos[2],
                              sub, g[u]);
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u)
#pragma unroll
      for (int i = 0; i < PER; ++i) mx = fmaxf(mx, fabsf(g[u][i]));
  }
  mx = block_max256(mx, red);
  if (threadIdx.x == 0) a.part[blockIdx.x] = mx;
}

// One workgroup: the power-of-two scale s with max |dO * s| < 2^14, and 1/s.
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void bwd_scale(KArgs a) {
  __shared__ float red[4];
  float m = 0.f;
  for (int i = threadIdx.x; i < NPART; i += 256) m = fmaxf(m, a.part[i]);
  m = block_max256(m, red);
  if (threadIdx.x == 0) {
    float s = 1.f;
    if (m > 0.f && m <= 3.4e38f) {
      int e;
      frexpf(m, &e);  // m < 2^e
      s = ldexpf(1.f, min(126, max(-126, 14 - e)));
    }
    a.dscale[0] = s;
    a.dscale[1] = 1.f / s;
  }
}

// 16 lanes per (b, q, h) row, 16 rows per workgroup.  MODE 0: delta only
// (float32 inputs); 1: also dO * s in float16 (float16 inputs); 2: also dO in
// bfloat16 (bfloat16 inputs).
template <int D, class Tag, bool O_F32, int MODE>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void bwd_pre(KArgs a) {
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  constexpr int PER = D / 16;
  const uint32_t nrows = (uint32_t)a.B * a.Lq * a.Hq;  // < 2^31 (checked by the C ABI)
  const uint32_t row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (row >= nrows) return;  // uniform per 16-lane group; no barrier below
  const float s = MODE > 0 ? a.dscale[0] : 1.f;
  const int h = (int)(row % (uint32_t)a.Hq);
  const uint32_t bq = row / (uint32_t)a.Hq;
  const int q = (int)(bq % (uint32_t)a.Lq), b = (int)(bq / (uint32_t)a.Lq);
  float x[PER], g[PER];
  load_row<D, Tag, O_F32>(a.o, (int64_t)b * a.os[0] + (int64_t)q * a.os[1] + (int64_t)h * a.os[2], sub, x);
  load_row<D, Tag, O_F32>(a.dO, (int64_t)b * a.dos[0] + (int64_t)q * a.dos[1] + (int64_t)h * a.dos[2],
                          sub, g);
  // delta = rowsum(dO * O) with dO as rounded in the copy whose dP it meets:
  // dS = P (dP - delta) then cancels exactly where it should (a row with one
  // allowed key has dS = 0), and its error scales with V - O rather than V.
  // MODE 0: float32 dO; MODE 1, 2: the float16 dO * s copy (divided by s),
  // and MODE 2 also delta16 from the bfloat16 copy (the dQ kernel's dP).
  uint32_t hp[PER / 2], bp[PER / 2];
  float acc = 0.f, acc16 = 0.f;
  if constexpr (MODE == 0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) acc = fmaf(x[i], g[i], acc);
  } else {
    const float inv = a.dscale[1];
#pragma unroll
    for (int i = 0; i < PER; i += 2) {
      hp[i / 2] = H::pack2(g[i] * s, g[i + 1] * s);
      acc = fmaf(x[i], H::to_f32(hp[i / 2] & 0xffffu) * inv, acc);
      acc = fmaf(x[i + 1], H::to_f32(hp[i / 2] >> 16) * inv, acc);
    }
  }
  if constexpr (MODE == 2) {
#pragma unroll
    for (int i = 0; i < PER; i += 2) {
      bp[i / 2] = E::pack2(g[i], g[i + 1]);
      acc16 = fmaf(x[i], E::to_f32(bp[i / 2] & 0xffffu), acc16);
      acc16 = fmaf(x[i + 1], E::to_f32(bp[i / 2] >> 16), acc16);
    }
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    acc += __shfl_xor(acc, o, 16);
    if constexpr (MODE == 2) acc16 += __shfl_xor(acc16, o, 16);
  }
  const int64_t rr = ((int64_t)b * a.Hq + h) * a.Lq + q;
  if (sub == 0) {
    a.delta[rr] = acc;
    if constexpr (MODE == 2) a.delta16[rr] = acc16;
  }
  if constexpr (MODE > 0) {
    // dense [B, Lq, Hq, D] copies
    uint16_t* w = (uint16_t*)a.dOhw + (int64_t)row * D + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4) *(u32x2*)(w + i) = u32x2{hp[i / 2], hp[i / 2 + 1]};
  }
  if constexpr (MODE == 2) {
    uint16_t* w = (uint16_t*)a.dO16w + (int64_t)row * D + sub * PER;
#pragma unroll
    for (int i = 0; i < PER; i += 4) *(u32x2*)(w + i) = u32x2{bp[i / 2], bp[i / 2 + 1]};
  }
}

// ---------------------------------------------------------------------------
// float32 SIMT backward
// ---------------------------------------------------------------------------

template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void bwd_dq_simt(KArgs a) {
  constexpr int SB = 32;
  constexpr int DP = D / 4;
  __shared__ __attribute__((aligned(16))) float Ks[SB * D];
  __shared__ __attribute__((aligned(16))) float Vs[SB * D];

  const int item = a.q_order[blockIdx.x];
  if (item < 0 || item >= a.B * a.Hq * a.nqt) return;  // idle slot (or an entry out of range)
  const int qt = item % a.nqt;
  const int bh = item / a.nqt;
  const int h = bh % a.Hq, b = bh / a.Hq, hk = h / a.G;
  const int mrow = map_row(a, b, h, a.nqt, qt);
  const int e0 = a.row_ptr[mrow], e1 = a.row_ptr[mrow + 1];
  const int tid = threadIdx.x, row = tid >> 2, part = tid & 3;
  const int q = qt * TILE + row;
  const int qc = min(q, a.Lq - 1);

  float qv[DP], gv[DP], dq[DP];
  {
    const float* qp = (const float*)a.q + (int64_t)b * a.qs[0] + (int64_t)qc * a.qs[1] +
                      (int64_t)h * a.qs[2] + part * DP;
    const float* gp = (const float*)a.dO + (int64_t)b * a.dos[0] + (int64_t)qc * a.dos[1] +
                      (int64_t)h * a.dos[2] + part * DP;
#pragma unroll
    for (int i = 0; i < DP; ++i) { qv[i] = qp[i]; gv[i] = gp[i]; dq[i] = 0.f; }
  }
  const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + qc;
  const float lse = a.lse[rs], dl = a.delta[rs];
  const float* kb = (const float*)a.k + (int64_t)b * a.ks[0] + (int64_t)hk * a.ks[2];
  const float* vb = (const float*)a.v + (int64_t)b * a.vs[0] + (int64_t)hk * a.vs[2];

  for (int e = e0; e < e1; ++e) {
    const int kt = a.row_ent[2 * e], mask = a.row_ent[2 * e + 1];
    for (int sb = 0; sb < TILE / SB; ++sb) {
      const int key0 = kt * TILE + sb * SB;
      if (key0 >= a.Lk) break;
      __syncthreads();
      for (int c = tid; c < SB * D / 4; c += 512) {
        const int r = c / (D / 4), col = 4 * (c % (D / 4));
        const int key = min(key0 + r, a.Lk - 1);
        *(f32x4*)&Ks[r * D + col] = *(const f32x4*)(kb + (int64_t)key * a.ks[1] + col);
        *(f32x4*)&Vs[r * D + col] = *(const f32x4*)(vb + (int64_t)key * a.vs[1] + col);
      }
      __syncthreads();
      uint32_t bits = 0xffffffffu;
      if (mask >= 0)
        bits = (uint32_t)(a.row_bits[((int64_t)mask * 2 + (sb >> 1)) * TILE + row] >> (32 * (sb & 1)));
      for (int j = 0; j < SB; ++j) {
        float s = 0.f, g = 0.f;
#pragma unroll
        for (int i = 0; i < DP; ++i) {
          s = fmaf(qv[i], Ks[j * D + part * DP + i], s);
          g = fmaf(gv[i], Vs[j * D + part * DP + i], g);
        }
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        g += __shfl_xor(g, 1);
        g += __shfl_xor(g, 2);
        float p = exp2f(s * a.scale_log2 - lse);
        if (!((bits >> j) & 1u)) p = 0.f;
        const float ds = p * (g - dl);
#pragma unroll
        for (int i = 0; i < DP; ++i) dq[i] = fmaf(ds, Ks[j * D + part * DP + i], dq[i]);
      }
    }
  }
  if (q >= a.Lq) return;
  float* op = (float*)a.dq + (int64_t)b * a.dqs[0] + (int64_t)q * a.dqs[1] + (int64_t)h * a.dqs[2] +
              part * DP;
#pragma unroll
  for (int i = 0; i < DP; ++i) op[i] = dq[i] * a.scale;
}

template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void bwd_dkdv_simt(KArgs a) {
  constexpr int SB = 32;
  constexpr int DP = D / 4;
  __shared__ __attribute__((aligned(16))) float Qs[SB * D];
  __shared__ __attribute__((aligned(16))) float Gs[SB * D];
  __shared__ float Ls[SB], Dl[SB];

  const int item = a.kv_order[blockIdx.x];
  if (item < 0 || item >= a.B * a.Hkv * a.nkt) return;  // idle slot (or an entry out of range)
  const int kt = item % a.nkt;
  const int bh = item / a.nkt;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;
  const int tid = threadIdx.x, row = tid >> 2, part = tid & 3;
  const int key = kt * TILE + row;
  const int kcl = min(key, a.Lk - 1);

  float kv[DP], vv[DP], dk[DP], dv[DP];
  {
    const float* kp = (const float*)a.k + (int64_t)b * a.ks[0] + (int64_t)kcl * a.ks[1] +
                      (int64_t)hk * a.ks[2] + part * DP;
    const float* vp = (const float*)a.v + (int64_t)b * a.vs[0] + (int64_t)kcl * a.vs[1] +
                      (int64_t)hk * a.vs[2] + part * DP;
#pragma unroll
    for (int i = 0; i < DP; ++i) { kv[i] = kp[i]; vv[i] = vp[i]; dk[i] = 0.f; dv[i] = 0.f; }
  }
  for (int g = 0; g < a.G; ++g) {
    const int h = hk * a.G + g;
    const int mc = map_row(a, b, h, a.nkt, kt);
    const int e0 = a.col_ptr[mc], e1 = a.col_ptr[mc + 1];
    const float* qb = (const float*)a.q + (int64_t)b * a.qs[0] + (int64_t)h * a.qs[2];
    const float* gb = (const float*)a.dO + (int64_t)b * a.dos[0] + (int64_t)h * a.dos[2];
    for (int e = e0; e < e1; ++e) {
      const int qt = a.col_ent[2 * e], mask = a.col_ent[2 * e + 1];
      for (int sb = 0; sb < TILE / SB; ++sb) {
        const int q0 = qt * TILE + sb * SB;
        if (q0 >= a.Lq) break;
        __syncthreads();
        for (int c = tid; c < SB * D / 4; c += 512) {
          const int r = c / (D / 4), col = 4 * (c % (D / 4));
          const int qq = min(q0 + r, a.Lq - 1);
          *(f32x4*)&Qs[r * D + col] = *(const f32x4*)(qb + (int64_t)qq * a.qs[1] + col);
          *(f32x4*)&Gs[r * D + col] = *(const f32x4*)(gb + (int64_t)qq * a.dos[1] + col);
        }
        if (tid < 2 * SB) {
          const int qq = min(q0 + (tid & (SB - 1)), a.Lq - 1);
          const int64_t rs = ((int64_t)b * a.Hq + h) * a.Lq + qq;
          if (tid < SB) Ls[tid] = a.lse[rs];
          else Dl[tid - SB] = a.delta[rs];
        }
        __syncthreads();
        uint32_t bits = 0xffffffffu;
        if (mask >= 0)
          bits = (uint32_t)(a.col_bits[((int64_t)mask * 2 + (sb >> 1)) * TILE + row] >> (32 * (sb & 1)));
        for (int j = 0; j < SB; ++j) {
          float s = 0.f, gd = 0.f;
#pragma unroll
          for (int i = 0; i < DP; ++i) {
            s = fmaf(kv[i], Qs[j * D + part * DP + i], s);
            gd = fmaf(vv[i], Gs[j * D + part * DP + i], gd);
          }
          s += __shfl_xor(s, 1);
          s += __shfl_xor(s, 2);
          gd += __shfl_xor(gd, 1);
          gd += __shfl_xor(gd, 2);
          float p = exp2f(s * a.scale_log2 - Ls[j]);
          if (!((bits >> j) & 1u)) p = 0.f;
          const float ds = p * (gd - Dl[j]);
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
  float* kp = (float*)a.dk + (int64_t)b * a.dks[0] + (int64_t)key * a.dks[1] + (int64_t)hk * a.dks[2] +
              part * DP;
  float* vp = (float*)a.dv + (int64_t)b * a.dvs[0] + (int64_t)key * a.dvs[1] + (int64_t)hk * a.dvs[2] +
              part * DP;
#pragma unroll
  for (int i = 0; i < DP; ++i) { kp[i] = dk[i] * a.scale; vp[i] = dv[i]; }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

hipError_t launch_dq(const KArgs& a, int D, int dtype, int grid, hipStream_t st);
hipError_t launch_dkdv(const KArgs& a, int D, int dtype, int grid, hipStream_t st);

hipError_t launch_bwd_stage(const KArgs& a, int D, int dtype, int o_dtype, int stage, int q_grid,
                            int kv_grid, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.Lq * a.Hq;
  const int pre_grid = (int)((rows + 15) / 16);
  const bool of32 = (o_dtype == MATTN_F32);
  if (dtype == MATTN_F32) {
    if (stage == MATTN_BWD_PRE) {
      if (D == 64) hipLaunchKernelGGL((bwd_pre<64, bf16_tag, true, 0>), dim3(pre_grid), dim3(256), 0, st, a);
      else hipLaunchKernelGGL((bwd_pre<128, bf16_tag, true, 0>), dim3(pre_grid), dim3(256), 0, st, a);
    } else if (stage == MATTN_BWD_DKDV) {
      if (D == 64) hipLaunchKernelGGL((bwd_dkdv_simt<64>), dim3(kv_grid), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((bwd_dkdv_simt<128>), dim3(kv_grid), dim3(512), 0, st, a);
    } else {
      if (D == 64) hipLaunchKernelGGL((bwd_dq_simt<64>), dim3(q_grid), dim3(512), 0, st, a);
      else hipLaunchKernelGGL((bwd_dq_simt<128>), dim3(q_grid), dim3(512), 0, st, a);
    }
    return hipGetLastError();
  }
  if (stage == MATTN_BWD_DKDV) return launch_dkdv(a, D, dtype, kv_grid, st);
  if (stage == MATTN_BWD_DQ) return launch_dq(a, D, dtype, q_grid, st);
#define MATTN_PRE(DD, TAG, OF32, MODE)                                                           \
  do {                                                                                           \
    hipLaunchKernelGGL((bwd_absmax<DD, TAG, OF32>), dim3(NPART), dim3(256), 0, st, a);           \
    hipLaunchKernelGGL(bwd_scale, dim3(1), dim3(256), 0, st, a);                                 \
    hipLaunchKernelGGL((bwd_pre<DD, TAG, OF32, MODE>), dim3(pre_grid), dim3(256), 0, st, a);     \
  } while (0)
  if (dtype == MATTN_BF16) {
    if (D == 64) { if (of32) MATTN_PRE(64, bf16_tag, true, 2); else MATTN_PRE(64, bf16_tag, false, 2); }
    else { if (of32) MATTN_PRE(128, bf16_tag, true, 2); else MATTN_PRE(128, bf16_tag, false, 2); }
  } else {
    if (D == 64) { if (of32) MATTN_PRE(64, f16_tag, true, 1); else MATTN_PRE(64, f16_tag, false, 1); }
    else { if (of32) MATTN_PRE(128, f16_tag, true, 1); else MATTN_PRE(128, f16_tag, false, 1); }
  }
#undef MATTN_PRE
  return hipGetLastError();
}

}  // namespace mattn
