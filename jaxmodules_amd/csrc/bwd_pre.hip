// Backward pass of the masked attention (the custom_vjp bwd rule,
// /root/reference/jaxmodules/attention.py:266-342).
//
// The reference recomputes each query block's key scan and back-propagates
// through it, adding full-size dK/dV contributions per query block.  Here the
// gradient is computed from the saved base-2 log-sum-exp in three kernels:
//   bwd_pre  : per (b, head, 128-row query tile) the float16 copy
//              doh = dO * dsc (a power of two from the tile's max |dO|),
//              delta = rowsum(O * doh), the tile's bounds on the dS the other
//              two kernels form, and the dK/dV kernel's dS scale f of the tile
//              as lse - log2(f), so that its exp2 yields f P (this file); in a
//              split tile (the forward found a row whose largest weight
//              reaches SPLIT_P) also what doh rounds off (dol), with delta
//              from the unrounded dO, and the tile marked by a negative asc;
//   bwd_dkdv : one workgroup per 128-key map column of (b, kv head); it walks
//              the column's present query tiles for every query head of the
//              GQA group and accumulates dK, dV in registers -- no atomics;
//              the columns where a split row has an allowed key (flagged by
//              the forward) then take the products of what float16 rounded
//              off there: by a second kernel at D = 128, in the same kernel
//              at D = 64 (bwd_dkdv.hip);
//   bwd_dq   : one workgroup per 128-query map row; dQ accumulated in
//              registers; the split tiles' rows by a kernel of their own, or
//              at D = 64 without stored dS in the same kernel (bwd_dq.hip).
// With P = exp2(scale_log2 * S - lse) and dS = P * (dO V^T - delta):
//   dV = P^T dO,  dK = scale * dS^T Q,  dQ = scale * dS K.
// Every product of the 16-bit paths runs on float16 operands (11 significant
// bits): a bfloat16 dS or dO (8 bits) leaves 2^-9 relative errors that the
// 2e-3 parity gate does not absorb where one term dominates a sum.
#include <type_traits>

#include "common.hpp"

namespace mattn {

// ---------------------------------------------------------------------------
// preprocess
// ---------------------------------------------------------------------------

// PER consecutive values of a row (o_dtype float32 or the 16-bit Tag) as floats.
template <int PER, class Tag, bool F32>
__device__ __forceinline__ void load_vals(const void* base, int64_t off, float* g) {
  using E = Elt<Tag>;
  if constexpr (F32) {
    const float* p = (const float*)base + off;
#pragma unroll
    for (int i = 0; i < PER; i += 4) {
      const f32x4 y = *(const f32x4*)(p + i);
      g[i] = y[0]; g[i + 1] = y[1]; g[i + 2] = y[2]; g[i + 3] = y[3];
    }
  } else {
    const uint16_t* p = (const uint16_t*)base + off;
#pragma unroll
    for (int i = 0; i < PER; i += 8) {
      const u32x4 y = *(const u32x4*)(p + i);
#pragma unroll
      for (int j = 0; j < 8; ++j) g[i + j] = E::to_f32(elt16(y, j));
    }
  }
}

// A row's values held by its 4 threads in 16-byte chunks: thread p holds
// chunks p + 4 j (CS values each: 4 float32 or 8 16-bit values), so that the
// row's 4 threads read 64 contiguous bytes per access.  g[CS j + e] is value
// CS (p + 4 j) + e of the row.
template <int D, class Tag, bool F32>
__device__ __forceinline__ void load_row(const void* base, int64_t row_off, int part, float* g) {
  constexpr int CS = F32 ? 4 : 8, NJ = D / 4 / CS;
#pragma unroll
  for (int j = 0; j < NJ; ++j) load_vals<CS, Tag, F32>(base, row_off + CS * (part + 4 * j), g + CS * j);
}

// One workgroup of 512 threads per (b, head, 128-row query tile), 4 threads
// per row.  Rows past Lq (up to the tile's end) are written as zeros.
template <int D, class Tag, bool O_F32>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512)))
void bwd_pre(KArgs a) {
  using H = Elt<f16_tag>;
  constexpr int PER = D / 4;
  constexpr int CS = O_F32 ? 4 : 8;  // values per 16-byte input chunk
  __shared__ f32x2 red[8];
  // Launch position -> (b, h, qt).  When a row of O holds all heads ([B, L, H,
  // D]), the head runs fastest, so that the workgroups running together read
  // whole rows of O and dO between them; otherwise the query tile does.
  int b, h, qt;
  if (a.os[2] < a.os[1]) {
    h = blockIdx.x % a.Hq;
    qt = (blockIdx.x / a.Hq) % a.nqt;
    b = blockIdx.x / (a.Hq * a.nqt);
  } else {
    qt = blockIdx.x % a.nqt;
    h = (blockIdx.x / a.nqt) % a.Hq;
    b = blockIdx.x / (a.nqt * a.Hq);
  }
  const int bh = b * a.Hq + h;
  const int tile = bh * a.nqt + qt;  // (b * Hq + h) * nqt + qt
  const int tid = threadIdx.x, part = tid & 3;
  const int q = qt * TILE + (tid >> 2);
  const bool live = q < a.Lq;

  float o[PER], g[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = g[i] = 0.f;
  if (live) {
    load_row<D, Tag, O_F32>(a.o, (int64_t)b * a.os[0] + (int64_t)q * a.os[1] + (int64_t)h * a.os[2], part, o);
    load_row<D, Tag, O_F32>(a.dO, (int64_t)b * a.dos[0] + (int64_t)q * a.dos[1] + (int64_t)h * a.dos[2], part, g);
  }
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) mx = fmaxf(mx, fabsf(g[i]));
  // max |V| of the kv head (the forward's per-tile maxima)
  float vm = 0.f;
  const int tb = (b * a.Hkv + h / a.G) * a.nkt;
  for (int t = tid; t < a.nkt; t += 512) vm = fmaxf(vm, a.vmax[tb + t]);
  const f32x2 m1 = block_max2_512(f32x2{mx, vm}, red);
  const float s = copy_scale(m1[0]);
  // A split tile (the forward found a row whose largest weight reaches
  // SPLIT_P; uniform per workgroup) also keeps what the float16 copy rounds
  // off, and its products in the other kernels see dO' unrounded.
  const bool split = a.pmx != nullptr && a.pmx[tile] >= SPLIT_P;
  // the float16 copy; delta and the row's L1 norm from doh exactly as the
  // products see it (rounded, or with the rounded-off part in a split tile),
  // so that dS = P (dP - delta) cancels exactly where the exact dS is zero
  // (a row with a single allowed key) and its rounding error scales with V - O
  uint32_t hp[PER / 2], lp[PER / 2];
  float dl = 0.f, l1 = 0.f;
#pragma unroll
  for (int i = 0; i < PER; i += 2) {
    const float e0 = g[i] * s, e1 = g[i + 1] * s;  // exact: s is a power of two
    hp[i / 2] = H::pack2(e0, e1);
    const float h0 = H::to_f32(hp[i / 2] & 0xffffu), h1 = H::to_f32(hp[i / 2] >> 16);
    lp[i / 2] = H::pack2(e0 - h0, e1 - h1);  // the rounded-off parts (differences exact in float32)
    dl = split ? fmaf(o[i], e0, fmaf(o[i + 1], e1, dl)) : fmaf(o[i], h0, fmaf(o[i + 1], h1, dl));
    l1 += fabsf(h0) + fabsf(h1);
  }
#pragma unroll
  for (int m = 1; m < 4; m <<= 1) {
    dl += __shfl_xor(dl, m);
    l1 += __shfl_xor(l1, m);
  }
  // a row of halves: 16-byte stores, the row's 4 threads covering 64 contiguous bytes each time
  auto store_row = [&](uint16_t* wd, const uint32_t* hv) {
    if constexpr (CS == 8) {
      // chunk j (8 values) -> 8 halves at 8 (part + 4 j)
#pragma unroll
      for (int j = 0; j < PER / 8; ++j)
        *(u32x4*)(wd + 8 * (part + 4 * j)) = u32x4{hv[4 * j], hv[4 * j + 1], hv[4 * j + 2], hv[4 * j + 3]};
    } else {
      // chunk j (4 values) -> 4 halves at 4 (part + 4 j).  Threads p and p ^ 1
      // swap one chunk of each pair (2k, 2k + 1): the even thread then holds the
      // 8 halves at 16 (2k) + 4 p, the odd thread those at 16 (2k + 1) + 4 (p - 1).
      const bool odd = part & 1;
#pragma unroll
      for (int k = 0; k < PER / 8; ++k) {
        const u32x2 c0 = {hv[4 * k], hv[4 * k + 1]};        // chunk 2k
        const u32x2 c1 = {hv[4 * k + 2], hv[4 * k + 3]};    // chunk 2k + 1
        const u32x2 send = odd ? c0 : c1;
        const u32x2 recv = {(uint32_t)__shfl_xor((int)send[0], 1), (uint32_t)__shfl_xor((int)send[1], 1)};
        const u32x4 w = odd ? u32x4{recv[0], recv[1], c1[0], c1[1]} : u32x4{c0[0], c0[1], recv[0], recv[1]};
        const int h0 = odd ? 16 * (2 * k + 1) + 4 * (part - 1) : 16 * (2 * k) + 4 * part;
        *(u32x4*)(wd + h0) = w;
      }
    }
  };
  const int64_t crow = ((int64_t)bh * (a.nqt * TILE) + q) * D;
  store_row(a.doh + crow, hp);
  if (split) store_row(a.dol + crow, lp);
  const f32x2 st = block_max2_512(f32x2{l1, fabsf(dl)}, red);
  // |dS s| <= |dP s| + |delta s| <= max_q |doh_q|_1 max |V| + max |delta s|
  const float f = ds_scale(fmaf(st[0], m1[1], st[1]));
  if (live && part == 0) {
    const int64_t rr = (int64_t)bh * a.Lq + q;
    a.delta[rr] = dl;
    a.lsf[rr] = a.lse[rr] - (float)((int)(__float_as_uint(f) >> 23) - 127);  // log2 f, exact
  }
  if (tid == 0) {
    a.dsc[tile] = s;
    a.tst[tile] = float2{st[0], st[1]};
    a.asc[tile] = split ? -(f * s) : f * s;  // the sign marks a split tile
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

hipError_t launch_dq(const KArgs& a, int D, int dtype, int grid, hipStream_t st);
hipError_t launch_dkdv(const KArgs& a, int D, int dtype, int grid, hipStream_t st);

template <int D, class Tag, bool OF32>
static void launch_pre_16(const KArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((bwd_pre<D, Tag, OF32>), dim3(a.B * a.Hq * a.nqt), dim3(512), 0, st, a);
}

hipError_t launch_bwd_simt(const KArgs& a, int D, int dtype, int o_dtype, int stage, int q_grid, int kv_grid,
                           hipStream_t st);

hipError_t launch_bwd_stage(const KArgs& a, int D, int dtype, int o_dtype, bool simt, int stage, int q_grid,
                            int kv_grid, hipStream_t st) {
  const bool of32 = (o_dtype == MATTN_F32);
  if (simt) return launch_bwd_simt(a, D, dtype, o_dtype, stage, q_grid, kv_grid, st);
  if (stage == MATTN_BWD_DKDV) return launch_dkdv(a, D, dtype, kv_grid, st);
  if (stage == MATTN_BWD_DQ) return launch_dq(a, D, dtype, q_grid, st);
  if (dtype == MATTN_BF16) {
    if (D == 64) { if (of32) launch_pre_16<64, bf16_tag, true>(a, st); else launch_pre_16<64, bf16_tag, false>(a, st); }
    else { if (of32) launch_pre_16<128, bf16_tag, true>(a, st); else launch_pre_16<128, bf16_tag, false>(a, st); }
  } else {
    if (D == 64) { if (of32) launch_pre_16<64, f16_tag, true>(a, st); else launch_pre_16<64, f16_tag, false>(a, st); }
    else { if (of32) launch_pre_16<128, f16_tag, true>(a, st); else launch_pre_16<128, f16_tag, false>(a, st); }
  }
  return hipGetLastError();
}

}  // namespace mattn
