// dK/dV kernel of the masked-attention backward (the custom_vjp bwd rule,
// /root/reference/jaxmodules/attention.py:266-342): one workgroup per
// 128-key map column of (b, kv head) walking the column's present query tiles
// for every query head of the GQA group; dK and dV accumulated in registers and
// written once each -- no atomics.  Every product runs on float16 operands.
#include <type_traits>

#include "common.hpp"

namespace mattn {

// ---------------------------------------------------------------------------
// dK / dV (MFMA, no atomics)
// ---------------------------------------------------------------------------
// 8 waves (2 per SIMD).  Wave w owns keys 32 (w % 4) .. +31 of the tile and
// query half w / 4 of every 64-query sub-block.  With the float16 copies
// Q' = Q r, V' = V v (the forward's), dO' = dO s (bwd_pre) and K' = K k (the
// prologue), each times a power of two per 128-row tile:
//   S'   = Q' K'^T          (A: Q' rows, B: K' rows; both from LDS)
//   dP'  = dO' V'^T         (B: V' rows from LDS)
//   P~   = exp2(S' c2 / (r k) - (lse - log2 f)) = f P
//   dS~  = P~ (dP' / v - delta s)   = f s dS
//   dV^T += dO'^T P~      (A: transposed reads of the dO' tile)
//   dK^T += Q'^T dS~      (A: transposed reads of the Q' tile)
// f is bwd_pre's power of two per query tile that keeps |dS~| < 2^14, so dS~
// loses nothing to float16's range; bwd_pre folds it into the lse copy (lsf)
// this kernel reads.  The accumulators are in units of f s (dV) and f s r
// (dK) of the query tile last walked, rescaled when a tile with other scales
// comes (rare: the scales move in steps of 2^4).
// The K' and V' tiles of the workgroup's 128 keys stay in LDS for the whole
// column (K' is also written to kh for the dQ kernel); Q', dO', lse, delta
// and the partial-tile mask words are double-buffered and filled by direct
// global->LDS loads.  The MFMA operand reads are pipelined by hand: asm LDS
// reads issued two k-steps ahead of their MFMAs, with counted lgkmcnt waits.
// The two query halves' dK/dV partials of a key are summed through LDS at the
// end, and the rows leave through an LDS-staged tile, 16 bytes per lane along
// each row.
// DS (MATTN_BWD_DS): each wave also leaves its 32 x 32 block of dS~ for the
// dQ kernel, as it holds it for the dK product (lane = key; the DS_TILE layout
// in common.hpp: the dQ kernel, which streams it from HBM with LDS to spare,
// does the transposition).  The two 16-byte stores per lane go out
// (nontemporal: read once, much later) right after the next sub-block's
// barrier, or after the loop, so that they have a whole step to complete
// before the wait ahead of the following barrier, which counts stores too.
//
// Split tiles.  A query tile whose rows put a weight of at least SPLIT_P on
// a key is a split tile (bwd_pre marks it by a negative asc); the forward's
// walk of its split rows flags the columns where they have allowed keys
// (scol).  The kernel (SPLIT = false) computes its sub-blocks like any other;
// a flagged column also leaves its reduced dK and dV unrounded (float32, free
// of the accumulator scales) in kvp.  The SPLIT = true
// kernel, launched after it, takes those columns (its other workgroups
// return at once), starts from kvp, and adds for each split sub-block the
// products of what float16 rounded off there (correct() below), so that the
// tile's terms enter dK and dV with 22 significant bits; it then stores the
// column's dK and dV over the first kernel's.  At D = 64 the registers allow
// both in one kernel (FUSED): a column whose walk met a split row runs the
// same correction pass right after its walk, from the accumulators it holds
// and the resident K' / V' tiles, and no second kernel is launched.
template <int D, class Tag, bool DS, bool SPLIT>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
void bwd_dkdv_mfma(KArgs a) {
  static_assert(!(DS && SPLIT), "the split kernel stores no dS");
  constexpr bool FUSED = !SPLIT && D == 64;  // the correction pass in this kernel
  using E = Elt<Tag>;
  using H = Elt<f16_tag>;
  using TL = TileLoad<D>;
  constexpr int BM = 64;              // queries per sub-block
  constexpr int NKD = D / 16;
  constexpr int NMD = D / 32;
  constexpr int BLK = 512;            // elements one load instruction fills
  constexpr int NS = BM * D / BLK / 8;  // load slots per wave for a 64-row tile

  // one array per buffer: the compiler then knows the loads landing in one
  // buffer cannot alias the operand reads of the other (no vmcnt waits mid-step)
  __shared__ __attribute__((aligned(16))) float L0[BM], L1[BM];        // lse
  __shared__ __attribute__((aligned(16))) float G0[BM], G1[BM];        // delta
  __shared__ __attribute__((aligned(16))) uint64_t M0[TILE], M1[TILE];  // partial-tile mask words
  // per buffer: Q' rows, then dO' rows (BM * D elements each); K' tile, then V' tile
  __shared__ __attribute__((aligned(16))) uint16_t QH0[2 * BM * D], QH1[2 * BM * D];
  __shared__ __attribute__((aligned(16))) uint16_t KV[2 * TILE * D];
  // SPLIT: the rounded-off part of dO' of the split sub-block being corrected
  __shared__ __attribute__((aligned(16))) uint16_t DL[SPLIT || FUSED ? BM * D : 8];
  uint16_t* const Q0 = QH0;
  uint16_t* const H0 = QH0 + BM * D;
  uint16_t* const Q1 = QH1;
  uint16_t* const H1 = QH1 + BM * D;
  uint16_t* const Ks = KV;
  uint16_t* const Vs = KV + TILE * D;
  __shared__ f32x2 red[8];

  // the slot's descriptor (item, first head / entry / end of its column list,
  // sub-block count, first entry's query tile, mask and row index): the first
  // loads need this one read, not a chain of dependent ones
  const u32x4 dA = ((const u32x4*)a.kv_desc)[2 * blockIdx.x];
  const u32x4 dB = ((const u32x4*)a.kv_desc)[2 * blockIdx.x + 1];
  const int item = (int)dA[0];
  if (item < 0 || item >= a.B * a.Hkv * a.nkt) return;  // idle slot (or an entry out of range)
  const bool col_split = a.scol[item] != 0;  // a split row has an allowed key in this column
  if constexpr (SPLIT) {
    if (!col_split) return;  // the first kernel's dK, dV stand
  }
  const int kt = item % a.nkt;
  const int bh = item / a.nkt;
  const int hk = bh % a.Hkv, b = bh / a.Hkv;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int kg = wave & 3, qh = wave >> 2;
  const int kloc = 32 * kg + l32;
  const float c2 = a.scale_log2;

  // the forward's V' tile of the column, by direct loads into LDS, and this
  // thread's share of its K rows (4 threads per key row), converted to
  // float16 once the tile's max |K| is known; both issued now so that their
  // latency overlaps the first sub-block's
  const int col = item;  // (b * Hkv + hk) * nkt + kt
  {
    const uint16_t* vsrc = a.vh + (int64_t)col * TILE * D;
    const uint16_t* ksrc = a.kh + (int64_t)col * TILE * D;  // SPLIT: the first kernel's K' tile
#pragma unroll
    for (int i = 0; i < 2 * NS; ++i) {
      const int n = 2 * NS * wave + i;
      const int64_t off = (int64_t)TL::row_of(n, lane) * D + 8 * TL::chunk_of(n, lane);
      lds_load16(vsrc + off, Vs + n * BLK);
      if constexpr (SPLIT) lds_load16(ksrc + off, Ks + n * BLK);
    }
  }
  TileRows<D> tkr;
  if constexpr (!SPLIT)
    tile_load<D>(tkr, (const uint16_t*)a.k + (int64_t)b * a.ks[0] + (int64_t)(kt * TILE) * a.ks[1] +
                          (int64_t)hk * a.ks[2], a.ks[1], a.Lk - kt * TILE);

  // Flattened walk over (query head g of the group, column entry, half):
  // tot sub-blocks; the cursor of the next sub-block to load starts at the
  // descriptor's first entry
  const int tot = SPLIT ? 0 : (int)dB[0];  // (the split kernel walks the split sub-blocks alone)
  int lg = (int)dA[1], le = (int)dA[2], lend = (int)dA[3], lhalf = 0;

  // loop-invariant source byte offsets of this lane's load slots (Q' and dO'
  // rows are dense: row stride D in both copies)
  uint32_t qld[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) qld[i] = 2 * TL::src_off(NS * wave + i, lane, D);
  // LDS operand addresses, formed per use from lane seeds (one v_xad_u32 each)
  // rather than held in 24 registers across the loop (element offsets):
  //   row read, chunk 2 kd + hi of row r:   r D + ((16 kd) ^ rx),  rx = 8 hi ^ 8 swz(r)
  //   transposed read (mt, sec):            tb[sec] + ((32 mt) ^ tz)
  // Rows 32 qh + l32 (queries) and 32 kg + l32 (keys) share swz(l32); only the
  // swizzle's bits from 2 up meet mt in a transposed read, and they do not depend on sec.
  const int rx = (8 * hi) ^ (swz<D>(l32) << 3);
  const int qrow = (32 * qh + l32) * D, krow_l = kloc * D;
  const int tz = 32 * (swz<D>(4 * hi + ((lane & 15) >> 2)) >> 2);
  const int tb0 = tr_src<D>(lane, 0, 0) + 32 * qh * D - tz;
  const int tb1 = tr_src<D>(lane, 0, 1) + 32 * qh * D - tz;
  const int wofs = __builtin_amdgcn_readfirstlane(NS * wave * BLK);  // this wave's load block
  EntryCache ec;
  int mid0 = -1, mid1 = -1;  // mask id of the sub-block in each buffer (-1: full tile)
  // dO' and Q' tile scales (s, r) of the sub-block in each buffer
  float sh0 = 1.f, rh0 = 1.f, sh1 = 1.f, rh1 = 1.f;
  // buffer resources of the current query head's Q' and dO' slices
  const int64_t hrows = (int64_t)a.nqt * TILE;  // rows per head in the copies
  const uint32_t hbytes = (uint32_t)(hrows * D * 2);
  __amdgpu_buffer_rsrc_t rq, rh;
  int rh_head = -1;
  const float* qsc_h = a.qsc;  // the current query head's per-tile scales
  const float* asc_h = a.asc;
  float cur_s = 1.f, cur_r = 1.f;  // scales f s and r of the prepared sub-block's query tile
  // Tile loads of the next sub-block on the fast path, prepared by launch()
  // and issued by the step, one per S / dP k-step, so that the 1 KiB DMA
  // instructions of the eight waves enter the load unit behind the MFMA chains
  // rather than all at the top of the step.
  bool dma_on = false;
  uint32_t dma_so = 0;
  auto dma = [&](auto bufc, auto ic) {  // load i of the sub-block that goes into buffer BUF
    constexpr int BUF = decltype(bufc)::value, i = decltype(ic)::value, k = i / 2;
    if (dma_on) {
      if constexpr (i % 2 == 0) lds_load16_buf(rq, qld[k], dma_so, (BUF ? Q1 : Q0) + wofs + k * BLK);
      else lds_load16_buf(rh, qld[k], dma_so, (BUF ? H1 : H0) + wofs + k * BLK);
    }
  };

  // Entry of the column list at the cursor (the same for both 64-query halves
  // of a query tile), and per query head the row pointers of lse / delta, the
  // Q' / dO' buffer resources and the head's scales: updated only when they change.  The branches
  // below test wave-uniform values (scalar registers), not per-lane ones.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  int cur_qt = 0, cur_mid = -1;
  int cur_ri = 0;                      // row-entry index of the column entry (DS)
  uint16_t* dsp0 = nullptr;            // DS: dS slot of the sub-block in each buffer
  uint16_t* dsp1 = nullptr;
  uint16_t* dpend = nullptr;           // DS: where the chunks in sf go (null: none)
  u32x4 sf[2];                         // DS: the last sub-block's dS~ chunks (sk)
  const float* lrow = nullptr;  // lse - log2 f (wave 6) or delta (wave 7) row of the current head

  // The next sub-block's loads in two parts: prep() advances the cursor
  // before the step's barrier (waves that reach the barrier early do it while
  // they would wait anyway; per-wave stamps put the whole bookkeeping at 400-
  // 600 cycles when all eight waves ran it right after the barrier); launch()
  // issues the loads after the barrier, once the buffer they fill is free.
  int nq0 = 0;  // first query row of the prepared sub-block
  // FIRST (the first sub-block): its entry comes from the descriptor, and the
  // query tile's scales are read back after the K' tile (first_r, first_s),
  // so that its loads are issued without waiting for any list read
  float first_r = 1.f, first_s = 1.f;
  auto prep = [&](auto bufc, auto firstc) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr bool FIRST = decltype(firstc)::value;
    if (lhalf == 0) {
      while (!FIRST && le >= lend) {  // next query head of the group: another column list
        ++lg;
        const int mc = map_row(a, b, hk * a.G + lg, a.nkt, kt);
        le = a.col_ptr[mc];
        lend = a.col_ptr[mc + 1];
        ec.reset();
      }
      const int h = hk * a.G + lg;
      if (h != rh_head) {
        rh_head = h;
        const int64_t hb = ((int64_t)b * a.Hq + h) * hrows * D;
        rq = make_rsrc(a.qh + hb, hbytes);
        rh = make_rsrc(a.doh + hb, hbytes);
        lrow = (wv == 6 ? a.lsf : a.delta) + ((int64_t)b * a.Hq + h) * a.Lq;
        qsc_h = a.qsc + (b * a.Hq + h) * a.nqt;
        asc_h = a.asc + (b * a.Hq + h) * a.nqt;
      }
      if constexpr (FIRST) {
        cur_qt = (int)dB[1];
        cur_mid = (int)dB[2];
        cur_ri = (int)dB[3];
        first_r = qsc_h[cur_qt];
        first_s = asc_h[cur_qt];
      } else if constexpr (DS)
        ec.get(a.col_ent, le, lend, lane, cur_qt, cur_mid, qsc_h, asc_h, cur_r, cur_s, a.col_row, cur_ri);
      else
        ec.get(a.col_ent, le, lend, lane, cur_qt, cur_mid, qsc_h, asc_h, cur_r, cur_s);
    }
    if constexpr (DS)  // this query half's two dQ waves (2 lhalf, 2 lhalf + 1) of the tile's slot
      (BUF ? dsp1 : dsp0) = a.ds + (ds_rep(a, b, rh_head) + cur_ri) * DS_TILE + lhalf * (2 * 8 * 512);
    (BUF ? mid1 : mid0) = cur_mid;
    (BUF ? sh1 : sh0) = fabsf(cur_s);  // (negative for a split tile)
    (BUF ? rh1 : rh0) = cur_r;
    nq0 = cur_qt * TILE + lhalf * BM;
    if (lhalf == 0) {
      lhalf = 1;
    } else {
      lhalf = 0;
      ++le;
    }
  };
  auto launch = [&](auto bufc) {  // global -> LDS loads of the prepared sub-block into buffer BUF
    constexpr int BUF = decltype(bufc)::value;
    const int mid = BUF ? mid1 : mid0;
    const int q0 = nq0;
    const int mh = (q0 / BM) & 1;  // query half of its tile
    if (mid >= 0 && wv < 4) {  // 32 keys' mask words per wave (256 bytes), one dword per lane
      const uint32_t* src = (const uint32_t*)(a.col_bits + ((int64_t)mid * 2 + mh) * TILE + wv * 32);
      __builtin_amdgcn_global_load_lds(src + lane, (__attribute__((address_space(3))) void*)((BUF ? M1 : M0) + wv * 32),
                                       4, 0, 0);
    }
    // the step issues the 2 NS tile loads, one per S / dP k-step (the Q' and
    // dO' copies are padded to whole tiles, so no row is out of range)
    dma_on = true;
    dma_so = (uint32_t)(q0 * D * 2);
    if (wv >= 6)  // lse (wave 6) and delta (wave 7) of the 64 rows; rows past Lq re-read row Lq-1
      __builtin_amdgcn_global_load_lds(lrow + min(q0 + lane, a.Lq - 1),
                                       (__attribute__((address_space(3))) void*)(wv == 6 ? (BUF ? L1 : L0) : (BUF ? G1 : G0)),
                                       4, 0, 0);
  };

  f32x16 dk[NMD], dv[NMD];
#pragma unroll
  for (int i = 0; i < NMD; ++i) { dk[i] = f32x16{}; dv[i] = f32x16{}; }
  // the column's unrounded dK, dV (units of 1): wave kg's [2][NMD][64][16]
  // floats of its 32 keys, dK then dV, each lane's 16 registers of an MFMA
  // tile contiguous
  float* const part = a.kvp + ((int64_t)col * 8 + 2 * kg) * (NMD * 16 * 64);
  if constexpr (SPLIT) {
    // the first kernel's sums (the other query half starts from zero), loaded
    // while the K' / V' tiles come
    if (qh == 0) {
#pragma unroll
      for (int mt = 0; mt < NMD; ++mt) {
        dk[mt] = *(const f32x16*)&part[(mt * 64 + lane) * 16];
        dv[mt] = *(const f32x16*)&part[((NMD + mt) * 64 + lane) * 16];
      }
    }
  }

  const int dsp_l0 = ds_pos(lane, 0) * 8, dsp_l1 = 512 + ds_pos(lane, 1) * 8;  // chunk offsets per t
  auto store_ds = [&]() {
    __builtin_nontemporal_store(sf[0], (u32x4*)(dpend + dsp_l0));
    __builtin_nontemporal_store(sf[1], (u32x4*)(dpend + dsp_l1));
  };
  // set by the prologue: the column's K' / V' tile scales
  float ksc = 1.f, ivs = 1.f;
  float acc_s = 1.f, acc_r = 1.f;  // scales f s and r the accumulators are in
  float m2c = c2;                   // c2 / (r k) of those scales

  auto step = [&](auto bufc, bool masked) {
    constexpr int BUF = decltype(bufc)::value;
    // the sub-block's dO' / Q' scales (uniform); other scales than the
    // accumulators' rescale them (powers of two: exact)
    const float ss = BUF ? sh1 : sh0, rr = BUF ? rh1 : rh0;
    if (ss != acc_s || rr != acc_r) {
      const float fv = ss / acc_s, fk = fv * (rr / acc_r);
#pragma unroll
      for (int i = 0; i < NMD; ++i) { dv[i] *= fv; dk[i] *= fk; }
      acc_s = ss;
      acc_r = rr;
      m2c = c2 * pow2_rcp(rr * ksc);
    }
    const float mc = m2c;
    const float* Lb = (BUF ? L1 : L0) + 32 * qh;
    const float* Gb = (BUF ? G1 : G0) + 32 * qh;
    // seeds re-defined here, so the addresses derived from them stay per use;
    const int rxo = opaque(rx);
    f32x16 st = f32x16{}, dp = f32x16{};
    {
      // S / dP pipelined by hand: the eight S MFMAs, then the eight dP MFMAs;
      // step i reads its two 16-byte operands PS steps ahead (dO' sits BM * D
      // elements after Q', V' TILE * D after K': immediate offsets)
      constexpr int PS = 2;
      const uint32_t qa0 = lds_addr(BUF ? Q1 : Q0) + 2 * (uint32_t)qrow;
      const uint32_t ka0 = lds_addr(Ks) + 2 * (uint32_t)krow_l;
      u32x4 oa[PS + 1], ob[PS + 1];
      auto rd = [&](auto ic) {
        constexpr int i = decltype(ic)::value, kd = i % NKD, isdp = i / NKD, sl = i % (PS + 1);
        const uint32_t x = 2 * (uint32_t)((16 * kd) ^ rxo);
        oa[sl] = ds_read128<isdp ? 2 * BM * D : 0>(qa0 + x);
        ob[sl] = ds_read128<isdp ? 2 * TILE * D : 0>(ka0 + x);
      };
      static_for<PS>(rd);
      static_for<2 * NKD>([&](auto ic) {
        constexpr int i = decltype(ic)::value, isdp = i / NKD, sl = i % (PS + 1);
        if constexpr (i + PS < 2 * NKD) rd(std::integral_constant<int, i + PS>{});
        lgkm_wait<2 * (i + PS < 2 * NKD ? PS : 2 * NKD - 1 - i)>();
        hold(oa[sl]);
        hold(ob[sl]);
        if constexpr (isdp) {
          dp = H::mfma(oa[sl], ob[sl], dp);
          hold(dp);
        } else {
          st = H::mfma(oa[sl], ob[sl], st);
          hold(st);
        }
        if constexpr (i < 2 * NS) dma(std::integral_constant<int, 1 - BUF>{}, ic);
      });
      dma_on = false;
    }

    // lse, delta and the mask words read together: one LDS round trip
    const uint64_t mw = (BUF ? M1 : M0)[kloc];
    f32x4 dv4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 lv = *(const f32x4*)&Lb[8 * j + 4 * hi];
      dv4[j] = *(const f32x4*)&Gb[8 * j + 4 * hi];
#pragma unroll
      for (int i = 0; i < 4; ++i) st[4 * j + i] = fast_exp2(fmaf(st[4 * j + i], mc, -lv[i]));
    }
    asm volatile("" ::"v"(mw));  // keeps the mask-word read with the others (not sunk into the branch)
    if (masked) {
      const uint32_t w32 = (uint32_t)(mw >> (32 * qh)) >> (4 * hi);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        st[r] = mask_zero(st[r], mask_ones(w32, r));
    }
    u32x4 pk[2], sk[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * j + i;
        dp[r] = st[r] * fmaf(dp[r], ivs, -dv4[j][i]);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      pk[r >> 3][(r & 7) >> 1] = H::pack2(st[r], st[r + 1]);
      sk[r >> 3][(r & 7) >> 1] = H::pack2(dp[r], dp[r + 1]);
    }
    if constexpr (DS) {
      // sk[t] holds queries 16 t + 4 hi + 8 j + i of key kloc (slots 4 j + i):
      // the chunk of lane `lane` in block (2 lhalf + qh, kg, t)
      sf[0] = sk[0];
      sf[1] = sk[1];
      dpend = (BUF ? dsp1 : dsp0) + (8 * qh + 2 * kg) * 512;
    }
    {
      // dV^T / dK^T pipelined by hand like S / dP.  Per 16-query k-step ks, the
      // four dV MFMAs (one per 32-row d tile mt), then the four dK MFMAs (an
      // accumulator recurs 8 MFMAs later).  Step i reads the two transposed
      // 8-byte halves of its A operand, issued PT steps ahead.
      constexpr int PT = 2;
      const uint32_t qb0 = lds_addr(BUF ? Q1 : Q0);  // dO' rows at +2 BM D bytes
      const int tzo = opaque(tz);
      uint32_t am0[NMD], am1[NMD];
#pragma unroll
      for (int mt = 0; mt < NMD; ++mt) {
        const uint32_t xm = 2 * (uint32_t)((32 * mt) ^ tzo);
        am0[mt] = qb0 + 2 * (uint32_t)tb0 + xm;
        am1[mt] = qb0 + 2 * (uint32_t)tb1 + xm;
      }
      constexpr int NSTEP = 4 * NMD;  // (ks, product, mt)
      u32x2 lo[PT + 1], up[PT + 1];
      auto rd = [&](auto ic) {
        constexpr int i = decltype(ic)::value, ks = i / (2 * NMD), isdv = (i / NMD) % 2 == 0, mt = i % NMD;
        constexpr int sl = i % (PT + 1);
        constexpr int off = (isdv ? 2 * BM * D : 0) + 32 * ks * D;
        lo[sl] = ds_read_tr8<off>(am0[mt]);
        up[sl] = ds_read_tr8<off>(am1[mt]);
      };
      static_for<PT>(rd);
      static_for<NSTEP>([&](auto ic) {
        constexpr int i = decltype(ic)::value, ks = i / (2 * NMD), isdv = (i / NMD) % 2 == 0, mt = i % NMD;
        constexpr int sl = i % (PT + 1);
        if constexpr (i + PT < NSTEP) rd(std::integral_constant<int, i + PT>{});
        lgkm_wait<2 * (i + PT < NSTEP ? PT : NSTEP - 1 - i)>();
        hold(lo[sl]);
        hold(up[sl]);
        const u32x4 aop = u32x4{lo[sl][0], lo[sl][1], up[sl][0], up[sl][1]};
        if constexpr (isdv) {
          dv[mt] = H::mfma(aop, pk[ks], dv[mt]);
          hold(dv[mt]);
        } else {
          dk[mt] = H::mfma(aop, sk[ks], dk[mt]);
          hold(dk[mt]);
        }
      });
    }
  };

  // SPLIT: one split sub-block in buffer 0 (Q', dO', lse - log2 f, delta,
  // mask words) and DL (dO'_lo, the rounded-off part of dO' that bwd_pre
  // left in dol; delta of a split tile is taken from the unrounded dO), with
  // the accumulators in its scales: the products of what float16 rounded off
  // when the first kernel's step() computed it.  S, dP, P~ and dS~ are formed
  // again exactly as step() formed them (same operands, same order: the same
  // float32 values), then
  //   dP_e    = dP' + dO'_lo V'^T,   dS~_e = P~ (dP_e / v - delta s)
  //   dV^T   += dO'^T (P~ - float16(P~)) + dO'_lo^T float16(P~)
  //   dK^T   += Q'^T (dS~_e - float16(dS~))
  // with P~ held as float16(P~) + its rounded-off part once packed.  Operands
  // are read with a full wait each (rare work: at the target shape one query
  // tile in 64 of every head).
  auto correct = [&](bool masked) {
    const float mc = m2c;
    const float* Lb = L0 + 32 * qh;
    const float* Gb = G0 + 32 * qh;
    const int rxo = opaque(rx), tzo = opaque(tz);
    const uint32_t qa0 = lds_addr(Q0) + 2 * (uint32_t)qrow;
    const uint32_t la0 = lds_addr(DL) + 2 * (uint32_t)qrow;
    const uint32_t ka0 = lds_addr(Ks) + 2 * (uint32_t)krow_l;
    // acc += A B over the head dimension, A and B row reads at base + offset:
    // at D = 64 each k-step's two reads are issued one step ahead (counted
    // waits); at D = 128, where the split kernel's registers are spent, each
    // read is waited for at once
    constexpr int PC = D == 64 ? 1 : 0;
    auto chain = [&](f32x16& acc, uint32_t ab, auto aoc, uint32_t bb, auto boc) {
      constexpr int AO = decltype(aoc)::value, BO = decltype(boc)::value;
      u32x4 ra[PC + 1], rb[PC + 1];
      auto rd = [&](auto kc) {
        constexpr int kd = decltype(kc)::value, sl = kd % (PC + 1);
        const uint32_t x = 2 * (uint32_t)opaque((16 * kd) ^ rxo);
        ra[sl] = ds_read128<AO>(ab + x);
        rb[sl] = ds_read128<BO>(bb + x);
      };
      static_for<PC>(rd);
      static_for<NKD>([&](auto kc) {
        constexpr int kd = decltype(kc)::value, sl = kd % (PC + 1);
        if constexpr (kd + PC < NKD) rd(std::integral_constant<int, kd + PC>{});
        lgkm_wait<2 * (kd + PC < NKD ? PC : NKD - 1 - kd)>();
        hold(ra[sl]);
        hold(rb[sl]);
        acc = H::mfma(ra[sl], rb[sl], acc);
        hold(acc);
      });
    };
    f32x16 st = f32x16{};
    chain(st, qa0, std::integral_constant<int, 0>{}, ka0, std::integral_constant<int, 0>{});
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 lv = *(const f32x4*)&Lb[8 * j + 4 * hi];
#pragma unroll
      for (int i = 0; i < 4; ++i) st[4 * j + i] = fast_exp2(fmaf(st[4 * j + i], mc, -lv[i]));
    }
    if (masked) {
      const uint64_t mw = M0[kloc];
      const uint32_t w32 = (uint32_t)(mw >> (32 * qh)) >> (4 * hi);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        st[r] = mask_zero(st[r], mask_ones(w32, r));
    }
    u32x4 pk[2], plo[2], slo[2];
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const uint32_t wp = H::pack2(st[r], st[r + 1]);
      pk[r >> 3][(r & 7) >> 1] = wp;
      plo[r >> 3][(r & 7) >> 1] = H::pack2(st[r] - H::to_f32(wp & 0xffffu), st[r + 1] - H::to_f32(wp >> 16));
    }
    f32x16 dp = f32x16{};
    chain(dp, qa0, std::integral_constant<int, 2 * BM * D>{}, ka0, std::integral_constant<int, 2 * TILE * D>{});
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // step()'s dS~, in place of dP'
      const f32x4 gv = *(const f32x4*)&Gb[8 * j + 4 * hi];
#pragma unroll
      for (int i = 0; i < 4; ++i) dp[4 * j + i] = st[4 * j + i] * fmaf(dp[4 * j + i], ivs, -gv[i]);
    }
    f32x16 dl = f32x16{};
    chain(dl, la0, std::integral_constant<int, 0>{}, ka0, std::integral_constant<int, 2 * TILE * D>{});
    // dS~_e - float16(dS~) = (dS~ - float16(dS~)) + P~ (dO'_lo V'^T) / v
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const uint32_t ws = H::pack2(dp[r], dp[r + 1]), wp = pk[r >> 3][(r & 7) >> 1], wl = plo[r >> 3][(r & 7) >> 1];
      const float p0 = H::to_f32(wp & 0xffffu) + H::to_f32(wl & 0xffffu);
      const float p1 = H::to_f32(wp >> 16) + H::to_f32(wl >> 16);
      slo[r >> 3][(r & 7) >> 1] = H::pack2(fmaf(p0 * dl[r], ivs, dp[r] - H::to_f32(ws & 0xffffu)),
                                           fmaf(p1 * dl[r + 1], ivs, dp[r + 1] - H::to_f32(ws >> 16)));
    }
    const uint32_t qb0 = lds_addr(Q0), lb = lds_addr(DL);
    // the six transposed reads of step i (dO', Q', dO'_lo), issued PC steps ahead
    u32x2 tr[PC + 1][6];
    auto rt = [&](auto ic) {
      constexpr int i = decltype(ic)::value, ks = i / NMD, mt = i % NMD, sl = i % (PC + 1);
      const uint32_t xm = 2 * (uint32_t)opaque((32 * mt) ^ tzo);
      const uint32_t x0 = 2 * (uint32_t)tb0 + xm, x1 = 2 * (uint32_t)tb1 + xm;
      tr[sl][0] = ds_read_tr8<2 * BM * D + 32 * ks * D>(qb0 + x0);
      tr[sl][1] = ds_read_tr8<2 * BM * D + 32 * ks * D>(qb0 + x1);
      tr[sl][2] = ds_read_tr8<32 * ks * D>(qb0 + x0);
      tr[sl][3] = ds_read_tr8<32 * ks * D>(qb0 + x1);
      tr[sl][4] = ds_read_tr8<32 * ks * D>(lb + x0);
      tr[sl][5] = ds_read_tr8<32 * ks * D>(lb + x1);
    };
    static_for<PC>(rt);
    static_for<2 * NMD>([&](auto ic) {
      constexpr int i = decltype(ic)::value, ks = i / NMD, mt = i % NMD, sl = i % (PC + 1);
      if constexpr (i + PC < 2 * NMD) rt(std::integral_constant<int, i + PC>{});
      lgkm_wait<6 * (i + PC < 2 * NMD ? PC : 2 * NMD - 1 - i)>();
#pragma unroll
      for (int r = 0; r < 6; ++r) hold(tr[sl][r]);
      const u32x2* t = tr[sl];
      dv[mt] = H::mfma(u32x4{t[0][0], t[0][1], t[1][0], t[1][1]}, plo[ks], dv[mt]);
      hold(dv[mt]);
      dv[mt] = H::mfma(u32x4{t[4][0], t[4][1], t[5][0], t[5][1]}, pk[ks], dv[mt]);
      hold(dv[mt]);
      dk[mt] = H::mfma(u32x4{t[2][0], t[2][1], t[3][0], t[3][1]}, slo[ks], dk[mt]);
      hold(dk[mt]);
    });
  };
  // SPLIT: the column's split sub-blocks (every wave finds the same ones: a
  // ballot over the column list of each query head, 64 entries at a time),
  // each loaded into buffer 0 and DL as launch() loads a sub-block, then
  // correct() in that sub-block's scales.  The K' / V' tiles are resident.
  auto split_pass = [&]() {
    for (int g = 0; g < a.G; ++g) {
      const int h = hk * a.G + g;
      const int mc = map_row(a, b, h, a.nkt, kt);
      const int c0 = a.col_ptr[mc], c1 = a.col_ptr[mc + 1];
      const int64_t hb = (int64_t)b * a.Hq + h;
      for (int base = c0; base < c1; base += 64) {
        const int idx = min(base + lane, c1 - 1);
        const int qt_l = a.col_ent[2 * idx], mk_l = a.col_ent[2 * idx + 1];
        const float as_l = a.asc[hb * a.nqt + qt_l];
        uint64_t todo = __ballot(base + lane < c1 && as_l < 0.f);
        while (todo) {
          const int j = __builtin_ctzll(todo);
          todo &= todo - 1;
          const int qt = __builtin_amdgcn_readlane(qt_l, j), mid = __builtin_amdgcn_readlane(mk_l, j);
          const float sp_s = -__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, as_l), j));
          const float sp_r = a.qsc[hb * a.nqt + qt];
          for (int half = 0; half < 2; ++half) {
            const uint32_t* sr = a.srow + (hb * a.nqt + qt) * 4 + 2 * half;
            if ((sr[0] | sr[1]) == 0u) continue;  // no split row in this half (uniform)
            const int q0 = qt * TILE + half * BM;
            const int64_t rows = (hb * hrows + q0) * D;
#pragma unroll
            for (int k = 0; k < NS; ++k) {
              lds_load16((const char*)(a.qh + rows) + qld[k], Q0 + wofs + k * BLK);
              lds_load16((const char*)(a.doh + rows) + qld[k], H0 + wofs + k * BLK);
              lds_load16((const char*)(a.dol + rows) + qld[k], DL + wofs + k * BLK);
            }
            if (mid >= 0 && wv < 4) {
              const uint32_t* src = (const uint32_t*)(a.col_bits + ((int64_t)mid * 2 + half) * TILE + wv * 32);
              __builtin_amdgcn_global_load_lds(src + lane, (__attribute__((address_space(3))) void*)(M0 + wv * 32),
                                               4, 0, 0);
            }
            if (wv >= 6)
              __builtin_amdgcn_global_load_lds((wv == 6 ? a.lsf : a.delta) + hb * a.Lq + min(q0 + lane, a.Lq - 1),
                                               (__attribute__((address_space(3))) void*)(wv == 6 ? L0 : G0), 4, 0, 0);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (sp_s != acc_s || sp_r != acc_r) {  // the sub-block's scales, as step() takes them
              const float fv = sp_s / acc_s, fk = fv * (sp_r / acc_r);
#pragma unroll
              for (int i = 0; i < NMD; ++i) { dv[i] *= fv; dk[i] *= fk; }
              acc_s = sp_s;
              acc_r = sp_r;
              m2c = c2 * pow2_rcp(sp_r * ksc);
            }
            {  // this wave's split rows of the sub-block, and their allowed keys among the wave's 32
              const uint32_t ws = sr[qh];
              const uint32_t w = mid >= 0 ? (uint32_t)(M0[kloc] >> (32 * qh)) : 0xffffffffu;
              if (__any((w & ws) != 0u)) correct(mid >= 0);
            }
            __syncthreads();  // buffer 0 and DL are read: the next loads may come
          }
        }
      }
    }
  };

  // sub-block s computes from buffer s % 2 while s + 1 loads into the other;
  // the loop is unrolled by two so that every buffer index is static
  auto iter = [&](int s, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    if (s + 1 < tot) prep(std::integral_constant<int, 1 - BUF>{}, std::false_type{});
    if (s > 0) {  // (sub-block 0: the prologue's wait and barrier)
      __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of sub-block s have landed
      __syncthreads();                // ... and every wave's; sub-block s-1 fully consumed
    }
    const bool masked = (BUF ? mid1 : mid0) >= 0;
    if (s + 1 < tot) launch(std::integral_constant<int, 1 - BUF>{});
    if constexpr (DS) {
      if (dpend) store_ds();  // sub-block s - 1's fragments
    }
    step(bufc, masked);
  };
  if (tot > 0) {
    prep(std::integral_constant<int, 0>{}, std::true_type{});
    launch(std::integral_constant<int, 0>{});
    static_for<2 * NS>([&](auto ic) { dma(std::integral_constant<int, 0>{}, ic); });  // no step to carry them
    dma_on = false;
  }
  if constexpr (SPLIT) {
    ksc = a.ksc[col];
    ivs = pow2_rcp(a.vsc[col]);
    m2c = c2 * pow2_rcp(acc_r * ksc);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // this wave's K' and V' loads have landed
    barrier_lds();                               // the K' / V' tiles are complete
  } else {
    // K' tile: float16 times the tile's copy_scale, into the resident LDS tile
    // and to kh for the dQ kernel.  4 threads per key row.  The tile's max
    // |K| meets through an LDS-only barrier (the V' and first sub-block loads
    // stay in flight); the kh stores go out after the barrier that completes
    // the tiles, so that no wait before the first sub-block covers them.
    constexpr int CPL = TileRows<D>::CPL;
    float km = tile_absmax<D, Tag>(tkr);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) km = fmaxf(km, __shfl_xor(km, o));
    if (lane == 0) red[wave] = f32x2{km, 0.f};
    barrier_lds_dma_in_flight();
#pragma unroll
    for (int w = 0; w < 8; ++w) km = fmaxf(km, red[w][0]);
    const float kscl = copy_scale(km);
    const int r = tid >> 2, part = tid & 3;
    u32x4 yk[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = TileRows<D>::chunk(part, j);
      yk[j] = chunk_f16<Tag>(tkr.x[j], kscl);
      *(u32x4*)&Ks[sw_off<D>(r, c)] = yk[j];
    }
    ksc = kscl;
    ivs = pow2_rcp(a.vsc[col]);
    m2c = c2 * pow2_rcp(acc_r * ksc);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // this wave's V' and sub-block 0 loads have landed
    barrier_lds();                               // the K' / V' tiles and sub-block 0 are complete
    uint16_t* kd = a.kh + ((int64_t)col * TILE + r) * D;
#pragma unroll
    for (int j = 0; j < CPL; ++j) __builtin_nontemporal_store(yk[j], (u32x4*)(kd + 8 * TileRows<D>::chunk(part, j)));
    if (tid == 0) a.ksc[col] = kscl;
  }
  if (tot > 0) {  // the first sub-block's scales, loaded with its entry
    cur_r = rh0 = first_r;
    cur_s = first_s;
    sh0 = fabsf(first_s);
  }
  for (int s = 0; s < tot; s += 2) {
    iter(s, std::integral_constant<int, 0>{});
    if (s + 1 < tot) iter(s + 1, std::integral_constant<int, 1>{});
  }
  if constexpr (SPLIT) {
    split_pass();
  } else if constexpr (FUSED) {
    // a flagged column corrects its split sub-blocks now, once every wave is
    // done with the LDS of the walk (uniform)
    if (col_split) {
      __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // (no load is in flight after the walk; stores may be)
      barrier_lds();
      if constexpr (DS) {
        if (dpend) {  // the last sub-block's fragments, before the pass reuses the registers
          store_ds();
          dpend = nullptr;
        }
      }
      split_pass();
    }
  }

  // dK / dV: the second query half's partials join the first's through LDS
  // (wave kg + 4 -> wave kg; per key group a dK slab in the K / V tiles and a
  // dV slab in a Q / dO_h buffer, all free now; lane-major 16-byte chunks).  Wave kg
  // then writes the finished rows of its 32 keys, scaled and rounded, over its
  // own slabs as [32 keys][D + 8] tiles, and all 8 waves store the 128 x D
  // tiles with 16-byte accesses along the rows.
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // (the dS~ stores of the sub-block before the last)
  barrier_lds();                               // every wave is done with the LDS
  if constexpr (DS) {
    if (dpend) store_ds();  // the last sub-block's fragments, in flight during the reduction below
  }
  constexpr int SLAB = NMD * 16 * 64;  // floats
  constexpr int OR = D + 8;            // staged row (elements): 16-byte aligned, spreads banks
  static_assert(2 * SLAB * 4 <= TILE * D * 2 && SLAB * 4 <= BM * D * 2 && 32 * OR * 2 <= SLAB * 4,
                "reduction slabs");
  float* redk = (float*)(kg < 2 ? Ks : Vs) + (kg & 1) * SLAB;
  float* redv = (float*)(kg == 0 ? Q0 : kg == 1 ? Q1 : kg == 2 ? H0 : H1);
  // slab layout: float j of lane-chunk (mt, c) at ((mt * 4 + c) * 64 + lane) * 4 + j
  if (qh == 1) {
#pragma unroll
    for (int mt = 0; mt < NMD; ++mt)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        ((f32x4*)redk)[(mt * 4 + c) * 64 + lane] = f32x4{dk[mt][4 * c], dk[mt][4 * c + 1], dk[mt][4 * c + 2], dk[mt][4 * c + 3]};
        ((f32x4*)redv)[(mt * 4 + c) * 64 + lane] = f32x4{dv[mt][4 * c], dv[mt][4 * c + 1], dv[mt][4 * c + 2], dv[mt][4 * c + 3]};
      }
  }
  barrier_lds();
  if (qh == 0) {
    // the slabs are this wave's alone: the rows overwrite them after the reads
    auto finish = [&](f32x16 (&acc)[NMD], float* red, float sc, float unit, float* keep) {
#pragma unroll
      for (int mt = 0; mt < NMD; ++mt)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 x = ((const f32x4*)red)[(mt * 4 + c) * 64 + lane];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[mt][4 * c + j] += x[j];
        }
      if constexpr (!SPLIT && !FUSED) {
        if (col_split) {  // for the split kernel, in units of 1 (powers of two: exact)
#pragma unroll
          for (int mt = 0; mt < NMD; ++mt) *(f32x16*)&keep[(mt * 64 + lane) * 16] = acc[mt] * unit;
        }
      }
      uint16_t* o = (uint16_t*)red + l32 * OR;
#pragma unroll
      for (int mt = 0; mt < NMD; ++mt) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *(u32x2*)(o + 32 * mt + 8 * j + 4 * hi) =
              u32x2{E::pack2(acc[mt][4 * j] * sc, acc[mt][4 * j + 1] * sc),
                    E::pack2(acc[mt][4 * j + 2] * sc, acc[mt][4 * j + 3] * sc)};
      }
    };
    finish(dk, redk, a.scale * pow2_rcp(acc_s * acc_r), pow2_rcp(acc_s * acc_r), part);
    finish(dv, redv, pow2_rcp(acc_s), pow2_rcp(acc_s), part + NMD * 16 * 64);
  }
  barrier_lds();
  constexpr int CPR = D / 8;  // 16-byte chunks per row
#pragma unroll
  for (int i = 0; i < TILE * CPR / 512; ++i) {
    const int n = tid + 512 * i;
    const int kl = n / CPR, c = n % CPR;  // key within the tile, chunk
    const int key_n = kt * TILE + kl;
    const int g = kl >> 5, off = (kl & 31) * OR + 8 * c;
    const float* sk = (const float*)(g < 2 ? Ks : Vs) + (g & 1) * SLAB;
    const float* sv = (const float*)(g == 0 ? Q0 : g == 1 ? Q1 : g == 2 ? H0 : H1);
    const u32x4 xk = *(const u32x4*)((const uint16_t*)sk + off);
    const u32x4 xv = *(const u32x4*)((const uint16_t*)sv + off);
    if (key_n < a.Lk) {
      __builtin_nontemporal_store(xk, (u32x4*)((char*)a.dk + 2 * ((int64_t)b * a.dks[0] + (int64_t)key_n * a.dks[1] + (int64_t)hk * a.dks[2] + 8 * c)));
      __builtin_nontemporal_store(xv, (u32x4*)((char*)a.dv + 2 * ((int64_t)b * a.dvs[0] + (int64_t)key_n * a.dvs[1] + (int64_t)hk * a.dvs[2] + 8 * c)));
    }
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------

template <int D, class Tag>
static void launch_dkdv_t(const KArgs& a, int grid, hipStream_t st) {
  if (a.ds) hipLaunchKernelGGL((bwd_dkdv_mfma<D, Tag, true, false>), dim3(grid), dim3(512), 0, st, a);
  else hipLaunchKernelGGL((bwd_dkdv_mfma<D, Tag, false, false>), dim3(grid), dim3(512), 0, st, a);
  // the columns that met a split tile again (the others' workgroups return at
  // once); at D = 64 the first kernel corrects them itself
  if constexpr (D != 64) hipLaunchKernelGGL((bwd_dkdv_mfma<D, Tag, false, true>), dim3(grid), dim3(512), 0, st, a);
}

hipError_t launch_dkdv(const KArgs& a, int D, int dtype, int grid, hipStream_t st) {
  if (dtype == MATTN_BF16) {
    if (D == 64) launch_dkdv_t<64, bf16_tag>(a, grid, st);
    else launch_dkdv_t<128, bf16_tag>(a, grid, st);
  } else {
    if (D == 64) launch_dkdv_t<64, f16_tag>(a, grid, st);
    else launch_dkdv_t<128, f16_tag>(a, grid, st);
  }
  return hipGetLastError();
}

}  // namespace mattn
