// C ABI of the library (declared in include/mattn.h): argument validation,
// workspace layouts, kernel-argument packing and launch selection.  Host code
// only; the kernels live in fwd.hip, bwd_pre.hip, bwd_dkdv.hip, bwd_dq.hip
// (16-bit inputs, D = 64 and 128: MFMA) and simt.hip (float32 inputs, and
// every input dtype at D = 256 and 512: float32 SIMT arithmetic).
#include <math.h>

#include <mutex>

#include "common.hpp"

namespace mattn {
hipError_t launch_fwd(const KArgs& a, int D, int dtype, int o_dtype, bool simt, int grid, hipStream_t st);
hipError_t launch_bwd_stage(const KArgs& a, int D, int dtype, int o_dtype, bool simt, int stage, int q_grid,
                            int kv_grid, hipStream_t st);
}  // namespace mattn

using namespace mattn;

namespace {

constexpr int kAbiVersion = 8;

int elem_size(int dt) { return dt == MATTN_F32 ? 4 : 2; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool strides_ok(const int64_t s[3], int esz) {
  for (int i = 0; i < 3; ++i)
    if (s[i] < 0 || (s[i] * esz) % 16 != 0) return false;
  return true;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// problems served by the SIMT kernels (float32 arithmetic), which need no
// residual and no backward workspace beyond one float per query row
bool simt_path(const mattn_problem* p) {
  return p->dtype == MATTN_F32 || p->D > 128 || (p->flags & MATTN_PRECISE);
}

// the backward keeps dS (MATTN_BWD_DS on the MFMA path)
bool ds_path(const mattn_problem* p) { return (p->flags & MATTN_BWD_DS) && !simt_path(p); }

// dS tiles of the whole problem: the map's present tiles once per (b, h) it covers
size_t ds_slots(const mattn_problem* p, const mattn_blockmap* bm) {
  return (size_t)bm->nnz * (bm->map_b == 1 ? p->B : 1) * (bm->map_h == 1 ? p->Hq : 1);
}

// Forward residual (16-bit inputs, D <= 128): V as float16 times a power of two per
// 128-key tile, [B, Hkv, nkt * 128, D]; Q likewise per 128-query tile,
// [B, Hq, nqt * 128, D] (written when MATTN_FWD_FOR_BWD is set); each tile's
// scale, each V tile's max |V|, and per query tile the largest attention
// weight of its rows and the mask of its split rows (rows whose largest
// weight reaches SPLIT_P: their forward and backward terms are formed free of
// the float16 rounding of their operands), and per key tile a flag: a split
// row has an allowed key there (its dK/dV column then takes the split
// products; cleared by the V' conversion, set by the split rows' walk).
// MATTN_PRECISE on the SIMT kernels: what the stored lse and O round off
// (float32, [B, Hq, Lq] and [B, Hq, Lq, D]), which the backward adds back.
struct FwdWs {
  size_t vh, qh, vsc, vmax, qsc, pmx, srow, scol, lse_lo, o_lo, total;
};

FwdWs fwd_ws_layout(const mattn_problem* p) {
  FwdWs w{};
  if (simt_path(p)) {
    if (p->flags & MATTN_PRECISE) {
      const size_t rows = (size_t)p->B * p->Hq * p->Lq;
      w.o_lo = align256(rows * sizeof(float));
      w.total = w.o_lo + align256(rows * p->D * sizeof(float));
    }
    return w;
  }
  const size_t ktiles = (size_t)p->B * p->Hkv * cdiv(p->Lk, MATTN_TILE_K);
  const size_t qtiles = (size_t)p->B * p->Hq * cdiv(p->Lq, MATTN_TILE_Q);
  w.vh = 0;
  w.qh = align256(ktiles * MATTN_TILE_K * p->D * 2);
  w.vsc = w.qh + align256(qtiles * MATTN_TILE_Q * p->D * 2);
  w.vmax = w.vsc + align256(ktiles * sizeof(float));
  w.qsc = w.vmax + align256(ktiles * sizeof(float));
  w.pmx = w.qsc + align256(qtiles * sizeof(float));
  w.srow = w.pmx + align256(qtiles * sizeof(float));
  w.scol = w.srow + align256(qtiles * 4 * sizeof(uint32_t));
  w.total = w.scol + align256(ktiles * sizeof(int));
  return w;
}

// Backward workspace: delta (f32 per query row); for 16-bit inputs at D <= 128
// (the MFMA kernels) also the
// shifted lse (f32 per query row), the float16 copies dO' ([B, Hq, nqt * 128,
// D]) and K' ([B, Hkv, nkt * 128, D]), and per 128-row tile the dO' scale, the
// dS bounds and scale of the query tiles and the K' scale of the key tiles;
// then the rounded-off part of dO' ([B, Hq, nqt * 128, D] float16, written and
// read only in the rows of split tiles) and the unrounded dK and dV of a key
// tile whose column a split row reaches (float32, [ktiles][2][128][D], written
// and read only for those columns; the flags are in the forward's residual).
struct WsLayout {
  size_t delta, lsf, doh, kh, dsc, tst, asc, ksc, dol, kvp, total;
};

WsLayout ws_layout(const mattn_problem* p) {
  const size_t rows = (size_t)p->B * p->Hq * p->Lq;
  WsLayout w{};
  w.delta = 0;
  w.total = align256(rows * sizeof(float));
  if (simt_path(p)) return w;
  const size_t qtiles = (size_t)p->B * p->Hq * cdiv(p->Lq, MATTN_TILE_Q);
  const size_t ktiles = (size_t)p->B * p->Hkv * cdiv(p->Lk, MATTN_TILE_K);
  w.lsf = w.total;
  w.doh = w.lsf + align256(rows * sizeof(float));
  w.kh = w.doh + align256(qtiles * MATTN_TILE_Q * p->D * 2);
  w.dsc = w.kh + align256(ktiles * MATTN_TILE_K * p->D * 2);
  w.tst = w.dsc + align256(qtiles * sizeof(float));
  w.asc = w.tst + align256(qtiles * 8);
  w.ksc = w.asc + align256(qtiles * sizeof(float));
  w.dol = w.ksc + align256(ktiles * sizeof(float));
  w.kvp = w.dol + align256(qtiles * MATTN_TILE_Q * p->D * 2);
  w.total = w.kvp + align256(ktiles * MATTN_TILE_K * p->D * 2 * sizeof(float));
  return w;
}

KArgs make_args(const mattn_problem* p, const mattn_blockmap* bm) {
  KArgs a{};
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = p->q_stride[i];
    a.ks[i] = p->k_stride[i];
    a.vs[i] = p->v_stride[i];
    a.os[i] = p->o_stride[i];
    a.dos[i] = p->do_stride[i];
    a.dqs[i] = p->dq_stride[i];
    a.dks[i] = p->dk_stride[i];
    a.dvs[i] = p->dv_stride[i];
  }
  a.B = p->B;
  a.Lq = p->Lq;
  a.Lk = p->Lk;
  a.Hq = p->Hq;
  a.Hkv = p->Hkv;
  a.G = p->Hq / p->Hkv;
  a.scale = p->scale;
  a.scale_log2 = p->scale * 1.4426950408889634f;
  a.map_b = bm->map_b;
  a.map_h = bm->map_h;
  a.nqt = bm->nqt;
  a.nkt = bm->nkt;
  a.row_ptr = bm->row_ptr;
  a.row_ent = bm->row_ent;
  a.col_ptr = bm->col_ptr;
  a.col_ent = bm->col_ent;
  a.row_bits = bm->row_bits;
  a.col_bits = bm->col_bits;
  a.q_order = bm->q_order;
  a.kv_order = bm->kv_order;
  a.kv_desc = bm->kv_desc;
  a.precise = (p->flags & MATTN_PRECISE) ? 1 : 0;
  return a;
}

}  // namespace

extern "C" {

int mattn_abi_version(void) { return kAbiVersion; }

const char* mattn_strerror(int status) {
  switch (status) {
    case MATTN_OK: return "success";
    case MATTN_ERR_NULL: return "a required pointer is NULL";
    case MATTN_ERR_SHAPE: return "invalid shape (sizes must be positive and Hq divisible by Hkv)";
    case MATTN_ERR_HEAD_DIM: return "unsupported head dimension (supported: 64, 128, 256, 512)";
    case MATTN_ERR_DTYPE: return "unsupported dtype combination";
    case MATTN_ERR_STRIDE: return "pointer or stride not 16-byte aligned";
    case MATTN_ERR_BLOCKMAP: return "block map inconsistent with the problem";
    case MATTN_ERR_LAUNCH: return "kernel launch failed";
    case MATTN_ERR_TOO_LARGE: return "problem exceeds 32-bit index ranges";
    case MATTN_ERR_SCRATCH: return "backward workspace exceeds the library's static scratch (MATTN_SCRATCH_BYTES; clear MATTN_BWD_DS)";
    case MATTN_ERR_DEVICE: return "the HIP runtime could not resolve the device or its scratch, or the stream belongs to another device";
    case MATTN_ERR_WORKSPACE: return "workspace smaller than mattn_bwd_workspace_bytes(p, bm)";
    case MATTN_ERR_RESIDUAL: return "the backward needs the float16 Q copy: run the forward with MATTN_FWD_FOR_BWD and pass that flag to the backward";
    default: return "unknown status";
  }
}

int mattn_validate(const mattn_problem* p, const mattn_blockmap* bm) {
  if (!p) return MATTN_ERR_NULL;
  if (p->B <= 0 || p->Lq <= 0 || p->Lk <= 0 || p->Hq <= 0 || p->Hkv <= 0 || p->D <= 0)
    return MATTN_ERR_SHAPE;
  if (p->Hq % p->Hkv != 0) return MATTN_ERR_SHAPE;
  if (p->D != 64 && p->D != 128 && p->D != 256 && p->D != 512) return MATTN_ERR_HEAD_DIM;
  if (p->dtype != MATTN_BF16 && p->dtype != MATTN_F16 && p->dtype != MATTN_F32) return MATTN_ERR_DTYPE;
  if (p->o_dtype != p->dtype && p->o_dtype != MATTN_F32) return MATTN_ERR_DTYPE;
  if (!(p->scale > 0.f) || isinf(p->scale)) return MATTN_ERR_SHAPE;  // positive, finite
  if (p->flags & ~(MATTN_FWD_FOR_BWD | MATTN_BWD_DS | MATTN_PRECISE)) return MATTN_ERR_SHAPE;
  const int es = elem_size(p->dtype), eo = elem_size(p->o_dtype);
  if (!strides_ok(p->q_stride, es) || !strides_ok(p->k_stride, es) || !strides_ok(p->v_stride, es) ||
      !strides_ok(p->dq_stride, es) || !strides_ok(p->dk_stride, es) ||
      !strides_ok(p->dv_stride, es) || !strides_ok(p->o_stride, eo) || !strides_ok(p->do_stride, eo))
    return MATTN_ERR_STRIDE;
  const int64_t nqt = cdiv(p->Lq, MATTN_TILE_Q), nkt = cdiv(p->Lk, MATTN_TILE_K);
  if ((int64_t)p->B * p->Hq * p->Lq >= (1ll << 31) || (int64_t)p->B * p->Hkv * p->Lk >= (1ll << 31) || (int64_t)p->B * p->Hq * nqt >= (1ll << 31) || (int64_t)p->B * p->Hkv * nkt >= (1ll << 31) ||
      (int64_t)p->Lq + MATTN_TILE_Q >= (1ll << 31) || (int64_t)p->Lk + MATTN_TILE_K >= (1ll << 31))
    return MATTN_ERR_TOO_LARGE;
  // kernels address rows inside one (batch, head) slice with 32-bit offsets:
  // element offsets along the inputs' sequence strides, and byte offsets
  // (buffer resources of the dK/dV kernel) inside one head's float16 copy
  const int64_t lim = (1ll << 31) - 1;
  if ((int64_t)(nqt * MATTN_TILE_Q) * p->q_stride[1] > lim ||
      (int64_t)(nkt * MATTN_TILE_K) * p->k_stride[1] > lim ||
      (int64_t)(nkt * MATTN_TILE_K) * p->v_stride[1] > lim ||
      (int64_t)(nqt * MATTN_TILE_Q) * p->D * 2 > lim || (int64_t)(nkt * MATTN_TILE_K) * p->D * 2 > lim)
    return MATTN_ERR_TOO_LARGE;
  if (!bm) return MATTN_OK;
  if (bm->nqt != nqt || bm->nkt != nkt) return MATTN_ERR_BLOCKMAP;
  if (!(bm->map_b == 1 || bm->map_b == p->B) || !(bm->map_h == 1 || bm->map_h == p->Hq))
    return MATTN_ERR_BLOCKMAP;
  if (bm->n_masks < 0 || bm->nnz < 0 || bm->n_q_order <= 0 || bm->n_kv_order <= 0)
    return MATTN_ERR_BLOCKMAP;
  if (bm->n_q_order < p->B * p->Hq * nqt || bm->n_kv_order < p->B * p->Hkv * nkt)
    return MATTN_ERR_BLOCKMAP;
  if (!bm->row_ptr || !bm->col_ptr || !bm->q_order || !bm->kv_order) return MATTN_ERR_NULL;
  if (bm->nnz > 0 && (!bm->row_ent || !bm->col_ent)) return MATTN_ERR_NULL;
  if (bm->n_masks > 0 && (!bm->row_bits || !bm->col_bits)) return MATTN_ERR_NULL;
  return MATTN_OK;
}

size_t mattn_workspace_bytes(const mattn_problem* p) {
  if (mattn_validate(p, nullptr) != MATTN_OK) return 0;
  return ws_layout(p).total;
}

size_t mattn_bwd_workspace_bytes(const mattn_problem* p, const mattn_blockmap* bm) {
  if (!bm || mattn_validate(p, bm) != MATTN_OK) return 0;
  const size_t base = ws_layout(p).total;
  return ds_path(p) ? base + ds_slots(p, bm) * DS_TILE * 2 : base;
}

size_t mattn_fwd_workspace_bytes(const mattn_problem* p) {
  if (mattn_validate(p, nullptr) != MATTN_OK) return 0;
  return fwd_ws_layout(p).total;
}

int mattn_fwd(const mattn_problem* p, const mattn_blockmap* bm, const void* q, const void* k,
              const void* v, void* o, float* lse, void* workspace, void* stream) {
  int rc = mattn_validate(p, bm);
  if (rc != MATTN_OK) return rc;
  if (!bm) return MATTN_ERR_NULL;
  if (!q || !k || !v || !o || !lse) return MATTN_ERR_NULL;
  const FwdWs w = fwd_ws_layout(p);
  if (w.total > 0 && !workspace) return MATTN_ERR_NULL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || ((uintptr_t)workspace & 255u))
    return MATTN_ERR_STRIDE;
  KArgs a = make_args(p, bm);
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = o;
  a.lse = lse;
  char* ws = (char*)workspace;
  if (w.total > 0 && simt_path(p)) {
    a.lse_lo = (float*)(ws + w.lse_lo);
    a.o_lo = (float*)(ws + w.o_lo);
  } else if (w.total > 0) {
    a.vh = (uint16_t*)(ws + w.vh);
    a.vsc = (float*)(ws + w.vsc);
    a.vmax = (float*)(ws + w.vmax);
    a.qsc = (float*)(ws + w.qsc);
    a.qh = (p->flags & MATTN_FWD_FOR_BWD) ? (uint16_t*)(ws + w.qh) : nullptr;
    a.pmx = (float*)(ws + w.pmx);
    a.srow = (uint32_t*)(ws + w.srow);
    a.scol = (int*)(ws + w.scol);
  }
  hipError_t e = launch_fwd(a, p->D, p->dtype, p->o_dtype, simt_path(p), bm->n_q_order, (hipStream_t)stream);
  return e == hipSuccess ? MATTN_OK : MATTN_ERR_LAUNCH;
}

int mattn_bwd_stage(const mattn_problem* p, const mattn_blockmap* bm, int stage, const void* q,
                    const void* k, const void* v, const void* o, const void* do_, const float* lse,
                    const void* residual, void* workspace, size_t workspace_bytes, void* dq, void* dk,
                    void* dv, void* stream) {
  int rc = mattn_validate(p, bm);
  if (rc != MATTN_OK) return rc;
  if (!bm) return MATTN_ERR_NULL;
  if (stage != MATTN_BWD_PRE && stage != MATTN_BWD_DKDV && stage != MATTN_BWD_DQ) return MATTN_ERR_SHAPE;
  if (!q || !k || !v || !o || !do_ || !lse || !workspace || !dq || !dk || !dv) return MATTN_ERR_NULL;
  if (workspace_bytes < mattn_bwd_workspace_bytes(p, bm)) return MATTN_ERR_WORKSPACE;
  if (!simt_path(p) && !(p->flags & MATTN_FWD_FOR_BWD)) return MATTN_ERR_RESIDUAL;
  if (mattn_fwd_workspace_bytes(p) > 0 && !residual) return MATTN_ERR_NULL;
  if (ds_path(p) && bm->nnz > 0 && !bm->col_row) return MATTN_ERR_NULL;
  if (!simt_path(p) && stage == MATTN_BWD_DKDV && !bm->kv_desc) return MATTN_ERR_NULL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(do_) ||
      !aligned16(dq) || !aligned16(dk) || !aligned16(dv) || ((uintptr_t)workspace & 255u) ||
      ((uintptr_t)residual & 255u))
    return MATTN_ERR_STRIDE;
  KArgs a = make_args(p, bm);
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.dO = do_;
  a.lse = const_cast<float*>(lse);
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  const WsLayout w = ws_layout(p);
  char* ws = (char*)workspace;
  a.delta = (float*)(ws + w.delta);
  if (simt_path(p) && (p->flags & MATTN_PRECISE)) {
    const FwdWs r = fwd_ws_layout(p);
    a.lse_lo = (float*)((const char*)residual + r.lse_lo);
    a.o_lo = (float*)((const char*)residual + r.o_lo);
  } else if (!simt_path(p)) {
    a.lsf = (float*)(ws + w.lsf);
    a.doh = (uint16_t*)(ws + w.doh);
    a.kh = (uint16_t*)(ws + w.kh);
    a.dsc = (float*)(ws + w.dsc);
    a.tst = (float2*)(ws + w.tst);
    a.asc = (float*)(ws + w.asc);
    a.ksc = (float*)(ws + w.ksc);
    a.dol = (uint16_t*)(ws + w.dol);
    a.kvp = (float*)(ws + w.kvp);
    const FwdWs r = fwd_ws_layout(p);
    const char* res = (const char*)residual;
    a.vh = (uint16_t*)(res + r.vh);
    a.qh = (uint16_t*)(res + r.qh);
    a.vsc = (float*)(res + r.vsc);
    a.vmax = (float*)(res + r.vmax);
    a.qsc = (float*)(res + r.qsc);
    a.pmx = (float*)(res + r.pmx);
    a.srow = (uint32_t*)(res + r.srow);
    a.scol = (int*)(res + r.scol);
    if (ds_path(p)) {  // dS after the workspace's other parts (w.total is 256-byte aligned)
      a.ds = (uint16_t*)(ws + w.total);
      a.col_row = bm->col_row;
      a.ds_nnz = bm->nnz;
    }
  }
  hipError_t e = launch_bwd_stage(a, p->D, p->dtype, p->o_dtype, simt_path(p), stage, bm->n_q_order,
                                  bm->n_kv_order, (hipStream_t)stream);
  return e == hipSuccess ? MATTN_OK : MATTN_ERR_LAUNCH;
}

int mattn_bwd(const mattn_problem* p, const mattn_blockmap* bm, const void* q, const void* k,
              const void* v, const void* o, const void* do_, const float* lse, const void* residual,
              void* workspace, size_t workspace_bytes, void* dq, void* dk, void* dv, void* stream) {
  for (int stage = MATTN_BWD_PRE; stage <= MATTN_BWD_DQ; ++stage) {
    const int rc = mattn_bwd_stage(p, bm, stage, q, k, v, o, do_, lse, residual, workspace, workspace_bytes,
                                   dq, dk, dv, stream);
    if (rc != MATTN_OK) return rc;
  }
  return MATTN_OK;
}

// ---------------------------------------------------------------------------
// allocation-free backward
// ---------------------------------------------------------------------------
// The workspace of mattn_bwd_noalloc: one array per device, held from module
// load to process end.  Host code must not pass `scratch` itself to a kernel
// (in host code it names a host-side stand-in): the device address comes
// from hipGetSymbolAddress, looked up once per device.
static __device__ __align__(256) unsigned char scratch[MATTN_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// The device address of this device's scratch (nullptr on failure); the
// lookup runs once per device, with that device current.
void* device_scratch(int dev) {
  std::call_once(g_scratch_once[dev], [dev] {
    void* ptr = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? ptr : nullptr;
  });
  return g_scratch_ptr[dev];
}
}  // namespace

int mattn_bwd_noalloc(const mattn_problem* p, const mattn_blockmap* bm, const void* q, const void* k,
                      const void* v, const void* o, const void* do_, const float* lse,
                      const void* residual, void* dq, void* dk, void* dv, void* stream) {
  const int rc = mattn_validate(p, bm);
  if (rc != MATTN_OK) return rc;
  const size_t need = bm ? mattn_bwd_workspace_bytes(p, bm) : ws_layout(p).total;
  if (need > (size_t)MATTN_SCRATCH_BYTES) return MATTN_ERR_SCRATCH;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MATTN_ERR_DEVICE;
  if (stream) {  // the scratch is the current device's: the stream must run there
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || sdev != dev) return MATTN_ERR_DEVICE;
  }
  void* ws = device_scratch(dev);
  if (!ws) return MATTN_ERR_DEVICE;
  return mattn_bwd(p, bm, q, k, v, o, do_, lse, residual, ws, (size_t)MATTN_SCRATCH_BYTES, dq, dk, dv, stream);
}

}  // extern "C"
