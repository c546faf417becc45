/*
 * mattn.h -- C ABI of the MI355X (gfx950) masked-attention library.
 *
 * This is the drop-in boundary for jaxmodules' memory-efficient masked
 * attention.  The reference implements the path in pure JAX:
 *
 *   masked_attention_via_map   /root/reference/jaxmodules/attention.py:347-455
 *   _masked_attention_via_map  attention.py:180-241   (custom_vjp primal)
 *   custom_vjp fwd rule        attention.py:244-264
 *   custom_vjp bwd rule        attention.py:266-342
 *   BlockMask tile lists       /root/reference/jaxmodules/block_mask.py:17-42
 *
 * The reference has no FFI, custom call or plugin registry of its own; these
 * entry points are what a jax.ffi / XLA custom-call target for the custom_vjp
 * rules binds (the primal -> mattn_fwd, the bwd rule -> mattn_bwd).  The host
 * layer (Python) keeps the reference's signature, traces mask_fn into the
 * tile map described by mattn_blockmap and calls these functions.
 *
 * Conventions
 *   - Q is [B, Lq, Hq, D], K and V are [B, Lk, Hkv, D] (the reference's BLHD
 *     layout).  The innermost (D) dimension is contiguous; the batch, sequence
 *     and head strides are given in ELEMENTS.
 *   - Query head h reads key/value head h / (Hq / Hkv) (attention.py:66-68).
 *   - The attention weights are exp(scale * q.k) normalised over the allowed
 *     keys of the row; a row with no allowed key yields O = 0 and zero
 *     gradients (attention.py:91-100).
 *   - All buffers are caller-owned device memory.  The library never
 *     allocates, frees or synchronises on the call path; every launch is
 *     enqueued on the caller's stream.  No kernel uses atomics, so results
 *     are bitwise reproducible.
 *   - Return value 0 is success, a negative value is an error code whose text
 *     is given by mattn_strerror().
 */
#ifndef MATTN_H
#define MATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types.  Q, K, V, dQ, dK, dV share `dtype`; O and dO share `o_dtype`
 * (the reference returns float32 O for bfloat16 inputs, attention.py:173). */
enum mattn_dtype { MATTN_BF16 = 0, MATTN_F16 = 1, MATTN_F32 = 2 };

enum mattn_status {
  MATTN_OK = 0,
  MATTN_ERR_NULL = -1,          /* a required pointer is NULL                  */
  MATTN_ERR_SHAPE = -2,         /* non-positive size or Hq % Hkv != 0          */
  MATTN_ERR_HEAD_DIM = -3,      /* D not in {64, 128, 256, 512}                */
  MATTN_ERR_DTYPE = -4,         /* unsupported dtype / o_dtype combination     */
  MATTN_ERR_STRIDE = -5,        /* misaligned pointer or stride                */
  MATTN_ERR_BLOCKMAP = -6,      /* tile map inconsistent with the problem      */
  MATTN_ERR_LAUNCH = -7,        /* the HIP runtime rejected a launch           */
  MATTN_ERR_TOO_LARGE = -8,     /* a size exceeds 32-bit index ranges          */
  MATTN_ERR_SCRATCH = -9,       /* mattn_bwd_noalloc: workspace > scratch      */
  MATTN_ERR_DEVICE = -10,       /* mattn_bwd_noalloc: no current device/scratch,
                                   or the stream belongs to another device     */
  MATTN_ERR_WORKSPACE = -11,    /* workspace_bytes < mattn_bwd_workspace_bytes */
  MATTN_ERR_RESIDUAL = -12      /* MFMA backward without MATTN_FWD_FOR_BWD: the
                                   residual holds no float16 copy of Q         */
};

/* mattn_problem.flags: the forward also leaves in its residual the float16
 * copy of Q that mattn_bwd reads (set it for a forward whose backward runs). */
#define MATTN_FWD_FOR_BWD 1
/* mattn_problem.flags: the backward keeps dS: the dK/dV stage stores dS of
 * every present tile (float16, 32 KiB per 128 x 128 tile) in the workspace and
 * the dQ stage computes dQ = dS K from it instead of recomputing S and dP.
 * The workspace then takes mattn_bwd_workspace_bytes(p, bm) bytes.  For
 * 16-bit inputs at D <= 128 (ignored on the SIMT path).  Faster at D = 128,
 * where recomputing costs more than streaming 2 bytes per allowed pair. */
#define MATTN_BWD_DS 2
/* mattn_problem.flags: float32 arithmetic for 16-bit inputs.  The problem runs
 * on the SIMT kernels (every product and sum in float32, the inputs read
 * exactly), as float32 inputs do, instead of the MFMA kernels, whose
 * operands P, dS and dO are rounded to float16 (11 significant bits) -- except
 * in split tiles: 128-row query tiles with a row whose largest attention
 * weight reaches 1/32, whose O, lse and gradient terms the MFMA path forms
 * again with those operands' rounded-off parts (22 significant bits) by
 * kernels of their own after the main ones (at D = 64 inside them).  Set it
 * for a forward and for its backward alike; the forward then has no residual.
 * For kernels sharper than the default scale 1/sqrt(d) (the reference's
 * threshold_kernel has scale 1, attention.py:18-36), where rows concentrate
 * on single keys and dS = P (dP - delta) cancels below the float16 operand
 * rounding.  The scores are then compensated dot products (about twice
 * float32's precision) for every dtype, O and the row sums accumulate in
 * float64, and the forward's residual (mattn_fwd_workspace_bytes) holds what
 * the stored lse and O round off (one float per query row and per element of
 * O), which the backward reads. */
#define MATTN_PRECISE 4

/* Tile size of the block map, in queries x keys. */
#define MATTN_TILE_Q 128
#define MATTN_TILE_K 128

typedef struct mattn_problem {
  int32_t B, Lq, Lk, Hq, Hkv, D;
  int32_t dtype;     /* enum mattn_dtype of Q, K, V, dQ, dK, dV            */
  int32_t o_dtype;   /* enum mattn_dtype of O and dO: dtype, or MATTN_F32  */
  float scale;       /* softmax scale; the reference's default_kernel uses
                        1/sqrt(D) (attention.py:39-50)                     */
  int32_t flags;     /* MATTN_FWD_FOR_BWD | MATTN_BWD_DS | MATTN_PRECISE   */
  /* element strides {batch, sequence, head}; D is contiguous */
  int64_t q_stride[3], k_stride[3], v_stride[3], o_stride[3];
  int64_t do_stride[3], dq_stride[3], dk_stride[3], dv_stride[3];
} mattn_problem;

/*
 * Tile map of the effective mask (mask_fn AND the window's visited key blocks
 * AND the unpadded range), at MATTN_TILE_Q x MATTN_TILE_K granularity.  Tiles
 * that are fully masked are absent.  Present tiles are either full (mask id
 * -1) or partial (mask id >= 0 into the bit arrays).  This is the reference
 * BlockMask (block_mask.py:17-42: kv_num_blocks/kv_indices and
 * full_kv_num_blocks/full_kv_indices, plus the transposed q_* lists) in CSR
 * form with the partial tiles' element masks attached.
 *
 * The map may be broadcast over batch and/or heads (map_b == 1, map_h == 1),
 * the way the reference's create_block_mask takes B and H (block_mask.py:454).
 * Map row index of (b, h, tile) = ((b % map_b) * map_h + h % map_h) * n + tile.
 * Every pointer is device memory.
 */
typedef struct mattn_blockmap {
  int32_t map_b, map_h;      /* 1 or B, 1 or Hq                             */
  int32_t nqt, nkt;          /* ceil(Lq / TILE_Q), ceil(Lk / TILE_K)        */
  int32_t n_masks;           /* number of distinct partial-tile masks       */
  int32_t nnz;               /* number of present tiles in the whole map    */
  const int32_t* row_ptr;    /* [map_b*map_h*nqt + 1]                        */
  const int32_t* row_ent;    /* [2*nnz]: (key tile, mask id) per row entry   */
  const int32_t* col_ptr;    /* [map_b*map_h*nkt + 1]                        */
  const int32_t* col_ent;    /* [2*nnz]: (query tile, mask id) per column    */
  /* row_bits[m][w][q]: bit j = key 64*w + j of tile m allowed for query row
   * q; col_bits[m][w][k]: bit j = query 64*w + j allowed for key k.
   * [n_masks][2][128] uint64 each.                                          */
  const uint64_t* row_bits;
  const uint64_t* col_bits;
  /* Launch order of the work items, one workgroup each, -1 = idle slot.
   * q item   = (b * Hq  + h ) * nqt + query tile   (forward and dQ)
   * kv item  = (b * Hkv + hk) * nkt + key tile     (dK/dV)
   * Each item should appear once.  Entries outside [0, B*Hq*nqt) and
   * [0, B*Hkv*nkt) are skipped by the kernels (their outputs are not
   * written), since device arrays cannot be checked on the host.           */
  const int32_t* q_order;
  const int32_t* kv_order;
  int32_t n_q_order, n_kv_order;
  /* [nnz]: for each col_ent entry, the index in row_ent of the same tile (the
   * slot of its dS under MATTN_BWD_DS; may be NULL without that flag).     */
  const int32_t* col_row;
  /* [n_kv_order][8], read by the dK/dV stage of 16-bit problems at D <= 128:
   * per kv_order slot p with item = kv_order[p] = (b * Hkv + hk) * nkt + kt,
   * { item, g, e, e_end, n_sub, qt, mask, row } where g is the first query
   * head hk * G + g of the group whose column list (map row of (b, hk*G+g),
   * key tile kt) is not empty, [e, e_end) that list, n_sub twice the total
   * entry count over the group's heads, and (qt, mask) = col_ent[e],
   * row = col_row[e] (0 without it); { -1, 0, ... } for idle slots and
   * { item, 0, ... } for an empty column.  It lets each workgroup issue its
   * first loads after a single read instead of a chain of dependent ones. */
  const int32_t* kv_desc;
} mattn_blockmap;

/* Host-only check of a problem (and, when bm != NULL, of the map's sizes).
 * No GPU call; usable without a device. */
int mattn_validate(const mattn_problem* p, const mattn_blockmap* bm);

/* Bytes of device workspace mattn_bwd needs without MATTN_BWD_DS (256-byte
 * aligned pointer); with it, mattn_bwd_workspace_bytes(p, bm).  0 for an
 * invalid problem.
 * Head dimensions 64 and 128 with 16-bit inputs run on the MFMA kernels;
 * float32 inputs, D = 256 and 512 for every dtype (the host pads d in (128, 512]
 * with zeros) and MATTN_PRECISE problems run on float32 SIMT kernels, whose
 * workspace is one float32 per query row. */
size_t mattn_workspace_bytes(const mattn_problem* p);

/* Bytes of device workspace mattn_bwd needs for this map, MATTN_BWD_DS
 * included: mattn_workspace_bytes(p) plus, with that flag on the MFMA path,
 * 32 KiB per present tile of every (batch, head) -- nnz * (B / map_b) *
 * (Hq / map_h) tiles.  Host only; 0 for an invalid problem or map. */
size_t mattn_bwd_workspace_bytes(const mattn_problem* p, const mattn_blockmap* bm);

/* Bytes of the forward's residual buffer (256-byte aligned pointer): float16
 * copies of V and (with MATTN_FWD_FOR_BWD) Q, each times a power of two per
 * 128-row tile, which the forward's P V product and the backward read, with
 * the split tiles' rows and key tiles (16-bit inputs at D <= 128); (1 + D)
 * float32 per query row under MATTN_PRECISE; 0 otherwise (float32 inputs,
 * D >= 256). */
size_t mattn_fwd_workspace_bytes(const mattn_problem* p);

/* Forward (replaces the custom_vjp primal and fwd rule, attention.py:180-264).
 *   o         : [B, Lq, Hq, D] of o_dtype
 *   lse       : [B, Hq, Lq] float32, base-2 log-sum-exp of the scaled scores
 *               (-inf for a row with no allowed key); a residual for mattn_bwd
 *   residual  : mattn_fwd_workspace_bytes(p) bytes (NULL when 0), written
 *               here; with MATTN_FWD_FOR_BWD in p->flags, mattn_bwd reads it. */
int mattn_fwd(const mattn_problem* p, const mattn_blockmap* bm,
              const void* q, const void* k, const void* v,
              void* o, float* lse, void* residual, void* stream);

/* Backward (replaces the custom_vjp bwd rule, attention.py:266-342).
 *   do_       : upstream gradient, [B, Lq, Hq, D] of o_dtype
 *   o, lse    : the forward's outputs
 *   residual  : the forward's residual buffer (16-bit inputs at D <= 128;
 *               that forward ran with MATTN_FWD_FOR_BWD, which p->flags must
 *               carry, else MATTN_ERR_RESIDUAL), read only; may be NULL when
 *               mattn_fwd_workspace_bytes(p) == 0
 *   workspace : workspace_bytes bytes of scratch, at least
 *               mattn_bwd_workspace_bytes(p, bm) (else MATTN_ERR_WORKSPACE)
 *   dq, dk, dv: gradients of dtype, every element written (no pre-zeroing). */
int mattn_bwd(const mattn_problem* p, const mattn_blockmap* bm,
              const void* q, const void* k, const void* v,
              const void* o, const void* do_, const float* lse, const void* residual,
              void* workspace, size_t workspace_bytes, void* dq, void* dk, void* dv, void* stream);

/* The three stages of mattn_bwd, in the order they must run on one stream:
 * MATTN_BWD_PRE (delta = rowsum(dO * O) and the float16 copy of dO, into the
 * workspace), MATTN_BWD_DKDV (also writes the float16 copy of K, and with
 * MATTN_BWD_DS every tile's dS, into the workspace), then MATTN_BWD_DQ (reads
 * them).  On the SIMT path MATTN_BWD_PRE does nothing: those kernels take
 * dP - delta as dO . (V - O) per pair.  mattn_bwd == the three stages
 * in order.  Same arguments as mattn_bwd; exposed so a caller can time the
 * stages. */
enum mattn_bwd_stage { MATTN_BWD_PRE = 0, MATTN_BWD_DKDV = 1, MATTN_BWD_DQ = 2 };
int mattn_bwd_stage(const mattn_problem* p, const mattn_blockmap* bm, int stage,
                    const void* q, const void* k, const void* v,
                    const void* o, const void* do_, const float* lse, const void* residual,
                    void* workspace, size_t workspace_bytes, void* dq, void* dk, void* dv,
                    void* stream);

/* Size of the library's static device scratch used by mattn_bwd_noalloc. */
#define MATTN_SCRATCH_BYTES (512u << 20)

/* mattn_bwd without a workspace argument: the backward's workspace is a
 * static device array of MATTN_SCRATCH_BYTES (512 MiB) inside the library, one
 * per device, so the call makes no allocation of any kind (B=1 L=8192 H=32
 * D=128 needs 450 MiB).  It has no
 * counterpart in the reference (whose backward is a jax custom_vjp rule); it
 * is for callers that cannot allocate: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Problems whose
 * mattn_bwd_workspace_bytes(p, bm) exceeds MATTN_SCRATCH_BYTES return
 * MATTN_ERR_SCRATCH (clear MATTN_BWD_DS to run a larger one here).  The
 * stream must belong to the current device (MATTN_ERR_DEVICE otherwise: the
 * scratch used is that device's).  Every call on one device shares that device's scratch:
 * calls that overlap on one device (other streams, other threads) race.  No
 * scratch content carries over between calls (each call writes all it reads). */
int mattn_bwd_noalloc(const mattn_problem* p, const mattn_blockmap* bm,
                      const void* q, const void* k, const void* v,
                      const void* o, const void* do_, const float* lse, const void* residual,
                      void* dq, void* dk, void* dv, void* stream);

/*
 * Device tile-map classifier, for masks given in closed form.  It replaces the
 * element-by-element evaluation of create_block_mask (block_mask.py:454-498,
 * get_partial_block :381-408) and of the host tracer of mask_fn; the host
 * assembles the mattn_blockmap lists from its per-tile output.
 *
 * The effective mask of map row (mb, mh) at query q, key k is the AND of
 *   - the unpadded range q < Lq, k < Lk                       (attention.py:426-437)
 *   - when blk_size > 0, the reference's visited key blocks: the block of k in
 *     [s, s + blk_left + blk_right), s = min(max(q / blk_size - blk_left, 0),
 *     blk_nk - blk_left - blk_right)                      (attention.py:161-167,199-204)
 *   - when tab_b > 0, the table entry of the tile: 0 no element, 1 every
 *     element, 2 the element predicates below
 *   - the element predicates: k <= q when causal; q - k <= win_left and
 *     k - q <= win_right where those are >= 0; doc_q[b][q] == doc_k[b][k]
 *     when doc_b > 0 (b = 0 when doc_b == 1); (q - k) % res_period == 0 when
 *     res_period > 1 (the strided mask k % P == q % P of check_attn.py:9-32).
 * Every pointer is device memory.
 */
typedef struct mattn_maskspec {
  int32_t causal;                /* 0 or 1                                       */
  int32_t win_left, win_right;   /* element window, -1 = unbounded               */
  int32_t doc_b;                 /* 0: no document ids; 1: shared; map_b: per b  */
  const int32_t* doc_q;          /* [doc_b][Lq] document id of each query        */
  const int32_t* doc_k;          /* [doc_b][Lk] document id of each key          */
  int32_t tab_b, tab_h;          /* 0: no table; else 1 or map_b, 1 or map_h     */
  const uint8_t* tiles;          /* [tab_b][tab_h][nqt][nkt] table entries       */
  int32_t blk_size;              /* 0: no visited-block window                   */
  int32_t blk_left, blk_right;   /* blocks before / from the query's block        */
  int32_t blk_nk;                /* key blocks of the padded key length          */
  int32_t res_period;            /* 0 or 1: none; P > 1: (q - k) % P == 0        */
} mattn_maskspec;

/* Host-only check of a mask spec for a map_b x map_h map of Lq x Lk. */
int mattn_maskspec_validate(const mattn_maskspec* ms, int32_t Lq, int32_t Lk,
                            int32_t map_b, int32_t map_h);

/* Classifies every tile t = ((mb * map_h + mh) * nqt + qt) * nkt + kt:
 *   state[t]            int8: 0 absent, 1 full, 2 partial
 *   count[t]            int32: allowed elements of the tile
 *   hash[2t], hash[2t+1] 128-bit hash of a partial tile's row bits (else 0). */
int mattn_tilemap_classify(const mattn_maskspec* ms, int32_t Lq, int32_t Lk,
                           int32_t map_b, int32_t map_h,
                           int8_t* state, int32_t* count, uint64_t* hash, void* stream);

/* For n (tile index, mask id) pairs in list (int32 [2n]):
 *   write != 0: writes row_bits[id] and col_bits[id] (mattn_blockmap layout,
 *               [n_masks][2][128] each) from the tile's mask;
 *   write == 0: compares the tile's mask with row_bits[id] and stores 1 into
 *               *mismatch when they differ (the caller zeroes it first).
 * Pairs with a tile index or mask id out of range are skipped. */
int mattn_tilemap_bits(const mattn_maskspec* ms, int32_t Lq, int32_t Lk,
                       int32_t map_b, int32_t map_h, const int32_t* list, int32_t n,
                       int32_t n_masks, int32_t write, uint64_t* row_bits,
                       uint64_t* col_bits, int32_t* mismatch, void* stream);

/* Static text of a status code. */
const char* mattn_strerror(int status);

/* Library ABI version (bumped on any change of the structs above). */
int mattn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MATTN_H */
