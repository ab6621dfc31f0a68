/*
 * helix_kv.h -- C ABI of the MI355X (gfx950) KV-cache hot-path library
 * (libhelix_kv.so).
 *
 * Plain pointers and sizes only.  Every pointer argument named as device data
 * is device memory; `stream` is a hipStream_t (NULL = the default stream).
 * Calls are asynchronous on `stream`, never allocate device memory, never
 * synchronise, and return an hkv_status (0 = success).  Shapes are checked
 * before anything is launched.  Layouts are contiguous row-major.
 *
 * Each entry point names the reference interface it replaces (paths relative to
 * the helix-lite checkout).
 */
#ifndef HELIX_KV_H
#define HELIX_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum hkv_status {
  HKV_OK = 0,
  HKV_ERR_ARG = 1,       /* null pointer / bad enum / negative size */
  HKV_ERR_SHAPE = 2,     /* unsupported or inconsistent shape */
  HKV_ERR_DTYPE = 3,     /* unsupported dtype */
  HKV_ERR_CAPACITY = 4,  /* output capacity too small (result still sized) */
  HKV_ERR_LAUNCH = 5,    /* kernel launch failed */
  HKV_ERR_WORKSPACE = 6, /* workspace missing or too small */
  HKV_ERR_SCRATCH = 7    /* problem larger than the fixed scratch of a no-allocation entry point */
};

enum hkv_dtype {
  HKV_DT_F16 = 0, HKV_DT_F32 = 1, HKV_DT_BF16 = 2,
  HKV_DT_I64 = 3, HKV_DT_U8 = 4, HKV_DT_I32 = 5 /* index / mask tensors */
};

/* A strided view: element i of a broadcast shape is at data + sum_d k_d *
 * strides[d] (in elements; stride 0 broadcasts). */
typedef struct hkv_tensor_desc {
  const void *data;
  int32_t dtype;
  int32_t reserved;
  int64_t strides[6];
} hkv_tensor_desc;

/* Bytes of one nearest-pole decision table (device record). */
#define HKV_TABLE_BYTES 80

const char *hkv_version(void);
const char *hkv_status_string(int status);

/*
 * Scale description shared by the nuq entry points.  A "table" is one row of
 * poles (levels entries) with its two thresholds:
 *   per_token == 0 (Keys, per-channel): table index = h*D + d; poles (H,D,L),
 *       thresholds (H,D).  src/kvquant/scales.py:13-39.
 *   per_token == 1 (Values, per-token): table index = h*rows + min(pos, rows-1)
 *       with pos = positions[t] if positions else pos_offset + t; poles
 *       (H,rows,L), thresholds (H,rows).  src/kvquant/scales.py:42-69, clamp as
 *       src/kvquant/compact_pool.py:467 / src/kvquant/vllm_backend.py:151-155.
 * `tables` (optional for the dense pack, required for the compact path) are
 * built from the same poles/thresholds by hkv_nuq_build_tables; the original
 * poles/thresholds are still required (they decide the rare inputs the tables
 * do not cover, bit-exactly).
 */
typedef struct hkv_nuq_scales {
  const void *tables;   /* n_tables * HKV_TABLE_BYTES, or NULL */
  const void *poles;    /* n_tables * levels */
  const void *upper;    /* n_tables */
  const void *lower;    /* n_tables */
  int32_t poles_dtype;  /* hkv_dtype */
  int32_t thr_dtype;    /* hkv_dtype */
  int32_t levels;       /* 1..16 */
  int32_t per_token;    /* 0 = per-channel (K), 1 = per-token (V) */
  int64_t rows;         /* per-token scale rows (T_cal); unused for per-channel */
  const int64_t *positions; /* (T,) absolute positions or NULL */
  int64_t pos_offset;   /* absolute position of token 0 when positions == NULL */
} hkv_nuq_scales;

/*
 * Build n_tables decision tables (nearest-pole breakpoints, canonical fp16
 * thresholds, fp16 dequant poles).  Replaces the per-element level scan of
 * src/kvquant/triton_batched.py:65-72 with an equivalent breakpoint search;
 * tables that do not meet the exactness criterion are flagged and scanned.
 * Host-side cost: none; device: one thread per table.
 */
int hkv_nuq_build_tables(const void *poles, int poles_dtype, const void *upper,
                         const void *lower, int thr_dtype, int64_t n_tables, int levels,
                         void *tables_out, void *stream);

/*
 * Dense-outlier pack (the reference's byte-per-code format): values (T,H,D)
 * fp16 -> codes u8, outlier_v fp16 (0 where not an outlier), outlier_m u8, each
 * (T,H,D).  Replaces pack_keys_per_channel_batched / pack_values_per_token_
 * batched (src/kvquant/triton_batched.py:125-148, :275-303) and, with H = 1,
 * pack_keys_per_channel / pack_values_per_token (src/kvquant/triton_kernels.py:
 * 96-125, :258-280).
 */
int hkv_nuq_pack_dense(const void *values, int64_t T, int H, int D,
                       const hkv_nuq_scales *scales, void *codes, void *outlier_v,
                       void *outlier_m, void *stream);

/*
 * Dense unpack: where(outlier_m, outlier_v, fp16(pole[code])) -> out (T,H,D)
 * fp16.  Replaces unpack_*_batched (src/kvquant/triton_batched.py:151-171,
 * :306-326) and unpack_* (src/kvquant/triton_kernels.py:175-194, :321-339).
 * Uses scales->poles only (tables may be NULL).
 */
int hkv_nuq_unpack_dense(const void *codes, const void *outlier_v, const void *outlier_m,
                         int64_t T, int H, int D, const hkv_nuq_scales *scales, void *out,
                         void *stream);

/*
 * Compact pack: values (T,H,D) fp16 -> bit-packed codes (T,H,D*bits/8) u8
 * (nuq4: byte j = c[2j] | c[2j+1]<<4; nuq2: byte j = c[4j] | c[4j+1]<<2 |
 * c[4j+2]<<4 | c[4j+3]<<6) plus CSR outliers over rows r = t*H + h:
 * row_ptr (T*H+1) int32, col u8 (channel d), val fp16 (original value), in
 * ascending (row, col) order.  Entries beyond `capacity` are not written;
 * row_ptr is always complete, so row_ptr[T*H] is the true nnz, which a
 * caller compares with `capacity` once the stream has run (the call itself
 * cannot know it).  bits = 2 or 4 (levels <= 2^bits).  Requires
 * scales->tables, D % 8 == 0, D <= 256.  The planned format of
 * src/kvquant/triton_kernels.py:7-18 and src/kvquant/compact_pool.py:11-12
 * (the reference never implemented it).  One kernel on `stream`.
 * `workspace` (256-byte aligned) holds a work counter and per-chunk status
 * words: hkv_nuq_pack_compact_workspace_bytes(T, H, D) bytes, ZERO-FILLED
 * before its first use and then passed unchanged to later calls (each call
 * leaves its counters ready for the next; a workspace serves calls of any
 * size up to the one it was sized for).  Word 3 of the workspace (uint32)
 * becomes nonzero if a chunk ever gave up waiting for its predecessors'
 * counts (a bounded wait that guards against a stalled device; not expected
 * to happen).  Calls that may overlap must not share a workspace.
 */
size_t hkv_nuq_pack_compact_workspace_bytes(int64_t T, int H, int D);
int hkv_nuq_pack_compact(const void *values, int64_t T, int H, int D, int bits,
                         const hkv_nuq_scales *scales, void *packed, int32_t *row_ptr,
                         uint8_t *col, uint16_t *val, int64_t capacity, void *workspace,
                         size_t workspace_bytes, void *stream);

/* One tensor of a batched compact pack: the arguments of hkv_nuq_pack_compact. */
typedef struct hkv_pack_item {
  const void *values;   /* (T,H,D) fp16 */
  int64_t T;
  int32_t H, D, bits, reserved;
  hkv_nuq_scales scales;
  void *packed;         /* (T,H,D*bits/8) u8 */
  int32_t *row_ptr;     /* (T*H+1) */
  uint8_t *col;
  uint16_t *val;
  int64_t capacity;
} hkv_pack_item;

/*
 * Batched compact pack: n independent hkv_nuq_pack_compact calls (a prefill
 * step: every layer's K and V) in as few launches as their kernel variants
 * allow (one per variant and 16 tensors), each tensor's result identical to
 * its own call.  Same workspace contract, sized by
 * hkv_nuq_pack_compact_batch_workspace_bytes(items, n).  The batch form of
 * the per-layer pack calls of the reference's prefill
 * (src/kvquant/compact_pool.py:447-489, called per layer).
 */
size_t hkv_nuq_pack_compact_batch_workspace_bytes(const hkv_pack_item *items, int n);
int hkv_nuq_pack_compact_batch(const hkv_pack_item *items, int n, void *workspace,
                               size_t workspace_bytes, void *stream);

/*
 * Compact unpack: packed codes + CSR -> out (T,H,D) fp16.  Inverse of
 * hkv_nuq_pack_compact; requires scales->tables.  `capacity` is the length of
 * col/val: CSR entries at or beyond it are never read (a row_ptr from a pack
 * that overflowed its capacity then decodes those outliers as their poles).
 */
int hkv_nuq_unpack_compact(const void *packed, const int32_t *row_ptr, const uint8_t *col,
                           const uint16_t *val, int64_t capacity, int64_t T, int H, int D,
                           int bits, const hkv_nuq_scales *scales, void *out, void *stream);

/* One tensor of a batched compact unpack: the arguments of hkv_nuq_unpack_compact. */
typedef struct hkv_unpack_item {
  const void *packed;
  const int32_t *row_ptr;
  const uint8_t *col;
  const uint16_t *val;
  int64_t capacity;
  int64_t T;
  int32_t H, D, bits, reserved;
  hkv_nuq_scales scales;
  void *out;            /* (T,H,D) fp16 */
} hkv_unpack_item;

/*
 * Batched compact unpack: n independent hkv_nuq_unpack_compact calls, each
 * result identical to its own call.  Per-channel (K) tensors share launches
 * (one per variant and 16 tensors; the launch's blocks are split among the
 * tensors in proportion to their rows); per-token (V) tensors are launched
 * one by one, since their pole rows are read through L2.  No workspace.  The
 * batch form of the per-layer dequantisation the reference runs for every
 * layer (src/kvquant/triton_batched.py:151-171, :306-326).
 */
int hkv_nuq_unpack_compact_batch(const hkv_unpack_item *items, int n, void *stream);

/*
 * Broadcasting quantise with the CPU spec's dtype semantics: over a shape of
 * up to 6 dims, code = first argmin_l |round_cdt(v - pole_l)| (NaN differences
 * win, first one first), mask = v < lower || v > upper (omit both thresholds
 * for no mask), recon = mask ? v : pole[code] in recon_dtype.  Any output may
 * be NULL (codes int64, mask u8, recon contiguous).  Pole l of element i is at
 * poles->data + offset_i + l*level_stride.  src/kvquant/nuq.py:22-38
 * (round_to_nearest_pole), :41-94 (find_outliers, without the cap/first-N
 * options), :97-132 (quantize_nuq).
 */
int hkv_nuq_quantize_generic(int ndim, const int64_t *shape, const hkv_tensor_desc *values,
                             const hkv_tensor_desc *poles, int64_t level_stride, int levels,
                             const hkv_tensor_desc *upper, const hkv_tensor_desc *lower,
                             int compute_dtype, int64_t *codes, void *recon, int recon_dtype,
                             uint8_t *mask, void *stream);

/*
 * Broadcasting dequantise: out = mask ? outliers : round_out(pole[code]) in
 * out_dtype (contiguous).  Codes outside [0, levels) set *err (device int32)
 * and read pole 0.  src/kvquant/nuq.py:135-156.
 */
int hkv_nuq_dequantize_generic(int ndim, const int64_t *shape, const hkv_tensor_desc *codes,
                               const hkv_tensor_desc *outliers, const hkv_tensor_desc *outlier_mask,
                               const hkv_tensor_desc *poles, int64_t level_stride, int levels,
                               void *out, int out_dtype, int32_t *err, void *stream);

/*
 * Compact KV pool write (one layer, K or V): token t of values (T,H,D) fp16
 * is quantised into slot slot_mapping[t] of the layer's pool tensors codes u8,
 * outlier_v fp16 (0 where not an outlier) and outlier_m u8, each
 * (num_blocks, block_size, H, D); slot < 0 (padding) and slot >=
 * num_blocks * block_size are skipped.  For V pass per-token scales with
 * scales->positions = the tokens' absolute positions (row min(pos, rows-1)).
 * For K, k_min / k_max (num_blocks, H, D) fp32 (or both NULL) receive the
 * running min / max of the reconstructed values (input for outliers, fp32
 * pole otherwise), -0 below +0; initialise them to +inf / -inf.  Requires
 * scales->tables; D/8 a power of two <= 32.  Replaces CompactKVPool.write_kv
 * (src/kvquant/compact_pool.py:447-489; kernels :160-287).
 */
int hkv_pool_write(const void *values, int64_t T, int H, int D, const hkv_nuq_scales *scales,
                   const int64_t *slot_mapping, int64_t num_blocks, int block_size, void *codes,
                   void *outlier_v, void *outlier_m, float *k_min, float *k_max, void *stream);

/*
 * Compact KV pool gather-dequant (one layer, K or V): staging (NK,
 * block_size, H, D) fp16 row k = dequantised pool block block_ids[k]; for V
 * (per-token scales) position p of kept block k uses scale row
 * min(first_pos[k] + p, rows - 1).  Block ids outside [0, num_blocks) give
 * zero rows.  Replaces CompactKVPool.unpack_to_staging
 * (src/kvquant/compact_pool.py:492-537; kernels :292-395).
 */
int hkv_pool_gather(const void *codes, const void *outlier_v, const void *outlier_m,
                    int64_t num_blocks, int block_size, int H, int D,
                    const hkv_nuq_scales *scales, const int64_t *block_ids,
                    const int64_t *first_pos, int64_t NK, void *staging, void *stream);

/*
 * Paged compact pool: one layer and side (K or V) of a paged KV cache, head
 * dim 128, 16 slots per block, described by hkv_paged_side:
 *   codes (num_blocks, heads, 16, 128*bits/8) u8 -- page-head blocks, slot
 *     rows in order, codes little-endian within a byte (nuq4: byte j = c[2j] |
 *     c[2j+1] << 4; nuq2: c[4j] in the low bits);
 *   ocnt (num_blocks, heads) int32 -- outliers of the page-head;
 *   oent (num_blocks, heads, cap) u32 -- its first cap outliers, (slot,
 *     channel) ascending, as fp16 value | channel << 16 | slot << 24;
 *   ovf (num_blocks, heads) int32 -- the page-head's overflow chunk (-1: none),
 *     holding its entries cap.. in ovf_ent (n_chunks, 2048 - cap) u32; chunks
 *     are handed out from ovf_next on first need and stay with the page-head.
 *     ovf NULL: no arena (entries past cap are dropped);
 *   kmin / kmax (num_blocks, heads, 128) fp16 -- K only (else NULL): min / max
 *     over the written slots of the dequantised values (outlier value, else
 *     fp16 pole), a zero stored as +0;
 *   status (1) int32 -- bit 0 set once outliers were dropped (no room left).
 * The reference's pool is byte-per-code with dense outliers
 * (src/kvquant/compact_pool.py:398-446); this is its planned bit-packed
 * layout with outliers kept per block (compact_pool.py:11-12,
 * src/kvquant/vllm_integration.md:51-55), page-head contiguous.
 */
typedef struct hkv_paged_side {
  uint8_t *codes;
  int32_t *ocnt;
  uint32_t *oent;
  int32_t *ovf;
  uint32_t *ovf_ent;
  int32_t *ovf_next;
  uint16_t *kmin;
  uint16_t *kmax;
  int32_t *status;
  int64_t num_blocks;
  int32_t heads;    /* <= 16 */
  int32_t bits;     /* 2 or 4 */
  int32_t cap;      /* 0..2048 */
  int32_t n_chunks;
} hkv_paged_side;

/*
 * hkv_paged_write replaces CompactKVPool.write_kv (compact_pool.py:447-489,
 * kernels :160-287): token t of values (T, heads, 128) fp16 goes to slot
 * slot_mapping[t] (block slot / 16, row slot % 16; slots < 0 or past the pool
 * are skipped).  A run -- consecutive tokens with consecutive slots in one
 * block -- starting at row w0 keeps the page-head's outliers of rows < w0
 * and replaces the rest; kmin / kmax restart at w0 = 0 and otherwise fold in.
 * The tokens of one call that fall in one block must form one run.  V:
 * per-token scales with scales->positions = absolute positions (row
 * min(pos, rows - 1)).  values / codes / kmin / kmax 16-byte aligned.
 *
 * hkv_paged_gather replaces CompactKVPool.unpack_to_staging
 * (compact_pool.py:492-537, kernels :292-395): staging (NK, 16, heads, 128)
 * fp16 row k = block block_ids[k] dequantised (ids outside the pool give
 * zeros); V row p of kept block k uses scale row min(first_pos[k] + p,
 * rows - 1).
 */
int hkv_paged_write(const void *values, int64_t T, const hkv_nuq_scales *scales,
                    const int64_t *slot_mapping, const hkv_paged_side *side, void *stream);
int hkv_paged_gather(const hkv_paged_side *side, const hkv_nuq_scales *scales,
                     const int64_t *block_ids, const int64_t *first_pos, int64_t NK, void *staging,
                     void *stream);

/*
 * Quest selection over a paged pool's K statistics (kside->kmin / kmax): as
 * hkv_quest_select with the group-summed bound, logical page p's statistics
 * at block block_table[p] (P logical pages); a block outside the pool gets
 * bound -inf.  The selection (sinks + k_eff, heads) holds logical pages, the
 * sinks being the first logical pages: positions follow from the block
 * table, not from block ids (src/kvquant/quest_selector.py:38-90 takes the
 * first used block ids as sinks and id * block_size as positions, :85-89).
 * Same workspace as hkv_quest_select.
 */
int hkv_quest_select_paged(const void *q, int q_dtype, int Hq, const hkv_paged_side *kside,
                           const int64_t *block_table, int64_t P, int64_t k, int64_t sink_pages,
                           float *scores, int64_t *out, int64_t *n_out, void *workspace,
                           size_t workspace_bytes, void *stream);

/*
 * Fused dequant + sparse decode attention over a paged pool (batch 1, head
 * dim 128): hkv_decode_attn with logical page p of the sequence (tokens
 * [16p, 16p+16), tokens >= T masked) read from block block_table[p] of the
 * paged K / V (the page-head's outliers patched over its codes); sel (nsel,
 * heads) holds logical pages, ids outside [0, ceil(T/16)) or whose block is
 * outside the pool are skipped; V rows min(16p + slot, v_rows - 1).  The
 * counterpart of the compact backend's forward over its block table
 * (src/kvquant/compact_backend.py:194-299).  Hq / heads <= 16.  Workspace:
 * hkv_decode_workspace_bytes(nsel, Hq, pages_per_split).
 */
int hkv_paged_decode_attn(const void *q, int Hq, int64_t T, const int64_t *block_table,
                          const hkv_paged_side *k, const void *k_tables, const hkv_paged_side *v,
                          const void *v_tables, int64_t v_rows, const int64_t *sel, int64_t nsel,
                          int pages_per_split, float scale, void *out, int out_dtype,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * Quest page statistics: K_pages (P,S,H,D) -> kmin, kmax (P,H,D), same dtype
 * (f16 or f32).  -0 orders below +0; a NaN in a page-channel gives NaN.
 * src/quest/reference.py:38-56.
 */
int hkv_quest_page_stats(const void *k_pages, int dtype, int64_t P, int S, int H, int D,
                         void *kmin, void *kmax, void *stream);

/*
 * Quest upper bound per (page, KV head):
 *   sum_d clamp(q,0)*kmax + clamp(q,max=0)*kmin   (fp32, fixed order)
 * q is (Hq,D); gqa_group = Hq / H: 1 = one query per KV head
 * (src/quest/reference.py:59-93, src/kvquant/quest_selector.py:68-70);
 * > 1 = the group's per-head bounds summed (query head h -> KV head h / group).
 * kmin/kmax (P,H,D) f16 or f32; out (P,H) f32 or f16 (f16 = the rounding of
 * page_upper_bound_triton, src/quest/triton_kernels.py:57).
 */
int hkv_quest_page_bound(const void *q, int q_dtype, int Hq, const void *kmin,
                         const void *kmax, int k_dtype, int64_t P, int H, int D,
                         void *out, int out_dtype, void *stream);

/*
 * Quest top-K with sinks over a bound (P,H) (f32 or f16):
 * sinks = clamp(sink_pages, 0, P); k_eff = clamp(k, 0, P - sinks); out
 * (sinks + k_eff, H) int64, per head the sinks then the k_eff highest-bound
 * non-sink pages, ascending; ties go to the lower page index; NaN ranks highest.
 * src/quest/reference.py:96-133.  Returns sinks + k_eff through *n_out.
 * workspace: unused (may be NULL); hkv_quest_topk_workspace_bytes is kept for
 * callers that size one.
 */
size_t hkv_quest_topk_workspace_bytes(int64_t P, int H);
int hkv_quest_topk(const void *bound, int b_dtype, int64_t P, int H, int64_t k,
                   int64_t sink_pages, int64_t *out, int64_t *n_out, void *workspace,
                   size_t workspace_bytes, void *stream);

/*
 * Quest selection for one decode step: the bound (as hkv_quest_page_bound,
 * f32, written head-major to scores (H,P)) then the top-K with sinks (as
 * hkv_quest_topk).  The per-layer path of src/kvquant/quest_selector.py:64-78
 * without the union.  With a workspace of hkv_quest_select_workspace_bytes(P,
 * H) bytes (256-byte aligned, zero-filled once before its first use; every
 * call leaves it reusable; calls that may overlap must not share it), large
 * fp16 columns take the multi-block top-K (the bound kernel also records the
 * key range of its blocks; a histogram kernel over slices of each column whose
 * last block resolves the threshold; a write kernel): three launches.
 * Without one (NULL / too small), the single-block top-K: two launches.  Both
 * give identical results.
 */
size_t hkv_quest_select_workspace_bytes(int64_t P, int H);
int hkv_quest_select(const void *q, int q_dtype, int Hq, const void *kmin, const void *kmax,
                     int k_dtype, int64_t P, int H, int D, int64_t k, int64_t sink_pages,
                     float *scores, int64_t *out, int64_t *n_out, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * hkv_quest_select without a workspace argument and without allocating: the
 * multi-block top-K keeps its state in a fixed device array of the library
 * (hkv_quest_select_noalloc_max_workspace() = 8 MiB per GPU, held until the
 * process ends) instead of a caller buffer.  No counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops that forbid hipMalloc).  Results are
 * identical to hkv_quest_select's.  A problem whose workspace
 * (hkv_quest_select_workspace_bytes(P, H)) exceeds the array returns
 * HKV_ERR_SCRATCH before anything is launched.  The array's address on a
 * device is looked up at the first call there, which also clears it with a
 * fill kernel on `stream`; every call leaves it cleared for the next.  All
 * calls on one GPU share the array: calls that may overlap on one GPU (other
 * streams without ordering between them) race.
 */
size_t hkv_quest_select_noalloc_max_workspace(void);
int hkv_quest_select_noalloc(const void *q, int q_dtype, int Hq, const void *kmin, const void *kmax,
                             int k_dtype, int64_t P, int H, int D, int64_t k, int64_t sink_pages,
                             float *scores, int64_t *out, int64_t *n_out, void *stream);

/*
 * Compact page metadata: u8 codes of the page minima / maxima with a per
 * (head, channel) lo and step (f32), half the bytes of fp16 statistics.  No
 * counterpart in the reference, whose pool keeps f32 page statistics
 * (src/kvquant/compact_pool.py:434-441); for callers whose selection is bound
 * by reading the statistics.
 *
 * hkv_quest_page_stats_u8: from (P,H,D) f16/f32 kmin / kmax (as
 * hkv_quest_page_stats writes them) to qmin / qmax (P,H,D) u8 and lo / step
 * (H,D) f32.  Per (head, channel) over the finite statistics of all pages:
 * lo = the smallest, hi = the largest; step = fl((hi - lo) / 255) raised one
 * ulp at a time until fl(lo + fl(255 * step)) >= hi (1 when hi <= lo).
 * Codes are rounded conservatively: fl(lo + fl(qmin * step)) <= min and
 * fl(lo + fl(qmax * step)) >= max for every finite statistic, so the bound
 * from the codes is never below the bound from the statistics; a non-finite
 * statistic codes as 0 (minimum) / 255 (maximum).  D a multiple of 4; qmin /
 * qmax 4-byte aligned.  workspace: hkv_quest_page_stats_u8_workspace_bytes(H,
 * D) bytes, 4-byte aligned (no initial contents needed).  Four launches.
 *
 * hkv_quest_select_u8: hkv_quest_select over the u8 metadata: the bound of
 * every page from the dequantised statistics fl(lo + fl(code * step)) in the
 * fp16 path's products and order (scores (H,P) f32), then the same top-K with
 * sinks and the same workspace (hkv_quest_select_workspace_bytes).  D a
 * multiple of 8 with D/8 a power of two <= 64 and H dividing 64/(D/8)
 * (D = 128: H in {1, 2, 4}); qmin / qmax 8-byte aligned.
 */
size_t hkv_quest_page_stats_u8_workspace_bytes(int H, int D);
int hkv_quest_page_stats_u8(const void *kmin, const void *kmax, int dtype, int64_t P, int H, int D,
                            uint8_t *qmin, uint8_t *qmax, float *lo, float *step, void *workspace,
                            size_t workspace_bytes, void *stream);
int hkv_quest_select_u8(const void *q, int q_dtype, int Hq, const uint8_t *kmin,
                        const uint8_t *kmax, const float *lo, const float *step, int64_t P, int H,
                        int D, int64_t k, int64_t sink_pages, float *scores, int64_t *out,
                        int64_t *n_out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Quest block selection over a compact pool layer
 * (src/kvquant/quest_selector.py:38-90): q (H,D) (one query per KV head),
 * pool statistics kmin/kmax (num_blocks,H,D) (f32 or f16), the sequence's
 * used blocks used_block_ids (NU,) int64.  Bound of every used block (as
 * hkv_quest_page_bound with page p -> statistics row used_block_ids[p]; an id
 * outside [0, num_blocks) gets bound -inf), per-head top-K with the first
 * min(sink_blocks, NU) used blocks as sinks (as hkv_quest_topk), union over
 * heads.  Writes the selected block ids ascending to out_ids, id * block_size
 * to out_first_pos, and their number to *n_selected (device int64).
 * Workspaces: scores H*NU f32, sel (min(sink,NU) + min(top_k, NU - sinks))*H
 * int64, flags num_blocks bytes (16-byte aligned), zero-filled before the first
 * call (the call leaves them zero).  out_ids / out_first_pos need min(num_blocks, NU)
 * entries.
 */
int hkv_quest_select_blocks(const void *q, int q_dtype, int H, const void *kmin, const void *kmax,
                            int k_dtype, int64_t num_blocks, int D, const int64_t *used_block_ids,
                            int64_t NU, int64_t top_k, int64_t sink_blocks, int64_t block_size,
                            float *scores, int64_t *sel, uint8_t *flags, int64_t *out_ids,
                            int64_t *out_first_pos, int64_t *n_selected, void *stream);

/*
 * Fused dequant + Quest-sparse decode attention, batch 1, head_dim 128, page
 * size 16.  Replaces unpack_to_staging + flash_attn_varlen_func over the fp16
 * staging copy (src/kvquant/compact_backend.py:233-299) and restates
 * selected_attention (src/quest/reference.py:136-168) with the standard GQA
 * map: query head hq attends with KV head hq / (Hq / H), over the tokens of
 * pages sel[0..nsel)[hq / (Hq / H)] (sel (nsel, H) int64, as hkv_quest_topk
 * returns; page p = tokens [16p, 16p+16), tokens >= T masked, page ids outside
 * [0, ceil(T/16)) skipped at no cost: a list with holes, such as the union of
 * the heads' pages padded with -1, is fine), softmax(q.K^T * scale) in fp32.
 * K and V are in the compact format of hkv_nuq_pack_compact over (T, H, 128)
 * (packed 16-byte aligned); tables are the decision tables of the K scales
 * (H*128 per-channel) and of the V scales (H*v_rows per-token, row
 * min(t, v_rows - 1)).  q (Hq, 128) fp16, 8-byte aligned; out (Hq, 128) fp16
 * or fp32.  Hq / H <= 16.  The workspace holds per-split partials (m, l, o):
 * hkv_decode_workspace_bytes(nsel, Hq, pages_per_split) bytes, no zeroing.
 */
size_t hkv_decode_workspace_bytes(int64_t nsel, int Hq, int pages_per_split);
/* pages_per_split in [1, 256]. */
int hkv_decode_attn(const void *q, int Hq, int H, int D, int64_t T,
                    const void *k_packed, const int32_t *k_row_ptr, const uint8_t *k_col,
                    const uint16_t *k_val, int64_t k_cap, int k_bits, const void *k_tables,
                    const void *v_packed, const int32_t *v_row_ptr, const uint8_t *v_col,
                    const uint16_t *v_val, int64_t v_cap, int v_bits, const void *v_tables,
                    int64_t v_rows, const int64_t *sel, int64_t nsel, int pages_per_split,
                    float scale, void *out, int out_dtype, void *workspace,
                    size_t workspace_bytes, void *stream);

/*
 * Batched decode: hkv_decode_attn for B <= 64 sequences held in one
 * compact-format K / V of T tokens, in one decode launch and one merge
 * launch (the reference decodes one sequence per forward,
 * src/kvquant/compact_backend.py:184-203; its per-sequence path is
 * :194-299).  Sequence b is tokens [tok_offsets[b], tok_offsets[b] +
 * seq_lens[b]) (tok_offsets multiples of 16), with query q[b] (q (B, Hq,
 * 128) fp16) and selection rows sel_offsets[b] .. sel_offsets[b+1]-1 of sel
 * (rows, H) int64, page ids local to the sequence (ids outside its pages are
 * skipped); V per-token tables are indexed by the position within the
 * sequence, row min(t, v_rows - 1).  out (B, Hq, 128) fp16 or fp32.
 * tok_offsets, seq_lens (B) and sel_offsets (B+1) are HOST arrays.  Each
 * sequence's result equals hkv_decode_attn over its view with the same
 * pages_per_split.  Workspace: hkv_decode_batch_workspace_bytes (no zeroing).
 */
size_t hkv_decode_batch_workspace_bytes(int B, const int64_t *sel_offsets, int Hq,
                                        int pages_per_split);
int hkv_decode_attn_batch(const void *q, int B, int Hq, int H, int D, int64_t T,
                          const int64_t *tok_offsets, const int64_t *seq_lens,
                          const void *k_packed, const int32_t *k_row_ptr, const uint8_t *k_col,
                          const uint16_t *k_val, int64_t k_cap, int k_bits, const void *k_tables,
                          const void *v_packed, const int32_t *v_row_ptr, const uint8_t *v_col,
                          const uint16_t *v_val, int64_t v_cap, int v_bits, const void *v_tables,
                          int64_t v_rows, const int64_t *sel, const int64_t *sel_offsets,
                          int pages_per_split, float scale, void *out, int out_dtype,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * Batched decode over a paged pool: hkv_paged_decode_attn for B <= 64
 * sequences sharing one pool, in one decode launch and one merge launch (the
 * compact backend's forward over the block tables of a batch,
 * src/kvquant/compact_backend.py:184-299, which attends one sequence at a
 * time).  Sequence b has seq_lens[b] tokens, query q[b] (q (B, Hq, 128)
 * fp16), its logical page p in block block_table[bt_offsets[b] + p]
 * (block_table a device array holding ceil(seq_lens[b] / 16) entries from
 * bt_offsets[b] on), and selection rows sel_offsets[b] .. sel_offsets[b+1]-1
 * of sel (rows, heads), logical page ids of the sequence.  V rows min(16p +
 * slot, v_rows - 1).  seq_lens, bt_offsets (B) and sel_offsets (B+1) are HOST
 * arrays.  Each sequence's result equals hkv_paged_decode_attn over its view
 * with the same pages_per_split.  Workspace: hkv_decode_batch_workspace_bytes
 * (no zeroing).  out (B, Hq, 128) fp16 or fp32.
 */
int hkv_paged_decode_attn_batch(const void *q, int B, int Hq, const int64_t *seq_lens,
                                const int64_t *block_table, const int64_t *bt_offsets,
                                const hkv_paged_side *k, const void *k_tables,
                                const hkv_paged_side *v, const void *v_tables, int64_t v_rows,
                                const int64_t *sel, const int64_t *sel_offsets,
                                int pages_per_split, float scale, void *out, int out_dtype,
                                void *workspace, size_t workspace_bytes, void *stream);

/*
 * Per-sequence union of the KV heads' selected pages, the page set the
 * reference's decode attends for every query head
 * (src/kvquant/quest_selector.py:80, then all heads of each kept block,
 * src/kvquant/compact_pool.py:492-537).  Sequence b (B <= 64) owns rows
 * row_offsets[b] .. row_offsets[b+1]-1 of sel (rows, H) int64 (page ids local
 * to the sequence, as hkv_quest_select_ragged writes them) and pages
 * [0, page_offsets[b+1] - page_offsets[b]); its union goes, ascending, to rows
 * page_offsets[b] .. of out (page_offsets[B], H) int64, every column alike,
 * with -1 in the rows after it.  row_offsets / page_offsets (B+1, first entry
 * 0) are HOST arrays.  flags: hkv_union_pages_workspace_bytes(page_offsets[B])
 * bytes, zero-filled before the first call; each call leaves it zero.  Three
 * launches over the whole batch, no host reads.
 */
size_t hkv_union_pages_workspace_bytes(int64_t total_pages);
int hkv_union_pages_ragged(const int64_t *sel, int H, int B, const int64_t *row_offsets,
                           const int64_t *page_offsets, int64_t *out, void *flags,
                           size_t flags_bytes, void *stream);

/*
 * Ragged batched Quest selection: B <= 64 sequences, sequence b owning pages
 * [page_offsets[b], page_offsets[b+1]) of the concatenated statistics kmin /
 * kmax (P_total, H, D) fp16 (D % 8 == 0, D/8 a power of two), with its own
 * decode query q[b] (Hq, D).  Per sequence and KV head: the group-summed bound
 * (as hkv_quest_select) and topk_pages_with_sinks (src/quest/reference.py:
 * 96-133) with the first sink_pages pages as sinks and top_k[b] more, indices
 * local to the sequence, ascending.  page_offsets (B+1, page_offsets[0] == 0)
 * and top_k (B) are HOST arrays; out_offsets (B+1, host) receives the row
 * offsets of each sequence's selection in out (rows, H) int64.  scores (H,
 * P_total) fp32 receives the bounds.  One bound launch over every sequence and
 * one top-K launch of H x B blocks.  (The reference selects per sequence,
 * src/kvquant/quest_selector.py:38-90; this is the batched form.)
 */
int hkv_quest_select_ragged(const void *q, int q_dtype, int B, int Hq, const void *kmin,
                            const void *kmax, int k_dtype, int H, int D,
                            const int64_t *page_offsets, const int64_t *top_k, int64_t sink_pages,
                            float *scores, int64_t *out, int64_t *out_offsets, void *stream);

/*
 * hkv_quest_select_ragged over a paged pool's K statistics (kside->kmin /
 * kmax, D = 128): sequence b has page_offsets[b+1] - page_offsets[b] logical
 * pages, logical page p's statistics at block block_table[bt_offsets[b] + p]
 * (a block outside the pool gets bound -inf), as hkv_quest_select_paged per
 * sequence (src/kvquant/quest_selector.py:38-90 per sequence).  scores (H,
 * page_offsets[B]) fp32.  bt_offsets (B) is a HOST array, block_table a
 * device array.  kside->heads must divide 16 (1, 2, 4, 8 or 16: a bound
 * lane's KV head is fixed); HKV_ERR_SHAPE otherwise.
 */
int hkv_quest_select_paged_ragged(const void *q, int q_dtype, int B, int Hq,
                                  const hkv_paged_side *kside, const int64_t *block_table,
                                  const int64_t *bt_offsets, const int64_t *page_offsets,
                                  const int64_t *top_k, int64_t sink_pages, float *scores,
                                  int64_t *out, int64_t *out_offsets, void *stream);

/*
 * Gather + dequantise the selected pages of a compact-format K or V (as
 * hkv_nuq_pack_compact writes it over the concatenated tokens of B <= 64
 * sequences; page p = tokens [16p, 16p+16)) into staging (rows, 16, H, 128)
 * fp16, per KV head: staging[i, j, h] = token (page_offsets[b] + sel[i][h])*16
 * + j of head h, for row i of sequence b (rows out_offsets[b] ..
 * out_offsets[b+1]-1).  Per-token (V) scales use row min(sel[i][h]*16 + j,
 * rows - 1), the position within the sequence (scales->positions and
 * pos_offset are not used); pages outside the sequence give zero rows.  The
 * compact-format, per-head counterpart of unpack_to_staging
 * (src/kvquant/compact_pool.py:492-537).  page_offsets / out_offsets are HOST
 * arrays (out_offsets as hkv_quest_select_ragged returns them); sel (rows, H)
 * int64 device.  D = 128, page_size = 16; packed and out 16-byte aligned.
 */
int hkv_nuq_gather_pages(const void *packed, const int32_t *row_ptr, const uint8_t *col,
                         const uint16_t *val, int64_t capacity, int64_t T, int H, int D, int bits,
                         const hkv_nuq_scales *scales, int page_size, int B,
                         const int64_t *page_offsets, const int64_t *out_offsets,
                         const int64_t *sel, void *out, void *stream);

/*
 * Attention of each query head over its selected dense pages: the drop-in for
 * selected_attention (src/quest/reference.py:136-168).  q (Hq, D); k_pages
 * (P, page_size, Hk, D) and v_pages (P, page_size, Hv, Dv) in kv_dtype; sel
 * (nsel, sel_cols) int64 with sel_cols = Hq (a column per query head, the
 * reference's layout) or Hk (a column per KV head).  head_map 0: the
 * reference's map (K head h, V head h % Hv; needs Hk == Hq); 1: GQA (K and V
 * head h / (Hq / Hk)).  softmax(q.K^T * scale) in fp32, result rounded once to
 * out_dtype; page ids outside [0, P) are skipped.  D, Dv <= 512, page_size <=
 * 1024; dtypes fp16 / fp32 / bf16.  Workspace:
 * hkv_selected_attention_workspace_bytes(nsel, page_size, Hq, Dv).
 */
size_t hkv_selected_attention_workspace_bytes(int64_t nsel, int page_size, int Hq, int Dv);
int hkv_selected_attention(const void *q, int q_dtype, int Hq, int D, const void *k_pages,
                           const void *v_pages, int kv_dtype, int64_t P, int page_size, int Hk,
                           int Hv, int Dv, const int64_t *sel, int64_t nsel, int sel_cols,
                           int head_map, float scale, void *out, int out_dtype, void *workspace,
                           size_t workspace_bytes, void *stream);

/*
 * Batched 1-D k-means for nuq calibration: replaces the per-(head, channel)
 * and per-(head, position) sklearn fits of src/kvquant/calibration.py:106-188
 * (_kmeans_1d in the _calibrate_keys / _calibrate_values loops).  Problem p is
 * values[offsets[p] .. offsets[p+1]) (fp32, finite; offsets int64,
 * n_problems + 1 entries, each problem < 2^31 values).  k <= 16 centres start
 * at order statistics, c_l = sorted[floor((2l + 1) n / 2k)], for n <= 8192
 * values, else evenly spread over [min, max] (c_l = min + (max - min) *
 * (2l + 1) / 2k in fp32), and take `iters` Lloyd steps: each value joins the
 * first centre of least fp32 |v - c|, a centre with members moves to their
 * mean (float64 sum / count, rounded to fp32), one without stays.  centers
 * (n_problems, k) fp32 receive the centres sorted ascending.  As the
 * reference's _kmeans_1d: no values give k zeros, n < k values give the
 * values and k - n zeros, sorted.  Malformed offsets give NaN centres.
 * Deterministic; no workspace.
 */
int hkv_kmeans_1d(const float *values, const int64_t *offsets, int64_t n_problems, int k,
                  int iters, float *centers, void *stream);

/*
 * Optimal batched 1-D k-means: the same problems and output as
 * hkv_kmeans_1d, solved exactly by dynamic programming over the sorted values
 * (least within-cluster sum of squares; partial costs rounded to fp32 per DP
 * row, the leftmost split wins ties), so the fit is never worse than any
 * k-means run, the reference's sklearn fit included (src/kvquant/
 * calibration.py:106-123).  Problems of at most 6144 values (the calibration
 * subsample is 5000); larger ones get NaN centres.  `workspace` holds each
 * resident block's split table: hkv_kmeans_1d_optimal_workspace_bytes()
 * bytes for a full grid (less runs fewer blocks at once; at least one
 * block's 184,320 bytes).
 */
size_t hkv_kmeans_1d_optimal_workspace_bytes(void);
int hkv_kmeans_1d_optimal(const float *values, const int64_t *offsets, int64_t n_problems, int k,
                          float *centers, void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HELIX_KV_H */
