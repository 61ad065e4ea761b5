/*
 * miburn.h -- the C ABI of the MI355X (gfx950) Burn-backend engine.
 *
 * One entry point per method of the reference's `Engine` trait that the hot
 * path uses (crates/burn-tt/src/server.rs:42-788): the device engine that the
 * Burn backend's server thread drives.  A Rust `-sys` crate binds these names
 * one for one; the C++ and Python hosts in this repository bind them too.
 *
 * Conventions (mirroring the trait):
 *  - A buffer is a row-major `[rows, cols]` matrix of one element kind, named
 *    by a `mi_id` (the trait's `BufferId = u64`, server.rs:862).  Ids are
 *    process-unique and never reused (server.rs:2421-2446).  Rank-N tensors
 *    fold to `[prod(leading dims), last dim]` on the host, as the reference's
 *    `stored_dims` does (crates/burn-tt/src/tensor.rs:905-908).
 *  - Every call returns an `int` status: 0 on success, a negative `MI_E_*`
 *    code otherwise, with a message in `mi_last_error`.  A call that fails
 *    argument checks creates nothing.
 *  - Work is stream-ordered and asynchronous on the context's one HIP
 *    stream: an op returns its result id at once.  A failure found by a
 *    kernel (an index out of range) is recorded and returned by the next
 *    waiting call (`mi_sync`, a download), and the first such failure sticks
 *    -- the trait's deferred `Ids.failed` (server.rs:2951-2991, 2390-2425).
 *  - A context is used by one thread at a time (the reference serialises its
 *    engine behind one server thread, server.rs:2886-2914); the library
 *    takes a per-context lock so concurrent callers are serialised, not
 *    undefined.
 */
#ifndef MIBURN_H
#define MIBURN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mi_ctx mi_ctx;
typedef uint64_t mi_id;

/* Element kinds: the trait's `Elem` (server.rs:862 ff.).  I32 and Bool are
 * 32-bit words (a Bool is 0 or 1), BF16 two-byte slots.  MI_BFP8 is the
 * reference's block floating point storage StorageFormat::Bfp8
 * (crates/burn-tt/src/storage.rs:24-40): a logical F32 [rows, cols] whose
 * rows are blocks of 16 consecutive columns (the last may be shorter)
 * sharing one exponent byte E, each value q * 2^(E - 133) with an integer
 * |q| <= 127 -- 1 + 1/16 bytes a value.  It is made by mi_cast_bfp, read
 * back decoded (mi_download, mi_cast_bfp to F32), and taken as the weight
 * operand of mi_matmul, mi_linear, mi_norm_matvec, mi_norm_qkv_rope(_at) and
 * mi_norm_qkv_attention; other ops refuse it.  Layout: q as [rows, cols]
 * two's-complement bytes, then, from the first multiple of 256 bytes after
 * them, E as [rows, ceil(cols / 16)] bytes. */
enum mi_elem { MI_F32 = 0, MI_I32 = 1, MI_BOOL = 2, MI_BF16 = 3, MI_BFP8 = 5 };

/* A result form, not a buffer kind: an F32 result [rows, cols] delivered as
 * its two BF16 parts in a BF16 buffer [rows, 2 cols], each row's heads (the
 * values rounded to nearest even; a finite value that would round to
 * infinity keeps its truncated head) then its remainders (value - head,
 * exact in F32, rounded to nearest even; 0 for an infinite or NaN value):
 * head + remainder is within 2^-17 relative of the value.  It is the operand
 * form of the fast matmul mode's split of F32 activations (a product taken as
 * head . w + remainder . w); mi_rms_norm and mi_silu_mul_halves produce it as
 * their `out_elem`, mi_linear_parts reads it, so a producer's F32 result
 * reaches the product with no separate split pass.  No Engine counterpart.
 *
 * MI_TILES_BF16 / MI_TILES_PARTS: an [r, c] operand (r a multiple of 32, c of
 * 16) in the matrix cores' operand order ("tiles"), the form mi_linear's
 * short-row path reads: blocks of 32 rows x 16 columns, block (t, s) at
 * element ((t (c / 16) + s) 64 + l) 8, its lane l holding row 32 t + l % 32,
 * columns 16 s + 8 (l / 32) .. + 7 -- the registers of one
 * v_mfma_f32_32x32x16_bf16 step, so each step's operand is one contiguous
 * KiB.  MI_TILES_BF16: the BF16 values (an F32 source rounded to nearest
 * even), a BF16 buffer [r, c]; MI_TILES_PARTS: an F32 value's two parts (as
 * MI_BF16_PARTS) in two planes, the heads' tiles then the remainders', a
 * BF16 buffer [r, 2 c].  A buffer holding tiles is marked so: mi_linear,
 * mi_linear_swiglu and mi_linear_qkv_rope_cache read a tiled weight (and
 * tiled activations) with it, mi_matmul and mi_reshape refuse it, and other
 * ops see its datums as BF16 values in that order.  No Engine counterpart
 * (the reference's weights are tiled for its cores by tt-layout). */
enum mi_result_form { MI_BF16_PARTS = 4, MI_TILES_BF16 = 6, MI_TILES_PARTS = 7 };

/* Status codes.  `MI_E_DOMAIN` is the reference's DOMAIN error for an index
 * out of range (crates/burn-tt/src/ops.rs:995-1000). */
enum mi_status {
  MI_OK = 0,
  MI_E_ARG = -1,         /* bad argument: shape, kind, elem mismatch */
  MI_E_ID = -2,          /* unknown or freed id (a stale tensor) */
  MI_E_HIP = -3,         /* HIP runtime failure */
  MI_E_OOM = -4,         /* device or pinned memory exhausted */
  MI_E_DOMAIN = -5,      /* an index out of range, found by a kernel */
  MI_E_UNSUPPORTED = -6, /* an op this engine does not run */
  MI_E_STICKY = -7       /* an earlier asynchronous failure, not yet cleared */
};

/* ---- context: server.rs `attach` / `KmdEngine` (server.rs:2738, 4071) ---- */
int mi_ctx_create(int device, mi_ctx **out);
int mi_ctx_destroy(mi_ctx *ctx);
/* The last message of this context (or of the process for a NULL ctx). */
const char *mi_last_error(const mi_ctx *ctx);
/* Wait for all submitted work; return the first asynchronous failure and
 * clear it (`Backend::sync`, crates/burn-tt/src/lib.rs:218-226). */
int mi_sync(mi_ctx *ctx);
/* The HIP stream (`hipStream_t`) work is submitted on, for callers that
 * order their own work with it. */
int mi_stream(mi_ctx *ctx, void **stream);

/* ---- storage: Engine::upload / upload_bits / upload_bf16 / download* /
 *      free / metadata (server.rs:91-174) ---- */
int mi_upload(mi_ctx *ctx, const float *values, int64_t rows, int64_t cols,
              mi_id *out);
int mi_upload_bits(mi_ctx *ctx, const uint32_t *bits, int64_t rows,
                   int64_t cols, int elem, mi_id *out);
int mi_upload_bf16(mi_ctx *ctx, const uint16_t *bits, int64_t rows,
                   int64_t cols, mi_id *out);
/* Read back `rows * cols` datums; `n` is the capacity of `out` in datums. */
int mi_download(mi_ctx *ctx, mi_id id, float *out, int64_t n);
int mi_download_bits(mi_ctx *ctx, mi_id id, uint32_t *out, int64_t n);
int mi_download_bf16(mi_ctx *ctx, mi_id id, uint16_t *out, int64_t n);
int mi_free(mi_ctx *ctx, mi_id id);
int mi_metadata(mi_ctx *ctx, mi_id id, int64_t *rows, int64_t *cols,
                int *elem);
/* Change a buffer's `[rows, cols]` in place, the element count kept: the
 * reference's free `float_reshape` over the same storage
 * (crates/burn-tt/src/views.rs:1-30, tensor.rs:905-908). */
int mi_reshape(mi_ctx *ctx, mi_id id, int64_t rows, int64_t cols);
/* A fresh `[rows, cols]` buffer of `elem` filled with the 32-bit pattern
 * `bits` (the low 16 bits for BF16): Engine::zeros_dram (server.rs:285). */
int mi_fill(mi_ctx *ctx, int64_t rows, int64_t cols, int elem, uint32_t bits,
            mi_id *out);
/* A fresh `[rows, cols]` buffer of `elem` whose contents are unspecified
 * until written (Burn's float_empty, crates/burn-tt/src/generated/ops.rs:130):
 * the destination of in-place writers such as mi_matmul_items. */
int mi_empty(mi_ctx *ctx, int64_t rows, int64_t cols, int elem, mi_id *out);

/* ---- products: Engine::matmul_dram / matmul_dram_bf16 (server.rs:178-204)
 * `op(A) @ op(B)`: `a` is `[m, k]` or, transposed, `[k, m]`; `b` is `[k, n]`
 * or, transposed, `[n, k]`.  F32 or BF16 operands (either mix); BF16
 * operands are multiplied exactly and accumulated in F32.  The result is F32,
 * or BF16 rounded once, ties to even, when `out_elem` is MI_BF16. */
int mi_matmul(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b,
              int b_transposed, int out_elem, mi_id *out);
/* Engine::matmul_dram_batched (server.rs:229): `batch` products of one shape
 * over stacked operands.  `a` holds `batch_a` matrices stacked by rows
 * (`[batch_a * m, k]`, or `[batch_a * k, m]` transposed), `b` likewise; a
 * stack of one is broadcast to every product.  The result stacks the
 * products by rows: `[batch * m, n]`. */
int mi_matmul_batched(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b,
                      int b_transposed, int64_t batch, int64_t m, int64_t k,
                      int64_t n, int out_elem, mi_id *out);

/* Engine::matmul_dram_batched with explicit items (server.rs:229: the items
 * are blocks of resident buffers): product i multiplies the block of `a` at
 * element a_offset + i * a_stride by the block of `b` at b_offset +
 * i * b_stride, each block read with its buffer's row pitch (its cols), e.g.
 * the first ctx rows of a KV-cache slot.  A stride of 0 broadcasts one
 * block.  Result `[batch * m, n]`. */
int mi_matmul_blocks(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b,
                     int b_transposed, int64_t batch, int64_t m, int64_t k,
                     int64_t n, int64_t a_offset, int64_t a_stride,
                     int64_t b_offset, int64_t b_stride, int out_elem,
                     mi_id *out);

/* Engine::matmul_dram_batched (server.rs:229-237) over an arbitrary list of
 * operand blocks (the trait's `&[(Block, Block)]`; Block,
 * crates/tt-kernels/src/tensor.rs:3479-3483): item i multiplies the block of
 * `a` whose top-left element is (a_at[2i], a_at[2i + 1]), `[m, k]` or,
 * transposed (a_transposed[i]), `[k, m]`, by the block of `b` at
 * (b_at[2i], b_at[2i + 1]), `[k, n]` or `[n, k]`.  Result `[items * m, n]`,
 * item i in rows i m .. i m + m - 1.  Runs of items stepping by constant
 * offsets are one launch. */
int mi_matmul_pairs(mi_ctx *ctx, mi_id a, mi_id b, int64_t items,
                    const int64_t *a_at, const int *a_transposed,
                    const int64_t *b_at, const int *b_transposed, int64_t m,
                    int64_t k, int64_t n, int out_elem, mi_id *out);

/* Products over strided items, the result written in place: what Burn's
 * multi-head attention runs as reshape + swap_dims + batched matmul (the
 * reference's batched_matmul, crates/burn-tt/src/ops.rs:2981-3052, after
 * float_swap_dims, ops.rs:3168), without materialising the head-split
 * operands.  There are groups x per_group items; item (g, i) of each operand
 * is the `[rows, cols]` block at element at[0] + g * at[1] + i * at[2] of its
 * buffer, read with the buffer's row pitch (its cols) -- e.g. head i of
 * sequence g inside a `[batch * seq, heads * d_head]` projection.  The result
 * item (g, i), `[m, n]`, is written likewise into the existing buffer `out`
 * (F32 or BF16, not `a` or `b`); the rest of `out` is left as it was.  Items
 * of the result must not overlap.  m, k, n >= 1; at most 65535 items. */
int mi_matmul_items(mi_ctx *ctx, mi_id a, int a_transposed,
                    const int64_t a_at[3], mi_id b, int b_transposed,
                    const int64_t b_at[3], int64_t groups, int64_t per_group,
                    int64_t m, int64_t k, int64_t n, mi_id out,
                    const int64_t out_at[3]);

/* op(A) @ op(B) left as the engine's split-K slices: `out` is [S * m, n], S
 * partial products over consecutive k ranges (S = 1: the product itself),
 * whose sum in slice order is what mi_matmul returns.  For a consumer that
 * folds the slices itself (mi_sgd_update: a weight gradient x^T dy over many
 * rows), so no reduce launch runs.  No Engine counterpart; F32 result. */
int mi_matmul_slices(mi_ctx *ctx, mi_id a, int a_transposed, mi_id b,
                     int b_transposed, mi_id *out, int64_t *slices);

/* A linear layer's forward with its residual add in the product's epilogue:
 * out = residual + (x @ op(w) + bias), each sum rounded to F32 in that order,
 * so the result is bit-identical to mi_matmul followed by the two broadcast
 * adds.  No single Engine call corresponds: the reference runs burn's
 * nn::Linear as float_matmul (crates/burn-tt/src/generated/ops.rs:532) then
 * float_add (ops.rs:159), and a residual connection as another float_add.
 * `x` is `[m, k]` (F32 or BF16), `w` is `[k, n]` or, transposed, `[n, k]`;
 * `bias` (F32, n elements) and `residual` (F32 `[m, n]`) may each be 0 for
 * none.  The result is F32, or BF16 rounded once after both adds.
 *
 * A weight in tiles (mi_tile of a BF16 [n, k] weight; w_transposed 1) takes
 * the short-row path (a batch-1 prefill's products: few output tiles, so the
 * k range is split over the waves of a block instead of over launches):
 * each wave loads its k steps of both operands straight into the matrix
 * cores' registers, sums its range in k order, and the block adds the
 * ranges in order -- one fixed order for a given (m, n, k), not the other
 * kernels'.  `x` is then F32 [m, k] (its parts' products, as the fast
 * matmul mode splits it; the accurate mode refuses it), BF16 [m, k], or
 * tiles of an [m, k] operand (MI_TILES_PARTS: the parts' products;
 * MI_TILES_BF16).  m a multiple of 32, n of 32, k of 16 and at most 3072
 * (else MI_E_UNSUPPORTED). */
int mi_linear(mi_ctx *ctx, mi_id x, mi_id w, int w_transposed, mi_id bias,
              mi_id residual, int out_elem, mi_id *out);
/* A row-major F32 or BF16 `a` [r, c] (r a multiple of 32, c of 16) in tiles:
 * `form` MI_TILES_BF16 (BF16 values; F32 rounded to nearest even) or
 * MI_TILES_PARTS (an F32 source's parts).  A weight is tiled once, where it
 * is made; activations come in tiles from their producers (mi_rms_norm,
 * mi_linear_swiglu).  No Engine counterpart. */
int mi_tile(mi_ctx *ctx, mi_id a, int form, mi_id *out);
/* mi_linear then mi_rms_norm of its result, in one call and bit for bit the
 * two: `y` = residual + x op(w) + bias (F32 [m, n]) and `y_norm` =
 * rms_norm(y) * gamma (eps; gamma F32 [1, n] or 0 for none) as `norm_elem`
 * (MI_F32, MI_BF16 or MI_BF16_PARTS), n <= 8192.  Where the product splits
 * over k (few output tiles: a short prompt's o and down projections) the
 * split's reduce forms the norm as it writes y: one launch and one pass over
 * y fewer.  The reference's Engine::add_rms_norm (server.rs:466-475) on a
 * Linear's output and its residual; the fusion has no Engine counterpart. */
int mi_linear_add_rms_norm(mi_ctx *ctx, mi_id x, mi_id w, int w_transposed,
                           mi_id bias, mi_id residual, mi_id gamma, float eps,
                           int norm_elem, mi_id *y, mi_id *y_norm);
/* mi_linear of an F32 `x` [m, k] given as its parts (MI_BF16_PARTS, a BF16
 * `x_parts` [m, 2 k]) against a BF16 `w`: the product runs as head . op(w) +
 * remainder . op(w), accumulated in F32 over the 2 k parts in that order --
 * what the fast matmul mode computes from `x` itself where it splits it (F32
 * x BF16 products filling the chip: m a multiple of 256, k of 32), and then
 * bit for bit the same result; in either matmul mode.  Other shapes run the
 * same sums on the plain BF16 product against `w` repeated along k.  Bias,
 * residual and result as mi_linear.  No Engine counterpart: the reference
 * fuses operation chains in its fusion runtime (crates/burn-tt/src/fusion/
 * mod.rs:1-12) instead. */
int mi_linear_parts(mi_ctx *ctx, mi_id x_parts, mi_id w, int w_transposed,
                    mi_id bias, mi_id residual, int out_elem, mi_id *out);
/* A SwiGLU MLP's first half from an F32 `x` [m, k] given as its parts: with
 * the gate and up weights' rows interleaved in 32-row groups (`w_pairs`
 * [2 i, k] BF16: gate rows 0..31, up rows 0..31, gate rows 32..63, ...), the
 * result is silu(x gate^T) * (x up^T) ([m, i]) as its parts (MI_BF16_PARTS,
 * [m, 2 i] BF16), each product as mi_linear_parts computes it and
 * silu * up as MI_K_SILU_MUL does -- the same bits as mi_linear_parts against
 * the [gate; up] weight followed by mi_silu_mul_halves to parts, without the
 * F32 [m, 2 i] product between them.  Whole tiles only: m a multiple of
 * 128, k of 32, i of 128 (else MI_E_UNSUPPORTED).  No Engine counterpart
 * (the reference's MLP, crates/tt-models/src/llama.rs:494-498, runs the two
 * products and the SwiGLU as separate ops). */
int mi_linear_swiglu_parts(mi_ctx *ctx, mi_id x_parts, mi_id w_pairs,
                           mi_id *out);
/* The same for BF16 activations `x` [m, k] (the performance numeric
 * contract's operands): silu(x gate^T) * (x up^T) [m, i] as F32, or rounded
 * once to BF16 (`out_elem`) -- the same bits as the BF16 product against
 * [gate; up] on the direct kernel followed by mi_silu_mul_halves.  Whole
 * tiles only, as mi_linear_swiglu_parts.
 *
 * With `w_pairs` in tiles (mi_tile of the interleaved weight), mi_linear's
 * short-row path: `x` F32, BF16 or tiles as there, each product's sums as
 * mi_linear forms them against the same tiled weight, silu * up as
 * MI_K_SILU_MUL; `out_elem` MI_F32, MI_BF16, MI_BF16_PARTS, or tiles of the
 * [m, i] result (MI_TILES_BF16 / MI_TILES_PARTS: the down product's operand
 * as it reads it).  m a multiple of 32, i of 32. */
int mi_linear_swiglu(mi_ctx *ctx, mi_id x, mi_id w_pairs, int out_elem,
                     mi_id *out);
/* The q|k|v product and mi_qkv_rope_cache in one launch: `x` BF16 [rows, k]
 * activations, or with `x_parts` an F32 operand's parts ([rows, 2 k],
 * MI_BF16_PARTS), against `w_qkv` [(heads + 2 kv_heads) 64, k] BF16; RoPE,
 * the cache writes and q's layout as mi_qkv_rope_cache (its q returned), on
 * the product's accumulators -- the same bits as the product (mi_matmul /
 * mi_linear_parts) followed by mi_qkv_rope_cache, without the F32 q|k|v
 * rows between them.  64-wide heads, rows a multiple of 128 and k of 32
 * (else MI_E_UNSUPPORTED).  With `w_qkv` in tiles, mi_linear's short-row
 * path (`x` F32, BF16 or tiles as there, `x_parts` 0; rows a multiple of
 * 32): the same bits as mi_linear against that tiled weight followed by
 * mi_qkv_rope_cache.  No Engine counterpart (the reference's
 * attention block, crates/tt-models/src/llama.rs:403-446, runs the
 * projection, RoPE and the cache writes as separate ops). */
int mi_linear_qkv_rope_cache(mi_ctx *ctx, mi_id x, int x_parts, mi_id w_qkv,
                             mi_id cos_table, mi_id sin_table, int64_t seq,
                             int64_t heads, int64_t kv_heads, int64_t pos0,
                             mi_id k_cache, mi_id v_cache, int grouped,
                             mi_id *q_out);

/* ---- matmul mode: Engine::matmul_mode (server.rs:48) and the reference's
 * MatmulMode (crates/burn-tt/src/matmul_mode.rs:1-43), fixed per context as
 * TtConfig::matmul fixes it per attachment.  Applies to products with an F32
 * operand; BF16 x BF16 products are the same in both.
 *  FAST (the default, as the reference's): where a product is large enough to
 *   be bound by the matrix cores (>= 2^33 multiply-adds over >= 128 tiles of
 *   128 x 128), and for F32 activations (>= 256 rows) against BF16 weights at
 *   any size, each F32 operand element is split as bf16 hi + bf16 lo and
 *   a b = hi hi + hi lo + lo hi runs on the BF16 matrix cores with F32
 *   accumulation (hi b + lo b for a BF16 b); error per product <= 3 * 2^-18
 *   |a||b| (the reference's fast mode rounds operands to TF32, 2^-11).  Other
 *   products run as in ACCURATE.  A non-finite operand element gives NaN in
 *   its row or column where F32 arithmetic could give an infinity.
 *  ACCURATE: F32 products on the F32 matrix cores, F32 accumulation.
 * The reference's EXACT mode (k-ordered sequential F32 sums) is not offered:
 * MI_E_UNSUPPORTED. ---- */
enum mi_matmul_mode { MI_MATMUL_FAST = 0, MI_MATMUL_ACCURATE = 1 };
int mi_set_matmul_mode(mi_ctx *ctx, int mode);
int mi_get_matmul_mode(mi_ctx *ctx, int *mode);

/* ---- element-wise: Engine::eltwise_op_as (server.rs:519) ----
 * `kind` is one of the MI_K_* ids below (the reference's op ids,
 * crates/tt-kernels/src/kind.rs:11-27 and sfpu/ops.rs:24-250).  `b` and `c`
 * are 0 when the op takes fewer operands.  Each operand is `[rows, cols]`,
 * or broadcasts a `[1, cols]` row, a `[rows, 1]` column or a `[1, 1]` value
 * over the output, which takes the largest extent of each axis.  F32 and BF16
 * inputs are read as F32; the result is F32 (BF16 rounded once when
 * `out_elem` is MI_BF16), or Bool for a comparison. */
int mi_eltwise(mi_ctx *ctx, uint32_t kind, float scalar, float scalar2,
               mi_id a, mi_id b, mi_id c, int out_elem, mi_id *out);

/* Element-wise op ids (the reference's numbering). */
enum mi_kind {
  MI_K_ADD = 1, MI_K_SUB = 2, MI_K_MUL = 3, MI_K_MUL_SCALAR = 4,
  MI_K_RELU = 5, MI_K_RELU_BACKWARD = 6, MI_K_ADD_ROW = 7,
  MI_K_ADD_SCALAR = 11,
  MI_K_RECIP = 0x100, MI_K_DIV = 0x101, MI_K_DIV_SCALAR = 0x102,
  MI_K_EXP = 0x103, MI_K_LOG = 0x104,
  MI_K_BOOL_NOT = 0x105, MI_K_BOOL_AND = 0x106, MI_K_BOOL_OR = 0x107,
  MI_K_BOOL_XOR = 0x108,
  MI_K_NEG = 0x109, MI_K_ABS = 0x10a, MI_K_SIGN = 0x10b,
  MI_K_CLAMP = 0x10c, MI_K_CLAMP_MIN = 0x10d, MI_K_CLAMP_MAX = 0x10e,
  MI_K_LEAKY_RELU = 0x10f, MI_K_HARD_SIGMOID = 0x110,
  MI_K_EQ = 0x111, MI_K_NE = 0x112, MI_K_GT = 0x113, MI_K_GE = 0x114,
  MI_K_LT = 0x115, MI_K_LE = 0x116,
  MI_K_EQ_S = 0x117, MI_K_NE_S = 0x118, MI_K_GT_S = 0x119, MI_K_GE_S = 0x11a,
  MI_K_LT_S = 0x11b, MI_K_LE_S = 0x11c,
  MI_K_IS_NAN = 0x11d, MI_K_IS_INF = 0x11e,
  MI_K_MASK_FILL = 0x11f, MI_K_MASK_WHERE = 0x120,
  MI_K_FILL = 0x122, MI_K_SQRT = 0x123, MI_K_RSQRT = 0x124,
  MI_K_LOG1P = 0x125, MI_K_POW = 0x126, MI_K_POW_S = 0x127,
  MI_K_I32_TO_F32 = 0x129, MI_K_EXPM1 = 0x12a,
  MI_K_SIGMOID = 0x12b, MI_K_SIGMOID_BACKWARD = 0x12c,
  MI_K_TANH = 0x12d, MI_K_ERF = 0x12e,
  MI_K_GELU = 0x12f, MI_K_GELU_BACKWARD = 0x130,
  MI_K_SIN = 0x138, MI_K_COS = 0x139,
  MI_K_BOOL_TO_F32 = 0x13f,
  MI_K_ADD_RELU = 0x1f0, MI_K_SILU = 0x1f1, MI_K_SILU_MUL = 0x1f2,
  MI_K_SUB_EXP = 0x1f3, MI_K_MUL_ADD = 0x1f4, MI_K_SCALE_MASK_FILL = 0x1f5,
  /* Fused kinds of this engine, numbered above the reference's. */
  MI_K_RSQRT_ABS_ADD = 0x200 /* 1 / sqrt(|a| + scalar) */
};

/* ---- reductions: Engine::reduce (server.rs:404), Engine::full_reduce ----
 * `axis` MI_AXIS_ROWS reduces over rows (Burn dim 0): `[r, c] -> [1, c]`;
 * MI_AXIS_COLS over columns (dim 1): `[r, c] -> [r, 1]`.  MI_R_MEAN is the
 * sum divided by the count.  F32 or BF16 in, F32 out. */
enum mi_reduce_op { MI_R_SUM = 0, MI_R_MAX = 1, MI_R_MEAN = 2, MI_R_MIN = 3 };
enum mi_axis { MI_AXIS_ROWS = 0, MI_AXIS_COLS = 1 };
int mi_reduce(mi_ctx *ctx, mi_id a, int op, int axis, mi_id *out);
/* The whole buffer to `[1, 1]` (float_sum / float_mean, ops.rs:3246-3400). */
int mi_reduce_all(mi_ctx *ctx, mi_id a, int op, mi_id *out);
/* Engine::reduce with its `then` (server.rs:404-412; ReduceThen,
 * crates/tt-kernels/src/tensor.rs:6038): the reduction, then the unary kind
 * `then_kind` (0 for none) with scalar `then_scalar` applied to its result --
 * a softmax's clamp_min of a row max, say -- bit for bit the two ops. */
int mi_reduce_then(mi_ctx *ctx, mi_id a, int op, int axis, uint32_t then_kind,
                   float then_scalar, mi_id *out);

/* ---- softmax: Engine::softmax_rows (server.rs:428) and the
 * softmax/log_softmax composition (ops.rs:5133-5166) ----
 * Over each row: `softmax(scale * x)` with entries where `mask` (a Bool
 * `[mask_rows, cols]`, row `r % mask_rows` read for row `r`; 0 for none) is
 * true set to -inf first.  With a mask the max is clamped below at -FLT_MAX
 * and the sum at FLT_MIN, so a fully masked row gives zeros (ops.rs:
 * 4572-4590).  `log` selects `(x - max) - ln(sum)` instead. */
int mi_softmax_rows(mi_ctx *ctx, mi_id x, mi_id mask, float scale, int log,
                    int out_elem, mi_id *out);

/* ---- RMSNorm: Engine::rms_norm_as (server.rs:449) ----
 * `a / sqrt(mean(a * a) + eps) * gamma` over each row; `gamma` a `[1, cols]`
 * row or 0.  `out_elem` MI_F32, MI_BF16, MI_BF16_PARTS (the F32 result's
 * parts, [rows, 2 cols] BF16), or tiles of the result (MI_TILES_BF16 /
 * MI_TILES_PARTS; rows a multiple of 32, cols of 16). */
int mi_rms_norm(mi_ctx *ctx, mi_id a, mi_id gamma, float eps, int out_elem,
                mi_id *out);
/* Engine::add_rms_norm (server.rs:466-475): `sum = a + b` and
 * rms_norm(sum, gamma, eps), both new buffers; bit for bit the two ops. */
int mi_add_rms_norm(mi_ctx *ctx, mi_id a, mi_id b, mi_id gamma, float eps,
                    mi_id *sum, mi_id *norm);
/* LayerNorm over each row, `(a - mean) / sqrt(var + eps) * gamma + beta`
 * (Burn's `LayerNorm`, biased variance); gamma/beta `[1, cols]` or 0. */
int mi_layer_norm(mi_ctx *ctx, mi_id a, mi_id gamma, mi_id beta, float eps,
                  mi_id *out);

/* ---- backward rows for the training harnesses.  No Engine counterpart:
 * Burn's autodiff composes these gradients from the forward's primitive ops
 * (burn-nn LayerNorm; softmax's exp / sum / divide, ops.rs:5133-5166); the
 * fused forms are this engine's, for the transformer training step. ---- */
/* LayerNorm's gradient: with xh = (x - mean) / sqrt(var + eps) and
 * g = dy * gamma, dx = (g - mean(g) - xh * mean(g * xh)) / sqrt(var + eps)
 * (+ residual_grad if not 0), dgamma = sum_rows(dy * xh), dbeta =
 * sum_rows(dy) ([1, cols] each).  x, dy F32 [rows, cols], cols <= 1024;
 * gamma [1, cols] or 0.  Three new ids. */
int mi_layer_norm_backward(mi_ctx *ctx, mi_id x, mi_id gamma, mi_id dy,
                           mi_id residual_grad, float eps, mi_id *dx,
                           mi_id *dgamma, mi_id *dbeta);
/* Softmax's gradient over rows, p = softmax(scale * x):
 * ds = scale * p * (dp - sum_row(p * dp)).  F32 [rows, cols]. */
int mi_softmax_backward(mi_ctx *ctx, mi_id p, mi_id dp, float scale,
                        mi_id *out);
/* Cross-entropy against integer targets and its gradient in one pass over
 * the logits: burn-nn's CrossEntropyLoss as the reference runs it --
 * log_softmax (crates/burn-tt/src/ops.rs:5133-5166), the target's value
 * gathered (pick_columns_native, ops.rs:1001), and under autodiff the
 * gradient exp(logp) * s plus the one-hot -s scattered at the target
 * (scatter_add_columns_native, ops.rs:1043), s = grad_scale (1 / rows for a
 * mean).  logits F32 [rows, cols], cols <= 16384; targets I32, one per row.
 * picked [rows, 1] = logp[row, target]; dlogits [rows, cols], the same bits
 * as the composition (log-softmax, exp, MUL_ADD against the scattered
 * one-hot).  A target outside [0, cols) is MI_E_DOMAIN at the next wait
 * (picked 0, no one-hot term), as the gather and scatter report it. */
int mi_log_softmax_ce(mi_ctx *ctx, mi_id logits, mi_id targets,
                      float grad_scale, mi_id *picked, mi_id *dlogits);

/* The optimizer step `param <- param - grad * lr` (burn-optim `Sgd`, no
 * momentum or decay; the reference applies it per parameter, and its traced
 * training step writes the weights in place, crates/burn-tt/src/trace.rs:
 * 989-1010) for `count` parameters in place, in one launch per 48.  params[i]
 * and grads[i] are F32 buffers; grads[i] holds the parameter's element count
 * (any [rows, cols] folding) or S <= 64 times it -- S stacked slices, as
 * mi_matmul_slices returns them, whose sum in slice order is the gradient.
 * The same bits as the reduce-then-two-op form. */
int mi_sgd_update(mi_ctx *ctx, int64_t count, const mi_id *params,
                  const mi_id *grads, float lr);

/* ---- indexing (ops.rs:1001-1240) ---- */
/* Engine::argmax_row (server.rs:477) over every row: `[r, c] -> [r, 1]` I32,
 * the first maximum, a NaN ranking above every number. */
int mi_argmax_rows(mi_ctx *ctx, mi_id a, mi_id *out);
/* A decode step's tail for a caller that chains steps on the device: with
 * p the device position of the step's input tokens, `ids[b] = next[b]` (the
 * next step's input), `log[b, p + 1] = next[b]` and the position becomes
 * p + 1.  next, ids: I32 with B elements; pos: I32 [1, 1]; log: I32 [B,
 * cols].  A position with p + 1 outside [0, cols) writes no log entry,
 * leaves the position and raises MI_E_DOMAIN at the next wait.  No
 * counterpart in the reference, whose generator hands each step's token to
 * the host (crates/tt-models/src/generate.rs:12-22): this one lets a traced
 * decode step be replayed token after token with no host transfer between,
 * the tokens read back once. */
int mi_decode_advance(mi_ctx *ctx, mi_id next, mi_id ids, mi_id pos, mi_id log);
/* Engine::select_rows (server.rs:300): `out[i, :] = table[idx[i], :]`, raw
 * bits; `idx` an I32 buffer of any dims, read in row-major order.  An index
 * outside `[0, table rows)` is an MI_E_DOMAIN failure. */
int mi_select_rows(mi_ctx *ctx, mi_id table, mi_id idx, mi_id *out);
/* mi_select_rows then mi_cast to `out_elem` (F32 or BF16) in one call: a
 * BF16 table's rows are widened as they are gathered (one launch; rows of a
 * multiple of 8 columns), other pairs run the two ops.  The gathered values
 * are those of the two ops.  No Engine counterpart (the reference's
 * embedding is the gather then a cast of the rows to the stream's dtype,
 * crates/tt-models/src/llama.rs:756-764). */
int mi_select_rows_as(mi_ctx *ctx, mi_id table, mi_id idx, int out_elem,
                      mi_id *out);
/* Engine::pick_columns (server.rs:349): `out[r] = x[r, idx[r]]`, raw bits,
 * `[r, 1]`. */
int mi_pick_columns(mi_ctx *ctx, mi_id x, mi_id idx, mi_id *out);
/* Burn's float_gather along any dim of a rank <= 4 tensor (ops.rs:1102-1160,
 * gather_native): `x` holds the row-major tensor of dims `dims[0..3]`
 * (leading dims 1 for a lower rank), `idx` an I32 buffer of the same
 * element count as dims `idims` (equal to `dims` except along `dim`);
 * `out[i] = x[i with its coordinate along dim replaced by idx[i]]`, raw
 * bits (4- or 2-byte elements), as [idims[0] idims[1] idims[2], idims[3]].
 * An index outside [0, dims[dim]) writes zero bits and is an MI_E_DOMAIN
 * failure at the next wait (ops.rs:995-1000).  The reference stages each
 * output element's candidates as a row (its repack, 32 rows at a time) and
 * picks with Engine::gather_indexed (server.rs:293), which is this
 * library's mi_pick_columns; here one launch reads the candidates in place. */
int mi_gather(mi_ctx *ctx, mi_id x, const int64_t dims[4], int dim, mi_id idx,
              const int64_t idims[4], mi_id *out);
/* The gather's backward (ops.rs:1043-1100): a copy of `x` with `v[r]` added
 * at `[r, idx[r]]`. */
int mi_scatter_add_columns(mi_ctx *ctx, mi_id x, mi_id idx, mi_id v,
                           mi_id *out);
/* Engine::select_add_rows (server.rs:358): a copy of `t` with row `i` of
 * `value` added to row `idx[i]`, duplicates folded in index order. */
int mi_select_add_rows(mi_ctx *ctx, mi_id t, mi_id idx, mi_id value,
                       mi_id *out);

/* ---- layout: Engine::repack / copy_blocks (server.rs:269-284) ----
 * A new `[rows, cols]` buffer whose element `(i, j)` is
 * `src[offset + i * row_stride + j * col_stride]` (strides in elements):
 * transposes, head splits and slices as one strided copy. */
int mi_copy_strided(mi_ctx *ctx, mi_id src, int64_t rows, int64_t cols,
                    int64_t offset, int64_t row_stride, int64_t col_stride,
                    mi_id *out);
/* A strided copy over a 4-D index space `[d0, d1, d2, d3]` (row-major
 * output of `d0*d1*d2` rows by `d3` columns), source strides s0..s3: a
 * `swap_dims`/`permute` materialised in one pass. */
int mi_copy_strided4(mi_ctx *ctx, mi_id src, const int64_t dims[4],
                     int64_t offset, const int64_t strides[4], mi_id *out);
/* Write `src` into `dst` (in place) at rows `[row0, row0 + src rows)`,
 * columns `[col0, col0 + src cols)`: a `slice_assign` (KV-cache writes). */
int mi_assign_block(mi_ctx *ctx, mi_id dst, mi_id src, int64_t row0,
                    int64_t col0);
/* A strided 4-D copy into an existing buffer (in place): element
 * (i0, i1, i2, i3) of `dims` goes from src[src_offset + sum i * src_strides]
 * to dst[dst_offset + sum i * dst_strides]; both ranges are bounds-checked.
 * KV-cache appends (crates/tt-models/src/llama.rs:415-435: `slice_assign`
 * into the cache) and Engine::scatter_rows_into (server.rs:389). */
int mi_copy_into4(mi_ctx *ctx, mi_id dst, int64_t dst_offset,
                  const int64_t dst_strides[4], mi_id src, int64_t src_offset,
                  const int64_t src_strides[4], const int64_t dims[4]);
/* Engine::rope_blocks (server.rs:566; crates/burn-tt/src/ops/rope.rs:27-240):
 * rows of `x` ([rows, d] F32) laid out (sequence, position, head) -- row r
 * at position pos0 + (r / heads) % seq -- become x * cos + rotate(x) * sin,
 * rotate swapping the halves; `cos`/`sin` are [positions, d] tables with
 * sin's first half negated (crates/tt-models/src/rope.rs:6-60). */
int mi_rope(mi_ctx *ctx, mi_id x, mi_id cos_table, mi_id sin_table,
            int64_t heads, int64_t seq, int64_t pos0, mi_id *out);
/* Engine::attention_rows (server.rs:255-265; crates/tt-kernels/src/
 * attention.rs:1-20; the composition of crates/burn-tt/src/ops.rs:4520-4595):
 * causal grouped-query attention of `t` new positions per sequence against a
 * KV cache.  q: [batch * t, heads * d] F32, rows (sequence, position), head h
 * reading kv head h / (heads / kv_heads).  k_cache, v_cache: both F32 or
 * both BF16 (the performance contract's cache, crates/tt-models/src/
 * llama.rs:1276-1278; widened exactly, F32 arithmetic either way)
 * [batch * kv_heads * max_ctx, d], item (sequence, kv head), the new
 * positions already written at pos0 .. pos0 + t - 1.  Query position p sees
 * cache positions 0 .. pos0 + p.  out: [batch * t, heads * d] =
 * softmax(scale * q k^T) v per head (max clamped at -FLT_MAX, sum at
 * FLT_MIN).  d in {16, 32, 64, 128}; at most 8 query heads per kv head. */
int mi_attention_rows(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache,
                      int64_t batch, int64_t t, int64_t heads,
                      int64_t kv_heads, int64_t pos0, float scale,
                      mi_id *out);
/* mi_attention_rows with its result in `out_form`: MI_F32 (mi_attention_rows
 * itself), MI_BF16 (each value rounded once), MI_BF16_PARTS (the F32
 * values' parts, [batch t, 2 heads d]), or tiles of the [batch t,
 * heads d] result (MI_TILES_BF16 / MI_TILES_PARTS; batch t a multiple of 32)
 * -- the operand an o projection against a tiled weight reads, stored by the
 * matrix-core (many new positions) kernel itself; other paths convert their
 * F32 rows.  The same values as mi_attention_rows, then rounded or split.
 * No Engine counterpart. */
int mi_attention_rows_as(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache,
                         int64_t batch, int64_t t, int64_t heads,
                         int64_t kv_heads, int64_t pos0, float scale,
                         int out_form, mi_id *out);
/* mi_attention_rows for a traced decode step, whose positions are device
 * data (the reference's position tensors and its step traced per attended
 * length, crates/tt-models/src/generate.rs:1-22, 770-790): pos0 read on the
 * device from `pos` ([1, 1] I32) when `pos` is nonzero, else the immediate
 * pos0; the key chunks planned for `span` positions (pos0 + t <= span <=
 * max_ctx), so every call with one span runs the same launches whatever the
 * position and a graph captured once replays at any position of its span.
 * The same results as mi_attention_rows up to the order of the chunk sums,
 * and bit for bit the same between an immediate and a device pos0 of one
 * value and span.  A device pos0 with pos0 < 0 or pos0 + t > span attends
 * from position 0 and raises MI_E_DOMAIN at the next wait.  The prompt's
 * matrix-core kernel is not used. */
int mi_attention_rows_at(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache,
                         int64_t batch, int64_t t, int64_t heads,
                         int64_t kv_heads, mi_id pos, int64_t pos0,
                         int64_t span, float scale, mi_id *out);
/* mi_attention_rows writing into an existing F32 `[batch * t, heads * d]`
 * buffer `out` (not one of the inputs), with no allocation of any kind: no
 * device or host memory is allocated, freed or grown, so callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation -- can call it.  No counterpart in the reference
 * (its attention_rows returns a new buffer).  The key-chunk partials live in
 * a fixed 4 MiB device array per GPU, held until the process ends; a call
 * whose partials need more (items * chunks * G * (d + 2) floats: long
 * prompts of many sequences) is refused with MI_E_UNSUPPORTED.  Every call on
 * one GPU shares that array: calls from different contexts or streams that
 * overlap in time on one GPU race; calls on one context's stream never do.
 * Same kernels and chunking as mi_attention_rows, so the same bits. */
int mi_attention_rows_into(mi_ctx *ctx, mi_id q, mi_id k_cache, mi_id v_cache,
                           int64_t batch, int64_t t, int64_t heads,
                           int64_t kv_heads, int64_t pos0, float scale,
                           mi_id out);
/* ---- fused decode projections: the fused q|k|v and gate|up matrices of
 * crates/tt-models/src/llama.rs:655-672 (`Llama::fused`) composed with the
 * ops around them in a decode step -- Engine::rms_norm_as (server.rs:449),
 * rope_blocks (server.rs:566), the KV-cache slice_assign (llama.rs:415-435),
 * the residual add and silu_mul (crates/burn-tt/src/ops.rs:2622-2651).  x is
 * [M, K] F32 with 1 <= M <= 32 (one row per sequence), K a multiple of 8; w is
 * BF16 [N, K] (each output row's weights k-contiguous, as the projections are
 * stored); gamma a [1, K] F32 RMSNorm gain or 0 for no norm. ---- */
/* out = residual + rmsnorm(x) w^T ([M, N]; residual [M, N] or 0), or with
 * silu_mul != 0 and w = [gate; up] ([2 I, K]): out = silu(g) * u, [M, I]. */
int mi_norm_matvec(mi_ctx *ctx, mi_id x, mi_id gamma, float eps, mi_id w,
                   mi_id residual, int silu_mul, mi_id *out);
/* A greedy decode step's head and pick in one call: logits = rmsnorm(x) w^T
 * (mi_norm_matvec with no residual, its bits) and ids = mi_argmax_rows of
 * them ([M, 1] I32, its rule) -- the reference's vocabulary head then the
 * greedy argmax of its generation loop (crates/tt-models/src/generate.rs:
 * 176-183), no Engine counterpart.  For one row against a weight of 32 MiB
 * or more (BF16, k <= 1024: a vocabulary head) the head's launch also folds
 * each block's logits to a best (value, index), and one block folds those:
 * no pass over the logits afterwards.  Otherwise the two calls. */
int mi_norm_matvec_argmax(mi_ctx *ctx, mi_id x, mi_id gamma, float eps,
                          mi_id w, mi_id *logits, mi_id *ids);
/* w_qkv = [wq; wk; wv] ([(heads + 2 kv_heads) * d, K]): q = rope(rmsnorm(x)
 * wq^T) returned [M, heads * d]; k = rope(.. wk^T) and v = .. wv^T written
 * into the caches ([M * kv_heads * max_ctx, d], both F32 or both BF16
 * (rounded to nearest even), item (row, kv head)) at
 * position `pos`; the rotary tables as mi_rope's, read at row `pos`. */
int mi_norm_qkv_rope(mi_ctx *ctx, mi_id x, mi_id gamma, float eps,
                     mi_id w_qkv, mi_id cos_table, mi_id sin_table,
                     int64_t heads, int64_t kv_heads, int64_t pos,
                     mi_id k_cache, mi_id v_cache, mi_id *q_out);
/* mi_norm_qkv_rope with the position read on the device from `pos` ([1, 1]
 * I32; a traced decode step's input, as mi_attention_rows_at's), the rotary
 * tables covering every position below max_ctx.  Bit for bit
 * mi_norm_qkv_rope at the position's value; a position outside [0, max_ctx)
 * writes no cache row and no q and raises MI_E_DOMAIN at the next wait. */
int mi_norm_qkv_rope_at(mi_ctx *ctx, mi_id x, mi_id gamma, float eps,
                        mi_id w_qkv, mi_id cos_table, mi_id sin_table,
                        int64_t heads, int64_t kv_heads, mi_id pos,
                        mi_id k_cache, mi_id v_cache, mi_id *q_out);
/* A decode step's attention up to its rows, in one call: mi_norm_qkv_rope
 * (or _at; the new key and value stored into the caches at the position)
 * then mi_attention_rows_at over the keys up to and including it (t = 1),
 * returning the attention rows [M, heads * d] F32 -- the reference's
 * attention block from its normed input to the attention output (crates/
 * tt-models/src/llama.rs:380-470), no Engine counterpart.  pos: a [1, 1]
 * I32 device position, or 0 for the immediate pos0; span as
 * mi_attention_rows_at's.  Up to 6 sequences with 64-wide heads, a gain and
 * k a multiple of 32 up to 1024: one launch forms each head's queries, the
 * new key and value rows and the key chunks' partials over the earlier
 * positions, and a combine adds the new key as one more chunk -- the two
 * calls' values up to the order of the sums.  Otherwise those two calls. */
int mi_norm_qkv_attention(mi_ctx *ctx, mi_id x, mi_id gamma, float eps,
                          mi_id w_qkv, mi_id cos_table, mi_id sin_table,
                          int64_t heads, int64_t kv_heads, mi_id pos,
                          int64_t pos0, int64_t span, mi_id k_cache,
                          mi_id v_cache, float scale, mi_id *out);
/* A decode step's whole attention block: x + o w_o^T, o the attention rows
 * mi_norm_qkv_attention returns for the same arguments, w_o the output
 * projection [hidden, heads * d] (BF16 or BFP8) and x [M, hidden] the
 * residual -- the reference's attention block through its output
 * projection and residual add (crates/tt-models/src/llama.rs:380-478; the
 * add at :478), no Engine counterpart.  Bit for bit mi_norm_qkv_attention then
 * mi_norm_matvec(o, 0, 0, w_o, x).  For one sequence on the fused launch
 * (up to 16 heads) the combine of the key chunks runs inside the
 * projection's launch, one launch fewer a step; otherwise those two calls. */
int mi_norm_qkv_attention_o(mi_ctx *ctx, mi_id x, mi_id gamma, float eps,
                            mi_id w_qkv, mi_id cos_table, mi_id sin_table,
                            int64_t heads, int64_t kv_heads, mi_id pos,
                            int64_t pos0, int64_t span, mi_id k_cache,
                            mi_id v_cache, float scale, mi_id w_o,
                            mi_id *out);
/* silu(gate) * up over the halves of a fused gate|up product: gate_up
 * [rows, 2 i] F32 -> [rows, i] of out_elem (the reference's MLP, crates/
 * tt-models/src/llama.rs:494-498, on the two row blocks of its gate|up
 * weight); no Engine counterpart.  F32: bit-identical to MI_K_SILU_MUL of the
 * two halves; BF16: that value rounded once (the performance contract's
 * activation operand, llama.rs:1270-1274); MI_BF16_PARTS: the F32 value's
 * parts ([rows, 2 i] BF16). */
int mi_silu_mul_halves(mi_ctx *ctx, mi_id gate_up, int out_elem, mi_id *out);
/* The q|k|v tail of a prefill in one launch: the composition the reference's
 * attention block makes of RoPE on the query and key heads, the key/value
 * cache write and the queries' grouping per kv head (crates/tt-models/src/
 * llama.rs:403-446; crates/tt-models/src/rope.rs:1-140), with no Engine
 * counterpart.  qkv: [batch * seq, (heads + 2 kv_heads) * d] F32 rows
 * (sequence, position) of the fused q|k|v projection; RoPE as mi_rope at
 * positions pos0 + p; keys and values written into the caches ([batch *
 * kv_heads * max_ctx, d] F32, item (sequence, kv head)) at positions pos0 ..
 * pos0 + seq - 1; q_out [batch * seq * heads, d]: rows (sequence, position,
 * head), or with `grouped` rows (sequence, kv head j, position, g) for head
 * j * heads / kv_heads + g.  Bit-identical to mi_rope + mi_copy_into4 +
 * mi_copy_strided4. */
int mi_qkv_rope_cache(mi_ctx *ctx, mi_id qkv, mi_id cos_table, mi_id sin_table,
                      int64_t seq, int64_t heads, int64_t kv_heads, int64_t pos0,
                      mi_id k_cache, mi_id v_cache, int grouped, mi_id *q_out);
/* Engine::cast_float (server.rs:128): F32 <-> BF16, ties to even, NaN kept
 * a NaN; and I32 -> F32 (`as f32`).  `out_elem` MI_BF16_PARTS: an F32
 * buffer's parts (columns a multiple of 4). */
int mi_cast(mi_ctx *ctx, mi_id a, int out_elem, mi_id *out);
/* Engine::cast_bfp (server.rs:141-147, 1035-1050; Session::store_bfp and
 * bfp_to_f32): `format` MI_BFP8 stores an F32 or BF16 buffer as BFP8 by the
 * reference's packer rule (crates/tt-models/src/quant.rs:185-235): each
 * value's BF16 truncation in quanta of 2^(E - 133), E the largest biased
 * exponent of its block, rounded half away from zero and clamped to 127
 * quanta (a zero or subnormal value is 0).  The reference refuses a
 * non-finite value; here one raises MI_E_DOMAIN at the next wait and its
 * block is held as zeros.  `format` 0 decodes a BFP8 buffer to F32 (exact).
 * A new buffer either way. */
int mi_cast_bfp(mi_ctx *ctx, mi_id a, int format, mi_id *out);

/* ---- traces: Engine::begin_trace / end_trace / run_trace /
 * run_generic_trace / release_trace (server.rs:591-660, 746), the reference's
 * TracedTrainingStep (crates/burn-tt/src/trace.rs:989-1010), as HIP graphs
 * captured from the context's stream.  Between begin and end, ops are
 * recorded, not run; host transfers, waits and event timing are refused
 * (MI_E_UNSUPPORTED), as is an embedding backward of more than 8192 indices.
 * Memory a capture allocates or frees stays reserved for the trace until it
 * is released, so replays never touch memory handed to other work; buffers
 * the trace reads that existed before the capture must outlive it.  A replay
 * overwrites each input buffer with the host bytes given, launches the graph
 * and reads each output buffer back whole.  The host slices' lengths are
 * passed as the reference passes its slices (`values: &[f32]`, server.rs:
 * 650-656; the payloads of run_generic_trace, 746-751): value_bytes[i] must
 * be input i's buffer size in bytes exactly, out_bytes[i] the room at
 * out_values[i], at least output i's buffer size; any mismatch is MI_E_ARG
 * before anything is written or launched. ---- */
int mi_trace_begin(mi_ctx *ctx);
int mi_trace_end(mi_ctx *ctx, uint64_t *trace);
int mi_trace_run(mi_ctx *ctx, uint64_t trace, int64_t n_inputs,
                 const mi_id *inputs, const void *const *values,
                 const int64_t *value_bytes, int64_t n_outputs,
                 const mi_id *outputs, void *const *out_values,
                 const int64_t *out_bytes);
int mi_trace_release(mi_ctx *ctx, uint64_t trace);
/* Engine::copy_into (server.rs:742): src's bytes into dst (equal byte size),
 * no allocation. */
int mi_copy_into(mi_ctx *ctx, mi_id src, mi_id dst);

/* ---- random: Engine::random_dram (server.rs:768) with the draw's 64-bit
 * base (crates/burn-tt/src/random.rs:42-56) ---- */
enum mi_draw {
  MI_DRAW_UNIT = 0,    /* [0, 1) */
  MI_DRAW_UNIFORM = 1, /* [p1, p2) */
  MI_DRAW_NORMAL = 2,  /* N(p1, p2^2) */
  MI_DRAW_BERNOULLI = 3, /* 1 with probability p1, as F32 */
  MI_DRAW_INT_RANGE = 4  /* integers in [p1, p2), I32 */
};
int mi_random(mi_ctx *ctx, int64_t rows, int64_t cols, int draw, float p1,
              float p2, uint64_t base, mi_id *out);

/* ---- timing on the context's stream (bench support; the reference's
 * session profiler, session.rs:9811-9830) ---- */
int mi_event_record(mi_ctx *ctx, int slot); /* slot in [0, 16) */
int mi_event_elapsed_ms(mi_ctx *ctx, int from, int to, float *ms);

/* ---- the op report (crates/burn-tt/src/report.rs:29-51) ---- */
typedef struct mi_report {
  uint64_t ops;            /* kernels submitted */
  uint64_t uploads;        /* host-to-device copies */
  uint64_t downloads;      /* device-to-host copies */
  uint64_t bytes_up;       /* host-to-device bytes */
  uint64_t bytes_down;     /* device-to-host bytes */
  uint64_t live_buffers;   /* ids not yet freed */
  uint64_t device_bytes;   /* bytes held by live buffers */
  uint64_t cached_bytes;   /* bytes held by the allocator's free lists */
} mi_report;
int mi_get_report(mi_ctx *ctx, mi_report *out);

#ifdef __cplusplus
}
#endif
#endif /* MIBURN_H */
