/* mbq — MI355X (gfx950) quantized linear: the C ABI of libmbq.so.
 *
 * The drop-in boundary for mashbox's quantized-linear path. mashbox's kernel-package surface
 * (reference src/mashbox/ops/__init__.py:11-34: TYPES, repack, repack_host, matmul, dequant, plane_bytes, kq_covers,
 * picks_layer) and its int8 per-channel linear (reference src/mashbox/models/qwen3_8_27b/model.py:72-82) are served by
 * these entry points; the Python package mashbox_amd binds them with ctypes.
 *
 * Conventions
 *   - Plain pointers and sizes only. "dev" pointers are device (HBM) addresses owned by the caller; "host" pointers are
 *     host memory. Every device entry point is stream-ordered on `stream` (a hipStream_t; NULL = the default stream)
 *     and returns before the work finishes; none allocates, except the GEMM's split-K workspaces of mbq_matmul
 *     and mbq_int8_linear, once per stream (see mbq_gemm_plan; mbq_matmul_noalloc never allocates), and none waits on
 *     the GPU except for that allocation.
 *   - Matrices are row-major. Activations x are bfloat16 bits (uint16) of shape (M, K); results y are (M, N) as
 *     float32 (out_dtype MBQ_OUT_F32) or bfloat16 bits rounded to nearest even (MBQ_OUT_BF16).
 *   - Weights have N rows (outputs) and K columns (inputs), as the GGUF reader orders them (reference
 *     src/mashbox/gguf/reader.py:85-87).
 *   - Return value: MBQ_OK (0) or a negative MBQ_E* code; mbq_last_error() gives the message of the calling
 *     thread's last failure. A failure launches nothing.
 *   - Device pointers must be 16-byte aligned (the kernels issue 128-bit loads and stores).
 */
#ifndef MBQ_H
#define MBQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids on this path (reference src/mashbox/ops/reference.py:22-29); MBQ_INT8 is not a ggml type: it names the
 * int8 per-output-channel weights of reference src/mashbox/models/qwen3_8_27b/model.py:72-82 */
#define MBQ_Q4_0 2
#define MBQ_Q8_0 8
#define MBQ_Q4_K 12
#define MBQ_Q5_K 13
#define MBQ_Q6_K 14
#define MBQ_INT8 (-8)
/* int8 per-output-channel weights repacked once at load into 16-row tiles (mbq_int8_repack_host / _dev): the planes
 * mbq_matmul, mbq_matmul_noalloc, mbq_plane_bytes, mbq_covers and mbq_gemm_plan take with this type id */
#define MBQ_I8T (-9)
/* Q4_K weights repacked once at load into 16-row tiles: mbq_repack_host / mbq_repack_dev / mbq_unpack_host with this
 * type id take the same Q4_K file blocks (rows, row_bytes) and write (read) planes whose 16 rows x 128 values of a
 * tile are one contiguous KiB, then the tiles' super-block headers (the Q4_K MFMA operand tile the K-group kernel
 * loads); mbq_plane_bytes, mbq_covers, mbq_matmul, mbq_matmul_noalloc, mbq_dequant, mbq_dequant_rows and
 * mbq_gemm_plan take them with this id, and give the results of the row-major MBQ_Q4_K planes (dequant bit for bit;
 * matmul within the same bars, and bit for bit from 65 rows on, where both run the same plans). Not a ggml type:
 * mbq_has_type and mbq_row_bytes refuse it. A layout of this library, with no counterpart in the reference: it serves
 * decode batches of several rows (the engine's row buckets 4 and 16, reference src/mashbox/runtime/engine.py:424-428)
 * better than the row-major planes. */
#define MBQ_Q4KT (-12)
/* Q8_0 weights repacked once at load into 16-row tiles, as MBQ_Q4KT for Q4_K: the same entry points take the Q8_0 file
 * blocks with this id and write (read) planes whose 16 rows x 64 quants of a tile are one contiguous KiB (the MBQ_I8T
 * quant layout), then the tiles' block scales; K a multiple of 32 (a last half chunk is zero padding). Dequant and
 * row gathers give the row-major MBQ_Q8_0 planes' values bit for bit, matmul the same bars. Not a ggml type. */
#define MBQ_Q8T (-10)
/* Q6_K weights repacked once at load into 16-row tiles, as MBQ_Q4KT for Q4_K: each of the four Q6_K planes (low
 * nibbles, high bits, sub-block scales, super-block scales) tiled by 16 rows x 128 values, the low nibbles' KiB
 * holding one 32-value unit per lane of a wave-wide load. Dequant bit for bit, matmul the same bars. Not a ggml type. */
#define MBQ_Q6KT (-14)
/* Q5_K weights in 16-row tiles, as MBQ_Q4KT (low nibbles and super-block headers tiled the same way) plus the high-bit
 * words tiled by 16 rows x 128 values. Dequant bit for bit, matmul the same bars. Not a ggml type. */
#define MBQ_Q5KT (-13)
/* Q4_0 weights in 16-row tiles, as MBQ_Q4KT (16 rows x 128 values of 16-byte units per KiB), the blocks' fp16 scales
 * tiled beside them; K a multiple of 32 (the last chunk's blocks past K are zero padding). Not a ggml type. */
#define MBQ_Q40T (-11)

#define MBQ_OUT_F32 0
#define MBQ_OUT_BF16 1

#define MBQ_OK 0
#define MBQ_E_ARG (-1)      /* bad type, shape, pointer or alignment */
#define MBQ_E_HIP (-2)      /* a HIP runtime call failed (launch, device query) */
#define MBQ_E_CAP (-3)      /* the output buffer is smaller than mbq_plane_bytes */

/* Library version (major*10000 + minor*100 + patch). */
int mbq_version(void);

/* Message of the calling thread's last failure ("" if none). The pointer stays valid until the thread's next call. */
const char* mbq_last_error(void);

/* 1 if type t is a ggml type with kernel planes here (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K: the types of reference
 * src/mashbox/ops/bundle.py:39), else 0.
 * Replaces the membership test `t in mod.TYPES` (reference src/mashbox/ops/__init__.py:21,303). */
int mbq_has_type(int t);

/* 1 if mbq_dequant_raw reads the file blocks of ggml type t, else 0: the five types above and F32, F16, BF16, Q4_1,
 * Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4 and NVFP4 (every ggml type but the seven that decode
 * through gguf-py's code books: IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M). Replaces the membership test
 * `t in BLOCKS` of the reference's dequant (src/mashbox/ops/reference.py:383-387,400-401), whose exact path takes every
 * type. */
int mbq_has_raw_type(int t);

/* Bytes one packed row of `cols` values takes in the file (ggml row bytes) for any ggml type id, or a negative code if
 * t is not one or cols is not a multiple of the type's block. Restates reference src/mashbox/ops/reference.py:22-29,
 * 390-395. */
int64_t mbq_row_bytes(int t, int64_t cols);

/* 1 if the kernels run a (rows, cols) weight of type t at every batch size, else 0: cols must be a whole number of
 * blocks, and the weight's planes must fit one buffer range (at most 0x7FFFFF00 bytes; mbq_matmul cuts activations
 * into row chunks within that range itself). Replaces the optional kq_covers(t, (rows, cols)) (reference
 * src/mashbox/ops/__init__.py:359-363), whose contract is that a covered shape runs. */
int mbq_covers(int t, int64_t rows, int64_t cols);

/* Device bytes of one (rows, cols) weight's kernel planes, 256-byte aligned, so that a stack of L weights is
 * L * mbq_plane_bytes(...) bytes with weight l at byte offset l * mbq_plane_bytes(...).
 * Replaces plane_bytes(t, shape) (reference src/mashbox/ops/__init__.py:24,374-378). Negative on error. */
int64_t mbq_plane_bytes(int t, int64_t rows, int64_t cols);

/* Host repack: the file's blocks raw (rows, row_bytes) -> the kernel planes in planes_host (cap bytes, at least
 * mbq_plane_bytes). A lossless byte permutation (padding bytes are zero); uses up to `threads` host threads
 * (0 = all cores). Replaces repack_host(t, raw, shape) (reference src/mashbox/ops/__init__.py:22-23,473-474). */
int mbq_repack_host(int t, const uint8_t* raw, int64_t rows, int64_t cols, uint8_t* planes_host, size_t cap,
                    int threads);

/* Inverse of mbq_repack_host: planes -> the file's blocks (rows, row_bytes). Used to prove the repack lossless. */
int mbq_unpack_host(int t, const uint8_t* planes_host, int64_t rows, int64_t cols, uint8_t* raw, size_t cap);

/* Device repack: the same permutation as mbq_repack_host, run on the GPU from blocks already in HBM.
 * Replaces the traced repack(t, raw, shape) on a device array (reference src/mashbox/ops/__init__.py:16,475-485). */
int mbq_repack_dev(int t, const uint8_t* raw_dev, int64_t rows, int64_t cols, uint8_t* planes_dev, void* stream);

/* y (M, N) = x (M, K) @ W.T for the planes of one (N, K) weight of ggml type t, float32 accumulation.
 * planes_dev: a stack of weights laid out as mbq_plane_bytes apart; `layer` picks one of them (0 for a lone weight),
 * read in place. layer_dev, when not NULL, is a device int32 holding the layer index instead (read by the kernel, so a
 * captured graph or a device-side layer loop never syncs with the host); nlayers bounds it (an index outside
 * [0, nlayers) makes every output NaN and is never read out of range).
 * M = 0 launches nothing. Replaces matmul(x, planes[, layer=]) (reference src/mashbox/ops/__init__.py:17-19,613-616;
 * call contract src/mashbox/ops/bundle.py:559-598: x as bf16, f32 result). */
int mbq_matmul(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
               const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev, int out_dtype, void* stream);

/* mbq_matmul for callers that cannot allocate: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. No counterpart in the reference. It runs the same plans and kernels as mbq_matmul, with identical results,
 * and calls no hipMalloc, hipFree or allocating library routine: a batch that splits K keeps its float32 partial tiles
 * and arrival counters in the library's static scratch array (64 MiB of partials, the allocated workspace's size, and 4096 counters; every GPU the
 * library runs on holds its own copy until the process ends), instead of mbq_matmul's allocated workspace. A plan whose
 * partials exceed the scratch (none of the automatic plans on up to 256 CUs; a forced plan can) returns MBQ_E_ARG and
 * launches nothing. Every call on one GPU shares that GPU's scratch: calls that overlap in time on one GPU (two streams)
 * race, and must not both split K. */
int mbq_matmul_noalloc(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
                       const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev, int out_dtype, void* stream);

/* W (N, K) float32 from the planes of one weight (layer / layer_dev as in mbq_matmul). Bit for bit the reference
 * dequantization (NaN where it has NaN). Replaces dequant(planes) (reference src/mashbox/ops/__init__.py:20,691-705). */
int mbq_dequant(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers, int64_t N,
                int64_t K, float* w_dev, void* stream);

/* Rows of W as float32: w (count, K) row r = dequantized weight row rows_dev[r] (device int32 ids; an id below zero
 * counts from the end, and ids are then clamped to [0, N - 1], as jax.numpy indexes), bit for bit the rows of
 * mbq_dequant, reading only those rows. Replaces take_rows(h, ids) on kernel planes (reference
 * src/mashbox/ops/__init__.py:527-548: the embedding lookup of a quantized table). */
int mbq_dequant_rows(int t, const uint8_t* planes_dev, int64_t layer, const int32_t* layer_dev, int64_t nlayers,
                     int64_t N, int64_t K, const int32_t* rows_dev, int64_t count, float* w_dev, void* stream);

/* W (rows, cols) float32 straight from the file's blocks raw_dev (rows, row_bytes) in HBM, no planes: the exact path's
 * rebuild, bit for bit the reference dequantization (NaN where it has NaN), for every type mbq_has_raw_type names
 * (the float types take any cols; a block type whole blocks). Replaces dequant(raw, t, cols) of reference
 * src/mashbox/ops/reference.py:398-409 as the exact path calls it (src/mashbox/ops/__init__.py:574-576). */
int mbq_dequant_raw(int t, const uint8_t* raw_dev, int64_t rows, int64_t cols, float* w_dev, void* stream);

/* y (M, N) = x (M, K) bf16 @ W.T for 1-8 activation rows, W (N, K) the file's blocks raw_dev (N, row_bytes) of a type
 * mbq_has_raw_type names that has no kernel planes (F32, F16, BF16, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, IQ4_NL, IQ4_XS,
 * TQ1_0, TQ2_0, MXFP4, NVFP4): each weight row rebuilt in registers, bit for bit the values of mbq_dequant_raw, and
 * multiplied in float32 (float32 products summed in float32), without writing W. K must be a multiple of 32; M = 0
 * launches nothing; more than 8 rows is refused (mbq_dequant_raw and a GEMM serve those). The exact path's product of
 * reference src/mashbox/ops/__init__.py:574-576,624-632 (dequant, then a float32 dot) for decode-sized batches.
 * raw_dev starts at a multiple of the type's block alignment (4 bytes for Q2_K, Q4_1, Q5_1, IQ4_XS, NVFP4 and F32; 2
 * for Q3_K, Q5_0, IQ4_NL, TQ1_0, TQ2_0, F16 and BF16; any for MXFP4), as mbq_dequant_raw's does for these types. */
int mbq_matmul_raw(int t, const uint8_t* raw_dev, const uint16_t* x_dev, int64_t M, int64_t N, int64_t K, void* y_dev,
                   int out_dtype, void* stream);

/* int8 per-output-channel linear: y (M, N) = (x (M, K) @ bf16(q).T accumulated in float32) * s, then out_dtype.
 * q_dev int8 (N, K) row-major, s_dev float32 (N,). Replaces linear(x, {"q", "s"}) (reference
 * src/mashbox/models/qwen3_8_27b/model.py:72-82); with out_dtype MBQ_OUT_F32 it returns the float32 y*s that the
 * reference's pj hook receives (model.py:79). */
int mbq_int8_linear(const int8_t* q_dev, const float* s_dev, const uint16_t* x_dev, int64_t M, int64_t N, int64_t K,
                    void* y_dev, int out_dtype, void* stream);

/* Load-time repack of int8 per-output-channel weights (the (rows, cols) int8 quants q, row-major, and the (rows,)
 * float32 scales s of reference src/mashbox/models/qwen3_8_27b/weights.py:55-74) into planes of type MBQ_I8T: 16-row
 * tiles whose 16 rows x 64 bytes are one contiguous KiB (the MFMA operand tile the kernels load), then the scales;
 * cols a multiple of 16, padding zero; mbq_plane_bytes(MBQ_I8T, rows, cols) bytes. mbq_matmul(MBQ_I8T, planes, ...)
 * then returns (x @ bf16(q).T accumulated in float32) * s, as mbq_int8_linear does on the unpacked weights.
 * The host form uses up to `threads` host threads (0 = all cores); the device form runs from q and s in HBM
 * (16-byte aligned q). mbq_int8_unpack_host inverts the host form (q and s back, to prove it lossless). */
int mbq_int8_repack_host(const int8_t* q, const float* s, int64_t rows, int64_t cols, uint8_t* planes_host, size_t cap,
                         int threads);
int mbq_int8_repack_dev(const int8_t* q_dev, const float* s_dev, int64_t rows, int64_t cols, uint8_t* planes_dev,
                        void* stream);
int mbq_int8_unpack_host(const uint8_t* planes_host, int64_t rows, int64_t cols, int8_t* q, float* s);

/* int8 embedding rows: y (T, D) = f32(q[r]) * s[r] per token, r = toks[t] (int32, device), plus N when negative and
 * clamped to [0, N - 1] (jax.numpy indexing), then out_dtype (bfloat16 rounded to nearest even, or float32 for a pj
 * hook). q_dev int8 (N, D) row-major, s_dev float32 (N,). Bit for bit the gather of embed(E, toks) for an int8 table
 * E = {"q", "s"} (reference src/mashbox/models/qwen3_8_27b/model.py:132-139, whose int8_rows at :117-129 equals the
 * plain gather q[toks]). */
int mbq_int8_embed(const int8_t* q_dev, const float* s_dev, int64_t N, int64_t D, const int32_t* toks_dev, int64_t T,
                   void* y_dev, int out_dtype, void* stream);

/* Tuning and introspection (no counterpart in the reference, whose kernels are closed). For an activation batch of M
 * rows, mbq_gemm_plan reports how mbq_matmul / mbq_int8_linear would run a (N, K) weight of type t (MBQ_INT8 for the
 * int8 linear): the kernel (MBQ_KERNEL_*), *bm x *bn output tiles and *splits K ranges (1 = no split; a split K uses
 * the per-device workspace below).
 *   MBQ_KERNEL_GEMV    M <= 4 on row-major planes whose rows the GEMV's registers hold; M = 1 on tiled planes (the
 *                      tile GEMV: x staged in LDS, K up to about 58,000 values); bm = bn = splits = 0.
 *   MBQ_KERNEL_STREAM  weight-stream kernel, M <= 64 (M <= 4 when the GEMV has no plan: e.g. K = 17408 at 3-4 rows,
 *                      Q8_0 / int8 rows over 24576 values): bm = 16, bn = weight rows per block (64 or 128); from 17
 *                      rows on, a weight of at least 64 rows per CU runs MBQ_KERNEL_TILES instead (automatic plan).
 *   MBQ_KERNEL_TILES   LDS-tile kernel: 256x{256,192,128}, 128x{256,192,128,64}, 64x{256,192,128,64}.
 *   MBQ_KERNEL_KGROUP  K-group kernel of tiled planes (MBQ_I8T and the tiled GGUF types) at M <= 64:
 *                      bm = 16, bn = weight rows per block (any count: N is cut into equal ranges that fill the
 *                      CUs, or several rounds of them for a weight of more than about 96 rows per CU), splits = K
 *                      ranges. The automatic plan of tiled planes from 2 to 64 rows (and at one row
 *                      when the tile GEMV has no plan); they have no weight-stream plan.
 * mbq_force_gemm_plan makes every later GEMM call in the process use that kernel, tile and K ranges (row-major planes
 * at M <= 4 with a GEMV plan keep the GEMV; tiled planes at one row take the forced kernel)
 * (kernel MBQ_KERNEL_AUTO: automatic again; bm = bn = 0 with MBQ_KERNEL_TILES: that kernel with its own tile choice;
 * MBQ_KERNEL_KGROUP takes bm = bn = 0 and chooses its rows per block for the forced splits, 0 = its own choice).
 * Workspace: a GEMM that splits K adds float32 partial tiles in a 64 MiB workspace (plus 256 KiB of counters) of
 * uncached device memory, one per (device, stream), so split-K calls that overlap in time on two streams never share
 * partials or counters. A stream's workspace is allocated by its first eager split-K call and kept until the process
 * ends (at most 31 streams per device). Every eager split-K call also keeps one spare workspace per device, which the
 * first split-K call recorded into a HIP graph on a stream without a workspace of its own takes; a recorded call that
 * finds neither (no eager split-K call on the device yet, or the spare taken by another capturing stream since the last
 * eager call) returns MBQ_E_ARG and launches nothing. Graphs recorded on one stream share its workspace: their replays
 * must not overlap in time. */
#define MBQ_KERNEL_AUTO 0
#define MBQ_KERNEL_GEMV 0
#define MBQ_KERNEL_STREAM 1
#define MBQ_KERNEL_TILES 2
#define MBQ_KERNEL_KGROUP 3
int mbq_gemm_plan(int t, int64_t M, int64_t N, int64_t K, int* kernel, int* bm, int* bn, int* splits);
int mbq_force_gemm_plan(int kernel, int bm, int bn, int splits);

/* Measurement probes (no counterpart in the reference): the peaks a benchmark reports beside the kernels' rates.
 * mbq_probe_read reads every whole KiB of [p_dev, p_dev + bytes) once with 128-bit loads from a persistent grid (one
 * block of 4 waves per CU) and writes at most one word to sink_dev: bytes / time is the HBM read rate a streaming kernel
 * reaches. mbq_probe_mfma runs `iters` rounds of 8 independent v_mfma_f32_16x16x32_bf16 per wave, 8 waves per CU, and
 * returns the launch's flop count in *flops: flops / time is the bf16 matrix-core rate at the clock the GPU holds under
 * MFMA load. Both are stream-ordered and allocate nothing. */
int mbq_probe_read(const void* p_dev, int64_t bytes, void* sink_dev, void* stream);
int mbq_probe_mfma(int iters, void* sink_dev, int64_t* flops, void* stream);
/* A check of the same family (no counterpart in the reference): every bfloat16 output value is converted from float32
 * by one hardware instruction; mbq_probe_bf16 runs all 2^32 float32 bit patterns through it and through the integer
 * round-to-nearest-even form (NaN kept quiet) and ADDS the count of inputs whose bits differ to the uint64 at diff_dev
 * (the caller zeroes it). Zero on MI355X. Stream-ordered; allocates nothing. */
int mbq_probe_bf16(void* diff_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MBQ_H */
