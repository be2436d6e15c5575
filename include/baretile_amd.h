/* baretile_amd: the C ABI of the MI355X (gfx950) backend for baretile's hot path.
 *
 * One shared library, libbaretile_amd.so, loaded with ctypes the way baretile's pci.Sim loads its device library
 * (baretile/pci.py:50-60). Plain pointers and sizes only: device memory is a uint64_t address, sizes and strides are
 * int64_t element counts, and every function returns a status, with the message of the last failure on the calling
 * thread in bt_last_error().
 *
 * Status -> Python exception, as baretile's API promises (docs/api.md:51-63): BT_EINVAL -> ValueError,
 * BT_ESTATE -> RuntimeError, BT_ETIMEOUT -> TimeoutError, BT_ENOMEM -> MemoryError.
 *
 * Each declaration names the reference interface it replaces. In the reference those are Python functions that build
 * a Tensix kernel image and queue it with Runtime.launch(kernel, args: tuple[u32], units, name) (runtime.py:680-695);
 * here they are direct calls that queue HIP kernels on the runtime's stream, in order, without waiting.
 */
#ifndef BARETILE_AMD_H
#define BARETILE_AMD_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BT_ABI_VERSION 1

enum { BT_OK = 0, BT_EINVAL = 1, BT_ESTATE = 2, BT_ETIMEOUT = 3, BT_ENOMEM = 4 };

/* Storage formats (tensix.py:14-21: ITEMSIZE and BFP). */
enum { BT_BF16 = 0, BT_FP32 = 1, BT_INT32 = 2, BT_BFP8 = 3, BT_BFP4 = 4 };

typedef struct bt_runtime bt_runtime;

/* ---- runtime: replaces Runtime (runtime.py:543-880) and the device layer under it (pci.py, chip.py) ------------ */

const char *bt_last_error(void);
int bt_version(void);
int bt_device_count(int *n);
/* Runtime(chip) (runtime.py:543): a device and one in-order stream. */
int bt_open(int device, bt_runtime **rt);
/* Runtime.close (runtime.py:484-541): waits for queued work, then releases the stream. */
int bt_close(bt_runtime *rt);
/* Runtime.dram_alloc / dram_free (runtime.py:791-820). Frees are stream-ordered, so memory goes back once the
 * launches queued before the free are done (runtime.py:814-820). `captured` marks memory allocated while a graph
 * capture was open. The runtime keeps freed blocks of up to 256 MB, 4 GB in all, for its next allocations of the
 * same size (one stream, so reuse is in stream order), and gives them back when it closes or when an allocation
 * outside a capture runs out of memory. Freeing a kept block again returns BT_EINVAL. */
int bt_alloc(bt_runtime *rt, uint64_t bytes, uint64_t *addr);
int bt_free(bt_runtime *rt, uint64_t addr, int captured);
/* Tensor.frombytes / tobytes transfers (tensor.py:113-204, kernels.py:1374-1453 upload/readback_kernel). Both
 * return once the bytes have arrived. */
int bt_upload(bt_runtime *rt, uint64_t dst, const void *src, uint64_t bytes);
int bt_download(bt_runtime *rt, void *dst, uint64_t src, uint64_t bytes);
int bt_copy(bt_runtime *rt, uint64_t dst, uint64_t src, uint64_t bytes);
/* zeros_kernel (kernels.py:1436-1453): fills 32-bit words, by a kernel (never a memset node in a graph). */
int bt_fill32(bt_runtime *rt, uint64_t dst, uint32_t value, uint64_t words);
/* Runtime.wait(timeout) (runtime.py:851-880): BT_ETIMEOUT if the stream is still busy after timeout_s seconds. */
int bt_wait(bt_runtime *rt, double timeout_s);
/* No counterpart in the reference (a measurement aid, like probe.py's DRAM probes, probe.py:81): reads `bytes` once
 * with 16-byte non-temporal loads and folds them into a word written to scratch_word only for one unlikely value
 * (bytes: a multiple of 16, at most 4 GB - 16 KB). The plain streaming read that bench.py sets beside a kernel of the
 * same size, and the known-size read that calibrates the HBM byte counters. */
int bt_stream_read(bt_runtime *rt, uint64_t src, uint64_t bytes, uint64_t scratch_word);
/* No counterpart in the reference (a test aid, like test_device.py:962's kernel that never ends, but one that always
 * does): queues a kernel that stays busy for `seconds` (0 to 10) of the device's wall clock and then ends by itself,
 * so a wait with a shorter timeout raises TimeoutError and the stream still drains. */
int bt_sleep(bt_runtime *rt, double seconds);
/* Timing for Runtime.profile (runtime.py:773-786): events on the runtime's stream. */
int bt_event_create(bt_runtime *rt, void **ev);
int bt_event_record(bt_runtime *rt, void *ev);
int bt_event_elapsed(void *start, void *end, float *ms);
int bt_event_destroy(void *ev);
/* jit / Recording (tensor.py:1171-1293): record the launches queued between begin and end into a graph, then replay
 * it with one call. */
int bt_graph_begin(bt_runtime *rt);
int bt_graph_end(bt_runtime *rt, void **graph);
int bt_graph_launch(bt_runtime *rt, void *graph);
int bt_graph_destroy(void *graph);
/* The runtime's hipStream_t, for callers that time or order their own work against it. */
int bt_stream(bt_runtime *rt, void **stream);

/* ---- block floats: replaces the bfp8 packer cast (kernels.py:128-138), bfp4_kernel (kernels.py:1527-1567),
 * storage_kernel (kernels.py:1483-1525) and columns_kernel (kernels.py:1455-1481) --------------------------------
 *
 * Plain layout of a block-float batch of [rows, cols] matrices: an exponent plane, one byte per run of 16 values
 * along a row, [batch][rows][ceil(cols / 16)], then a value plane of signed magnitudes q in two's complement,
 * [batch][rows][cols16] int8 for bfp8 or [batch][rows][cols16 / 2] bytes of two 4-bit values for bfp4 (the first in
 * the low nibble), where cols16 rounds cols up to 16. A value is q * 2^(e - 133) (bfp8) or q * 2^(e - 129) (bfp4).
 *
 * Columns layout (Tensor.columns(), a matmul's B): tiles of 64 rows (K) by 16 columns (N), ordered
 * [batch][column run][64-row chunk]. A tile is 64 exponent bytes, then its values in the order the 16x16x32 matrix
 * instruction reads B: lane l (0..63) holds rows 32h + 8(l / 16) + j, j = 0..7, of column l % 16, for h = 0, 1.
 * Exponent byte p = 16g + 8h + j belongs to row 32h + 8g + j and holds (e - 133) mod 256 (bfp8) or (e - 120) mod 256
 * (bfp4). bfp8 tiles are 64 + 1024 bytes: lane l's 16 bytes at 64 + 16l, byte 8h + j the signed q of value j.
 * bfp4 tiles are 64 + 512: lane l's 8 bytes at 64 + 8l, 4 bytes a half h holding its values j = 0..7 as sign and
 * magnitude: for j < 4 byte j's bit 7 and bits 0-2, for j >= 4 bits 4-6 of byte j - 4 and bit 3 of byte
 * (j - 3) % 4. bf16 tiles are 2048 bytes (32 bytes at 32l, no exponents). Rows past K and columns
 * past N are zero. A matmul reads exponents as signed bytes, so it takes block floats whose nonzero runs' exponents e
 * lie in 5..255 (bfp8) or 3..247 (bfp4) (bt_bfp_range counts the others); readback is exact for any. */

/* bf16 (round to nearest even first, as gpt2.bfp does: models/gpt2.py:19-30) or fp32 matrices -> plain planes.
 * src strides are in elements. */
int bt_bfp_pack(bt_runtime *rt, int fmt, uint64_t src, int src_dtype, int64_t batch, int64_t rows, int64_t cols,
                int64_t src_bstride, int64_t src_rstride, int64_t src_cstride, uint64_t exps, uint64_t vals);
/* plain planes -> bf16 row-major [batch][rows][cols], bit for bit what the unpacker gives (tensor.py:1093-1104). */
int bt_bfp_unpack(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t rows, int64_t cols,
                  uint64_t dst);
/* plain planes -> columns tiles (Tensor.columns, tensor.py:597-611). */
int bt_bfp_columns(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t rows, int64_t cols,
                   uint64_t dst);
/* The number of runs of a plain block float that a matmul can't multiply, written to the uint32 at `bad` (no
 * counterpart in the reference, whose unpacker reads any exponent): runs with a nonzero value whose exponent lies
 * outside 5..255 (bfp8) or 3..247 (bfp4), the range the matmul kernels read exponents in. Tensor.columns() checks it
 * before a block float becomes a matmul's B. */
int bt_bfp_range(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t rows, int64_t cols,
                 uint64_t bad);
/* bf16 matrices with any strides -> bf16 columns tiles (a matmul's B read as it is, or transposed by strides). */
int bt_bf16_columns(bt_runtime *rt, uint64_t src, int64_t batch, int64_t rows, int64_t cols, int64_t sb, int64_t sr,
                    int64_t sc, uint64_t dst);
/* columns tiles of any format -> bf16 row-major [batch][rows][cols] (readback of a tensor by columns). */
int bt_columns_unpack(bt_runtime *rt, int fmt, uint64_t src, int64_t batch, int64_t rows, int64_t cols, uint64_t dst);

/* ---- fused expressions: replaces fused_kernel's elementwise and reduction kernels (kernels.py:41-727) ----------
 *
 * A program is a straight line of instructions over up to 16 registers, evaluated per element in one dtype: bf16
 * rounds every result half up as the packer does (so fused and unfused give the same bits, test_kernels.py:987-1004),
 * fp32 keeps it, int32 is integer arithmetic that wraps. Inputs are read with element strides; a stride of 0
 * broadcasts. Batch index b of the result reads stored matrix (b / rep) % cyc of an input (cyc 0: no wrap), as a
 * repeat or a spread view does (tensor.py:265-279, 414-424). */
#define BT_MAX_INPUTS 8
#define BT_MAX_INST 48
#define BT_MAX_REGS 16

enum {
  BT_OP_LOAD = 0,  /* dst = input a, converted to the program's dtype */
  BT_OP_CONST,     /* dst = imm (bits in the program's dtype) */
  BT_OP_MOV,
  BT_OP_ADD, BT_OP_SUB, BT_OP_MUL, BT_OP_DIV, BT_OP_MAX, BT_OP_MIN,
  BT_OP_CMPLT, BT_OP_CMPLE, BT_OP_CMPNE, BT_OP_CMPEQ, /* 1 or 0 */
  BT_OP_WHERE,     /* dst = a != 0 ? b : c, keeping the selected value's bits */
  BT_OP_NEG, BT_OP_RELU, BT_OP_EXP, BT_OP_EXP2, BT_OP_LOG, BT_OP_LOG2, BT_OP_SQRT, BT_OP_RECIP, BT_OP_RSQRT,
  BT_OP_SIN, BT_OP_COS, BT_OP_SIGMOID, BT_OP_SILU, BT_OP_GELU, BT_OP_TANH,
  BT_OP_FTOB,      /* round an fp32 value to bf16 (half up, as the bf16 cast does) and back */
  BT_OP_COUNT
};

typedef struct {
  uint64_t ptr;      /* address of element (0, 0, 0) */
  int64_t sb, sr, sc; /* element strides of batch, row and column */
  int32_t dtype;     /* BT_BF16, BT_FP32 or BT_INT32 */
  int32_t rep;       /* >= 1 */
  int32_t cyc;       /* 0, or the number of stored matrices the batch index wraps at */
  int32_t pad_;
} bt_operand;

typedef struct {
  uint8_t op, dst, a, b, c, pad_[3];
  uint32_t imm;
} bt_inst;

typedef struct {
  int32_t n_inst;
  int32_t n_inputs;
  int32_t dtype;   /* the dtype the program computes in */
  int32_t result;  /* the register holding the result */
  bt_inst inst[BT_MAX_INST];
  bt_operand in[BT_MAX_INPUTS];
} bt_program;

/* A fused elementwise kernel over [batch, rows, cols], written to out in out->dtype (a cast at the root converts:
 * to bf16 rounds half up, to int32 rounds to nearest, from int32 converts exactly where it can). */
int bt_elementwise(bt_runtime *rt, const bt_program *prog, int64_t batch, int64_t rows, int64_t cols,
                   const bt_operand *out);
/* A reduction (sum or max) along axis 0 (batch), 1 (rows) or 2 (columns) of the program's value over [batch, rows,
 * cols], accumulated in fp32 (int32 for an int32 max), written to out, whose extent along axis is 1. With sweep > 1,
 * axis 0 folds `sweep` matrices a `step` apart, as a reduction over a middle leading dimension does
 * (tensor.py:657-676). */
enum { BT_REDUCE_SUM = 0, BT_REDUCE_MAX = 1 };
int bt_reduce(bt_runtime *rt, const bt_program *prog, int kind, int axis, int64_t batch, int64_t rows, int64_t cols,
              int64_t sweep, int64_t step, const bt_operand *out);

/* ---- matmul: replaces fused_kernel's matmul schedules (kernels.py:41-727, 216-555) ------------------------------
 *
 * out[b, m, n] = epilogue(sum_k A[b, m, k] * B[b', k, n]), with exact bf16 products summed in fp32 by the matrix
 * instructions (fidelity 4, tensor.py:12, 756-757). A is bf16 with element strides. B is in columns layout (any of
 * bf16, bfp8, bfp4) with b' = b when b_batch > 1, else 0. The epilogue program, if any, reads the matmul's value
 * from register 0 (rounded to the program's dtype first) and may read other inputs at the same [b, m, n]. Without
 * one, the value is written to out as bf16 (rounded half up) or fp32. 5 to 32 rows of one A against K over 768 (a
 * multiple of 64) run split-K: fp32 partial sums in the runtime's scratch, summed in a fixed order (inside a capture
 * that would have to grow that scratch, a one-launch kernel instead, summing in another order). */
int bt_matmul(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t b_batch, int64_t batch, int64_t m,
              int64_t k, int64_t n, const bt_program *epilogue, const bt_operand *out);

/* ---- one-row products with their neighbours fused: the decode step of models/llama.py at batch 1 (its layer,
 * llama.py:106-130: rms then qkv, rms then gate_up, silu(gate) * up then down, each product then the residual add),
 * where fused_kernel would run the norm, the activation and the add as the matmul's prologue and epilogue
 * (kernels.py:41-727) ----------------------------------------------------------------------------------------------
 *
 * out[n] = (residual ? residual[n] : 0) + sum_k a'[k] * B[k, n] for n < N, where a' is
 *   BT_ROW_PLAIN:  a, bf16, k values;
 *   BT_ROW_RMS:    bf16(x[k] * r * norm[k]), x = bf16(a[k]) (rounded half up) for a an fp32 row of k values,
 *                  norm bf16, r = 1 / sqrt(mean over k of x^2 + eps), all in fp32;
 *   BT_ROW_SWIGLU: bf16(silu(g) * u) with g = a[k], u = a[k + K] (a: bf16, the gate then the up half, 2K values),
 *                  silu(g) = g / (1 + exp(-g)) in fp32.
 * B is in columns layout (bf16, bfp8 or bfp4) and is multiplied as bt_matmul does; residual is 0 or fp32, n values;
 * out is bf16 (rounded half up) or fp32. k <= 4096. */
#define BT_ROW_PLAIN 0
#define BT_ROW_RMS 1
#define BT_ROW_SWIGLU 2
typedef struct {
  uint64_t a, norm, residual, out, b;
  int64_t k, n;
  int32_t kind, b_fmt, out_dtype;
  float eps;
} bt_row_args;
int bt_matmul_row(bt_runtime *rt, const bt_row_args *args);

/* The MLP's first product for a block of tokens with silu(gate) * up as its epilogue (llama.py:174-183; the fused
 * SiLU-mul epilogue fused_kernel gives the prefill's gate_up): B holds gate then up side by side (n = 2 f columns,
 * n a multiple of 32) and out[i, j] = bf16(silu(g) * u) for j < f, with g, u the products at columns j and f + j
 * rounded to bf16 as stored, silu(g) = g / (1 + exp(-g)), in fp32. A is bf16 with contiguous rows, k a multiple of
 * 32; out is bf16 with contiguous, 16-byte aligned rows. Where the tiled GEMM runs it (more than 64 rows, unless its
 * grid would be small), a block-float B is unpacked to bf16 in the runtime's scratch first (BT_ESTATE inside a capture
 * when that scratch would have to grow); fewer rows read B as stored, 5 to 32 of them against a long K through split-K
 * partial sums in that scratch (inside a capture that would have to grow it, the one-launch kernel instead). */
int bt_matmul_swiglu(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t m, int64_t k, int64_t n,
                     const bt_operand *out);
/* RMSNorm of a block of token rows (llama.py:88-95): out[r, c] = bf16(x * s * w[c]) with x = bf16(x[r, c]) (half
 * up), s = 1 / sqrt(mean over c of x^2 + eps), in fp32; x fp32, w and out bf16, row strides in elements. */
int bt_rms_rows(bt_runtime *rt, uint64_t x, int64_t rows, int64_t k, int64_t x_sr, uint64_t w, float eps, uint64_t out,
                int64_t out_sr);

/* RoPE and the cache put of a decode step (llama.py:132-160: rope, then the key and value heads put at the tokens'
 * places). For each token i < rows and head h < heads + 2 kv of qkv (bf16, element (i, h, j) at
 * i * qkv_sr + h * head_dim + j):
 *   y = bf16(x[j] * cos[j] + t[j] * sin[j]), t[j] = -x[j + d/2] for j < d/2 and x[j - d/2] after (d = head_dim),
 * in fp32, with cos and sin bf16 rows laid out as qkv (row stride cs_sr). Query heads are written to q (as qkv, row
 * stride q_sr); key and value heads to cache[h - heads, place, :] (bf16, element strides cache_sh, cache_sr),
 * place = places[i] (places[0] for every token when one_place is nonzero), a place outside [0, cache_rows) skipped.
 * With vcache nonzero the value heads go to vcache[h - heads - kv, place, :] instead (laid out as cache), and
 * cache_tsh adds i * cache_tsh elements to token i's rows in both caches: a batch of sequences with caches of their
 * own side by side (the slots of llama.py:293-354, slot i's key heads at i * kv). RoPE's tables carry the query
 * scale, and cos 1, sin 0 for the value heads, so a value head is stored as it is. */
typedef struct {
  uint64_t qkv, cos, sin, q, cache, places;
  int64_t qkv_sr, cs_sr, q_sr, cache_sh, cache_sr, cache_rows;
  int32_t rows, heads, kv, head_dim;
  uint64_t vcache;     /* 0: value heads at cache heads kv .. 2 kv - 1 */
  int64_t cache_tsh;   /* elements between tokens' caches, or 0 */
  int32_t one_place, pad_;
} bt_rope_args;
int bt_rope_put(bt_runtime *rt, const bt_rope_args *args);
/* bt_matmul_row (BT_ROW_RMS, a bf16 product, no residual) with bt_rope_put run on its product in the same kernel: the
 * decode step's RMSNorm, qkv product, RoPE and cache put (llama.py:106-160) for one token. rope->qkv and args->out are
 * not used; rope->rows is 1, args->n is (heads + 2 kv) head_dim and head_dim a multiple of 32. The query heads land
 * in rope->q and the key and value heads in the cache, bit for bit what the two calls write. */
int bt_matmul_row_rope(bt_runtime *rt, const bt_row_args *args, const bt_rope_args *rope);

/* The batched decode step's products with their neighbours (llama.py:106-160 with slots, llama.py:293-354): where
 * fused_kernel would run RoPE and the residual add as a matmul's epilogue (kernels.py:41-727), here the product of 5 to
 * 32 rows of A (bf16, contiguous 16-byte aligned rows) against a long K (a multiple of 256, over 768) is left as
 * split-K partial sums in the runtime's scratch and the kernel that consumes it sums them, in split order as
 * bt_matmul's reduction does, so the product and its reduction are neither stored nor launched on their own. Each is
 * bit for bit the unfused calls. Inside a graph capture the runtime's scratch can't grow: make the call once before
 * capturing. BT_EINVAL for a product outside those shapes.
 *
 * bt_matmul_rope_put: bt_matmul (bf16 product, no epilogue) then bt_rope_put on its product. rope->qkv and qkv_sr
 * are not used; rope->rows is m, n is (heads + 2 kv) head_dim with head_dim a multiple of 16, and the tables, q and
 * caches 16-byte aligned with strides a multiple of 8.
 * bt_matmul_residual_rms: x = residual + a @ b (fp32, bt_matmul's residual epilogue; x may be the residual itself),
 * then h = bt_rms_rows(x, norm, eps) (bf16); n <= 8192 and a multiple of 4. */
int bt_matmul_rope_put(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t m, int64_t k, int64_t n,
                       const bt_rope_args *rope);
int bt_matmul_residual_rms(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t m, int64_t k, int64_t n,
                           uint64_t residual, int64_t res_sr, uint64_t x, int64_t x_sr, uint64_t norm, float eps,
                           uint64_t h, int64_t h_sr);


/* ---- attention: replaces attention_kernel and its division/combine launches (kernels.py:794-1005,
 * tensor.py:797-841) -------------------------------------------------------------------------------------------
 *
 * out[e, r, :] = softmax(q[e, r, :] . k[e / rep, j, :] + mask) @ v[e / rep, j, :] over keys j < keys, where the mask
 * hides j > places[r] and, with window > 0, j <= places[r] - window. Scores, maxima and sums are fp32, p is packed to
 * bf16 before it is summed and multiplied by v (as the reference packs it, kernels.py:815-823); out is bf16.
 * q, k, v, out are bf16 with element strides (head, row); places is int32 with a head stride of 0 or rows. No scale
 * is applied: baretile's RoPE pre-scales q (llama.py:210-216).
 *
 * firsts, when given, raises each row's first visible key (a batch of sequences with their own regions of one cache,
 * as the reference's slots use it, llama.py:293-318).
 *
 * parts splits a decode step's keys (at most 64 query rows per key head: rep * rows <= 64) between that many blocks,
 * as attention_kernel's parts does; 0 picks a count from the shape. With more than one part the blocks write fp32
 * partial sums into scratch (bt_attention_scratch gives the bytes; 16-byte aligned) and a second launch combines
 * them. Calls that share one scratch buffer must not overlap.
 *
 * A block-float cache (kv_fmt BT_BFP8 or BT_BFP4, test_kernels.py:2106-2132) is read in place and gives, bit for bit,
 * the result of the bf16 values it holds: k and v are then the value planes' and k_exps, v_exps the exponent planes'
 * addresses of element (0, 0) of key head 0, with the plain layout's rules (a value's q at its index, or index / 2
 * for bfp4, its exponent byte at index / 16); strides, in values, are multiples of 16. */
typedef struct {
  uint64_t q, k, v, out, places;
  int64_t q_sh, q_sr, k_sh, k_sr, v_sh, v_sr, o_sh, o_sr, places_sh;
  int32_t heads, rep, rows, keys, head_dim, window, parts, pad_;
  uint64_t scratch, scratch_bytes;
  uint64_t firsts;    /* 0, or int32 with the first key each row sees (head stride firsts_sh: 0 or rows) */
  int64_t firsts_sh;
  int32_t kv_fmt;     /* BT_BF16 (0), or a block-float cache: BT_BFP8, BT_BFP4 */
  int32_t pad2_;
  uint64_t k_exps, v_exps; /* with a block-float cache: k and v are value planes, these the exponent planes */
} bt_attention_args;
int bt_attention(bt_runtime *rt, const bt_attention_args *args);
/* The scratch bytes bt_attention needs for args (0 when it runs in one part). */
int bt_attention_scratch(const bt_attention_args *args, uint64_t *bytes);
/* No counterpart in the reference: bt_attention for callers that cannot allocate device memory (code under graph
 * capture, serving loops that must not call hipMalloc, harnesses that forbid it). The same kernels and results, with
 * args->scratch and scratch_bytes ignored: the split decode's partial sums go to a static array of
 * BT_ATTENTION_NOALLOC_BYTES on each GPU, held until the process ends, and nothing is allocated or freed. BT_EINVAL
 * when the plan needs more than that (bt_attention_scratch tells); nothing in it needs to start at zero. Every call
 * on one GPU shares that GPU's array, so calls that overlap on one GPU (other streams, other threads) race. */
#define BT_ATTENTION_NOALLOC_BYTES (8u << 20)
int bt_attention_noalloc(bt_runtime *rt, const bt_attention_args *args);

/* ---- rows in and out of a cache: replaces gather_kernel (kernels.py:1007-1049) and put_kernel
 * (kernels.py:1083-1168) ------------------------------------------------------------------------------------------ */
/* out[i, :] = table[ids[i], :] for i < n. An id outside [0, rows) gives a row of zeros. */
int bt_gather(bt_runtime *rt, int dtype, uint64_t table, int64_t rows, int64_t cols, int64_t table_rstride,
              uint64_t ids, int64_t n, uint64_t out, int64_t out_rstride);
/* dst[b, ids[i], :] = x[b, i, :] for i < n, in order, so a later duplicate wins. Places outside [0, dst_rows) are
 * skipped. dst and x share dtype (bf16, fp32, int32). */
int bt_put(bt_runtime *rt, int dtype, uint64_t dst, int64_t batch, int64_t dst_rows, int64_t cols, int64_t dst_sb,
           int64_t dst_sr, uint64_t ids, int64_t n, uint64_t x, int64_t x_sb, int64_t x_sr);
/* bt_put into a plain block-float tensor (a bfp8 or bfp4 KV cache, kernels.py:1083-1168): x is bf16 and each run of 16
 * of a row is rounded as bt_bfp_pack rounds it, bit for bit. exps and vals are the exponent and value planes'
 * addresses of element (0, 0, 0); cols and the destination's strides (in values) are multiples of 16. */
int bt_put_bfp(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t dst_rows, int64_t cols,
               int64_t dst_sb, int64_t dst_sr, uint64_t ids, int64_t n, uint64_t x, int64_t x_sb, int64_t x_sr);

/* ---- top-k: replaces topk_kernel (Tensor.topk, tensor.py:685-706) ----------------------------------------------
 * values[b, r, p * k + j] and ids[b, r, p * k + j]: the k largest of part p of row r (parts equal parts of cols), in
 * descending order with equal values in column order (numpy's stable argsort of -x), -0 equal to 0. ids are columns of
 * the whole row, or labels[b, r, column] when labels is nonzero (element strides lsb, lsr). x is bf16 or fp32 with
 * element strides sb, sr and contiguous columns; values has x's dtype and ids is int32, both contiguous. k <= 64. */
int bt_topk(bt_runtime *rt, int dtype, uint64_t x, int64_t batch, int64_t rows, int64_t cols, int64_t sb, int64_t sr,
            int32_t parts, int32_t k, uint64_t labels, int64_t lsb, int64_t lsr, uint64_t values, uint64_t ids);

#ifdef __cplusplus
}
#endif
#endif
