/*
 * q4rdna.h -- C ABI of the MI355X (gfx950) Q4_RDNA group-64 dequant-GEMV.
 *
 * A drop-in for the reference's llama.cpp entry points
 * (source/q4rdna.cuh:5-24, defined at source/q4rdna.cu:713-793) with ggml
 * types replaced by plain pointers and sizes.  The packed layout is the
 * reference's byte-exact Q4_RDNA sidecar: 32-row tiles of 1088 bytes (32 fp16
 * scales, then 32x32 lane-interleaved bytes of two's-complement nibbles, low
 * nibble = even k) in (row tile, group) order.
 *
 * Conventions
 *  - Every call returns a status.  Q4RDNA_NOT_APPLICABLE is the reference's
 *    "return false": the call touched nothing and the caller should run its
 *    own path.  Negative values are errors; q4rdna_last_error() describes the
 *    last one on the calling thread.
 *  - Device pointers are caller-owned except the sidecar's weights, which the
 *    library owns until q4rdna_sidecar_close().
 *  - `stream` is a hipStream_t (NULL = the null stream).  Launches are
 *    asynchronous on that stream; nothing here synchronises it.
 *  - A launch needs the weights' device to be the current device.
 */
#ifndef Q4RDNA_H
#define Q4RDNA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q4RDNA_ABI_VERSION 4

/* status codes */
#define Q4RDNA_OK 0
#define Q4RDNA_NOT_APPLICABLE 1
#define Q4RDNA_ERR_ARGUMENT (-1)
#define Q4RDNA_ERR_FORMAT (-2)
#define Q4RDNA_ERR_IO (-3)
#define Q4RDNA_ERR_HIP (-4)
#define Q4RDNA_ERR_MEMORY (-5)

/* format constants (source/q4rdna.cu:20-22) */
#define Q4RDNA_GROUP 64
#define Q4RDNA_TILE_ROWS 32
#define Q4RDNA_TILE_BYTES 1088

/* scale-search algorithms of the packers */
#define Q4RDNA_ALGO_SIDECAR 0 /* source/q4rdna_sidecar_pack.cpp:126-179 */
#define Q4RDNA_ALGO_ABSMAX 1  /* source/q4rdna_cpu_experiment.cpp:209-211 */
#define Q4RDNA_ALGO_RANGE 2   /* source/q4rdna_cpu_experiment.cpp:213-223 */
#define Q4RDNA_ALGO_MSE 3     /* source/q4rdna_cpu_experiment.cpp:225-236 */

/* GLU operations accepted by q4rdna_mul_mat_glu (source/q4rdna.cu:776) */
#define Q4RDNA_GLU_SWIGLU 0

/* A packed tensor resident on a device: rows x columns weights, rows%32 == 0,
 * columns%64 == 0, `tiles` 16-byte aligned, rows*columns*34/64 bytes. */
typedef struct q4rdna_weight {
    const uint8_t *tiles;
    uint32_t rows;
    uint32_t columns;
    int32_t device;
    uint32_t reserved;
} q4rdna_weight;

typedef struct q4rdna_sidecar q4rdna_sidecar;

/* Library version (Q4RDNA_ABI_VERSION) and the last error on this thread. */
int q4rdna_abi_version(void);
const char *q4rdna_last_error(void);

/* ---- sidecar container --------------------------------------------------
 * q4rdna_sidecar_inspect: host-only validation of a sidecar image prefix that
 * holds at least the header and the index; `file_size` is the size of the
 * whole file.  Applies the loader's acceptance rules of
 * source/q4rdna.cu:129-155 (magic, version, group 64, 32 rows, 1088-byte
 * tiles, NUL-terminated names, offsets inside the data region, rows%32,
 * columns%64, size = rows*columns*34/64) and the data-length check of
 * source/q4rdna.cu:163-170.  On success *count receives the entry count. */
int q4rdna_sidecar_inspect(const void *image, uint64_t image_size, uint64_t file_size,
                           uint32_t *count);

/* Open a sidecar file and upload its data region to `device` once
 * (source/q4rdna.cu:119-179, without the device-0 restriction). */
int q4rdna_sidecar_open(const char *path, int device, q4rdna_sidecar **out);
/* Same from an in-memory image of `size` bytes. */
int q4rdna_sidecar_open_memory(const void *image, uint64_t size, int device, q4rdna_sidecar **out);
/* Frees the sidecar's device buffer (hipFree waits for work in flight):
 * every q4rdna_weight found in it is invalid afterwards.  Not for the
 * process-wide sidecar of q4rdna_default_sidecar, which lives until exit. */
void q4rdna_sidecar_close(q4rdna_sidecar *sidecar);
uint32_t q4rdna_sidecar_count(const q4rdna_sidecar *sidecar);
/* Entry metadata; name receives up to 64 bytes including the NUL. */
int q4rdna_sidecar_entry(const q4rdna_sidecar *sidecar, uint32_t index, char name[64],
                         uint32_t *rows, uint32_t *columns, uint64_t *offset, uint64_t *size);

/* Name lookup with the reference's shape check: `ne0` = columns (K) and
 * `ne1` = rows (M) as ggml stores them.  NOT_APPLICABLE when the name is
 * absent or the shape differs (source/q4rdna.cu:682-705). */
int q4rdna_find(const q4rdna_sidecar *sidecar, const char *name, int64_t ne0, int64_t ne1,
                q4rdna_weight *out);

/* Describe tiles already resident on `device` (synthetic or externally
 * uploaded tensors). */
int q4rdna_weight_from_device(const void *tiles, uint32_t rows, uint32_t columns, int device,
                              q4rdna_weight *out);

/* Sidecar named by LLAMA_Q4_RDNA_SIDECAR, opened once per process on the
 * first call (source/q4rdna.cu:683,698) on that call's device, and kept
 * until exit (never pass it to q4rdna_sidecar_close).  NULL when unset or
 * invalid, or for another device. */
q4rdna_sidecar *q4rdna_default_sidecar(int device);
/* The reference's LLAMA_Q4_RDNA_SCOPE name filter (source/q4rdna.cu:685-696):
 * scope NULL/"" admits every name; "ffn", "qkv-fallback", "hotspot", "attn"
 * as in the reference.  Returns 1 if `name` is in scope, else 0. */
int q4rdna_scope_allows(const char *scope, const char *name);

/* ---- GEMV entry points ---------------------------------------------------
 * y[M] = W[M][K] x[K] in fp32 accumulation.  x_ne0 must equal K and y_ne0 M
 * (the reference's src1->ne[0] / dst->ne[0] checks); any mismatch, a weight
 * on another device or a NULL weight returns NOT_APPLICABLE with nothing
 * launched.  x and y are contiguous fp32 device buffers (4-byte aligned);
 * y may not overlap x, and an add vector is either y itself or apart from
 * it (argument errors otherwise).
 *
 * Launches with split K use a scratch buffer per (device, stream).  The
 * first call that needs more than the stream has allocates it (and waits
 * for the device), so it cannot run under HIP graph capture: make one call
 * of each shape on the stream before capturing.  Outgrown buffers are
 * never freed, so a graph captured earlier stays valid.  Calls on one
 * stream are ordered by it; a graph must not replay on another stream
 * while the stream it was captured on runs such calls.
 *
 * Replaces ggml_cuda_q4rdna_mul_mat (source/q4rdna.cuh:5-9, q4rdna.cu:713-745). */
int q4rdna_mul_mat(const q4rdna_weight *w, const float *x, int64_t x_ne0, float *y, int64_t y_ne0,
                   void *stream);

/* y = W x + add, add[M] fp32.
 * Replaces ggml_cuda_q4rdna_mul_mat_add (source/q4rdna.cuh:11-16, q4rdna.cu:747-767). */
int q4rdna_mul_mat_add(const q4rdna_weight *w, const float *x, int64_t x_ne0, const float *add,
                       int64_t add_ne, float *y, int64_t y_ne0, void *stream);

/* y = (W_up x) * silu(W_gate x), both weights of one shape; glu_op must be
 * Q4RDNA_GLU_SWIGLU (anything else is NOT_APPLICABLE).
 * Replaces ggml_cuda_q4rdna_mul_mat_glu (source/q4rdna.cuh:18-24, q4rdna.cu:769-793). */
int q4rdna_mul_mat_glu(const q4rdna_weight *up, const q4rdna_weight *gate, const float *x,
                       int64_t x_ne0, int glu_op, float *y, int64_t y_ne0, void *stream);

/* Launch options: split_k = number of K chunks reduced across workgroups of
 * the per-tensor kernel (0 = the shape policy, the reference's launch policy
 * at source/q4rdna.cu:578-680 and its LLAMA_Q4_RDNA_COOP override
 * :579-584); kernel = Q4RDNA_KERNEL_POLICY or Q4RDNA_KERNEL_VALU (the same
 * kernel) or Q4RDNA_KERNEL_SEQUENTIAL (any other value, 2 included, which
 * ABI 1 used for a kernel since withdrawn, is an argument error); reserved
 * words must be zero.  Zero-initialised options mean "policy" throughout. */
#define Q4RDNA_KERNEL_POLICY 0
#define Q4RDNA_KERNEL_VALU 1 /* the split-K VALU kernel (split_k applies) */
/* The reference's old mapping (LLAMA_Q4_RDNA_MAPPING=old, source/q4rdna.cu:
 * 190-234,626-634): one thread per row, its weights in k order, one fp32 fma
 * each, so y is bit for bit the reference bench's CPU loop
 * (source/q4rdna_gemv_bench.hip:189-210) before the epilogue.  split_k must be 0
 * or 1; q4rdna_mul_mat_batch runs it once per vector, q4rdna_mul_mat_group
 * refuses it (argument error).  Slow: an ablation and a bit-exact
 * reference, not a decode path. */
#define Q4RDNA_KERNEL_SEQUENTIAL 3
typedef struct q4rdna_launch_options {
    uint32_t split_k;
    uint32_t kernel;
    uint32_t reserved[6];
} q4rdna_launch_options;

/* q4rdna_mul_mat / _add / _glu with explicit options (add, gate may be NULL). */
int q4rdna_mul_mat_ex(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x,
                      const float *add, float *y, const q4rdna_launch_options *options,
                      void *stream);

/* n = 1..Q4RDNA_MAX_BATCH activation vectors against one weight in one
 * launch (no reference counterpart: the reference's hooks decline batches
 * above 1, source/q4rdna.cu:722,754,777).  x holds n vectors of `columns`
 * floats back to back, y (and add) n rows of `rows` floats, as ggml's src1
 * and dst with ne[1] = n, contiguous.  gate (may be NULL) makes it the
 * SwiGLU site.  options->split_k as in q4rdna_mul_mat_ex (0 = the shape
 * policy); for n >= 2 it is raised until every K chunk holds at most 32
 * groups (16 for n > 4).  Each tile is read once for all n vectors; each
 * vector's result is bit-identical to q4rdna_mul_mat_ex of that vector with
 * that split where that call runs eight-wave workgroups. */
int q4rdna_mul_mat_batch(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x, uint32_t n,
                         const float *add, float *y, const q4rdna_launch_options *options,
                         void *stream);

/* Several GEMVs that share one activation, in one launch: y_i = W_i x
 * (+ add_i), or with gate_tiles y_i = (W_i x + add_i) * silu(G_i x) -- e.g.
 * q, k and v of a decoder layer, or its gate and up projections.  count =
 * 1..Q4RDNA_MAX_GROUP; every weight has K = x_ne0 columns (else
 * NOT_APPLICABLE) and lives on the current device; gate_tiles is given for
 * every descriptor or for none, each of its weight's shape; no y may overlap
 * x, another descriptor's y or another descriptor's add, and a descriptor's
 * add is its own y or apart from it (argument error).  x is read once per
 * workgroup in the kernel (no separate prepare launch).  options->split_k
 * applies (0 = the shape policy for the group's total rows, raised until
 * every K chunk holds at most 64 groups; K above 262,144 columns, 64 chunks
 * of 64 groups, is NOT_APPLICABLE).  Each output equals q4rdna_mul_mat_ex of
 * its weight at the group's split bit for bit when both launches run the
 * same workgroup width: eight waves, which each launch uses while it has at
 * most four workgroups per CU (rows / 32 * split of the whole group, or of
 * the one weight), and four waves above that.  The split-K scratch is the stream's,
 * as for q4rdna_mul_mat.  No reference counterpart: the reference launches
 * one kernel per projection and fuses only gate/up
 * (source/q4rdna.cu:736-741,769-793). */
#define Q4RDNA_MAX_GROUP 8
typedef struct q4rdna_group_desc {
    q4rdna_weight weight;      /* W (the up projection for SwiGLU) */
    const uint8_t *gate_tiles; /* SwiGLU gate tiles of W's shape, or NULL */
    const float *add;          /* [rows] or NULL */
    float *y;                  /* [rows] */
} q4rdna_group_desc;
int q4rdna_mul_mat_group(const q4rdna_group_desc *descs, uint32_t count, const float *x, int64_t x_ne0,
                         const q4rdna_launch_options *options, void *stream);

/* Split-K factor the shape policy picks for rows x columns on `device`. */
uint32_t q4rdna_policy_split_k(uint32_t rows, uint32_t columns, int device);

/* q4rdna_mul_mat_ex that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The K
 * chunks of a split launch meet in exchange slots, which here live in a
 * fixed per-GPU device array of Q4RDNA_NOALLOC_SLOTS 32-bit slots (8 MiB,
 * held by every GPU the library runs on until the process ends).  A launch
 * at split_k s > 1 needs (p - 1) * rows slots, p the smallest power of two
 * >= s, doubled with a gate; one that would need more returns
 * Q4RDNA_ERR_ARGUMENT and launches nothing.  Arguments, statuses and results
 * are those of q4rdna_mul_mat_ex (bit-identical at the same split).  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU race,
 * so issue them on one stream or order them with events.  The first call on
 * a GPU looks the array's address up; its slots are zero from the start (a
 * zero-initialised device variable, left zero by every launch), so no set-up
 * runs on any stream and the first call may be captured into a graph. */
#define Q4RDNA_NOALLOC_SLOTS (1u << 21)
int q4rdna_mul_mat_ex_noalloc(const q4rdna_weight *w, const q4rdna_weight *gate, const float *x,
                              const float *add, float *y, const q4rdna_launch_options *options,
                              void *stream);

/* ---- multi-tensor stack --------------------------------------------------
 * One launch that sweeps many independent GEMVs (a decode step's weight
 * streaming).  The GEMVs run concurrently and in an order the plan picks
 * (longest K chunks first), so no descriptor's x, add or y may overlap
 * another's y, and an add is its own y or apart from it (plan creation
 * refuses these with an argument error).  A descriptor's x may overlap its
 * own y: the prepare launch reads every x before the sweep writes.  No
 * reference counterpart: the reference launches one kernel per tensor
 * (source/q4rdna.cu:736-741). */
typedef struct q4rdna_gemv_desc {
    q4rdna_weight weight;      /* W (the up projection for SwiGLU) */
    const uint8_t *gate_tiles; /* SwiGLU gate tiles of the same shape, or NULL */
    const float *x;            /* [columns], 16-byte aligned */
    const float *add;          /* [rows] or NULL */
    float *y;                  /* [rows] */
} q4rdna_gemv_desc;

typedef struct q4rdna_plan q4rdna_plan;

/* Build a plan for `count` descriptors (uploads the descriptor table once).
 * Single-vector plans also fix here which workgroup runs which item: a
 * load-balancing deal computed on the host, about 2 ms for the 252-tensor
 * Qwen3-8B stack and 0.2 s for 100,000 items. */
int q4rdna_plan_create(const q4rdna_gemv_desc *descs, uint32_t count, int device,
                       q4rdna_plan **out);
/* Batched plan: every descriptor's x holds n activation vectors of
 * `columns` floats one after another ([n][columns]), y and add hold n
 * results of `rows` floats ([n][rows]); n = 1..Q4RDNA_MAX_BATCH (the
 * small-batch decode shapes).  No reference counterpart: the reference's
 * hooks decline batches above 1 (source/q4rdna.cu:722,754,777). */
#define Q4RDNA_MAX_BATCH 8
int q4rdna_plan_create_batch(const q4rdna_gemv_desc *descs, uint32_t count, uint32_t n, int device,
                             q4rdna_plan **out);
/* Launch the whole plan on `stream` (prepare + sweep); allocates nothing.
 * Launches of one plan share its digit buffers, split-K partials and
 * counters, so they must not overlap: keep them on one stream or order
 * them with events.  Different plans are independent. */
int q4rdna_plan_launch(q4rdna_plan *plan, void *stream);
/* The two launches of q4rdna_plan_launch, for callers that time or overlap
 * them: prepare converts every activation x into the plan's int8 digit
 * buffers; sweep runs the GEMVs and must follow a prepare of the same x on
 * the same stream. */
int q4rdna_plan_prepare(q4rdna_plan *plan, void *stream);
int q4rdna_plan_sweep(q4rdna_plan *plan, void *stream);
void q4rdna_plan_destroy(q4rdna_plan *plan);
/* Workgroups the plan launches (persistent grid). */
uint32_t q4rdna_plan_workgroups(const q4rdna_plan *plan);

/* Launch statistics, the reference's q4rdna_launches and per-entry hits
 * (source/q4rdna.cu:57,73,706-709,742,764,789-791).  Every GEMV kernel
 * launch the entry points above make counts once (q4rdna_mul_mat_batch's
 * per-vector launches one each, a plan's sweep once), and every weight it
 * streams that starts an entry of an open sidecar counts a hit for that
 * entry (a SwiGLU launch hits both weights). */
uint64_t q4rdna_launch_count(void);
/* Hits of entry `index` of `sidecar` (0 for an invalid pair). */
uint64_t q4rdna_sidecar_hits(const q4rdna_sidecar *sidecar, uint32_t index);
/* The reference's report on stderr (source/q4rdna.cu:75-112, same lines):
 * "Q4_RDNA: launched N decode GEMV kernels", with LLAMA_Q4_RDNA_TRACE set
 * one "Q4_RDNA: hit <name> <hits>" line per entry that was hit, and the
 * unique / hits-by-shape summary, over every open sidecar.  Printed at
 * process exit once q4rdna_default_sidecar has loaded (source/q4rdna.cu:176). */
void q4rdna_report_stats(void);

/* ---- packing and dequantisation ------------------------------------------
 * Quantize fp32 W[rows][columns] (device, row-major) into tiles (device) with
 * the chosen scale search, bit-identical to the reference CPU packers
 * (source/q4rdna_sidecar_pack.cpp:126-179,259-279 for Q4RDNA_ALGO_SIDECAR;
 * source/q4rdna_cpu_experiment.cpp:136-273,387-399 for absmax/range/mse). */
int q4rdna_pack(const float *w, uint32_t rows, uint32_t columns, int algorithm, uint8_t *tiles,
                void *stream);

/* Test/inspection: out[rows][columns] = fp32(scale) * code, the exact
 * product (source/q4rdna_cpu_experiment.cpp:270-271). */
int q4rdna_dequantize(const q4rdna_weight *w, float *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* Q4RDNA_H */
