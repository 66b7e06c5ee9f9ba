/* thvm_hip.h -- C-ABI of libthvm_hip.so, the MI355X (gfx950) DEV=hip device
 * for thvm's tensor track.
 *
 * Every entry point takes plain integers, byte counts and host pointers.
 * Device memory is addressed by buffer ids (u32, 0 = "no buffer"), exactly as
 * the reference Backend vtable addresses it (reference src/thvm.h:751-829), so
 * a `struct Backend HIP_BACKEND` in the reference tree wires these functions in
 * field by field.  Each declaration names the reference entry it replaces.
 *
 * Errors: int entry points return 0 on success and -1 on failure; u32 entry
 * points return 0 on failure.  The reason is kept in a static string
 * (thvm_hip_last_error) and printed to stderr, as the CUDA backend does
 * (reference src/backend/cuda/init.c:95-102).
 *
 * Threading: one host thread, one device (ordinal 0), one stream.  Launches
 * are asynchronous; thvm_hip_dispatch_end drains.  buf_read drains first.
 */
#ifndef THVM_HIP_H
#define THVM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype ids: the reference DT_* numbering (reference src/thvm.h:254-271). */
enum {
  THVM_DT_BOOL = 0, THVM_DT_INT8 = 1, THVM_DT_UINT8 = 2, THVM_DT_INT16 = 3,
  THVM_DT_UINT16 = 4, THVM_DT_INT32 = 5, THVM_DT_UINT32 = 6, THVM_DT_INT64 = 7,
  THVM_DT_UINT64 = 8, THVM_DT_FP8E4M3 = 9, THVM_DT_FP8E5M2 = 10,
  THVM_DT_FP16 = 11, THVM_DT_BF16 = 12, THVM_DT_FP32 = 13, THVM_DT_FP64 = 14
};

/* Backend id the reference reserves for a fourth device: CPU=1, METAL=2,
 * CUDA=3 (reference src/codegen/hand_opts.c:174, src/thvm.c:676). */
#define THVM_HIP_BACKEND_ID 4u

/* ===================== lifecycle (Backend.init / .shutdown) ============= */

/* cuda_init (reference src/backend/cuda/init.c:110): pick device 0, create
 * the dispatch stream.  Idempotent.  -1 when no gfx950 device is present. */
int         thvm_hip_init(void);
/* cuda_shutdown: free every buffer, module, graph and the stream. */
void        thvm_hip_shutdown(void);
/* cuda available probe (reference src/backend/cuda/_.c:62). */
int         thvm_hip_available(void);
/* thvm_cuda_last_error (reference src/backend/cuda/init.c:95-102). */
const char *thvm_hip_last_error(void);
/* Library version string, e.g. "thvm-hip 0.1 gfx950". */
const char *thvm_hip_version(void);

/* ===================== buffers (Backend.buf_*) ========================== */

/* cuda_buf_alloc (reference src/backend/cuda/buf_alloc.c:19): zero-filled
 * device buffer, best-fit freelist recycle first.  0 on failure. */
uint32_t thvm_hip_buf_alloc(uint64_t nbytes);
/* cuda_buf_free (buf_free.c): drop the slot now (stream-ordered free). */
void     thvm_hip_buf_free(uint32_t buf_id);
/* cuda_buf_incref / cuda_buf_decref: refcount; decref to 0 parks the block
 * on the freelist (buf_decref.c, buf_freelist.c). */
void     thvm_hip_buf_incref(uint32_t buf_id);
void     thvm_hip_buf_decref(uint32_t buf_id);
/* cuda_buf_jit_pin / unpin: sticky hold by an active JIT capture. */
void     thvm_hip_buf_jit_pin(uint32_t buf_id);
void     thvm_hip_buf_jit_unpin(uint32_t buf_id);
/* cuda_buf_read / cuda_buf_write / cuda_buf_copy (buf_read.c, buf_write.c,
 * buf_copy.c).  Byte 0 based; nbytes must fit the buffer. */
int      thvm_hip_buf_read (uint32_t buf_id, void *dst, uint64_t nbytes);
int      thvm_hip_buf_write(uint32_t buf_id, const void *src, uint64_t nbytes);
int      thvm_hip_buf_copy (uint32_t dst_id, uint32_t src_id, uint64_t nbytes);
/* Backend.buf_write_at / buf_copy_at (reference src/thvm.h:780-787): the
 * KV-append form, bounds-checked against the destination. */
int      thvm_hip_buf_write_at(uint32_t buf_id, uint64_t byte_off,
                               const void *src, uint64_t nbytes);
int      thvm_hip_buf_copy_at(uint32_t dst_id, uint64_t dst_byte_off,
                              uint32_t src_id, uint64_t nbytes);
/* Inside an open graph capture buf_copy / buf_copy_at are recorded as copy
 * kernels and buf_zero as a fill kernel (the reference's jit_replay calls
 * buf_zero and, through tensor_assign, buf_copy_at inside its capture:
 * src/jit/capture.c:2779-2815); buf_read / buf_write are refused there.
 *
 * The KV-append ASSIGN at a symbolic row (capture.c:2797-2801 computes
 * kvar_runtime(kvar) * strides[0] on the host, which a captured graph would
 * freeze): copy nbytes of src to dst at byte offset
 *   base_off + row_bytes * row,  row = the int32 at row_buf + row_buf_off,
 * read on the device when the copy runs, so a replayed graph appends at the
 * current row.  A row outside the destination writes nothing.  0 / -1. */
int      thvm_hip_buf_copy_row(uint32_t dst_id, uint64_t base_off, uint64_t row_bytes,
                               uint32_t row_buf_id, uint64_t row_buf_off,
                               uint32_t src_id, uint64_t nbytes);
/* cuda_buf_refcount / freelist_push / freelist_remove / storage_root /
 * nbytes / zero (reference src/thvm.h:788-815). */
uint32_t thvm_hip_buf_refcount(uint32_t buf_id);
void     thvm_hip_buf_freelist_push(uint32_t buf_id);
void     thvm_hip_buf_freelist_remove(uint32_t buf_id);
uint32_t thvm_hip_buf_storage_root(uint32_t buf_id);
uint64_t thvm_hip_buf_nbytes(uint32_t buf_id);
void     thvm_hip_buf_zero(uint32_t buf_id);
/* Load nbytes of a file at byte file_off into a buffer at dst_off: the
 * region is mmapped read-only (page-aligned, as the reference's disk tensor
 * maps it, src/tensor/mmap.c:1-30) and streamed through a ring of pinned
 * staging buffers with asynchronous host-to-device copies; returns when the
 * bytes are on the device.  Refused inside a graph capture.  0 / -1. */
int      thvm_hip_buf_load_file(uint32_t buf_id, uint64_t dst_off, const char *path,
                                uint64_t file_off, uint64_t nbytes);
/* Arena view: a non-owning buffer id aliasing [off, off+nbytes) of parent
 * (cuda_buf_alloc_arena_view, reference src/backend/cuda/buf_alloc.c:189-205).
 * Holds a reference on the parent.  0 on failure. */
uint32_t thvm_hip_buf_view(uint32_t parent_id, uint64_t byte_off, uint64_t nbytes);
/* Raw device address of a buffer (cuda_buf_dptr), for interop only. */
uint64_t thvm_hip_buf_device_ptr(uint32_t buf_id);
/* Live / peak device bytes (cuda_buf_live_bytes / cuda_buf_peak_bytes). */
uint64_t thvm_hip_mem_live_bytes(void);
uint64_t thvm_hip_mem_peak_bytes(void);

/* ===================== pool watermarks and preserve marks =============== *
 * The per-realize memory scope of the reference's realize loop
 * (src/schedule/realize.c:132-152, :296-310, :326-340, :420-450), served by
 * its backend's buf_pool.c:9-183.  A watermark names every buffer allocated
 * after it (an allocation sequence number, not a slot index: dead slots are
 * reused here, with a per-slot generation in the id so a stale id stays
 * dead).  The caller marks the buffers that must survive, then rolls back. */
/* cuda_buf_pool_begin (buf_pool.c:9-11). */
uint32_t thvm_hip_buf_pool_begin(void);
/* cuda_buf_pool_rollback_with_preserve (:22-47): every buffer since wm that
 * is not preserved, not JIT-pinned and not already parked: owning blocks are
 * parked on the freelist (freed when it is full), arena blocks freed, views
 * freed.  Refcounts are not consulted (the planner knows these are dead). */
void     thvm_hip_buf_pool_rollback_with_preserve(uint32_t wm);
/* cuda_buf_pool_free_unpreserved (:54-64): the same set, freed outright. */
void     thvm_hip_buf_pool_free_unpreserved(uint32_t wm);
/* cuda_buf_mark_preserved (:66-69); called through tensor_mark_buf_preserved
 * (src/tensor/mark_buf_preserved.c:22), which also marks an arena view's
 * parent. */
void     thvm_hip_buf_mark_preserved(uint32_t buf_id);
/* cuda_buf_clear_preserved (:105-108): marks of buffers since wm (1: all). */
void     thvm_hip_buf_clear_preserved(uint32_t wm);
/* cuda_buf_clear_preserved_arena_views (:172-183): views since wm lose their
 * mark, and so does each one's parent when it too was allocated since wm. */
void     thvm_hip_buf_clear_preserved_arena_views(uint32_t wm);
/* cuda_buf_free_unpreserved_all (:122-160): table-wide, every live owning
 * buffer neither preserved nor JIT-pinned is parked (arena blocks freed);
 * views are left to their parent.  Drains the stream first.  Returns bytes. */
uint64_t thvm_hip_buf_free_unpreserved_all(void);
/* A per-realize arena block (the reference's skip_freelist CudaBuf,
 * src/thvm.h:1147-1158; thvm_metal_buf_arena_alloc): never recycled from or
 * parked on the freelist; a rollback or the sweep frees it outright. */
uint32_t thvm_hip_buf_arena_alloc(uint64_t nbytes);
/* Diagnostics: live buffer slots (parked blocks included), and the highest
 * slot index ever used.  A dead slot is reused with the next generation; a
 * slot retires after 2^14 generations (so an id is never issued twice), so
 * the high-water mark grows by one per 2^14 buffer deaths beyond the peak
 * live count, not by one per allocation. */
uint32_t thvm_hip_buf_slots_used(void);
uint32_t thvm_hip_buf_slot_highwater(void);

/* ===================== dispatch (Backend.dispatch_*) ==================== */

void thvm_hip_dispatch_begin(void);
void thvm_hip_dispatch_flush(void);
/* cuda_dispatch_end (reference src/backend/cuda/_.c:23-27): drain the
 * stream; a no-op while a graph capture is open. */
void thvm_hip_dispatch_end(void);

/* Custom-kernel dispatch: the body of Backend.dispatch_kernel for a
 * KernelEntry carrying custom_program (cuda_custom_dispatch, reference
 * src/backend/cuda/jit.c:802; ABI reference src/schedule/kernel_custom.c:14-35).
 *   name/program : KernelEntry.custom_name / custom_program
 *   grid/block   : custom_grid[3] / custom_block[3]
 *   shared_bytes : custom_shared_bytes (dynamic LDS; up to 160 KiB on gfx950)
 *   buf_ids      : one buffer id per argument slot, n_args <= 64
 *   outs_mask    : custom_outs_mask (slots the kernel writes)
 * Two program forms:
 *   - HIP source: `extern "C" __global__ void <name>(T *arg0, ...)`, compiled
 *     by hiprtc for gfx950 and cached by source hash (memory + disk);
 *   - "thvm-builtin:<kernel> key=value ...": a hand-written gfx950 kernel
 *     linked into this library (GEMV, norms, attention, routing, ...).  The
 *     library picks its own launch geometry; grid/block are ignored.
 * Inside a JIT capture the dispatch is also recorded for replay. */
int thvm_hip_dispatch_custom(const char *name, const char *program,
                             const uint32_t grid[3], const uint32_t block[3],
                             uint32_t shared_bytes,
                             const uint32_t *buf_ids, uint32_t n_args,
                             uint64_t outs_mask);

/* Compile-only probe of a custom program (hiprtc or builtin parse): 0 when
 * it would dispatch.  Used by hosts to fail early. */
int thvm_hip_program_check(const char *name, const char *program);

/* The attention builtin without its workspace: no counterpart in the
 * reference.  It is for callers that cannot allocate device memory (code
 * under graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * `program` is a "thvm-builtin:attn ..." spec exactly as for
 * thvm_hip_dispatch_custom; buf_ids are its first five slots (out, q, kcache,
 * vcache, len), and the partials live in a static device array of 16 MiB per
 * GPU (held until the process ends) instead of slot 5.  A spec whose
 * partials exceed 16 MiB fails with an error.  Nothing is allocated or freed.
 * Calls that overlap on one GPU share that array and race.  0 / -1. */
int thvm_hip_attn_decode_noalloc(const char *program, const uint32_t *buf_ids,
                                 uint32_t n_args);

/* ===================== renderer target ================================= */
/* One node of a kernel's lifted uop DAG, flattened for the C ABI, sources
 * before users.  `op` is the reference's UOP_* number (src/thvm.h:302-512);
 * a reference-side adapter walks its Term DAG (the root that
 * cg_render_uop_kernel_cuda_root takes, src/codegen/render_uop.c:4964) once
 * and fills this array.  Payloads:
 *   CONST(2)        arg0 = bits (an f32 pattern for every float dtype, the
 *                   integer value otherwise), as UOP_CONST holds them
 *   RANGE(25)       arg0 = axis id, arg1 = KAX_* axis type, arg2 = extent,
 *                   or src0 = an extent expression (symbolic)
 *   REDUCE(17)      src0 = value, src1..3 = the RANGEs reduced,
 *                   arg0 = REDUCE_SUM(0) / REDUCE_MAX(1)
 *   DEFINE_VAR(18)  arg0 = index into the kernel's int32 variable buffer,
 *                   arg1 / arg2 = min / max of the variable
 *   BUFFER(36)      arg0 = argument slot (0 = the output), dtype = element,
 *                   arg1 = capacity in elements (> 0: every load outside
 *                   reads 0 and every store outside is dropped)
 *   INDEX_E(26)     src0 = BUFFER, src1 = element index: the element's value
 *                   (the reference's lifted DAGs read buffers this way);
 *                   LOAD(21) src0 = INDEX is the same value
 *   STORE(37)       src0 = BUFFER slot 0, src1 = index, src2 = value (root,
 *                   the last node)
 *   CAST(23) / BITCAST(24): dtype = the target type
 *   ALU: ADD MUL NEG RECIP EXP2 LOG2 SQRT SIN CMPLT CMPEQ, IADD ISUB IMUL
 *   IDIV IMOD ILT IAND IOR IXOR ISHL ISHR IWHERE (src0 ? src1 : src2). */
typedef struct ThvmUop {
  uint32_t op;
  uint32_t dtype;
  int32_t  src[4];   /* earlier node indices, -1 = none */
  int64_t  arg[4];
} ThvmUop;

typedef struct ThvmRenderInfo {
  uint32_t n_slots;    /* argument slots: buffers 0..k-1, then the variable buffer */
  uint32_t kvar_slot;  /* slot of the int32 variable buffer, 0 = no variables */
  uint32_t group;      /* threads per output in its reductions (1: one thread) */
  uint32_t block;      /* threads per block */
  uint64_t grid_max;   /* blocks to launch (variables at their maxima) */
  uint32_t upcast;     /* consecutive outputs per thread */
  uint32_t reserved;
} ThvmRenderInfo;

/* Launch geometry of a rendered kernel -- the reference's LOCAL,
 * GROUP_REDUCE and UPCAST opts (src/thvm.h:433-437, applied by
 * src/codegen/apply_opt.c) as the gfx950 target realises them: `block`
 * threads per block (64..1024, a power of 2; 0 = 256), `group` consecutive
 * threads sharing one output's reductions (a power of 2 <= block, only for
 * un-nested reductions; 0 or 1 = one thread per output), `upcast`
 * consecutive outputs per thread (1..8, with group 1; 0 = 1). */
typedef struct ThvmRenderOpts {
  uint32_t block, group, upcast, reserved;
} ThvmRenderOpts;

/* cg_render_uop_kernel_cuda_root + the CUDA dispatch geometry (reference
 * src/codegen/render_uop.c:4964-5113, src/backend/cuda/jit.c:634-787) for
 * gfx950: writes `extern "C" __global__ void <name>(out, in1.., kv)` HIP
 * source into `out` (NUL-terminated) for thvm_hip_dispatch_custom with
 * grid = {grid_max,1,1}, block = {block,1,1}.  Pure host code (no device
 * needed).  0 / -1. */
int thvm_hip_render_kernel(const ThvmUop *nodes, uint32_t n, const char *name,
                           char *out, uint64_t cap, ThvmRenderInfo *info);
/* The same with explicit opts (NULL: the target's hand-coded choice, which
 * thvm_hip_render_kernel uses). */
int thvm_hip_render_kernel_opts(const ThvmUop *nodes, uint32_t n, const char *name,
                                const ThvmRenderOpts *opts, char *out, uint64_t cap,
                                ThvmRenderInfo *info);
/* The reference BEAM autotuner's role (src/codegen/autotune.c, candidates of
 * src/codegen/propose.c:382-415) on the device: search the opts of one
 * kernel over its own argument buffers (ids as thvm_hip_dispatch_custom
 * takes them; the kernel must not read its output), each candidate timed
 * over `reps` launches (0 = 20) and kept only when its output matches the
 * hand-coded choice's (floats 1e-5 relative, integers exactly).  Writes the
 * fastest opts and the two mean launch times; the output buffer holds the
 * winner's result.  Winners are cached by the rows' hash, in the process and
 * under $THVM_HIP_CACHE_DIR/tune/.  0 / -1. */
int thvm_hip_render_autotune(const ThvmUop *nodes, uint32_t n, const uint32_t *buf_ids,
                             uint32_t n_args, uint32_t reps, ThvmRenderOpts *best,
                             double *best_us, double *base_us);

/* ===================== JIT capture / replay ============================ */
/* The reference capture API (src/jit/capture.c:644-745, 2687-2884) restricted
 * to custom dispatches: ops fired between begin and end are recorded, every
 * argument buffer is JIT-pinned, and jit_replay re-issues the sequence.  The
 * first replay captures the stream into a hipGraph; later replays are one
 * hipGraphLaunch.  Slots are 1..15; 0 means failure. */
uint32_t thvm_hip_jit_capture_begin(void);
void     thvm_hip_jit_capture_end(void);
uint32_t thvm_hip_jit_capture_op_count(uint32_t slot);
int      thvm_hip_jit_replay(uint32_t slot);
/* jit_replay_with_inputs (capture.c:2615): rebind argument buffer ids
 * (old -> new) for this and later replays; the graph is re-captured when a
 * device address moved.  n pairs in old_ids/new_ids. */
int      thvm_hip_jit_rebind(uint32_t slot, const uint32_t *old_ids,
                             const uint32_t *new_ids, uint32_t n);
void     thvm_hip_jit_capture_drop(uint32_t slot);
int      thvm_hip_jit_is_capturing(void);

/* Backend graph hooks used by the reference's own jit_replay
 * (cuda_jit_graph_*, reference src/backend/cuda/jit.c:457-615). */
int  thvm_hip_graph_replay(uint32_t slot);
int  thvm_hip_graph_capture_begin(void);
int  thvm_hip_graph_capture_end_and_launch(uint32_t slot);
void thvm_hip_graph_invalidate(uint32_t slot);

/* ===================== timing =========================================== */
/* hipEvent pair on the dispatch stream (replaces THVM_CUDA_GPU_TIME,
 * reference src/backend/cuda/jit.c:990-1016).  Returns a timer id. */
uint32_t thvm_hip_timer_start(void);
/* Milliseconds between start and now (drains the stream). */
double   thvm_hip_timer_stop(uint32_t timer_id);
/* Per-builtin-kernel time: when enabled, every eager builtin dispatch binds
 * a hipEvent pair to the start of its first kernel and the end of its last
 * (hipExtLaunchKernel) and accumulates into a table keyed by kernel tag, so
 * the figures are kernel execution time, as a kernel trace reports it.
 * Dispatches made while a graph capture is open are not timed. */
void     thvm_hip_kprof_enable(int on);
void     thvm_hip_kprof_reset(void);
/* Total ms and launch count for kernel tag (e.g. "gemv"); -1 when absent. */
double   thvm_hip_kprof_query(const char *tag, uint64_t *count_out);
/* Algorithmic bytes credited to the timed launches of `tag` (weights, scales,
 * activations read and outputs written, each once; 0 for kernels whose bytes
 * depend on a device-resident length, e.g. attention). */
uint64_t thvm_hip_kprof_bytes(const char *tag);

/* ===================== decode models ==================================== */
/* C counterpart of the reference's decode drivers (bench/dsv2_decode_bench.c
 * step_build :2328-2430 and the GPT-2 driver bench/gpt2/thvm_gpt2.py): a
 * synthetic, seeded, random-init decoder whose whole decode step is a list of
 * custom dispatches, captured once and replayed with a device-resident token
 * and position (no host values per step). */
enum {
  THVM_ARCH_LLAMA = 1,   /* RMSNorm, GQA + RoPE, SwiGLU (config C4)      */
  THVM_ARCH_GPT2  = 2,   /* LayerNorm, learned positions, GELU (C1, C3)  */
  THVM_ARCH_DSV2  = 3    /* MLA latent cache + MoE (C5)                  */
};

typedef struct ThvmDecodeConfig {
  uint32_t arch;          /* THVM_ARCH_*                                   */
  uint32_t n_layers;
  uint32_t dim;           /* d_model                                       */
  uint32_t n_heads;
  uint32_t n_kv_heads;    /* GQA; = n_heads for MHA                        */
  uint32_t head_dim;
  uint32_t ffn;           /* FFN width (dense layers)                      */
  uint32_t vocab;
  uint32_t max_seq;       /* KV capacity (positions)                       */
  uint32_t batch;         /* rows decoded per step, 1..64 (above 4: MFMA GEMM projections) */
  uint32_t wdtype;        /* weight dtype: FP32 / FP16 / BF16 / FP8E4M3    */
  uint32_t adtype;        /* activation dtype: FP32 / FP16 / BF16          */
  float    eps;           /* norm epsilon                                  */
  float    rope_theta;    /* RoPE base (LLAMA, DSV2)                       */
  float    init_std;      /* weight N(0, init_std)                         */
  /* DSV2 (MLA + MoE) fields; ignored by the other archs                  */
  uint32_t kv_lora;       /* latent rank                                   */
  uint32_t d_nope, d_rope, d_v;
  uint32_t n_experts, n_shared, top_k, moe_inter, first_dense;
  /* LLAMA only: 1 runs the step as ONE persistent launch (one block per CU,
   * stages separated by grid barriers) instead of one launch per op; outputs
   * are identical.  Batch 1, 2 or 4; fp8 or bf16 weights, bf16 activations;
   * head_dim 64/128; 1, 2 or 4 query heads per kv head.                    */
  uint32_t step_mode;
  /* DSV2 above 4 rows: the expert-grouped MoE on MFMA (0 or 2, the default)
   * or on the VALU (1); at 4 rows and below the per-row kernels run.      */
  uint32_t moe_mode;
  /* 64-row cache chunks per attention split block (0 auto, else 1..64):
   * LLAMA / GPT2 attention, and the DSV2 latent split on MFMA.  The
   * persistent step's attention is the one-chunk form; an op-list decoder
   * with attn_cpb 1 computes it bit for bit.                              */
  uint32_t attn_cpb;
  /* next-token choice: temperature 0 is greedy (argmax, lowest index on
   * ties); above 0 each step samples an id from softmax(logits / temperature)
   * with a draw keyed on (sample_seed, row, position), so a replayed step
   * draws afresh and a rerun from the same state draws the same ids.      */
  float    temperature;
  uint32_t sample_seed_lo, sample_seed_hi;
  /* blind speculative decode (reference DSV2_SPEC, bench/dsv2_decode_bench.c:
   * 56-68, 2255-2745): spec_rows S in 2..4 builds a second step that drafts
   * S-1 ids from the most recent bigram match in the token history, verifies
   * the pending id and the drafts as S consecutive positions of one
   * sequence, and commits the longest verified prefix plus one id (L
   * advances by 1..S).  Each verify row folds exactly as the one-row step
   * does, so the committed ids are the greedy ids.  LLAMA, batch 1, greedy,
   * op-list step only; 0 = off.  spec_forced = 1 drafts the ids the host
   * seeded after the pending one instead (the acceptance gate).            */
  uint32_t spec_rows, spec_forced;
  /* attention form: 0 auto (one launch for caches of at most 512 rows, two
   * above), 1 one launch (the last split block of a row and kv head
   * merges), 2 two launches (split, then merge)                            */
  uint32_t attn_fused;
  /* attention split: 0 auto (on MFMA for 16-bit caches of head dim 64 or
   * 128 and up to 8 query heads per kv head, where the attention runs as two
   * launches), 1 the MFMA split, 2 the VALU split                           */
  uint32_t attn_mf;
} ThvmDecodeConfig;

/* Build the model on device: allocate, fill weights from `seed` (weights
 * N(0, init_std); fp8 weights per-row absmax/448 e4m3 with f32 scales; norm
 * gains 1), compile the step.  Returns a handle > 0, 0 on failure. */
uint32_t thvm_hip_decoder_create(const ThvmDecodeConfig *cfg, uint64_t seed);
void     thvm_hip_decoder_destroy(uint32_t dec);
/* Generation through the captured step (reference serve mode,
 * bench/dsv2_decode_bench.c:2749-2897): consume prompts [batch][n_prompt]
 * from position 0, one position per step (the prompt id written into the
 * device token), then decode up to max_new ids per row with the token kept
 * on the device; a row stops at `eos` (not emitted; eos < 0: never).  out
 * [batch][max_new] gets the ids (-1 after a row stops), n_out[batch] their
 * counts.  Greedy or sampled as the decoder's temperature says.  The step is
 * captured on first use.  0 / -1. */
int      thvm_hip_decoder_generate(uint32_t dec, const int32_t *prompts, uint32_t n_prompt,
                                   uint32_t max_new, int32_t eos, int32_t *out,
                                   uint32_t *n_out);
/* The reference's stdin serve protocol over file descriptors (batch 1):
 * writes "ready", then per request line "id,id,...[|max_new]" one line
 * "ids: id,id,..." (timing to stderr) until EOF on in_fd.  Requests with ids
 * outside the vocabulary get an empty reply.  0 at EOF, -1 on a failure. */
int      thvm_hip_decoder_serve(uint32_t dec, int in_fd, int out_fd, int32_t eos,
                                uint32_t default_max_new);
/* Fill the KV cache rows [0, ctx) of every layer and batch row with N(0,1)
 * values from `seed` and set the position so the next step writes row ctx. */
int      thvm_hip_decoder_prefill_synthetic(uint32_t dec, uint32_t ctx, uint64_t seed);
/* Set the current token of each batch row (n = batch) and the position
 * (the row the next step writes). */
int      thvm_hip_decoder_set_state(uint32_t dec, const int32_t *tokens, uint32_t pos);
/* One eager decode step: every kernel dispatched individually. */
int      thvm_hip_decoder_step(uint32_t dec);
/* Capture one step into a JIT slot (runs it once) and return the slot. */
uint32_t thvm_hip_decoder_capture(uint32_t dec);
/* Replay the captured step n_steps times (graph launches, no host values).
 * Each step writes its greedy token into the history buffer. */
int      thvm_hip_decoder_replay(uint32_t dec, uint32_t n_steps);
/* Speculative step (spec_rows > 0): one eager draft + verify + commit;
 * capture it into its own JIT slot (runs it once; returns the slot, 0 on
 * failure); replay the captured speculative step n_steps times.  Each step
 * advances the position by 1..spec_rows, written to the token history as
 * the one-row step writes it.  Reference: step_build_spec and run_spec,
 * bench/dsv2_decode_bench.c:2419-2745. */
int      thvm_hip_decoder_spec_step(uint32_t dec);
uint32_t thvm_hip_decoder_spec_capture(uint32_t dec);
int      thvm_hip_decoder_spec_replay(uint32_t dec, uint32_t n_steps);
/* Read back the token history rows [0, n) of batch row b (greedy ids), and
 * the logits [batch, vocab] f32 of the last step. */
int      thvm_hip_decoder_read_tokens(uint32_t dec, int32_t *dst, uint32_t n);
int      thvm_hip_decoder_read_logits(uint32_t dec, float *dst, uint64_t nfloats);
uint32_t thvm_hip_decoder_position(uint32_t dec);
/* Named tensor of the model (e.g. "l0.wqkv", "l0.kcache", "emb", "x"):
 * buffer id, dtype and byte size, so a host can read weights back. */
uint32_t thvm_hip_decoder_tensor(uint32_t dec, const char *name,
                                 uint32_t *dtype_out, uint64_t *nbytes_out);
/* Decoders above 4 rows keep a tiled copy ("<name>.tiled", the MFMA GEMM's
 * tile layout) of each projection weight: after writing a weight tensor
 * through its buffer, call this to refresh the copy (name NULL: every
 * tiled weight).  A tensor with no tiled copy is a no-op.  0 / -1. */
int      thvm_hip_decoder_sync_weights(uint32_t dec, const char *name);
/* Algorithmic HBM bytes one decode step reads+writes at the current
 * position (weights + KV over the live context + activations). */
uint64_t thvm_hip_decoder_step_bytes(uint32_t dec);
/* Number of dispatches in one step. */
uint32_t thvm_hip_decoder_step_kernels(uint32_t dec);
/* Persistent step (step_mode 1) only: the stage clock of the last step, in
 * microseconds after its start, as recorded by block 0: the opening of each
 * grid barrier and the end of the step (5 n_layers + 2 values), then for each
 * stage (l*5 + QKV, ATTN, O, GU, DOWN; then the LM head) its entry, barrier
 * open, work done and stores drained (4 values each).  Writes up to n values
 * and returns how many the step has (0 for a per-op decoder, -1 on error). */
int      thvm_hip_decoder_stage_clock(uint32_t dec, double *us_out, uint32_t n);
/* Per-sublayer probes of one step (counterpart of the reference bench's
 * DSV2_DUMP per-layer fingerprints, bench/dsv2_decode_bench.c:2516-2556,
 * which localise the first layer where a numerics change enters).
 * op_tags writes, for up to n of the step's dispatches, the sublayer each
 * belongs to: 2l for layer l's attention sublayer, 2l+1 for its FFN
 * sublayer, -1 before the first layer (embedding), -2 after the last (final
 * norm, LM head, argmax, length bump); returns the step's dispatch count.
 * run_ops dispatches ops [first, first + count) of the step eagerly -- the
 * same kernels the captured step replays -- so a host can run a step one
 * sublayer at a time and read the activations ("x", "q", "att", "h", ...)
 * in between.  Not during a JIT capture.  0 / -1. */
int      thvm_hip_decoder_op_tags(uint32_t dec, int32_t *tags, uint32_t n);
int      thvm_hip_decoder_run_ops(uint32_t dec, uint32_t first, uint32_t count);
/* Dispatch i of the step as thvm_hip_dispatch_custom would receive it: its
 * name and program text (NUL-terminated, truncated to the caps) and up to
 * ids_cap buffer ids; returns the op's buffer count, -1 on error.  A host
 * can re-dispatch an op with options of its own (e.g. a builtin's clk=). */
int      thvm_hip_decoder_op_info(uint32_t dec, uint32_t i, char *name, uint32_t name_cap,
                                  char *prog, uint32_t prog_cap, uint32_t *ids, uint32_t ids_cap);

#ifdef __cplusplus
}
#endif

#endif /* THVM_HIP_H */
