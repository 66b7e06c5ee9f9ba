/* internal.h -- shared state of the C host layer of libthvm_hip.so. */
#ifndef THVM_HIP_INTERNAL_H
#define THVM_HIP_INTERNAL_H

#include <stdint.h>
#include <stddef.h>
#include <hip/hip_runtime_api.h>
#include "thvm_hip.h"
#include "kern_api.h"

typedef uint8_t  u8;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int32_t  i32;

#define THVM_API __attribute__((visibility("default")))

/* ---- errors ---- */
void hb_set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
extern char HB_ERRBUF[512];

/* ---- device + stream ---- */
extern int         HB_READY;
extern hipStream_t HB_STREAM;
extern int         HB_GRAPH_CAPTURING;   /* stream capture open */
int hb_require_ready(const char *who);
int hb_stream_capturing(void);           /* HB_STREAM is being recorded */

/* ---- buffer table ---- */
void *hb_buf_ptr(u32 id);               /* NULL when id is dead/invalid */
u64   hb_buf_size(u32 id);              /* requested (logical) size     */

/* ---- custom programs ---- */
typedef struct HbOp {
  char *name;
  char *program;
  u32   grid[3], block[3], shared;
  u32   n_args;
  u32   args[64];
  u64   outs_mask;
} HbOp;
/* launch one custom op on HB_STREAM (no recording). */
int hb_launch_op(const char *name, const char *program, const u32 grid[3], const u32 block[3],
                 u32 shared, const u32 *buf_ids, u32 n_args);
int hb_builtin_launch(const char *program, const u32 *buf_ids, u32 n_args, int check_only);
int hb_rtc_launch(const char *name, const char *source, const u32 grid[3], const u32 block[3],
                  u32 shared, const u32 *buf_ids, u32 n_args, int check_only);
void hb_rtc_reset(void);
void hb_jit_reset(void);
void hb_graph_reset(void);
void hb_decoder_reset(void);
void hb_loader_reset(void);
int  hb_decoder_dims(u32 h, u32 *batch, u32 *max_seq, u32 *vocab);   /* -1: no such decoder */
u32  hb_decoder_slot(u32 h);                                          /* its JIT slot, 0 = none */
u32  hb_decoder_spec_rows(u32 h);                                     /* S of its speculative step, 0 = none */
u32  hb_decoder_spec_slot(u32 h);                                     /* that step's JIT slot, 0 = none */

/* kernel profiling hooks (builtin dispatches only, never under capture) */
int  hb_kprof_on(void);
void hb_kprof_begin(const char *tag, hipEvent_t *e0, hipEvent_t *e1);
void hb_kprof_end(const char *tag, hipEvent_t e0, hipEvent_t e1, u64 bytes);

/* small helpers */
u64 hb_hash64(const void *p, size_t n, u64 h);
u32 hb_dt_size(u32 dt);

#endif
