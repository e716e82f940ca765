/*
 * shaobo_fa3_ext.h -- extensions of libshaobo_fa3_bwd.so beyond the
 * reference ABI.
 */
#ifndef SHAOBO_FA3_EXT_H_
#define SHAOBO_FA3_EXT_H_

#include "shaobo_fa3_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* shaobo_fa3_bwd_v2 on a caller-chosen stream.  No counterpart in the
 * reference, whose ABI launches on the null stream only
 * (reference include/shaobo_fa3_api.h:119-130); this is for framework
 * bindings that order work on their own streams (a PyTorch custom op passes
 * torch.cuda.current_stream()).  `stream` is a hipStream_t (NULL = the null
 * stream, which makes this identical to shaobo_fa3_bwd_v2).  Validation,
 * statuses, workspace and outputs are those of shaobo_fa3_bwd_v2;
 * sync_after_launch synchronises `stream` (the device for NULL).  A stream
 * of another GPU than the current one returns
 * SHAOBO_FA3_STATUS_INVALID_VALUE (make its GPU current first).  The
 * workspace must not be shared by calls that may run concurrently. */
int shaobo_fa3_bwd_v2_on_stream(const void* dout,
                                const void* q,
                                const void* k,
                                const void* v,
                                const void* out,
                                const void* softmax_lse,
                                void* dq,
                                void* dk,
                                void* dv,
                                void* softmax_d,
                                const ShaoboFa3Params* params,
                                void* stream);

/* Test hook, no counterpart in the reference: the number of polls a split
 * job's second piece makes while waiting for the first piece's partial sums
 * before it gives up (default 1 << 24, each poll followed by a short sleep).
 * A wait that gives up still finishes its workgroup normally, writes the
 * launch's epoch into the workspace's error word and the synchronised call
 * (sync_after_launch = 1) returns SHAOBO_FA3_STATUS_HIP_ERROR (unsynchronised
 * calls: shaobo_fa3_ext_split_status / _split_error_count); 0 makes every
 * split wait give up at once (a wait that finds the partial sums already
 * published carries on, so whether a call fails depends on timing).
 * Process-wide; affects launches made after the call. */
void shaobo_fa3_ext_set_split_spin_limit(int polls);

/* Test hook, no counterpart in the reference: with on != 0 the launches
 * that follow (v2, its stream / timed / stages / no-allocation variants,
 * the legacy entry, fused5) run the race-check instantiation of the main
 * kernel.  It does the same arithmetic in the same order as the fast kernel
 * with the pipeline's concurrency taken out: every job starts on an LDS
 * filled with 0xFF bytes (a NaN in fp16, bf16 and fp32, so a read of LDS
 * the job did not write shows in its outputs), and after each LDS phase of
 * a pipeline step every wave waits for all its memory operations and meets
 * the others at a barrier.  Its outputs must equal the fast kernel's bit
 * for bit; it is several times slower.  0 restores the fast kernel.
 * Process-wide. */
void shaobo_fa3_ext_set_race_check(int on);

/* Whether a split wait of an earlier launch gave up on `workspace`, for
 * callers that launch without sync_after_launch.  No counterpart in the
 * reference, whose launches never wait on each other's workgroups.
 * `workspace` is a workspace given to shaobo_fa3_bwd_v2 / _on_stream /
 * shaobo_fa3_bwd / shaobo_fa3_bwd_fused5 (NULL: the no-allocation scratch
 * array of the current GPU).  Synchronises `stream` (a hipStream_t of the
 * current GPU; NULL = the null stream), so queue it behind the launches to
 * check, then reads the workspace's error word.  Returns
 * SHAOBO_FA3_STATUS_HIP_ERROR when a launch of this process wrote it there
 * (its gradients are wrong) and clears the word, so each give-up is
 * reported once; SUCCESS otherwise, whatever an uninitialised workspace
 * holds; INVALID_VALUE for a stream of another GPU. */
int shaobo_fa3_ext_split_status(const void* workspace, void* stream);

/* The number of split waits that gave up on the current GPU since the
 * library was loaded, in any launch on any workspace: *count never
 * decreases, so a caller that does not keep its workspaces (a framework
 * binding allocating one per call) compares it with the count it saw last.
 * No counterpart in the reference.  Synchronises `stream` first (as for
 * shaobo_fa3_ext_split_status).  Returns SUCCESS, INVALID_VALUE (null
 * count, or a stream of another GPU) or HIP_ERROR. */
int shaobo_fa3_ext_split_error_count(void* stream, unsigned long long* count);

/* shaobo_fa3_bwd_v2_on_stream that also records three caller-created
 * hipEvent_t on `stream`: events[0] before the delta preprocess, events[1]
 * between it and the main kernel, events[2] after the main kernel (a NULL
 * handle is skipped).  No counterpart in the reference; it is for
 * benchmarks that time each kernel inside a run of back-to-back calls
 * (bench.py).  Everything else is shaobo_fa3_bwd_v2_on_stream's. */
int shaobo_fa3_ext_bwd_v2_timed(const void* dout,
                                const void* q,
                                const void* k,
                                const void* v,
                                const void* out,
                                const void* softmax_lse,
                                void* dq,
                                void* dk,
                                void* dv,
                                void* softmax_d,
                                const ShaoboFa3Params* params,
                                void* stream,
                                void* const* events);

/* shaobo_fa3_bwd_v2_on_stream limited to some of its two kernels: stages
 * bit 0 launches the delta preprocess, bit 1 the main kernel (3 = both, the
 * same as shaobo_fa3_bwd_v2_on_stream; anything outside 1..3 returns
 * SHAOBO_FA3_STATUS_INVALID_VALUE).  No counterpart in the reference; it is
 * for benchmarks that time one kernel in back-to-back launches (bench.py).
 * The main kernel alone reads the row statistics the preprocess left in the
 * workspace, so it needs an earlier call with bit 0 on the same workspace,
 * inputs and shape, and its dQ / dK / dV then equal those of a full call;
 * with bit 0 alone only softmax_d and the workspace are written. */
int shaobo_fa3_ext_bwd_v2_stages(const void* dout,
                                 const void* q,
                                 const void* k,
                                 const void* v,
                                 const void* out,
                                 const void* softmax_lse,
                                 void* dq,
                                 void* dk,
                                 void* dv,
                                 void* softmax_d,
                                 const ShaoboFa3Params* params,
                                 void* stream,
                                 int stages);

/* Size of the device scratch array behind shaobo_fa3_ext_bwd_v2_no_alloc:
 * 32 MiB per GPU, held from the library's first use on that GPU until the
 * process ends. */
#define SHAOBO_FA3_EXT_SCRATCH_BYTES ((size_t)32 << 20)

/* shaobo_fa3_bwd_v2_on_stream without a workspace: no counterpart in the
 * reference.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The workspace_bytes / workspace fields of params are ignored;
 * the library uses a static device array of SHAOBO_FA3_EXT_SCRATCH_BYTES on
 * the current GPU instead, and calls no hipMalloc / hipFree.  A shape whose
 * workspace (shaobo_fa3_bwd_v2_workspace_bytes) exceeds that size returns
 * SHAOBO_FA3_STATUS_INVALID_VALUE before any HIP call -- except where the
 * excess is the head-split plan's per-chunk dK / dV (GQA with very few KV
 * heads): then the call runs the plan with one dKV job per KV head, whose
 * workspace is smaller, and its results meet the same bar but need not be
 * bit-equal to v2's.  Inputs, outputs,
 * statuses and results are those of shaobo_fa3_bwd_v2_on_stream.  Every
 * call on one GPU shares that GPU's array: calls that may overlap in time on
 * one GPU (other streams, other host threads) race and must not be made. */
int shaobo_fa3_ext_bwd_v2_no_alloc(const void* dout,
                                   const void* q,
                                   const void* k,
                                   const void* v,
                                   const void* out,
                                   const void* softmax_lse,
                                   void* dq,
                                   void* dk,
                                   void* dv,
                                   void* softmax_d,
                                   const ShaoboFa3Params* params,
                                   void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SHAOBO_FA3_EXT_H_ */
