/* presk_hip.h -- the C ABI of the MI355X (gfx950) executor of Presk's realized
 * loop nests: a drop-in `KernelExec` for `--backend hip`.
 *
 * The reference's seam is `trait KernelExec` (crates/presk-kernel/src/host.rs:
 * 28-95), whose native implementations compile each `Kernel` once
 * (`trait KernelCompiler`, crates/presk-cranelift/src/lib.rs:48-53) into a
 * `KernelFn = unsafe extern "C" fn(bufs: *const *mut u8, lo: i64, hi: i64)`
 * (crates/presk-cranelift/src/lib.rs:38-42) and call it over a pointer table
 * [inputs..., output, overflow flag iff the kernel stores f16/e8m15]
 * (crates/presk-cranelift/src/lib.rs:1609-1629).  This ABI keeps that shape,
 * with device pointers and a HIP stream:
 *
 *   presk_hip_compile  <->  KernelCompiler::compile(&Kernel) -> KernelFn
 *   presk_hip_run      <->  the KernelFn call f(bufs, lo, hi)
 *   presk_hip_alloc/free/h2d/d2h/sync
 *                      <->  the host's `Buf`s made device-resident
 *                           (crates/presk-rt/src/lib.rs:760-915)
 *
 * A kernel arrives as its text (`impl Display for Kernel`,
 * crates/presk-kernel/src/ir.rs:495-595) plus the two facts the text does not
 * carry: its storage type (`Kernel::dtype`) and its lane width
 * (`Kernel::lanes`).
 *
 * Errors: every function returns 0 on success and a negative code otherwise;
 * presk_hip_last_error() then gives the message, which starts with the
 * reference's code: "E10001" for an executor error
 * (crates/presk-cranelift/src/lib.rs:34-36), "E7005" for a kernel whose
 * formats the executor does not compute (crates/presk-rt/src/lib.rs:567-591),
 * "E7007" for the overflow guard (crates/presk-kernel/src/host.rs:140-177).
 *
 * Threading: one host thread drives a device (as `KernelBackend` is
 * single-threaded, crates/presk-kernel/src/host.rs:256); launches are
 * asynchronous on the given stream, and a buffer is read on the host only
 * after presk_hip_sync on that stream.
 */
#ifndef PRESK_HIP_H
#define PRESK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRESK_HIP_OK 0
#define PRESK_HIP_ERR (-1)       /* E10001: executor or HIP error */
#define PRESK_HIP_REFUSED (-2)   /* E7005: formats not computed natively */
#define PRESK_HIP_OVERFLOW (-3)  /* E7007: a narrowing store overflowed */

/* How a kernel's reductions are ordered.
 * EXACT: every sum in index order, bit-identical to `--backend kernel`
 *        (ReductionOrder::Sequential, crates/presk-rt/src/lib.rs:251-285).
 * FAST:  contractions on MFMA tiles with f32 accumulation, a reassociating
 *        order the kernel's info names (the declared-order rule of
 *        crates/presk-rt/src/lib.rs:262-268); every other nest as in EXACT.  */
#define PRESK_HIP_EXACT 0
#define PRESK_HIP_FAST 1

typedef struct presk_hip_kernel presk_hip_kernel;

/* What a compiled kernel is: no counterpart in the reference beyond
 * `KernelExec::name` and the launch log (host.rs:317-321); used by the
 * harness to report the class chosen and the roofline of each launch. */
typedef struct {
    char kind[32];        /* "gemm", "rows", "generic", ... */
    char order[32];       /* "sequential", "mfma-k32", ... */
    int32_t guarded;      /* the pointer table ends with a u32 flag */
    int32_t n_inputs;
    int64_t split_bound;  /* the [lo,hi) range of presk_hip_run, or -1 */
    double flops;         /* algorithmic flops of one launch (2*I*J*K for a contraction) */
    double bytes;         /* algorithmic bytes: inputs once + output once, at storage width
                             (crates/presk-kernel/src/cost.rs:26-95) */
} presk_hip_info;

/* Selects the device and sets the executor up.  No counterpart in the
 * reference (its executors need none); must be called before any other
 * function that touches the device.  `device` -1 takes PRESK_HIP_DEVICE
 * (an ordinal; device 0 when unset).  The environment's other switches are
 * checked here, a malformed one failing the call (E10001):
 *   PRESK_HIP_MODE=exact|fast       every kernel compiled in that mode, whatever
 *                                   presk_hip_compile is asked (exact: the
 *                                   interpreter's order in every kernel);
 *   PRESK_HIP_GEMM_TILE=<bm>x<bn>[w8][/<splits>]
 *                                   contraction tiles (128 x 64/96/128, w8
 *                                   after 128x128 or 128x96 (f32) for eight
 *                                   waves; 256 x
 *                                   96/128 on f32 storage, 256 x 128/256 on
 *                                   16-bit) and k splits (1-64, single-entry
 *                                   contractions) in place of the planner's,
 *                                   where they apply;
 *   PRESK_HIP_CACHE, PRESK_HIP_DUMP  the generated kernels' code-object cache
 *                                   and a directory to keep their sources in. */
int presk_hip_init(int device);

/* The message of the calling thread's last failed call ("" if none). */
const char *presk_hip_last_error(void);

/* KernelCompiler::compile (crates/presk-cranelift/src/lib.rs:48-53): reads the
 * kernel's text, chooses its HIP kernel, builds it.  `dtype` is "f64", "f32",
 * "bf16", "f16" or "e8m15"; `lanes` is Kernel::lanes; `mode` is
 * PRESK_HIP_EXACT or PRESK_HIP_FAST.  Refuses (PRESK_HIP_REFUSED) a kernel
 * whose formats are not its storage type's arithmetic (ir.rs:204-259), as
 * the native backend's `prepare` does (host.rs:416-434).  Integer weights
 * (`int8/<over>`, `int4/<over>..<end>`, BufKind::Quant, ir.rs:30) are
 * computed: each load is f32(q) * scale (crates/presk-rt/src/quant.rs:248-252).
 * After presk_hip_init, the kernel's code object is loaded here. */
int presk_hip_compile(const char *text, const char *dtype, int lanes, int mode, presk_hip_kernel **out);

/* The KernelFn call (crates/presk-cranelift/src/lib.rs:38-42): `bufs` holds
 * device pointers [inputs..., output, one f32 scales pointer per int8/int4
 * input in input order, overflow flag iff guarded] (lib.rs:1609-1629);
 * [lo, hi) is a range of the outermost loop's iterations when
 * presk_hip_kernel_info's split_bound is not -1 (Kernel::parallel_outer,
 * ir.rs:336-373): pieces that cover [0, split_bound) give the whole call's
 * bytes.  When split_bound is -1 the call is (0, 0).  `stream` is a hipStream_t (NULL: the
 * null stream).  Asynchronous: the overflow flag, a device u32 the caller
 * zeroes, is read after presk_hip_sync (E7007 if set). */
int presk_hip_run(const presk_hip_kernel *k, void *const *bufs, int64_t lo, int64_t hi, void *stream);

/* No counterpart in the reference: presk_hip_run for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The same kernels and bits as
 * presk_hip_run; a class kernel's workspace (split-K partials, chunk sums,
 * mask bits) is the library's fixed scratch array of 64 MiB per device,
 * held from the library's load to the process's end, instead of memory
 * allocated on first use.  It calls no hipMalloc, hipFree or allocating
 * routine; a kernel compiled before presk_hip_init (no code object loaded
 * yet) or needing more scratch than 64 MiB is refused with an E10001 error.
 * Calls on one device share its scratch: calls that overlap on one device
 * (on several streams, or from several threads) race. */
int presk_hip_run_noalloc(const presk_hip_kernel *k, void *const *bufs, int64_t lo, int64_t hi, void *stream);

int presk_hip_kernel_info(const presk_hip_kernel *k, presk_hip_info *info);
void presk_hip_release(presk_hip_kernel *k);

/* The kernel's text as the executor read it, printed back as the reference
 * prints a kernel (ir.rs:495-595): the round trip that pins the reader.
 * Writes at most `cap` bytes including the terminator; returns the full
 * length, or a negative code. */
int64_t presk_hip_kernel_text(const presk_hip_kernel *k, char *buf, size_t cap);

/* Device memory and streams: the host's buffers made resident
 * (crates/presk-rt/src/lib.rs:760-915 holds them in host memory). */
int presk_hip_alloc(size_t bytes, void **dev);
int presk_hip_free(void *dev);
int presk_hip_h2d(void *dev, const void *host, size_t bytes, void *stream);
int presk_hip_d2h(void *host, const void *dev, size_t bytes, void *stream);
int presk_hip_memset(void *dev, int value, size_t bytes, void *stream);
int presk_hip_sync(void *stream);
int presk_hip_stream_create(void **stream);
int presk_hip_stream_destroy(void *stream);

/* Timing of launches with HIP events on the launch stream, in the shape of the
 * reference's per-launch `TimedExec` (crates/presk-kernel/src/cost.rs:719-780):
 * runs `k` `reps` times on `stream` after `warmup` untimed runs and stores the
 * mean milliseconds per launch. */
int presk_hip_time(const presk_hip_kernel *k, void *const *bufs, int64_t lo, int64_t hi, void *stream, int warmup,
                   int reps, double *ms_per_launch);

/* The host's conversion of a buffer at a kernel's edge, on the device: n
 * elements of type `from` at src stored as type `to` at dst, as
 * Buf::of(to, b.to_f64()) stores them (crates/presk-rt/src/lib.rs:868-876,
 * called at crates/presk-kernel/src/host.rs:793-829 when a mixed realization
 * hands a kernel a buffer of another type; the C export's presk_convert,
 * crates/presk-export-c/c/presk_rt.h:409-417).  Types "f64", "f32", "bf16",
 * "f16", "e8m15".  A buffer of the same type is copied as it is.  When `to` is
 * f16 or e8m15 and a finite value reaches its overflow threshold, *flag gets
 * bit 0 (if flag is not null): the host's E7007. */
int presk_hip_convert(const void *src, const char *from, void *dst, const char *to, int64_t n, uint32_t *flag,
                      void *stream);

/* One leaf of a `.psk.d` file decoded on the device, replacing the reader's
 * per-element Enc::decode (crates/presk-data/src/lib.rs:205-219, called from
 * `decode`, lib.rs:816-843) followed by Buf::of into the storage type.  `src`
 * holds the leaf's n elements as the file stores them (copied to device
 * memory); `enc` is the header's code: 0 f64, 1 f32, 2 bf16, 3 a format given
 * by its parameters, whose six header bytes `desc` points to (host memory;
 * Enc::of_description, lib.rs:143-166).  Each element is the exact f64 its
 * code denotes (Float::decode, crates/presk-format/src/lib.rs:460-476), stored
 * as type `to` stores an f64 (as presk_hip_convert does, overflow guard
 * included).  A description that is no format fails with E9002. */
int presk_hip_pskd_decode(const void *src, int enc, const uint8_t *desc, int64_t n, void *dst, const char *to,
                          uint32_t *flag, void *stream);
/* An `idx[bound]` leaf: n elements of the smallest unsigned integer holding
 * bound-1 (idx_width, crates/presk-data/src/lib.rs:289-296), little-endian,
 * widened to i64 at dst. */
int presk_hip_pskd_decode_idx(const void *src, uint64_t bound, int64_t n, int64_t *dst, void *stream);

/* A recorded launch sequence: a function body's kernels in the order the
 * host's call loop issues them (crates/presk-kernel/src/host.rs:887-1030 runs
 * each `let` of the body as one or more launches through `KernelExec::run`).
 * No counterpart in the reference's interface: a host that calls the same
 * body again and again (a training loop, a serving loop) records it once and
 * replays it.  `presk_hip_batch_add` copies the kernel's pointer table (its
 * inputs, output and, for a guarded kernel, the flag); the kernels and
 * buffers must outlive the batch.  `presk_hip_batch_graph` makes every later
 * `presk_hip_batch_run` one HIP graph launch of the whole sequence (lazy
 * module loads and workspaces are done first, outside the capture, and
 * nothing the sequence launches is a memset); without it each run issues the
 * launches one by one.  Adding a launch discards the graph. */
typedef struct presk_hip_batch presk_hip_batch;
int presk_hip_batch_create(presk_hip_batch **out);
int presk_hip_batch_add(presk_hip_batch *b, const presk_hip_kernel *k, void *const *bufs, int64_t lo, int64_t hi);
/* An edge conversion (presk_hip_convert) as a step of the sequence. */
int presk_hip_batch_add_convert(presk_hip_batch *b, const void *src, const char *from, void *dst, const char *to,
                                int64_t n, uint32_t *flag);
/* A training dropout mask (presk_hip_dropout_mask) as a step of the sequence:
 * the key is read from device memory at each run, so a replayed graph draws
 * the mask of whatever key the host last wrote there. */
int presk_hip_batch_add_dropout(presk_hip_batch *b, const void *key, double rate, const char *type, int64_t n,
                                void *dst);
int presk_hip_batch_graph(presk_hip_batch *b);
/* presk_hip_batch_graph with independent steps on up to `branches` (1-8)
 * parallel branches of the graph: a step follows every earlier step that
 * writes bytes it reads or writes, or reads bytes it writes (the overflow
 * flag aside: its stores commute), and every earlier launch of the same
 * compiled kernel (one workspace a kernel).  1 is presk_hip_batch_graph.
 * More than one branch is switched off in this build (E10001): a branched
 * capture ended in a host segmentation fault whose cause is not found. */
int presk_hip_batch_graph_branches(presk_hip_batch *b, int branches);
int presk_hip_batch_run(presk_hip_batch *b, void *stream);
void presk_hip_batch_release(presk_hip_batch *b);

/* A training dropout mask on the device: `DropoutMask` with training on
 * (crates/presk-kernel/src/host.rs:1610-1627 calling dropout_mask,
 * host.rs:1893-1926, which draws it on the host's workers).  n elements of
 * type "f64", "f32", "bf16", "f16" or "e8m15": element e is 1/(1-rate) where
 * the key's e-th uniform draw (uniform01 of its ChaCha20Rng stream read from
 * word 2e, crates/presk-interp/src/key.rs:43-55) is below 1-rate, else 0,
 * rounded as Buf::of rounds it -- the host's bits.  `key`: the 32-byte key in
 * device memory (4-byte aligned).  A rate outside [0, 1) is E7001, as the
 * host refuses it. */
int presk_hip_dropout_mask(const void *key, double rate, const char *type, int64_t n, void *dst, void *stream);

/* Seeded synthetic values written in place: n elements mean + std * z of
 * type "f32", "bf16" or "f16", z ~ N(0, 1) a function of (seed, element
 * index) alone (a splitmix64 hash and Box-Muller in f32).  Stands in for the
 * host's parameter initialization (`Normal` and `ones` are host primitives,
 * crates/presk-kernel/src/host.rs:1476; their draws come from ChaCha20 keys,
 * crates/presk-interp/src/run.rs:56-100) where a model's parameters are too
 * large to draw on the host and copy: the values are seeded N(0, std) but not
 * the reference's draws.  std = 0 fills the constant `mean`. */
int presk_hip_fill_normal(void *dst, const char *type, int64_t n, uint64_t seed, double mean, double std, void *stream);

/* A measurement aid with no counterpart in the reference: the matrix cores'
 * rate measured on this device, reported beside the vendor's nominal peak.
 * One timed launch (after an untimed one) of independent MFMA loops, eight
 * waves on every CU, each wave `iters` rounds of eight MFMAs: `type` "bf16"
 * (32x32x16) or "f32" (16x16x4).  *ms the launch's duration (HIP events on
 * `stream`), *flops the flops it performed. */
int presk_hip_mfma_probe(const char *type, int64_t iters, void *stream, double *ms, double *flops);

/* Self-test of the device's scalar functions over a domain block: the digest
 * (sum of splitmix64 finalizers of (i << 32 | out_i)) of function `fn` over
 * inputs [lo, hi), as tests/golden/digests.json holds the reference's.  For
 * fn 50 (expf) and 51 (erff) the result is instead the largest distance in
 * units in the last place between FAST mode's function and the
 * interpreter's over the inputs, and for fn 60 / 61 the count of inputs
 * where the two differ; fn 70-77 count the f32 dividends (the inputs' bit
 * patterns) whose quotient by one of eight fixed divisors through the
 * printed nests' division by a constant differs from the correctly rounded
 * division.  No counterpart in the reference; for the exhaustive device
 * checks. */
int presk_hip_scalar_digest(int fn, uint64_t lo, uint64_t hi, uint64_t *digest);

#ifdef __cplusplus
}
#endif
#endif
