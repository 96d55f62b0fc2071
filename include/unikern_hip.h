/* libunikern_hip.so — the MI355X (gfx950) kernel hot path of UNIKERN behind a plain C ABI.
 *
 * One target (gfx950), one language (hand-written HIP for CDNA4). No OpenCL, Metal, CUDA
 * shims or Triton. Plain pointers and sizes only; streams are passed as void* (hipStream_t).
 *
 * The reference's boundary is a generate-then-run pipeline:
 *   IBackend::generate -> hip_runnable_program   (reference include/unikern/components.hpp:19-20,
 *                                                 include/unikern/codegen.hpp:40, src/codegen_hip.cpp:132-164)
 *   run_hip(program, workdir) -> RunOutcome       (include/unikern/codegen.hpp:49-93, src/runner.cpp:146-238)
 * which writes a program, compiles it with hipcc and parses one UNIKERN_RESULT line. Here the
 * kernels are compiled ahead of time and the same verify + time + report contract is one call,
 * uk_run(); uk_launch() is the raw operator a caller with its own device buffers uses.
 *
 * Exit-code classes are the reference's (src/codegen_hip.cpp:194-204, :240-292, :889-892;
 * src/main.cpp:472): 0 pass, 1 verify fail, 2 bad invocation / unsupported, 3 infeasible,
 * 4 HIP failure or refusal, 5 residency (oversubscription). Nothing throws across the ABI; the
 * text of the last error is available from uk_last_error().
 *
 * Threading: the reference's caller is single-threaded (src/main.cpp:416-436); so is this
 * library's contract. Calls on one device from several threads must be serialised by the caller.
 */
#ifndef UNIKERN_HIP_H
#define UNIKERN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UK_ABI_VERSION 4

enum uk_status {
  UK_OK = 0,
  UK_VERIFY_FAIL = 1,
  UK_BAD_INVOCATION = 2,
  UK_INFEASIBLE = 3,
  UK_HIP_FAILURE = 4,
  UK_RESIDENCY = 5
};

/* Op kinds: same order as the reference's OpKind (include/unikern/core.hpp:11). */
enum uk_op { UK_OP_GEMM = 0, UK_OP_CONV = 1, UK_OP_REDUCE = 2, UK_OP_SOFTMAX = 3, UK_OP_RMSNORM = 4, UK_OP_CHANNELSCALE = 5 };
/* DType (core.hpp:12) plus Q8_0 (GGUF block: binary16 scale + 32 int8 quants, 34 bytes). */
enum uk_dtype { UK_DT_F32 = 0, UK_DT_F16 = 1, UK_DT_I8 = 2, UK_DT_Q8_0 = 3 };
/* NT: the reference's only tag (A[M][K], B[K][N], C[M][N] row-major; conv HWC valid).
 * TN: gemm with B stored [N][K] (column-major B). NCHW: batched conv with zero padding. */
enum uk_layout { UK_LAYOUT_NT = 0, UK_LAYOUT_TN = 1, UK_LAYOUT_NCHW = 2 };
enum uk_epilogue { UK_EPI_NONE = 0, UK_EPI_CHANNELSCALE = 1 };
enum uk_input_mode { UK_INPUTS_BASELINE = 0, UK_INPUTS_EXACT = 1 };

/* The op spec: a parsed KML tree root (reference KmlTree, include/unikern/core.hpp:22-31).
 * dims as declared: gemm M,N,K | conv H,W,C,Kh,Kw,Oc | reduce L (scalar) or L,C (row-sum) |
 * softmax/rmsnorm/channelscale L,C. */
typedef struct uk_op_desc {
  int32_t op, dtype, layout, epilogue;
  int32_t ndims;
  int32_t dims[6];
  int32_t tile_m, tile_n;     /* KML tile hints (reference defaults 64, 128) */
  int32_t batch, pad, stride; /* conv NCHW (defaults 1, 0, 1) */
  float eps;                  /* rmsnorm epsilon (reference: 1e-6) */
  int32_t n_children;
} uk_op_desc;

/* A solver decision (reference Solution/Instance, include/unikern/core.hpp:66-82). */
typedef struct uk_plan {
  int32_t family;   /* 1 rows, 2 rows_stream, 3 channelscale, 4 reduce1d, 5 gemm_f16_mfma,
                       6 gemm_generic_mfma, 7 conv_igemm_mfma, 8 q8_0_gemm */
  int32_t variant;  /* index into the family's compiled variant table */
  int32_t tile_m, tile_n, tile_k;
  int32_t threads;  /* threads per workgroup */
  int32_t tpr, vec; /* rows family: threads per row, float4 registers per thread */
  int32_t split_k, stages;
  int64_t grid;     /* workgroups per launch */
  double predicted_us;
  int32_t feasible; /* candidates that passed the predicates */
  int32_t shard_rows; /* > 0: scenario B (reference src/codegen_hip.cpp:1143-1238): a GEMM whose
                         working set exceeds the device tier streams A and C in M-shards of this
                         many rows through pinned host buffers, B resident; 0: all resident */
  int32_t stream_path; /* scenario B's data path for A (reference Instance::Path,
                          include/unikern/core.hpp:70): 1 pinned copies (uk_stream_gemm), 2 mapped
                          staging (uk_stream_gemm_file: A read from a file into host-mapped
                          buffers that the kernel reads directly, src/codegen_hip.cpp:1239-1326);
                          0 with shard_rows 0 */
  char key[64];     /* canonical candidate key */
} uk_plan;

/* Result of uk_run (reference RunOutcome, include/unikern/codegen.hpp:49-83, plus roofline). */
typedef struct uk_result {
  int32_t built, ran, verified, exit_code;
  double max_rel;     /* reference metric: max |y-r| / max(|r|, 1e-6) */
  double err_metric;  /* the gate's own metric (see tol_kind) */
  double tol;         /* the gate */
  int32_t tol_kind;   /* 0 max_rel, 1 row-sum |y-r| <= tol*sum|x|, 2 frobenius, 3 bit-exact */
  double kernel_ms;   /* median per-launch time, device-resident inputs, rotating buffer sets */
  double measured_ms; /* end-to-end per pass: H2D + kernel + D2H */
  double achieved;    /* GB/s (bound 0) or TFLOP/s (bound 1) */
  double peak;
  double frac;
  int32_t bound;      /* 0 hbm, 1 mfma */
  int32_t migrations, checks;
  uint64_t vram_free, vram_total;
  int64_t algo_bytes, algo_flops, weight_bytes;
  int32_t launches, repeats, sets;
  uk_plan plan;
  char mode[16];
  char dtype[8];
  char perf[48];
  /* The host side of the run, the SURVEY's cpu_ms=/cpu_cores= tokens: wall time of uk_run's
   * own CPU reference pass (binary64, over the outputs it checks) on the inputs the device saw,
   * the host threads that pass ran on, and how many outputs it computed (all of them, or the
   * sampled rows/images of a GEMM or conv). -1 when not reported (a parsed line without them). */
  double cpu_ms;
  int32_t cpu_cores;
  int64_t cpu_outputs;
  /* The data path a streamed run took, "pinned" or "mmap" (the reference's stream_path= token,
   * src/codegen_hip.cpp:1716); empty for a resident run. */
  char stream_path[8];
} uk_result;

/* ---- library / device ---- */
int uk_abi_version(void);
/* 0 when device 0 reports a gcnArchName starting with gfx950; writes the name. */
int uk_device_check(char* arch, size_t cap);
/* Measured device facts: compute units, max LDS per workgroup, clock (kHz), total bytes. */
int uk_device_props(int32_t* cus, int32_t* lds_per_block, int32_t* clock_khz, uint64_t* total_bytes);
/* Matrix-core ceiling of the device, measured (no counterpart in the reference, which has no
 * matrix-core probe; its calibrate, src/solver.cpp:194-244, derives HCS constants from ledger
 * rows only). One wavefront per SIMD issues only independent f16 MFMAs for a few milliseconds
 * after at least 50 ms of the same load, first v_mfma_f32_16x16x32_f16 (the form of the f16
 * GEMM the solver picks at the BASELINE shape), then v_mfma_f32_32x32x16_f16. tflops: sustained
 * rate; clock_ghz: shader clock over the loop (s_memtime against the 100 MHz s_memrealtime),
 * which uk_calibrate turns into the HCS clock when no MFMA-bound row has been measured;
 * cycles_per_mfma: issue interval per wavefront. The part runs this load at its power limit, so
 * the two forms settle at different clocks; the _32x32 fields report the second form. */
typedef struct uk_mfma_probe {
  double tflops;
  double clock_ghz;
  double cycles_per_mfma;
  double ms_per_launch;
  int32_t workgroups;
  int32_t mfmas_per_wave;
  double tflops_32x32;
  double clock_ghz_32x32;
  double cycles_per_mfma_32x32;
} uk_mfma_probe;
int uk_probe_mfma(uk_mfma_probe* out);
const char* uk_last_error(void);

/* ---- KML op specs (reference src/kml_front.cpp:203-251, src/kml.cpp:57-177) ---- */
int uk_kml_import(const char* json, uk_op_desc* out, char* err, size_t cap); /* 0 ok, 2 rejected */
int uk_kml_export(const char* json, char* out, size_t cap);    /* canonical re-export of a KML text */
int uk_kml_canonical(const char* json, char* out, size_t cap); /* canonical form, children included */
int uk_kml_tree_hash(const char* json, char* out, size_t cap); /* fnv1a of the canonical form */
int uk_op_signature(const uk_op_desc* d, char* out, size_t cap);
int uk_workload(const uk_op_desc* d, int64_t* ops, int64_t* bytes, int64_t* weight_bytes);
int uk_support_gap(const uk_op_desc* d, char* reason, size_t cap); /* 0 covered, 2 refused */

/* ---- hardware description + solver (reference src/hcs.cpp, src/solver.cpp:141-186) ---- */
int uk_hcs_fingerprint(const char* hcs_json, char* out, size_t cap); /* NULL json: built-in MI355X */
int uk_hcs_export(const char* hcs_json, char* out, size_t cap);
/* log: the SOLVE line, one "  rejected KEY violates ..." line per candidate a predicate
   dropped, then one "  candidate KEY family=F variant=V predicted_us=T" line per feasible
   candidate, cheapest first (a plan with that family and variant runs it). */
int uk_solve(const char* hcs_json, const uk_op_desc* d, uk_plan* out, char* log, size_t cap);

/* ---- execution ----
 * uk_launch: enqueue the op on `stream` over caller-owned device buffers.
 *   gemm f32/f16:  in[0]=A, in[1]=B (layout NT: [K][N]; TN: [N][K]); out=C [M][N] (same dtype)
 *   gemm q8_0 TN:  in[0]=X f16 [M][K], in[1]=W blocks (N rows of K/32 blocks); out=Y f32 [M][N]
 *                  (X 16-byte aligned, Y 4-byte; W 16-byte aligned where K is a multiple of 256,
 *                  which every variant the solver picks there copies in 16-byte units, else 4-byte)
 *   conv NT:       in[0]=X [H][W][C], in[1]=Wt [Oc][Kh][Kw][C] (, in[2]=scale[Oc]); out=Y [Oc][Ho][Wo]
 *   conv NCHW:     in[0]=X [N][C][H][W], in[1]=W [Oc][C][Kh][Kw] (, in[2]=scale[Oc]); out=Y [N][Oc][Ho][Wo]
 *   reduce [L]:    in[0]=X; out=Y[1]           reduce [L,C]: in[0]=X; out=Y[L] (row sums)
 *   softmax:       in[0]=X; out=Y               rmsnorm: in[0]=X, in[1]=W[C]; out=Y
 *   channelscale:  in[0]=X, in[1]=S[C]; out=Y
 * plan may be NULL (solved against the built-in MI355X description).
 * Allocates nothing. The 1-D reduce keeps its pass-1 partials (8 KiB) in a static device array,
 * one per GPU, held until the process ends; a 1-D reduce waits (hipStreamWaitEvent on one event
 * per GPU) for the previous one enqueued on that GPU through uk_launch or uk_launch_n, whatever
 * its stream, so two never share the partials at once. That wait is an event recorded outside
 * any graph: callers under HIP graph capture use uk_launch_noalloc. */
int uk_launch(const uk_op_desc* d, const uk_plan* plan, const void* const* in, int32_t n_in, void* out,
              void* stream);
/* uk_launch that allocates nothing: no counterpart in the reference; for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments, kernels and results as uk_launch. The scratch a launch
 * needs beyond its inputs and output (the 1-D reduce's 8 KiB of pass-1 partials) comes from a
 * static 1 MiB device array, one per GPU, held until the process ends; its device address is
 * looked up on the first call on each device. A launch needing more is refused (class 2).
 * Every call on one GPU shares that array and nothing in it needs to start at zero: calls that
 * overlap on one GPU (concurrent streams, or threads) race on it and must be serialised. */
int uk_launch_noalloc(const uk_op_desc* d, const uk_plan* plan, const void* const* in, int32_t n_in, void* out,
                      void* stream);
/* Enqueue `iters` launches, launch i reading set (i % n_sets): in_sets[s*n_in + j], out_sets[s]. */
int uk_launch_n(const uk_op_desc* d, const uk_plan* plan, const void* const* in_sets, int32_t n_in,
                void* const* out_sets, int32_t n_sets, int32_t iters, void* stream);
/* Verify + time + report, the contract of one emitted reference program: seeded inputs
 * (base seed `seed`), GPU result checked against a CPU reference, kernel timed over rotating
 * device-resident buffer sets. With a streamed plan (shard_rows > 0, scenario B) the verified
 * result comes from one streamed pass, measured_ms is a whole pass and kernel_ms its shards'
 * kernels on resident buffers; mode= says which ran. Returns the exit-code class. */
int uk_run(const char* hcs_json, const uk_op_desc* d, const uk_plan* plan, uint64_t seed, int32_t input_mode,
           int32_t timing_iters, uk_result* out, char* log, size_t cap);
/* Scenario B (reference src/codegen_hip.cpp:1143-1238, uk_stream_pass): C = A . B for an f16 or
 * f32 GEMM whose operands live in host memory: hA [M][K], hB as the layout says ([K][N] NT,
 * [N][K] TN), hC [M][N], all host pointers. B is uploaded once and stays resident; A and C move
 * in M-shards of plan->shard_rows rows (0: the whole of M in one shard) through two pinned
 * buffers each on two streams, so the copies of one shard overlap the kernel of the other. plan
 * NULL: solved against hcs_json (NULL: the built-in MI355X description), which picks the shard
 * height when the working set exceeds the device tier. Device and pinned buffers are allocated
 * per call (the residency check applies to each). *pass_ms: the pass, first copy to last. */
int uk_stream_gemm(const char* hcs_json, const uk_op_desc* d, const uk_plan* plan, const void* hA, const void* hB,
                   void* hC, double* pass_ms);
/* Scenario B's mapped path (reference src/codegen_hip.cpp:1239-1326, uk_stream_pass_mmap): the
 * same GEMM with A on disk. a_path names a file holding A [M][K] row-major in the GEMM's element
 * type (f16 bits or f32), no header; hB and hC are host memory as for uk_stream_gemm. Per shard
 * the host reads A's rows from the file into one of two host-mapped, coherent pinned staging
 * buffers (the other still being read by the previous shard's kernel) and the kernel reads them
 * through the mapped device pointer: no copy of A to the device runs, so A's bytes cross the link
 * once per workgroup that consumes them, and A's host footprint is the two staging buffers. The
 * shard height is plan->shard_rows as in uk_stream_gemm (plan NULL: solved against hcs_json).
 * Refused (class 2) when the file is shorter than M K elements. *pass_ms: the pass. */
int uk_stream_gemm_file(const char* hcs_json, const uk_op_desc* d, const uk_plan* plan, const char* a_path,
                        const void* hB, void* hC, double* pass_ms);
/* The UNIKERN_RESULT line for a result (reference src/codegen_hip.cpp:1710-1722 tokens + roofline). */
int uk_format_result(const uk_result* r, char* line, size_t cap);
/* Parse the output of one program run into a result (reference run_hip's parse,
 * src/runner.cpp:195-237): the UNIKERN_RESULT line's verify, max_rel, measured_ms, kernel_ms,
 * migrations, checks, vram_free and vram_total; without a result line, the tokens of an
 * "UNIKERN_ERROR what=oversubscription" line. Absent migrations/checks stay -1. built and ran
 * are set, exit_code is the given one. Returns 0, or 2 when neither line is present. */
int uk_parse_result(const char* program_output, int32_t exit_code, uk_result* out);
/* The alarm criterion of a run's residency report (reference migration_rate_violation,
 * src/runner.cpp:240-255): 1 when migrations / checks > threshold, or when migrations > 0 with
 * no denominator (checks <= 0, rate 1.0); 0 otherwise (rate 0 when migrations <= 0). */
int uk_migration_alarm(int32_t migrations, int32_t checks, double threshold, double* rate);
/* Exit class of one allocation's residency probe (reference uk_resident,
 * src/codegen_hip.cpp:256-280): probe_status is the hipError_t of hipPointerGetAttributes,
 * memory_type its hipMemoryType. 4 when the probe failed, 5 when the memory is not device
 * memory (managed or host: oversubscription), 0 when it is device-resident. */
int uk_residency_class(int32_t probe_status, int32_t memory_type);

/* ---- seeded inputs (host memory): SplitMix64 per tensor ---- */
int uk_fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi);
int uk_fill_normal(float* out, size_t n, uint64_t seed, float mu, float sigma);
int uk_f32_to_f16(const float* in, uint16_t* out, size_t n);
int uk_f16_to_f32(const uint16_t* in, float* out, size_t n);
/* Pack N rows x K int8 quants and N x K/32 binary16 scales into Q8_0 blocks (34 B each). */
int uk_q8_0_pack(const int8_t* q, const uint16_t* d, uint8_t* blocks, int32_t N, int32_t K);

/* ---- solution ledger (reference ILedger, include/unikern/components.hpp:83-125; stores
 * src/runtime.cpp:29-176 and src/sqlite_ledger.cpp) ----
 * A path ending in ".jsonl" opens the TAB-separated text ledger, any other path an SQLite
 * database with the reference's schema (src/main.cpp:35-37). Keys are
 * "op_signature|hcs_fingerprint|tree_hash" of a KML text (children included) and an HCS
 * (NULL: the built-in MI355X description). One handle per thread. */
int uk_ledger_open(const char* path, void** ledger);
int uk_ledger_close(void* ledger);
int uk_ledger_key(const char* hcs_json, const char* kml_json, char* out, size_t cap); /* length, or -1 */
/* *hit = 1 and the recorded plan (family, variant, key, tiles; predicted_us = c_ms * 1e3) on a hit. */
int uk_ledger_lookup(void* ledger, const char* hcs_json, const char* kml_json, uk_plan* plan, double* c_ms,
                     double* measured_ms, double* kernel_ms, int32_t* hit);
/* Commit a plan with its measurement (measured_ms = 0 for a solve-only row); all-or-nothing.
 * replayed = 1 marks a measurement parsed from a recorded program output rather than a device
 * run (the CLI's --outcomes): the row is kept, and calibration leaves it out. */
int uk_ledger_commit(void* ledger, const char* hcs_json, const char* kml_json, const uk_plan* plan,
                     double measured_ms, double kernel_ms, int32_t replayed);
int uk_ledger_record_violation(void* ledger, const char* hcs_json, const char* kml_json, double rate,
                               double threshold, int32_t migrations, int32_t checks, uint64_t vram_free);
int uk_ledger_size(void* ledger, int32_t* solutions, int32_t* violations);
/* Measured rows of one HCS fingerprint, for calibration: up to cap rows of
 * (c_ms, measured_ms, kernel_ms); the count is returned. */
int uk_ledger_measured(void* ledger, const char* hcs_fp, double* rows3, int32_t cap);
/* Calibration closure (replaces the reference's calibrate, src/main.cpp:579-652 and
 * src/solver.cpp:194-244, which refits the host link only): the HCS with the three rate constants
 * the solver prices with refitted from this HCS's measured ledger rows, and constants_version + 1.
 *   hbm_bw_gbps  x geometric mean of predicted/kernel-only time over streaming rows;
 *   clock_mhz    x the same over MFMA-bound rows (GEMM, conv), or, with none, x the probe's
 *                sustained clock over the clock the variant efficiencies were fitted at
 *                (probe may be NULL);
 *   link_bw_gbps from a least-squares line copy_ms = latency + bytes / link through the rows'
 *                end-to-end minus kernel-only times (left alone on a unified-memory HCS).
 * detail: one line per refitted constant. 3 when nothing could be fitted. */
int uk_calibrate(const char* hcs_json, void* ledger, const uk_mfma_probe* probe, char* out_json, size_t cap,
                 char* detail, size_t detail_cap);
/* The HCS with its device tier set to `bytes` (re-solve on a measured capacity,
 * reference src/main.cpp:488-515). */
int uk_hcs_with_capacity(const char* hcs_json, uint64_t bytes, char* out_json, size_t cap);

/* ---- GGUF weights (format as read by the reference's probe/phase63_gguf_header.py; no
 * counterpart on the reference's execution path, which has no Q8_0 kernel) ----
 * Reads the header, metadata and tensor directory; Q8_0 tensors [ne0 = K, ne1 = N] are the
 * Q8_0 GEMM's weight layout byte for byte. ggml types: 0 f32, 1 f16, 8 q8_0, 30 bf16. */
int uk_gguf_open(const char* path, void** file);
int uk_gguf_close(void* file);
int32_t uk_gguf_tensor_count(void* file);
int32_t uk_gguf_find(void* file, const char* name); /* index, or -1 */
int uk_gguf_tensor_info(void* file, int32_t index, char* name, size_t cap, int32_t* ggml_type, int32_t* n_dims,
                        int64_t* ne4, uint64_t* file_offset, uint64_t* nbytes);
int uk_gguf_metadata(void* file, const char* key, char* out, size_t cap); /* length, or -1 */
int uk_gguf_read(void* file, int32_t index, void* host_dst, uint64_t cap);
/* Copy a tensor's bytes into device memory (host staging, then one copy). */
int uk_gguf_upload(void* file, int32_t index, void* dev_dst, uint64_t cap);
/* The Q8_0 GEMM of M activation rows against a 2-D Q8_0 tensor: gemm q8_0 TN [M, ne1, ne0]. */
int uk_gguf_q8_0_desc(void* file, int32_t index, int32_t M, uk_op_desc* out);

/* ---- device memory, streams and events (plumbing for callers without a runtime) ---- */
int uk_malloc(void** p, size_t bytes);
int uk_free(void* p);
int uk_memcpy_htod(void* dst, const void* src, size_t bytes);
int uk_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int uk_memset(void* p, int value, size_t bytes);
int uk_synchronize(void);
int uk_stream_create(void** stream);
int uk_stream_destroy(void* stream);
int uk_stream_synchronize(void* stream);
int uk_event_create(void** ev);
int uk_event_destroy(void* ev);
int uk_event_record(void* ev, void* stream);
int uk_event_elapsed_ms(void* start, void* stop, float* ms);

#ifdef __cplusplus
}
#endif
#endif /* UNIKERN_HIP_H */
