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

#define UK_ABI_VERSION 1

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
} uk_result;

/* ---- library / device ---- */
int uk_abi_version(void);
/* 0 when device 0 reports a gcnArchName starting with gfx950; writes the name. */
int uk_device_check(char* arch, size_t cap);
/* Measured device facts: compute units, max LDS per workgroup, clock (kHz), total bytes. */
int uk_device_props(int32_t* cus, int32_t* lds_per_block, int32_t* clock_khz, uint64_t* total_bytes);
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
int uk_solve(const char* hcs_json, const uk_op_desc* d, uk_plan* out, char* log, size_t cap);

/* ---- execution ----
 * uk_launch: enqueue the op on `stream` over caller-owned device buffers.
 *   gemm f32/f16:  in[0]=A, in[1]=B (layout NT: [K][N]; TN: [N][K]); out=C [M][N] (same dtype)
 *   gemm q8_0 TN:  in[0]=X f16 [M][K], in[1]=W blocks (N rows of K/32 blocks); out=Y f32 [M][N]
 *   conv NT:       in[0]=X [H][W][C], in[1]=Wt [Oc][Kh][Kw][C] (, in[2]=scale[Oc]); out=Y [Oc][Ho][Wo]
 *   conv NCHW:     in[0]=X [N][C][H][W], in[1]=W [Oc][C][Kh][Kw] (, in[2]=scale[Oc]); out=Y [N][Oc][Ho][Wo]
 *   reduce [L]:    in[0]=X; out=Y[1]           reduce [L,C]: in[0]=X; out=Y[L] (row sums)
 *   softmax:       in[0]=X; out=Y               rmsnorm: in[0]=X, in[1]=W[C]; out=Y
 *   channelscale:  in[0]=X, in[1]=S[C]; out=Y
 * plan may be NULL (solved against the built-in MI355X description). */
int uk_launch(const uk_op_desc* d, const uk_plan* plan, const void* const* in, int32_t n_in, void* out,
              void* stream);
/* Enqueue `iters` launches, launch i reading set (i % n_sets): in_sets[s*n_in + j], out_sets[s]. */
int uk_launch_n(const uk_op_desc* d, const uk_plan* plan, const void* const* in_sets, int32_t n_in,
                void* const* out_sets, int32_t n_sets, int32_t iters, void* stream);
/* Verify + time + report, the contract of one emitted reference program: seeded inputs
 * (base seed `seed`), GPU result checked against a CPU reference, kernel timed over rotating
 * device-resident buffer sets. Returns the exit-code class. */
int uk_run(const char* hcs_json, const uk_op_desc* d, const uk_plan* plan, uint64_t seed, int32_t input_mode,
           int32_t timing_iters, uk_result* out, char* log, size_t cap);
/* The UNIKERN_RESULT line for a result (reference src/codegen_hip.cpp:1710-1722 tokens + roofline). */
int uk_format_result(const uk_result* r, char* line, size_t cap);

/* ---- seeded inputs (host memory): SplitMix64 per tensor ---- */
int uk_fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi);
int uk_fill_normal(float* out, size_t n, uint64_t seed, float mu, float sigma);
int uk_f32_to_f16(const float* in, uint16_t* out, size_t n);
int uk_f16_to_f32(const uint16_t* in, float* out, size_t n);
/* Pack N rows x K int8 quants and N x K/32 binary16 scales into Q8_0 blocks (34 B each). */
int uk_q8_0_pack(const int8_t* q, const uint16_t* d, uint8_t* blocks, int32_t N, int32_t K);

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
