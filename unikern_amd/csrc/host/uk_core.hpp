// Core types of the MI355X kernel hot path: the KML op spec, the hardware description,
// the plan the solver picks, and the workload model.
//
// The op surface follows the reference's KmlTree (include/unikern/core.hpp:11-31); the
// hardware description follows its Hcs (core.hpp:44-63) plus CDNA4 fields.
#pragma once
#include <cstdint>
#include <optional>
#include <string>
#include <vector>

namespace uk {

// Same order as the reference's OpKind (include/unikern/core.hpp:11).
enum class OpKind : int { Gemm = 0, Conv = 1, Reduction = 2, Softmax = 3, RmsNorm = 4, ChannelScale = 5 };
// Reference DType (core.hpp:12) plus q8_0: GGUF 34-byte blocks {f16 d; int8 qs[32]}.
enum class DType : int { F32 = 0, F16 = 1, I8 = 2, Q8_0 = 3 };
// Layout tags. NT is the reference's only tag (src/codegen_hip.cpp:70): A[M][K], B[K][N],
// C[M][N] row-major; for conv it is the reference's HWC/valid semantics (src/reference.cpp:6-22).
// TN: A[M][K] row-major and B column-major, i.e. stored [N][K] (both operands K-contiguous).
// NCHW: batched conv, X[N][C][H][W], W[Oc][C][Kh][Kw], Y[N][Oc][Ho][Wo], zero padding.
enum class Layout : int { NT = 0, TN = 1, NCHW = 2 };
enum class Epilogue : int { None = 0, ChannelScale = 1 };

const char* to_string(OpKind k);
const char* to_string(DType d);
const char* to_string(Layout l);
const char* to_string(Epilogue e);
std::optional<OpKind> op_from_string(const std::string& s);
std::optional<DType> dtype_from_string(const std::string& s);
std::optional<Layout> layout_from_string(const std::string& s);
size_t dtype_size(DType d);  // bytes per element (q8_0: 34 bytes per 32 elements -> reported as 1)

struct KmlTree {
  OpKind op = OpKind::Gemm;
  DType dtype = DType::F32;
  int ndims = 3;
  int dims[6] = {4096, 4096, 4096, 0, 0, 0};
  int tile_m = 64;  // reference defaults (core.hpp:27-28)
  int tile_n = 128;
  Layout layout = Layout::NT;
  // extensions (absent from reference files; defaults reproduce reference semantics)
  int batch = 1;
  int pad = 0;
  int stride = 1;
  Epilogue epilogue = Epilogue::None;
  float eps = 1e-6f;  // rmsnorm; the reference hard-codes 1e-6f (src/codegen_hip.cpp:2162)
  bool has_eps = false;
  std::vector<KmlTree> children;
};

// Derived shape of a tree, resolved once for every consumer.
struct Shape {
  // gemm
  int64_t M = 0, N = 0, K = 0;
  // 2-D row ops and reduce: rows x cols (1-D reduce: rows = 1)
  int64_t L = 0, C = 0;
  // conv
  int64_t Nb = 1, Ci = 0, H = 0, W = 0, Co = 0, Kh = 0, Kw = 0, Ho = 0, Wo = 0, pad = 0, stride = 1;
};
Shape shape_of(const KmlTree& t);

struct Workload {
  int64_t ops = 0;           // algorithmic arithmetic (FLOP; adds for reductions)
  int64_t bytes = 0;         // compulsory HBM bytes (read once + write once)
  int64_t weight_bytes = 0;  // q8_0 only: the streamed weight bytes the metric is quoted on
};
Workload workload_of(const KmlTree& t);

// ---------------------------------------------------------------------------
// Hardware description (reference Hcs, include/unikern/core.hpp:44-63, plus CDNA4).
// ---------------------------------------------------------------------------
enum class Confidence : int { Official = 3, Measured = 2, Predicted = 1 };
struct StorageTier {
  std::string name;
  int64_t bytes = 0;
  double bw_gbps = 0;
  Confidence confidence = Confidence::Official;
};
struct MfmaShape {
  std::string name;  // e.g. "f32_32x32x16_f16"
  std::string in;    // "fp16", "fp32", ...
  int m = 0, n = 0, k = 0;
  int cycles = 0;    // issue-to-issue cycles on one SIMD
};
struct Hcs {
  // reference fields
  std::string vendor, device, toolchain;
  bool unified_memory = false;
  std::vector<StorageTier> tiers;
  double link_bw_gbps = 0, flops_gflops = 0;
  int compute_units = 0;
  Confidence confidence = Confidence::Official;
  int constants_version = 1;
  // CDNA4 fields (zero/empty when the file does not declare them)
  std::string arch;
  int wave_size = 0, simds_per_cu = 0, xcds = 0, max_waves_per_simd = 0;
  int vgprs_per_lane = 0;          // VGPR+AGPR budget of one lane at one wave per SIMD
  int64_t lds_bytes_per_cu = 0, lds_bytes_per_block = 0;
  int64_t l2_bytes_per_xcd = 0, mall_bytes = 0;
  double clock_mhz = 0, hbm_bw_gbps = 0;
  double peak_f16_mfma_tflops = 0, peak_f32_mfma_tflops = 0, peak_f32_valu_tflops = 0;
  double launch_overhead_us = 0;   // per-dispatch gap between back-to-back launches
  std::vector<MfmaShape> mfma;

  int64_t tier_bytes(const std::string& name) const;
  double tier_bw(const std::string& name) const;
  int64_t device_capacity() const;
  bool cdna4() const { return !arch.empty(); }
};

std::optional<Hcs> hcs_import(const std::string& json, std::string* err);
std::string hcs_export(const Hcs& h);
std::string hcs_fingerprint(const Hcs& h);
const Hcs& hcs_mi355x();          // built-in description of one MI355X (samples/hcs_mi355x.json)
const char* hcs_mi355x_json();

// ---------------------------------------------------------------------------
// KML front end (reference src/kml_front.cpp, src/kml.cpp).
// ---------------------------------------------------------------------------
std::optional<KmlTree> kml_import(const std::string& json, std::string* err);
std::string kml_export(const KmlTree& t);
std::string canonical_form(const KmlTree& t);
std::string op_signature(const KmlTree& t);
std::string fnv1a_hex(const std::string& data);
std::optional<KmlTree> tree_from_signature(const std::string& sig);  // inverse of op_signature
int kml_arity_min(OpKind op);
int kml_arity_max(OpKind op);
const char* kml_dim_spec(OpKind op);
// Capability gate (reference src/codegen_hip.cpp:81-130): empty = the kernels cover the tree.
std::string support_gap(const KmlTree& t);

// ---------------------------------------------------------------------------
// Plans (solver output) and kernel families.
// ---------------------------------------------------------------------------
enum class Family : int {
  None = 0,
  Rows = 1,          // row-sum / rmsnorm / softmax, row held in registers
  RowsStream = 2,    // same ops, any row length, row streamed twice
  ChannelScale = 3,  // standalone elementwise channelscale
  Reduce1D = 4,      // scalar sum, two deterministic passes
  GemmF16 = 5,       // MFMA f16 GEMM, LDS-staged, f32 accumulate
  GemmGeneric = 6,   // MFMA GEMM for any shape/layout (f16 or f32)
  ConvIgemm = 7,     // implicit-GEMM conv on f32 MFMA, fused channelscale
  Q8Gemm = 8,        // Q8_0 skinny GEMM (in-kernel dequant, MFMA f16, f32 accumulate)
  ConvDirect = 9,    // reference-semantics HWC valid conv (any shape)
};
const char* to_string(Family f);

struct Plan {
  Family family = Family::None;
  int variant = 0;      // index into the family's compiled variant table
  int tile_m = 0, tile_n = 0, tile_k = 0;
  int threads = 0;      // threads per workgroup
  int tpr = 0;          // rows family: threads per row
  int vec = 0;          // rows family: float4 per thread
  int split_k = 1;
  int stages = 1;
  int64_t grid = 0;     // workgroups per launch
  double predicted_us = 0;
  int feasible = 0;     // |X|, candidates that passed the predicates
  int shard_rows = 0;   // > 0: scenario B, the GEMM streams A and C through pinned host memory in
                        // M-shards of this many rows with B resident (0: everything resident)
  int stream_path = 0;  // scenario B's path for A: 1 pinned copies, 2 host-mapped staging read by
                        // the kernel (0 when resident)
  std::string key;      // canonical candidate key (tie-break)
  std::string why;      // one-line account of the choice
};

struct SolveLog {
  std::vector<std::string> rejected;                // violated predicates (sample)
  std::vector<std::pair<double, std::string>> ranked;  // feasible candidates ("key family=F variant=N") by predicted us
};
std::optional<Plan> solve(const Hcs& h, const KmlTree& t, SolveLog* log, std::string* err);

}  // namespace uk
