// CDNA4 tile/plan selection.
//
// Same contract as the reference's solver (src/solver.cpp:141-186): enumerate a bounded set
// of candidates, drop those that violate a predicate (recording a sample of violations),
// price the rest with a deterministic analytic cost, and take the argmin with ties broken
// by a canonical candidate key, so solve() is a pure function of (hcs, tree).
//
// What changes for MI355X: the candidate set is the table of compiled kernel variants
// (variants.hpp), and the predicates and costs read the CDNA4 description — LDS bytes per
// workgroup and per CU, the VGPR/AGPR budget per lane, MFMA shape divisibility, wavefront
// quantisation of tiles over 256 CUs, bytes in flight for HBM-bound kernels (Little's law)
// and L2/LDS feed rates for MFMA-bound kernels. The reference's predicate is only
// "tile working set <= VRAM" (src/solver.cpp:54-77).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <sstream>

#include "../variants.hpp"
#include "uk_core.hpp"

namespace uk {

namespace {

// Effective DRAM latency seen by a streaming wavefront (issue to data), used to turn bytes in
// flight into sustainable bandwidth.
constexpr double kMemLatencyUs = 1.2;
// L2 -> CU feed budget (bytes per clock per CU) and LDS read bandwidth per CU.
constexpr double kL2BytesPerClkPerCu = 64.0;
constexpr double kLdsBytesPerClkPerCu = 128.0;

struct Cand {
  Plan plan;
  double cost = 0;
};

void reject(SolveLog* log, const std::string& what) {
  if (log && log->rejected.size() < 8) log->rejected.push_back(what);
}

double hbm_gbps(const Hcs& h) {
  if (h.hbm_bw_gbps > 0) return h.hbm_bw_gbps;
  return h.tier_bw(h.unified_memory ? "unified" : "vram");
}
int cus(const Hcs& h) { return h.compute_units > 0 ? h.compute_units : 1; }
int simds(const Hcs& h) { return h.simds_per_cu > 0 ? h.simds_per_cu : 4; }
int max_waves_simd(const Hcs& h) { return h.max_waves_per_simd > 0 ? h.max_waves_per_simd : 8; }
int regs_lane(const Hcs& h) { return h.vgprs_per_lane > 0 ? h.vgprs_per_lane : 512; }
double clock_ghz(const Hcs& h) { return h.clock_mhz > 0 ? h.clock_mhz * 1e-3 : 2.1; }
int64_t lds_cu(const Hcs& h) { return h.lds_bytes_per_cu > 0 ? h.lds_bytes_per_cu : 65536; }
int64_t lds_block(const Hcs& h) { return h.lds_bytes_per_block > 0 ? h.lds_bytes_per_block : lds_cu(h); }
double launch_us(const Hcs& h) { return h.launch_overhead_us > 0 ? h.launch_overhead_us : 2.0; }

// Waves per SIMD that fit the register file (allocation granule of 8 registers).
int waves_by_regs(const Hcs& h, int regs) {
  regs = (regs + 7) / 8 * 8;
  int w = regs_lane(h) / std::max(regs, 8);
  return std::min(std::max(w, 0), max_waves_simd(h));
}

// Streaming time of `bytes` over `grid` workgroups, each keeping `inflight_wg` bytes of loads
// outstanding, with at most `resident_per_cu` workgroups per CU: rounds of resident
// workgroups, each round at min(peak, in-flight bytes / latency).
double stream_us(const Hcs& h, double bytes, int64_t grid, int resident_per_cu, double inflight_wg) {
  const double peak = hbm_gbps(h) * 1e3;  // bytes per microsecond
  const int64_t slots = int64_t(cus(h)) * std::max(resident_per_cu, 1);
  const double per_wg = bytes / double(std::max<int64_t>(grid, 1));
  double t = 0;
  for (int64_t done = 0; done < grid; done += slots) {
    const int64_t active = std::min(slots, grid - done);
    const double bw = std::min(peak, double(active) * inflight_wg / kMemLatencyUs);
    t += double(active) * per_wg / bw;
  }
  return t;
}

std::string fmt(const char* f, double a) {
  char b[64];
  std::snprintf(b, sizeof b, f, a);
  return b;
}

std::optional<Plan> pick(std::vector<Cand>& cs, const char* family_name, std::string* err) {
  if (cs.empty()) {
    if (err) *err = std::string("no feasible ") + family_name + " candidate";
    return std::nullopt;
  }
  const Cand* best = &cs[0];
  for (const Cand& c : cs)
    if (c.cost < best->cost || (c.cost == best->cost && c.plan.key < best->plan.key)) best = &c;
  Plan p = best->plan;
  p.predicted_us = best->cost;
  p.feasible = int(cs.size());
  return p;
}

// ---------------------------------------------------------------------------------------
std::optional<Plan> solve_rows(const Hcs& h, const KmlTree& t, const Shape& s, SolveLog* log, std::string* err) {
  const Workload w = workload_of(t);
  const bool rms = t.op == OpKind::RmsNorm;
  std::vector<Cand> cs;
  for (int i = 0; i < kNumRowsVariants; ++i) {
    const RowsVariant v = kRowsVariants[i];
    const int64_t cap = int64_t(v.tpr) * v.nv * 4;
    std::ostringstream key;
    key << "rows:tpr=" << v.tpr << ",nv=" << v.nv;
    if (s.C % 4 != 0) {
      reject(log, key.str() + " violates C%4==0 (float4 rows), C=" + std::to_string(s.C));
      continue;
    }
    if (s.C > cap) {
      reject(log, key.str() + " violates C<=tpr*nv*4=" + std::to_string(cap));
      continue;
    }
    if (cap >= 4 * s.C && cap > 256) {
      reject(log, key.str() + " violates capacity<4*C (three quarters of the lanes idle)");
      continue;
    }
    const int wg = std::max(v.tpr, 256);
    const int rows_per_wg = wg / v.tpr;
    const int64_t grid = (s.L + rows_per_wg - 1) / rows_per_wg;
    const int regs = v.nv * 4 * (rms ? 2 : 1) + 24;
    const int wps = waves_by_regs(h, regs);
    if (wps == 0) {
      reject(log, key.str() + " violates register budget");
      continue;
    }
    const int resident = std::max(1, (wps * simds(h)) / (wg / 64));
    const double useful = double(s.C) / double(cap);
    const double inflight = double(wg) * v.nv * 16.0 * useful;
    double cost = launch_us(h) + stream_us(h, double(w.bytes), grid, resident, inflight);
    if (v.tpr > 64) cost += 0.05 * (t.op == OpKind::Softmax ? 2 : 1);  // LDS fold + barrier per reduction
    Cand c;
    c.plan.family = Family::Rows;
    c.plan.variant = i;
    c.plan.tpr = v.tpr;
    c.plan.vec = v.nv;
    c.plan.threads = wg;
    c.plan.grid = grid;
    c.plan.key = key.str();
    c.plan.why = "row in registers, " + std::to_string(wps) + " waves/SIMD by registers, " +
                 std::to_string(resident) + " workgroups/CU resident";
    c.cost = cost;
    cs.push_back(c);
  }
  if (!cs.empty()) return pick(cs, "rows", err);
  // Fallback for any row length: stream the row.
  Plan p;
  p.family = Family::RowsStream;
  p.threads = kRowsStreamThreads;
  p.grid = s.L;
  const int passes = t.op == OpKind::Softmax ? 3 : (t.op == OpKind::RmsNorm ? 2 : 1);
  p.predicted_us = launch_us(h) + double(s.L * s.C * 4) * passes / (hbm_gbps(h) * 1e3) + double(s.L * s.C * 4) / (hbm_gbps(h) * 1e3);
  p.feasible = 1;
  p.key = "rows_stream";
  p.why = "row length not register-resident; streamed";
  return p;
}

// ---------------------------------------------------------------------------------------
std::optional<Plan> solve_gemm(const Hcs& h, const KmlTree& t, const Shape& s, SolveLog* log, std::string* err) {
  const double peak_tflops = t.dtype == DType::F16 ? (h.peak_f16_mfma_tflops > 0 ? h.peak_f16_mfma_tflops : h.flops_gflops * 1e-3)
                                                   : (h.peak_f32_mfma_tflops > 0 ? h.peak_f32_mfma_tflops : h.flops_gflops * 1e-3 / 16);
  const double flops = 2.0 * double(s.M) * double(s.N) * double(s.K);
  const double clk = clock_ghz(h) * 1e3;  // clocks per microsecond
  std::vector<Cand> cs;
  if (t.dtype == DType::F16 && t.layout == Layout::TN) {
    for (int i = 0; i < kNumGemmF16Variants; ++i) {
      const GemmF16Variant v = kGemmF16Variants[i];
      std::ostringstream key;
      key << "gemm_f16:" << v.bm << "x" << v.bn << "x" << v.bk << ",w" << v.wm << "x" << v.wn << ",s" << v.stages << ",z" << v.swz;
      if (s.M % v.bm || s.N % v.bn || s.K % v.bk) {
        reject(log, key.str() + " violates M%bm==0 && N%bn==0 && K%bk==0");
        continue;
      }
      const int waves = v.wm * v.wn;
      const int64_t stage_bytes = int64_t(v.bm + v.bn) * v.bk * 2;
      const int64_t epi_bytes = int64_t(waves) * (v.bm / v.wm) * ((v.bn / v.wn) * 2 + 16);
      const int64_t lds = std::max<int64_t>(v.stages * stage_bytes, epi_bytes);
      if (lds > lds_block(h)) {
        reject(log, key.str() + " violates LDS " + std::to_string(lds) + " <= " + std::to_string(lds_block(h)));
        continue;
      }
      const int fm = v.bm / v.wm / 32, fn = v.bn / v.wn / 32;
      const int acc_regs = fm * fn * 16;
      const int regs = acc_regs + (fm + fn) * 8 + 48;
      if (acc_regs > 256 || regs > regs_lane(h)) {
        reject(log, key.str() + " violates accumulator budget (" + std::to_string(acc_regs) + " AGPRs)");
        continue;
      }
      const int wps = waves_by_regs(h, regs);
      const int wg_by_waves = std::max(1, wps * simds(h) / waves);
      const int wg_by_lds = int(lds_cu(h) / lds);
      const int resident = std::max(1, std::min(wg_by_waves, wg_by_lds));
      const int64_t tiles = (s.M / v.bm) * (s.N / v.bn);
      const int64_t slots = int64_t(cus(h)) * resident;
      const int64_t rounds = (tiles + slots - 1) / slots;
      // Per k-tile of one workgroup: MFMA issue cycles on each SIMD, LDS fragment reads and the
      // L2 feed of the A/B panels; the slowest sets the pace, the others partly overlap it.
      const double cu_flops_per_clk = peak_tflops * 1e12 / (double(cus(h)) * clk * 1e6);
      const int wg_on_cu = int(std::min<int64_t>(resident, (tiles + cus(h) - 1) / cus(h)));
      const double k16 = double(v.bk) / 16.0;
      const double mfma_clk = double(wg_on_cu) * double(waves) / simds(h) * fm * fn * k16 *
                              (32768.0 * simds(h) / cu_flops_per_clk);
      const double lds_clk = double(wg_on_cu) * waves * (fm + fn) * 1024.0 * k16 / kLdsBytesPerClkPerCu;
      const double l2_clk = double(wg_on_cu) * double(v.bm + v.bn) * v.bk * 2.0 / kL2BytesPerClkPerCu;
      const double pace = std::max({mfma_clk, lds_clk, l2_clk}) + 0.25 * (lds_clk + l2_clk);
      const double eff = mfma_clk / pace;
      const double tile_flops = 2.0 * v.bm * v.bn * double(s.K);
      const double l2_need = l2_clk;
      // Workgroups resident on one CU share its MFMA pipes: a round lasts as long as the CU
      // with the most tiles takes to finish them.
      const int64_t per_cu = (std::min<int64_t>(tiles, slots) + cus(h) - 1) / cus(h);
      const double per_round_us = double(per_cu) * tile_flops / (cu_flops_per_clk * clk * eff);
      const double epi_us = double(s.M * s.N * 2) / (hbm_gbps(h) * 1e3);
      const double cost = launch_us(h) + double(rounds) * per_round_us + epi_us + 1.0;
      Cand c;
      c.plan.family = Family::GemmF16;
      c.plan.variant = i;
      c.plan.tile_m = v.bm;
      c.plan.tile_n = v.bn;
      c.plan.tile_k = v.bk;
      c.plan.stages = v.stages;
      c.plan.threads = waves * 64;
      c.plan.grid = tiles;
      c.plan.key = key.str();
      c.plan.why = std::to_string(tiles) + " tiles over " + std::to_string(slots) + " slots (" +
                   std::to_string(rounds) + " rounds), MFMA efficiency " + fmt("%.2f", eff) + " (L2 " + fmt("%.0f", l2_need) + " clk per k-tile), LDS " +
                   std::to_string(lds) + " B";
      c.cost = cost;
      cs.push_back(c);
    }
  }
  {
    Cand c;
    c.plan.family = Family::GemmGeneric;
    c.plan.tile_m = c.plan.tile_n = kGemmGenericTile;
    c.plan.tile_k = 16;
    c.plan.threads = 256;
    c.plan.grid = ((s.M + 63) / 64) * ((s.N + 63) / 64);
    c.plan.key = "gemm_generic:64x64x16";
    c.plan.why = "bounds-checked 64x64 MFMA tiles (any shape and layout)";
    c.cost = launch_us(h) + flops / (peak_tflops * 1e6 * 0.12) + 1.0;
    cs.push_back(c);
  }
  return pick(cs, "gemm", err);
}

// ---------------------------------------------------------------------------------------
std::optional<Plan> solve_q8(const Hcs& h, const KmlTree& t, const Shape& s, SolveLog* log, std::string* err) {
  const Workload w = workload_of(t);
  std::vector<Cand> cs;
  const int64_t nblk = s.K / 32;
  for (int i = 0; i < kNumQ8Variants; ++i) {
    const Q8Variant v = kQ8Variants[i];
    std::ostringstream key;
    key << "q8_0:waves=" << v.waves << ",kblocks=" << v.kblocks;
    if (nblk % v.kblocks != 0) {
      reject(log, key.str() + " violates (K/32)%kblocks==0");
      continue;
    }
    const int64_t ksplit = nblk / v.kblocks;          // wavefronts per 16 output columns
    if (ksplit % v.waves != 0 && v.waves % ksplit != 0) {
      reject(log, key.str() + " violates k-split divisibility by waves per workgroup");
      continue;
    }
    const int64_t col_tiles = (s.N + 15) / 16;
    const int64_t m_tiles = (s.M + 15) / 16;
    const int64_t waves_total = col_tiles * ksplit * m_tiles;
    const int64_t grid = (waves_total + v.waves - 1) / v.waves;
    const int regs = 96;
    const int wps = waves_by_regs(h, regs);
    const int resident = std::max(1, wps * simds(h) / v.waves);
    const double inflight = double(v.waves) * v.kblocks * 16 * 34.0;  // a wavefront's weight slice
    const double cost = launch_us(h) + stream_us(h, double(w.bytes), grid, resident, inflight) +
                        (ksplit > v.waves ? 0.5 : 0.1);
    Cand c;
    c.plan.family = Family::Q8Gemm;
    c.plan.variant = i;
    c.plan.threads = v.waves * 64;
    c.plan.split_k = int(ksplit);
    c.plan.grid = grid;
    c.plan.key = key.str();
    c.plan.why = std::to_string(grid) + " workgroups, split-K " + std::to_string(ksplit);
    c.cost = cost;
    cs.push_back(c);
  }
  return pick(cs, "q8_0", err);
}

// ---------------------------------------------------------------------------------------
std::optional<Plan> solve_conv(const Hcs& h, const KmlTree& t, const Shape& s, SolveLog* log, std::string* err) {
  const double peak = h.peak_f32_mfma_tflops > 0 ? h.peak_f32_mfma_tflops : h.flops_gflops * 1e-3 / 16;
  const double flops = double(workload_of(t).ops);
  const int64_t Mpix = s.Nb * s.Ho * s.Wo;
  std::vector<Cand> cs;
  for (int i = 0; i < kNumConvVariants; ++i) {
    const ConvVariant v = kConvVariants[i];
    std::ostringstream key;
    key << "conv_igemm:" << v.bm << "x" << v.bn << "x" << v.bk << ",w" << v.waves;
    const int64_t tiles = ((Mpix + v.bm - 1) / v.bm) * ((s.Co + v.bn - 1) / v.bn);
    const int64_t lds = int64_t(v.bm + v.bn) * v.bk * 4 * 2;
    if (lds > lds_block(h)) {
      reject(log, key.str() + " violates LDS");
      continue;
    }
    const int resident = std::max(1, std::min(int(lds_cu(h) / lds), 8 * simds(h) / v.waves));
    const int64_t slots = int64_t(cus(h)) * resident;
    const int64_t rounds = (tiles + slots - 1) / slots;
    // MFMA work per workgroup lands on `waves` SIMDs; balance = tiles spread over CUs x SIMDs.
    const double simd_slots = double(cus(h)) * simds(h);
    const double waves_total = double(tiles) * v.waves;
    const double per_simd = std::ceil(waves_total / simd_slots);
    const double balance = waves_total / (per_simd * simd_slots);
    const double pad_eff = double(Mpix) / double(((Mpix + v.bm - 1) / v.bm) * v.bm) *
                           double(s.Co) / double(((s.Co + v.bn - 1) / v.bn) * v.bn);
    const double cost = launch_us(h) + flops / (peak * 1e6 * 0.7 * balance * pad_eff) + 0.5 * double(rounds > 1);
    Cand c;
    c.plan.family = Family::ConvIgemm;
    c.plan.variant = i;
    c.plan.tile_m = v.bm;
    c.plan.tile_n = v.bn;
    c.plan.tile_k = v.bk;
    c.plan.threads = v.waves * 64;
    c.plan.grid = tiles;
    c.plan.key = key.str();
    c.plan.why = std::to_string(tiles) + " tiles, SIMD balance " + fmt("%.2f", balance);
    c.cost = cost;
    cs.push_back(c);
  }
  return pick(cs, "conv", err);
}

}  // namespace

std::optional<Plan> solve(const Hcs& h, const KmlTree& t, SolveLog* log, std::string* err) {
  if (const std::string gap = support_gap(t); !gap.empty()) {
    if (err) *err = gap;
    return std::nullopt;
  }
  const Shape s = shape_of(t);
  switch (t.op) {
    case OpKind::Gemm:
      if (t.dtype == DType::Q8_0) return solve_q8(h, t, s, log, err);
      return solve_gemm(h, t, s, log, err);
    case OpKind::Conv: return solve_conv(h, t, s, log, err);
    case OpKind::Reduction:
      if (t.ndims == 1) {
        Plan p;
        p.family = Family::Reduce1D;
        p.threads = kReduceThreads;
        p.grid = kReduceParts;
        p.predicted_us = 2 * launch_us(h) + double(workload_of(t).bytes) / (hbm_gbps(h) * 1e3);
        p.feasible = 1;
        p.key = "reduce1d:parts=" + std::to_string(kReduceParts);
        p.why = "two deterministic passes (partials, one-workgroup fold)";
        return p;
      }
      return solve_rows(h, t, s, log, err);
    case OpKind::Softmax:
    case OpKind::RmsNorm: return solve_rows(h, t, s, log, err);
    case OpKind::ChannelScale: {
      Plan p;
      p.family = Family::ChannelScale;
      p.threads = 256;
      p.grid = std::min<int64_t>((s.L * s.C / 4 + 255) / 256, 256 * 32);
      p.predicted_us = launch_us(h) + double(workload_of(t).bytes) / (hbm_gbps(h) * 1e3);
      p.feasible = 1;
      p.key = "channelscale:grid_stride";
      p.why = "elementwise float4 grid-stride";
      return p;
    }
  }
  if (err) *err = "unknown op";
  return std::nullopt;
}

}  // namespace uk
