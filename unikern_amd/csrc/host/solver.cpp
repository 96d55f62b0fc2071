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
// flight into sustainable bandwidth, and the fraction of the HBM peak a streaming kernel
// sustains on MI355X (a device-to-device copy reaches 5.05-5.37 TB/s of 8 TB/s). Both were
// calibrated on the device against the row-family variant sweep at 4096 x 4096.
constexpr double kMemLatencyUs = 2.0;
constexpr double kStreamEff = 0.72;
// Streams whose loads and stores carry the non-temporal hint sustain more of the peak (row
// family sweep at 4096 x 4096: +1.5% to +5.8% over the same geometry without the hint).
constexpr double kStreamEffNt = 0.75;
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

// The matrix cores are priced at clock_mhz. The published MFMA peak is quoted at the clock the
// HCS's MFMA table implies (CUs x SIMDs x FLOP per cycle of its fastest f16 shape); the ratio of
// the two scales every MFMA-bound prediction, so a calibrated clock moves them all.
double mfma_clock_scale(const Hcs& h) {
  double flop_per_cycle = 0;
  for (const MfmaShape& m : h.mfma)
    if (m.in == "fp16" && m.cycles > 0) flop_per_cycle = std::max(flop_per_cycle, 2.0 * m.m * m.n * m.k / m.cycles);
  if (flop_per_cycle <= 0 || h.peak_f16_mfma_tflops <= 0 || h.clock_mhz <= 0) return 1.0;
  const double nominal_mhz = h.peak_f16_mfma_tflops * 1e6 / (double(cus(h)) * simds(h) * flop_per_cycle);
  return h.clock_mhz / nominal_mhz;
}

// Waves per SIMD that fit the register file (allocation granule of 8 registers).
int waves_by_regs(const Hcs& h, int regs) {
  regs = (regs + 7) / 8 * 8;
  int w = regs_lane(h) / std::max(regs, 8);
  return std::min(std::max(w, 0), max_waves_simd(h));
}

// Streaming time of `bytes` over `grid` workgroups, each keeping `inflight_wg` bytes of loads
// outstanding, with at most `resident_per_cu` workgroups per CU (Little's law: sustained
// bandwidth = bytes in flight / latency, capped at the sustainable peak).
double stream_us(const Hcs& h, double bytes, int64_t grid, int resident_per_cu, double inflight_wg,
                 bool nontemporal = false, double calibrated_eff = 0.0, double latency_us = kMemLatencyUs) {
  const double eff = calibrated_eff > 0 ? calibrated_eff : (nontemporal ? kStreamEffNt : kStreamEff);
  const double peak = hbm_gbps(h) * 1e3 * eff;  // bytes per microsecond
  const int64_t slots = int64_t(cus(h)) * std::max(resident_per_cu, 1);
  const int64_t active = std::min(slots, std::max<int64_t>(grid, 1));
  const double bw = std::min(peak, double(active) * inflight_wg / latency_us);
  // Workgroups that retire while others load let reads and writes overlap; a grid that fits in
  // one round of resident workgroups loads everything first and writes everything last.
  const double rounds = double(std::max<int64_t>(grid, 1)) / double(slots);
  // A calibrated efficiency was measured on a full grid and already carries this effect.
  const double overlap = calibrated_eff > 0 ? 1.0 : 1.0 - 0.08 / std::max(rounds, 1.0);
  return bytes / (bw * overlap);
}

std::string fmt(const char* f, double a) {
  char b[64];
  std::snprintf(b, sizeof b, f, a);
  return b;
}

std::optional<Plan> pick(std::vector<Cand>& cs, const char* family_name, SolveLog* log, std::string* err) {
  if (cs.empty()) {
    if (err) *err = std::string("no feasible ") + family_name + " candidate";
    return std::nullopt;
  }
  const Cand* best = &cs[0];
  for (const Cand& c : cs)
    if (c.cost < best->cost || (c.cost == best->cost && c.plan.key < best->plan.key)) best = &c;
  if (log) {
    for (const Cand& c : cs)
      log->ranked.emplace_back(c.cost, std::string(c.plan.key) + " family=" + std::to_string(int(c.plan.family)) +
                                           " variant=" + std::to_string(c.plan.variant));
    std::sort(log->ranked.begin(), log->ranked.end());
  }
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
    key << "rows:tpr=" << v.tpr << ",nv=" << v.nv << (v.nt ? ",nt" : "");
    if (v.rpb > 1) key << ",rpb=" << v.rpb;
    if (v.grp) key << ",grp";
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
    // Grouped stores were measured at full rows only; with half of each row's lanes idle the
    // one-wavefront rows ran slower than the walking variants (RMSNorm 8192 x 2048: 24.3 against
    // 23.3-24.1 us).
    if (v.grp && cap >= 2 * s.C) {
      reject(log, key.str() + " violates capacity<2*C (grouped stores with half the lanes idle)");
      continue;
    }
    const int wg = std::max(v.tpr, 256);
    const int rows_per_wg = wg / v.tpr * v.rpb;
    const int64_t grid = (s.L + rows_per_wg - 1) / rows_per_wg;
    // Registers per lane: the row (two with a walk), the gain unless it is staged in LDS.
    const int regs = v.nv * 4 * ((rms && !v.grp ? 1 : 0) + (v.rpb > 1 ? 2 : 1)) + 24;
    const int wps = waves_by_regs(h, regs);
    if (wps == 0) {
      reject(log, key.str() + " violates register budget");
      continue;
    }
    const int resident = std::max(1, (wps * simds(h)) / (wg / 64));
    const double useful = double(s.C) / double(cap);
    // A walking workgroup keeps its next row in flight while it reduces the current one.
    const double inflight = double(wg) * v.nv * 16.0 * useful * (v.rpb > 1 ? 1.5 : 1.0);
    const double eff = t.op == OpKind::Softmax ? v.eff_softmax : (rms ? v.eff_rms : v.eff_sum);
    double cost = launch_us(h) + stream_us(h, double(w.bytes), grid, resident, inflight, v.nt != 0, eff);
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
  if (!cs.empty()) return pick(cs, "rows", log, err);
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
constexpr double kGemmF32Eff = 0.72;  // gemm_f32_kernel's fraction of the f32 MFMA rate (calibrated at 1024^3)

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
      key << "gemm_f16:" << v.bm << "x" << v.bn << "x" << v.bk << ",w" << v.wm << "x" << v.wn << ",s" << v.stages << ",z" << v.swz
          << (v.pp == 1   ? ",pp"
              : v.pp == 2 ? ",w4"
              : v.pp == 3 ? ",w4s"
              : v.pp == 4 ? ",w4k"
              : v.pp == 5 ? ",w4k16"
              : v.pp == 6 ? ",w8k16"
                          : "");
      if (s.M % v.bm || s.N % v.bn || s.K % v.bk) {
        reject(log, key.str() + " violates M%bm==0 && N%bn==0 && K%bk==0");
        continue;
      }
      const int waves = v.wm * v.wn;
      const int64_t stage_bytes = int64_t(v.bm + v.bn) * v.bk * 2;
      const int64_t epi_bytes = int64_t(waves) * (v.bm / v.wm) * ((v.bn / v.wn) * 2 + 16);
      // The 64-deep kernels (pp = 4, 5, 6) keep five operand slots: two for A, three for B.
      const int64_t ring = v.pp >= 4 ? 5 * int64_t(v.bm) * v.bk * 2 : v.stages * stage_bytes;
      const int64_t lds = std::max<int64_t>(ring, epi_bytes);
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
      // L2 feed of the A/B panels bound the pace from below (the model's feasibility check); the
      // sustained efficiency is the variant's calibrated one, capped by that bound.
      const double cu_flops_per_clk = peak_tflops * 1e12 / (double(cus(h)) * clk * 1e6);
      const int wg_on_cu = int(std::min<int64_t>(resident, (tiles + cus(h) - 1) / cus(h)));
      const double k16 = double(v.bk) / 16.0;
      const double mfma_clk = double(wg_on_cu) * double(waves) / simds(h) * fm * fn * k16 *
                              (32768.0 * simds(h) / cu_flops_per_clk);
      const double lds_clk = double(wg_on_cu) * waves * (fm + fn) * 1024.0 * k16 / kLdsBytesPerClkPerCu;
      const double l2_clk = double(wg_on_cu) * double(v.bm + v.bn) * v.bk * 2.0 / kL2BytesPerClkPerCu;
      const double bound = mfma_clk / std::max({mfma_clk, lds_clk, l2_clk});
      const double eff = std::min(bound, v.eff);
      const double tile_flops = 2.0 * v.bm * v.bn * double(s.K);
      const double l2_need = l2_clk;
      // Workgroups resident on one CU share its MFMA pipes: a round lasts as long as the CU
      // with the most tiles takes to finish them.
      const int64_t per_cu = (std::min<int64_t>(tiles, slots) + cus(h) - 1) / cus(h);
      const double per_round_us = double(per_cu) * tile_flops / (cu_flops_per_clk * clk * eff * mfma_clock_scale(h));
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
  if (t.dtype == DType::F32) {
    const std::string key = "gemm_f32:64x64x64,w8";
    if (!(s.M % 64 == 0 && s.N % 64 == 0 && s.K % 64 == 0)) {
      reject(log, key + " violates M%64==0 && N%64==0 && K%64==0");
    } else {
      // One 64x64 tile per workgroup, eight wavefronts (two per SIMD, splitting each k-tile):
      // the busiest CU's tiles at the calibrated fraction of its f32 MFMA rate.
      const int64_t tiles = (s.M / 64) * (s.N / 64);
      const double cu_flops_per_us = peak_tflops * 1e6 / double(cus(h));
      const double per_cu = std::ceil(double(tiles) / cus(h));
      Cand c;
      c.plan.family = Family::GemmGeneric;
      c.plan.variant = 1;
      c.plan.tile_m = c.plan.tile_n = c.plan.tile_k = 64;
      c.plan.threads = 512;
      c.plan.grid = tiles;
      c.plan.key = key;
      c.plan.why = std::to_string(tiles) + " tiles of 64x64, k-tiles of 64 copied into LDS one ahead, split over two wavefronts per SIMD";
      c.cost = launch_us(h) +
               per_cu * 2.0 * 64 * 64 * double(s.K) / (cu_flops_per_us * kGemmF32Eff * mfma_clock_scale(h)) + 1.0;
      cs.push_back(c);
    }
  }
  {
    Cand c;
    c.plan.family = Family::GemmGeneric;
    c.plan.variant = 0;
    c.plan.tile_m = c.plan.tile_n = kGemmGenericTile;
    c.plan.tile_k = 16;
    c.plan.threads = 256;
    c.plan.grid = ((s.M + 63) / 64) * ((s.N + 63) / 64);
    c.plan.key = "gemm_generic:64x64x16";
    c.plan.why = "bounds-checked 64x64 MFMA tiles (any shape and layout)";
    // Measured at the BASELINE shapes (element-wise staging, one 64x64 tile per workgroup):
    // 1.5% of the f16 MFMA peak at 4096^3, 9% of the f32 peak at 1024^3.
    const double eff = t.dtype == DType::F16 ? 0.016 : 0.09;
    c.cost = launch_us(h) + flops / (peak_tflops * 1e6 * eff * mfma_clock_scale(h)) + 1.0;
    cs.push_back(c);
  }
  return pick(cs, "gemm", log, err);
}

// ---------------------------------------------------------------------------------------
constexpr double kActBytesPerUsPerCu = 100e3;  // activation bytes per us per CU (fitted)
// Loaded latency of a Q8_0 weight copy: a wavefront's data lands about 0.8 us after its last copy
// issued, in a timeline of one launch at N = 4096 (the copies queue behind each other, so the
// row family's 2 us figure, which covers a cold start, overstates it here).
constexpr double kQ8LatencyUs = 1.0;

std::optional<Plan> solve_q8(const Hcs& h, const KmlTree& t, const Shape& s, SolveLog* log, std::string* err) {
  const Workload w = workload_of(t);
  std::vector<Cand> cs;
  const int64_t npairs = s.K / 64;
  for (int i = 0; i < kNumQ8Variants; ++i) {
    const Q8Variant v = kQ8Variants[i];
    if (v.gemv) {
      // One weight row per wavefront (M = 1): the weight stream in whole rows, the activation row
      // read from L2 once per workgroup, and the last row's vector-ALU reduction after it lands.
      const std::string key = "q8_0:gemv,waves=" + std::to_string(v.waves);
      const int64_t lds = int64_t(v.waves) * 17 * 64 * 4 + 64 * 128;
      if (s.M != 1) {
        reject(log, key + " violates M==1");
        continue;
      }
      if (s.K % 256 != 0 || npairs > 64) {
        reject(log, key + " violates K%256==0 && K<=4096");
        continue;
      }
      if (lds > lds_block(h)) {
        reject(log, key + " violates LDS " + std::to_string(lds) + " <= " + std::to_string(lds_block(h)));
        continue;
      }
      const int64_t grid = (s.N + v.waves - 1) / v.waves;
      const int resident =
          std::max(1, std::min<int>(waves_by_regs(h, 64) * simds(h) / v.waves, int(lds_cu(h) / lds)));
      const double inflight = double(v.waves) * double(npairs) * 68.0;
      const double stream = stream_us(h, double(w.bytes), grid, resident, inflight, false, 0.0, kQ8LatencyUs);
      const double act_cu = std::ceil(double(grid) / cus(h)) * double(s.K) * 2.0;
      // The last wavefront's reduction (about 170 vector instructions per lane per 64 pairs, a
      // quarter of a latency at K = 4096) runs after its row lands.
      const double tail_us = 0.25 * kQ8LatencyUs;
      Cand c;
      c.plan.family = Family::Q8Gemm;
      c.plan.variant = i;
      c.plan.threads = v.waves * 64;
      c.plan.split_k = 1;
      c.plan.tile_k = int(s.K);
      c.plan.grid = grid;
      c.plan.key = key;
      c.plan.why = std::to_string(grid) + " workgroups of " + std::to_string(v.waves) +
                   " weight rows (one per wavefront), vector-ALU dot products, " + std::to_string(resident) +
                   " resident per CU";
      c.cost = launch_us(h) + stream + act_cu / kActBytesPerUsPerCu + tail_us;
      cs.push_back(c);
      continue;
    }
    std::ostringstream key;
    key << "q8_0:waves=" << v.waves << ",pairs=" << v.pairs << ",vec=" << v.vec << (v.db ? ",db" : "");
    if (v.nt > 1) key << ",nt=" << v.nt;
    const int64_t lds = int64_t(v.waves) * v.nt * v.pairs * 16 * 17 * 4 * (v.db ? 2 : 1);
    if (v.vec == 4 && s.K % (64 * v.pairs) != 0) {
      reject(log, key.str() + " violates K%(64*pairs)==0 (16-byte aligned copies)");
      continue;
    }
    if (lds > lds_block(h)) {
      reject(log, key.str() + " violates LDS " + std::to_string(lds) + " <= " + std::to_string(lds_block(h)));
      continue;
    }
    const int64_t per_round = int64_t(v.waves) * v.pairs;
    const int64_t rounds = (npairs + per_round - 1) / per_round;
    // Pairs of the last round beyond K/64 re-copy pair 0 of the same rows and are skipped: those
    // copies hit in L2 and cost issue, not HBM bytes (charged as HBM bytes, the 16-wavefront
    // kernel was priced 1.4-1.7x its measured time at K = 4608-6144 and lost picks it wins).
    const double useful = double(npairs) / double(rounds * per_round);
    const int64_t grid = ((s.N + 16 * v.nt - 1) / (16 * v.nt)) * ((s.M + 15) / 16);
    // VGPRs per lane: activation fragments (8 per pair, twice with double buffering) and the
    // accumulators of each weight tile on a fixed base (the compiled variants use 70-133).
    const int regs = 40 + 10 * v.pairs * (v.db ? 2 : 1) + 16 * (v.nt - 1);
    const int wps = waves_by_regs(h, regs);
    const int resident = std::max(1, std::min<int>(wps * simds(h) / v.waves, int(lds_cu(h) / lds)));
    // Bytes in flight per workgroup: one round of copies (two with double buffering).
    const double inflight = double(per_round) * 16.0 * v.nt * 68.0 * useful * (v.db && rounds > 1 ? 2.0 : 1.0);
    // Copy instructions: 16-byte copies issue a quarter of the dword ones.
    const double issue_us = double(rounds) * (v.vec == 4 ? 0.1 : 0.4);
    // Each generation of resident workgroups waits one load latency before its first round
    // lands and folds its split-K partials after its last. Only the first generation's wait is
    // exposed whole: the CUs reach their later generations at different times, so a later one's
    // wait overlaps the other CUs' streams and a quarter of it shows (fitted over the Q8_0 sweep
    // of 20 shapes: any share from 0.1 to 0.3 gives the same picks; the whole wait for every
    // generation took a tile kernel of three or four 16-row tiles per workgroup 8-18% slower than
    // the 16-wavefront one at long-K single rows).
    const int64_t slots = int64_t(cus(h)) * resident;
    const int64_t generations = (grid + slots - 1) / slots;
    const double gen_us = (1.0 + 0.25 * double(generations - 1)) * 0.25 * kMemLatencyUs;
    // Every workgroup reads its activation rows over all of K (from L2); the n-tiles of a
    // workgroup share each activation fragment: the busiest CU's activation bytes.
    const double act_cu = std::ceil(double(grid) / cus(h)) * double(std::min<int64_t>(s.M, 16)) * double(s.K) * 2.0;
    const double act_us = act_cu / kActBytesPerUsPerCu;
    // Without double buffering a round's compute and the next round's load latency are serial
    // within a wavefront; the other resident wavefronts of the CU hide that (fitted over the
    // variants at the BASELINE shapes: half a latency at 16 resident wavefronts per CU).
    const double rounds_us = v.db ? 0.0 : double(rounds - 1) * 0.1 * kQ8LatencyUs;
    // (A wavefront with nt weight tiles carries nt tiles' copies and compute: it counts nt times.)
    const int64_t waves_cu = std::min<int64_t>(resident, (grid + cus(h) - 1) / cus(h)) * v.waves * v.nt;
    const double hide_us = 0.5 * kQ8LatencyUs * 16.0 / double(std::max<int64_t>(waves_cu, 1));
    // A grid narrower than the chip streams through fewer CUs, each of which sustains about 1.25x
    // its share of the peak (fitted: 64-row workgroups at N = 11008 leave 84 CUs idle).
    const double cu_share = hbm_gbps(h) * 1e3 * kStreamEff / double(cus(h)) * 1.25;  // bytes per us
    const double narrow_us = double(w.bytes) / (double(std::min<int64_t>(grid, cus(h))) * cu_share);
    const double stream =
        std::max(stream_us(h, double(w.bytes), grid, resident, inflight, false, 0.0, kQ8LatencyUs), narrow_us);
    const double cost = launch_us(h) + stream + issue_us + gen_us + act_us + rounds_us + hide_us;
    Cand c;
    c.plan.family = Family::Q8Gemm;
    c.plan.variant = i;
    c.plan.threads = v.waves * 64;
    c.plan.split_k = v.waves;
    c.plan.tile_k = int(per_round * 64);
    c.plan.grid = grid;
    c.plan.key = key.str();
    c.plan.why = std::to_string(grid) + " workgroups of " + std::to_string(16 * v.nt) + " weight rows, " + std::to_string(rounds) +
                 " round(s) of " + std::to_string(per_round) + " block pairs, " + std::to_string(resident) +
                 " resident per CU";
    c.cost = cost;
    cs.push_back(c);
  }
  return pick(cs, "q8_0", log, err);
}

// ---------------------------------------------------------------------------------------
std::optional<Plan> solve_conv(const Hcs& h, const KmlTree& t, const Shape& s, SolveLog* log, std::string* err) {
  const double peak = h.peak_f32_mfma_tflops > 0 ? h.peak_f32_mfma_tflops : h.flops_gflops * 1e-3 / 16;
  const double clk = clock_ghz(h) * 1e3;  // clocks per microsecond
  const int64_t taps = s.Kh * s.Kw;
  const int64_t strips = (s.Ho * s.Wo + 31) / 32;
  const int64_t units = s.Nb * strips;          // 32-pixel strips
  const int64_t oc_tiles = (s.Co + 63) / 64;
  const double simd_slots = double(cus(h)) * simds(h);
  // One 32x32 output tile over the whole reduction: one MFMA 32x32x2 f32 per (channel pair,
  // tap), each 4096 FLOP at the per-SIMD f32 rate.
  const double per_simd_flop_clk = peak * 1e12 / (simd_slots * clk * 1e6);
  const double tile_cycles = double((s.Ci + 1) / 2) * double(taps) * (4096.0 / per_simd_flop_clk);
  std::vector<Cand> cs;
  for (int i = 0; i < kNumConvVariants; ++i) {
    const ConvVariant v = kConvVariants[i];
    std::ostringstream key;
    const bool l16 = v.tile_strips == kConvL16;
    const bool tile = v.tile_strips > 0;
    const bool ldsk = v.tile_strips < 0 && !l16;
    if (l16) {
      // Runs of 16-pixel groups, one workgroup (8 wavefronts) per CU: the busiest SIMD multiplies
      // its 16-channel tile over the longest run, one v_mfma_f32_16x16x4f32 (2048 FLOP) per four
      // k values.
      const int64_t ocb = (s.Co + 63) / 64;
      const ConvL16Geom g = conv_l16_geom(s.Nb, s.Ho, s.Wo, ocb);
      const std::string k = "conv_lds16:g" + std::to_string(g.gmax) + "x64,cb16";
      if (!conv_l16_supported(t.layout == Layout::NCHW, s.Kh, s.Kw, s.stride, s.pad, s.Nb, s.W, s.Ho, s.Wo, s.Ci, s.Co) ||
          4 * kConvL16Rows * (s.W / 4) > 512) {
        reject(log, k + " violates NCHW 3x3 stride 1 pad<=1, W+2pad<=72, W%4==0, C%16==0, runs within 4 output rows, "
                       "index quotients below 2^21");
        continue;
      }
      const int64_t wgs = s.Nb * g.wpi * ocb;
      const int64_t lds = 2 * (4 * kConvL16Rows * kConvL16Pitch + 9 * 4 * kConvL16WQuad) * 16;
      if (lds > lds_block(h)) {
        reject(log, k + " violates LDS per workgroup");
        continue;
      }
      const double wg_per_cu = std::ceil(double(wgs) / cus(h));
      const double mfmas = double(g.gmax) * double(s.Ci) * 9.0 / 4.0;
      const double cycles = wg_per_cu * mfmas * (2048.0 / per_simd_flop_clk);
      Cand c;
      c.plan.family = Family::ConvIgemm;
      c.plan.variant = i;
      c.plan.tile_m = 64;
      c.plan.tile_n = int(16 * g.gmax);
      c.plan.tile_k = int(16 * taps);
      c.plan.threads = 512;
      c.plan.grid = wgs;
      c.plan.key = k;
      c.plan.why = std::to_string(wgs) + " workgroups of 8 wavefronts, runs of up to " + std::to_string(g.gmax) +
                   " 16-pixel groups, 16 channels per staged chunk, calibrated MFMA efficiency " + fmt("%.2f", v.eff);
      c.cost = launch_us(h) + cycles / (clk * v.eff * mfma_clock_scale(h));
      cs.push_back(c);
      continue;
    }
    if (ldsk) key << "conv_lds:" << -64 * v.tile_strips << "x64,cb" << v.bk_bytes;
    else if (tile) key << "conv_tile:s" << v.tile_strips << ",cb" << v.bk_bytes;
    else key << "conv_igemm:w" << v.waves << ",lds" << v.bk_bytes;
    int64_t cb = 0, lds = 0, wgs = 0;
    double tiles_per_wave = 0;
    if (ldsk) {
      const int64_t pix = -64 * v.tile_strips;
      if (!conv_lds_supported(t.layout == Layout::NCHW, s.Kh, s.Kw, s.stride, s.pad, s.W, s.Ho, s.Wo, s.Ci, pix)) {
        reject(log, key.str() + " violates NCHW 3x3 stride 1 pad<=1, W+2pad<=64, W%4==0, C%8==0, " + std::to_string(pix) +
                        " pixels within 6 output rows");
        continue;
      }
      cb = v.bk_bytes;
      lds = 2 * (2 * kConvLdsRows * kConvLdsCols * 4 + 64 * 76) * 4;
      wgs = ((s.Ho * s.Wo + pix - 1) / pix) * s.Nb * oc_tiles;
      tiles_per_wave = 1;
    } else if (tile) {
      if (taps != 9 && taps != 1) {
        reject(log, key.str() + " violates taps in {9, 1} (compiled kernel sizes)");
        continue;
      }
      cb = v.bk_bytes;
      lds = cb * taps * 97 * 4;
      wgs = ((units + v.tile_strips - 1) / v.tile_strips) * oc_tiles;
      tiles_per_wave = 1;
    } else {
      if (taps > 49) {
        reject(log, key.str() + " violates taps<=49 (per-lane tap table)");
        continue;
      }
      const int64_t per_channel = taps * 64 * 4;
      cb = (v.bk_bytes / per_channel) & ~int64_t(1);
      if (cb < 2) {
        reject(log, key.str() + " violates LDS budget >= 2 channels x taps x 64 oc");
        continue;
      }
      cb = std::min<int64_t>(cb, (s.Ci + 1) & ~int64_t(1));
      lds = cb * per_channel;
      wgs = ((units + v.waves - 1) / v.waves) * oc_tiles;
      tiles_per_wave = 2;
    }
    if (lds > lds_block(h)) {
      reject(log, key.str() + " violates LDS per workgroup");
      continue;
    }
    // Workgroups spread over the CUs; the busiest SIMD holds ceil(workgroups per CU) times
    // waves / SIMDs wavefronts and sets the time.
    const int64_t wg_per_cu = (wgs + cus(h) - 1) / cus(h);
    const double waves_per_simd = std::ceil(double(wg_per_cu) * v.waves / simds(h));
    const double cost =
        launch_us(h) + waves_per_simd * tiles_per_wave * tile_cycles / (clk * v.eff * mfma_clock_scale(h));
    Cand c;
    c.plan.family = Family::ConvIgemm;
    c.plan.variant = i;
    c.plan.tile_m = tile ? 32 : 64;
    c.plan.tile_n = ldsk ? -64 * v.tile_strips : 32 * (tile ? v.tile_strips : v.waves);
    c.plan.tile_k = int(cb * taps);
    c.plan.threads = v.waves * 64;
    c.plan.grid = wgs;
    c.plan.key = key.str();
    c.plan.why = std::to_string(wgs) + " workgroups of " + std::to_string(v.waves) + " wavefronts, " +
                 std::to_string(cb) + " channels per staged weight chunk, calibrated MFMA efficiency " +
                 fmt("%.2f", v.eff);
    c.cost = cost;
    cs.push_back(c);
  }
  return pick(cs, "conv", log, err);
}

// Scenario B (reference src/solver.cpp:14-44, src/codegen_hip.cpp:1143-1238): a GEMM whose
// payload exceeds the 0.85 share of the device tier that a run may occupy keeps B resident and
// streams A and C in M-shards through two pinned host buffers each, on two streams, so the copies
// of one shard overlap the kernel of the other. The kernel variant is the one the resident solve
// picks; the shard height is the largest multiple of its tile rows with about 64 MiB of A per
// shard (the reference's shard size) for which B and two shard pairs fit the 0.85 share. The
// cost adds the link time of every byte crossing it once.
std::optional<Plan> solve_stream_gemm(const Hcs& h, const KmlTree& t, const Shape& s, SolveLog* log,
                                      std::string* err) {
  constexpr double kRunShare = 0.85;               // the residency refusal's threshold
  constexpr int64_t kShardTarget = int64_t(64) << 20;
  const int64_t es = t.dtype == DType::F16 ? 2 : 4;
  const int64_t cap = h.device_capacity();
  const int64_t budget = int64_t(kRunShare * double(cap));
  auto kp = solve_gemm(h, t, s, log, err);
  if (!kp) return std::nullopt;
  const int64_t unit = kp->family == Family::GemmF16 ? kp->tile_m : (kp->variant == 1 ? 64 : 1);
  const int64_t b_bytes = s.K * s.N * es;
  const int64_t row_bytes = (s.K + s.N) * es;  // one row of A and one of C
  const int64_t fit = (budget - b_bytes) / (2 * row_bytes);
  int64_t rows = std::min<int64_t>({fit, std::max<int64_t>(unit, kShardTarget / (s.K * es)), s.M});
  rows = rows / unit * unit;
  if (rows < unit || budget <= b_bytes) {
    const std::string rec = "stream_working_set<=0.85*device_capacity need=" +
                            std::to_string(b_bytes + 2 * unit * row_bytes) + " cap=" + std::to_string(cap);
    reject(log, rec);
    if (err) *err = "infeasible: " + rec;
    return std::nullopt;
  }
  Plan p = *kp;
  const int64_t shards = (s.M + rows - 1) / rows;
  const double link_gbps = h.link_bw_gbps > 0 ? h.link_bw_gbps : 1.0;
  const double bytes = double(workload_of(t).bytes);
  const double overhead_us = double(shards) * launch_us(h);
  p.shard_rows = int(rows);
  // Two data paths for A (reference src/solver.cpp:14-44, :96-121). Pinned copies move every byte
  // over the link once and overlap the kernels. The mapped path pages A in from storage (the
  // nvme tier) and the kernel reads it over the link once per workgroup column that consumes
  // it (ceil(N / tile_n)); B and C move as copies. Its copy term is the pinned one plus two
  // non-negative terms, so the pinned path wins by the cost model; the mapped candidate exists
  // only where the description has an nvme tier (a named predicate otherwise).
  std::vector<Cand> cs;
  {
    Cand c;
    c.plan = p;
    c.plan.stream_path = 1;
    c.plan.key = kp->key + "+stream";
    c.cost = std::max(kp->predicted_us, bytes / (link_gbps * 1e3)) + overhead_us;
    c.plan.why = "scenario B: " + std::to_string(shards) + " M-shards of " + std::to_string(rows) +
                 " rows through pinned host buffers, B resident (" + std::to_string(b_bytes) + " B), link " +
                 fmt("%.0f", link_gbps) + " GB/s; kernel " + kp->key;
    cs.push_back(c);
  }
  const double nvme_gbps = h.tier_bw("nvme");
  if (nvme_gbps <= 0) {
    reject(log, kp->key + "+stream_mmap violates mmap_stream_requires_nvme_tier_bw>0");
  } else {
    const double streamed = double(s.M * s.K * es);
    const int64_t reuse = (s.N + std::max(1, kp->tile_n) - 1) / std::max(1, kp->tile_n);
    const double copy_us = streamed / (nvme_gbps * 1e3) + streamed * double(reuse) / (link_gbps * 1e3) +
                           (bytes - streamed) / (link_gbps * 1e3);
    Cand c;
    c.plan = p;
    c.plan.stream_path = 2;
    c.plan.key = kp->key + "+stream_mmap";
    c.cost = std::max(kp->predicted_us, copy_us) + overhead_us;
    c.plan.why = "scenario B: " + std::to_string(shards) + " M-shards of " + std::to_string(rows) +
                 " rows, A read by the kernel from host-mapped staging (read " + std::to_string(reuse) +
                 " times over the link), B resident, nvme " + fmt("%.0f", nvme_gbps) + " GB/s, link " +
                 fmt("%.0f", link_gbps) + " GB/s; kernel " + kp->key;
    cs.push_back(c);
  }
  const Cand* best = &cs[0];
  for (const Cand& c : cs)
    if (c.cost < best->cost || (c.cost == best->cost && c.plan.key < best->plan.key)) best = &c;
  if (log) {
    for (const Cand& c : cs)
      log->ranked.emplace_back(c.cost, c.plan.key + " family=" + std::to_string(int(c.plan.family)) +
                                           " variant=" + std::to_string(c.plan.variant) +
                                           " stream_path=" + (c.plan.stream_path == 2 ? "mmap" : "pinned"));
    std::sort(log->ranked.begin(), log->ranked.end());
  }
  Plan out = best->plan;
  out.predicted_us = best->cost;
  out.feasible = kp->feasible * int(cs.size());  // every kernel candidate with each data path
  return out;
}

}  // namespace

std::optional<Plan> solve(const Hcs& h, const KmlTree& t, SolveLog* log, std::string* err) {
  if (const std::string gap = support_gap(t); !gap.empty()) {
    if (err) *err = gap;
    return std::nullopt;
  }
  const Shape s = shape_of(t);
  // Capacity predicate (the reference's only one, tile_working_set<=device_capacity,
  // src/solver.cpp:14-60): every kernel here keeps the operation's whole working set resident,
  // so it must fit the device tier; an empty candidate set ends infeasible with the record.
  if (const int64_t cap = h.device_capacity(); cap > 0) {
    const int64_t need = workload_of(t).bytes;
    // A GEMM on the MFMA kernels streams instead (scenario B) when its payload exceeds what a
    // run may keep resident; every other op is resident-only, as the reference's programs are.
    const bool streams = t.op == OpKind::Gemm && (t.dtype == DType::F16 || t.dtype == DType::F32) && !h.unified_memory;
    if (streams && double(need) > 0.85 * double(cap)) return solve_stream_gemm(h, t, s, log, err);
    if (need > cap) {
      const std::string rec = "working_set<=device_capacity need=" + std::to_string(need) +
                              " cap=" + std::to_string(cap);
      reject(log, rec);
      if (err) *err = "infeasible: " + rec;
      return std::nullopt;
    }
  }
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
      p.predicted_us = launch_us(h) + double(workload_of(t).bytes) / (hbm_gbps(h) * 1e3);
      p.feasible = 1;
      // The launch takes the row form for these shapes when X, S and Y are 16-byte aligned.
      if (channelscale_rows_form(s.L, s.C)) {
        p.grid = (s.L + 3) / 4;
        p.key = "channelscale:rows";
        p.why = "one wavefront per row, S in LDS, grouped stores";
      } else {
        p.grid = std::min<int64_t>((s.L * s.C / 4 + 255) / 256, 256 * 32);
        p.key = "channelscale:grid_stride";
        p.why = "elementwise float4 grid-stride";
      }
      return p;
    }
  }
  if (err) *err = "unknown op";
  return std::nullopt;
}

}  // namespace uk
