// Calibration closure: refit the HCS rate constants the solver prices with, from the ledger's
// measured rows (the reference's closure, src/main.cpp:579-652, refits only the host link).
//
// Design:
//  * Every measured row carries the solver's prediction (c_ms) and the kernel-only time the
//    device delivered (kernel_ms). Rows split by what bounds their kernel: streaming rows
//    (row family, reduce, channelscale, Q8_0) are priced by hbm_bw_gbps, MFMA-bound rows (f16/f32
//    GEMM, conv) by clock_mhz. Within a class the speed factor is the geometric mean of
//    predicted/measured, i.e. the least-squares fit of one multiplicative constant in log time,
//    so a row twice too slow and a row twice too fast cancel rather than averaging to 1.25.
//  * With no MFMA-bound row, a matrix-core probe supplies the clock factor instead: the variant
//    efficiencies were fitted on parts whose probe sustained kEffFitProbeClockGhz, so a part that
//    sustains less under the same load runs every MFMA-bound plan proportionally slower.
//  * Streamed (scenario-B) rows and rows replayed from recorded outputs take no part in the fit:
//    the first are priced as copies overlapping shard kernels, the second were not measured here.
//  * The end-to-end time of a row minus its kernel time is the host copy of its inputs and
//    outputs. A straight line copy_ms = latency + bytes / link through all usable rows (ordinary
//    least squares; a single byte count gives the zero-latency ratio) separates the per-call
//    latency from the link rate. A unified-memory part has no copy, so its link is left alone.
#include "calibrate.hpp"

#include <cmath>
#include <cstdio>
#include <sstream>

#include "../variants.hpp"

namespace uk {

bool mfma_bound(const KmlTree& t) {
  return (t.op == OpKind::Gemm && t.dtype != DType::Q8_0) || t.op == OpKind::Conv;
}

namespace {

std::string num(double v) {
  char b[48];
  std::snprintf(b, sizeof b, "%.6g", v);
  return b;
}

// exp(mean(log x)): the least-squares scale of one multiplicative constant.
double geomean(const std::vector<double>& xs) {
  double s = 0;
  for (double x : xs) s += std::log(x);
  return std::exp(s / double(xs.size()));
}

}  // namespace

Calibration calibrate_hcs(const Hcs& in, const std::vector<LedgerMeasured>& rows, const ProbeClock& probe) {
  Calibration c;
  c.hcs = in;
  std::vector<double> stream_ratio, mfma_ratio, link_x, link_y;
  int streamed = 0, replayed = 0;
  for (const LedgerMeasured& r : rows) {
    const auto t = tree_from_signature(r.op_sig);
    if (!t) continue;
    // A replayed row was parsed from a recorded output, not measured here. A streamed row's
    // prediction is a pass of overlapping host copies and shard kernels, while its kernel_ms covers
    // the shard kernels only, so its ratio measures copy against kernel, not the clock or the
    // HBM rate, and its end-to-end time is not one copy of its inputs and outputs.
    if (r.replayed) {
      ++replayed;
      continue;
    }
    if (r.shard_rows > 0) {
      ++streamed;
      continue;
    }
    if (r.c_ms > 0 && r.kernel_ms > 0 && std::isfinite(r.c_ms / r.kernel_ms))
      (mfma_bound(*t) ? mfma_ratio : stream_ratio).push_back(r.c_ms / r.kernel_ms);
    const double copy_ms = r.measured_ms - r.kernel_ms;
    const int64_t bytes = workload_of(*t).bytes;
    if (r.kernel_ms > 0 && copy_ms > 0 && bytes > 0) {
      link_x.push_back(double(bytes));
      link_y.push_back(copy_ms);
    }
  }
  std::ostringstream d;
  if (replayed) d << "left out: " << replayed << " replayed row(s) (recorded outputs, not device measurements)\n";
  if (streamed)
    d << "left out: " << streamed << " streamed row(s) (pass of host copies and shard kernels; not a clock, HBM or "
         "link figure)\n";

  if (!stream_ratio.empty() && in.hbm_bw_gbps > 0) {
    c.hbm_rows = int(stream_ratio.size());
    c.hbm_scale = geomean(stream_ratio);
    c.hcs.hbm_bw_gbps = in.hbm_bw_gbps * c.hbm_scale;
    c.changed = true;
    d << "streaming: " << c.hbm_rows << " row(s), predicted/measured " << num(c.hbm_scale) << ", hbm_bw_gbps "
      << num(in.hbm_bw_gbps) << " -> " << num(c.hcs.hbm_bw_gbps) << "\n";
  }

  if (in.clock_mhz > 0) {
    if (!mfma_ratio.empty()) {
      c.mfma_rows = int(mfma_ratio.size());
      c.clock_scale = geomean(mfma_ratio);
      d << "matrix: " << c.mfma_rows << " row(s), predicted/measured " << num(c.clock_scale);
    } else if (probe.clock_ghz > 0) {
      c.clock_scale = probe.clock_ghz / kEffFitProbeClockGhz;
      d << "matrix: probe sustains " << num(probe.clock_ghz) << " GHz against " << num(kEffFitProbeClockGhz)
        << " GHz where the variant efficiencies were fitted";
    }
    if (c.clock_scale > 0) {
      c.hcs.clock_mhz = in.clock_mhz * c.clock_scale;
      c.changed = true;
      d << ", clock_mhz " << num(in.clock_mhz) << " -> " << num(c.hcs.clock_mhz) << "\n";
    }
  }

  if (!link_x.empty() && !in.unified_memory) {
    const double n = double(link_x.size());
    double mx = 0, my = 0;
    for (size_t i = 0; i < link_x.size(); ++i) {
      mx += link_x[i] / n;
      my += link_y[i] / n;
    }
    double sxx = 0, sxy = 0;
    for (size_t i = 0; i < link_x.size(); ++i) {
      sxx += (link_x[i] - mx) * (link_x[i] - mx);
      sxy += (link_x[i] - mx) * (link_y[i] - my);
    }
    // ms per byte; the line needs two distinct byte counts and a positive slope, otherwise the
    // latency is taken as zero and the slope is the ratio of the sums.
    double slope = sxx > 0 ? sxy / sxx : 0;
    double latency = my - slope * mx;
    if (!(slope > 0) || latency < 0) {
      slope = my / mx;
      latency = 0;
    }
    c.link_rows = int(link_x.size());
    c.link_latency_ms = latency;
    c.hcs.link_bw_gbps = 1.0 / (slope * 1e6);  // bytes per ms -> GB/s
    c.changed = true;
    d << "link: " << c.link_rows << " row(s), copy_ms = " << num(latency) << " + bytes / "
      << num(c.hcs.link_bw_gbps) << " GB/s, link_bw_gbps " << num(in.link_bw_gbps) << " -> "
      << num(c.hcs.link_bw_gbps) << "\n";
  } else if (!link_x.empty()) {
    d << "link: unified memory has no host copy; link_bw_gbps kept\n";
  }

  if (c.changed) {
    c.hcs.constants_version = in.constants_version + 1;
    c.hcs.confidence = Confidence::Measured;
  } else {
    d << "nothing to fit: " << rows.size()
      << " measured row(s), none with a prediction and a kernel time, and no probe clock\n";
  }
  c.detail = d.str();
  return c;
}

}  // namespace uk
