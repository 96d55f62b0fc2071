// Calibration closure (reference src/solver.cpp:194-244 and src/main.cpp:579-652): the host link
// bandwidth of an HCS, derived from the measured rows its ledger holds. A measured row's
// end-to-end time minus its kernel-only time is the host-to-device and device-to-host copy of
// the op's inputs and outputs; their bytes over that time is the link rate the row saw. The
// median over rows (mean of the two middle values for an even count) is deterministic and
// robust to outliers; it replaces link_bw_gbps and bumps constants_version.
#include <algorithm>
#include <sstream>

#include "calibrate.hpp"

namespace uk {

double calibrated_link_bw(const std::vector<LedgerMeasured>& rows, std::string* detail) {
  std::vector<double> bws;
  std::ostringstream log;
  for (const auto& r : rows) {
    if (r.measured_ms <= 0 || r.kernel_ms <= 0 || r.measured_ms <= r.kernel_ms) continue;  // no copy time
    const auto t = tree_from_signature(r.op_sig);
    if (!t) continue;
    const Workload w = workload_of(*t);
    if (w.bytes <= 0) continue;
    const double copy_ms = r.measured_ms - r.kernel_ms;
    const double bw = double(w.bytes) / (copy_ms * 1e6);  // GB/s
    bws.push_back(bw);
    log << r.op_sig << " bytes=" << w.bytes << " copy_ms=" << copy_ms << " eff_bw=" << bw << "GB/s; ";
  }
  if (bws.empty()) {
    if (detail) *detail = "no usable rows (need measured_ms > kernel_ms > 0)";
    return 0;
  }
  std::sort(bws.begin(), bws.end());
  const size_t n = bws.size();
  const double med = n % 2 ? bws[n / 2] : 0.5 * (bws[n / 2 - 1] + bws[n / 2]);
  if (detail) *detail = "usable_rows=" + std::to_string(n) + " median_link_bw=" + std::to_string(med) + "GB/s [" + log.str() + "]";
  return med;
}

}  // namespace uk
