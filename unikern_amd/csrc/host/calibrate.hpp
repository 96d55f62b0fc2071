// Calibration of HCS constants from measured ledger rows.
#pragma once

#include <string>
#include <vector>

#include "ledger.hpp"
#include "uk_core.hpp"

namespace uk {

// Median effective host link bandwidth (GB/s) over the usable rows; 0 when none is usable.
double calibrated_link_bw(const std::vector<LedgerMeasured>& rows, std::string* detail);

}  // namespace uk
