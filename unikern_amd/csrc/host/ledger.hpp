// Kernel solution ledger: solutions keyed by (op signature, HCS fingerprint, tree hash).
//
// Same contract as the reference's ILedger (include/unikern/components.hpp:83-125): lookup of a
// recorded solution, commit of a measured one (all-or-nothing), violation events kept apart from
// solution rows, the measured rows of one HCS for calibration. Two stores, chosen by the path as
// in the reference (src/main.cpp:35-37): a path ending in ".jsonl" is the append-only text ledger
// (TAB-separated lines, src/runtime.cpp:29-176), any other path an SQLite database with the
// reference's schema (src/sqlite_ledger.cpp). A ledger written by the reference opens here and
// the other way round.
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace uk {

struct LedgerKey {
  std::string op_sig, hcs_fp, tree_hash;
  std::string composite() const { return op_sig + "|" + hcs_fp + "|" + tree_hash; }
};

// One solution row. c_ms is the predicted time; measured_ms the end-to-end measurement and
// kernel_ms the kernel-only one (0 for a row committed by solve). placement carries the plan:
// "plan=<key> family=<n> variant=<n> | <why>".
struct LedgerRow {
  double c_ms = 0, measured_ms = 0, kernel_ms = 0;
  int tile_m = 0, tile_n = 0;
  std::string placement;
};

struct LedgerMeasured {
  std::string op_sig;
  double c_ms = 0, measured_ms = 0, kernel_ms = 0;
  int shard_rows = 0;     // > 0: a streamed (scenario-B) plan, priced as copies overlapping shard kernels
  bool replayed = false;  // parsed from a recorded program output, not measured on a device
};

// Marks the "why" part of a placement whose measurement was replayed from a recorded output.
inline constexpr const char* kReplayedTag = "replayed ";

class Ledger {
 public:
  virtual ~Ledger() = default;
  virtual std::optional<LedgerRow> lookup(const LedgerKey& key) = 0;
  // One row per key; a later commit replaces it (file ledger: the first matching line wins on
  // lookup, as in the reference, so a replacement is appended and older lines are ignored).
  virtual bool commit(const LedgerKey& key, const LedgerRow& row, std::string* err) = 0;
  virtual bool record_violation(const LedgerKey& key, double rate, double threshold, int migrations, int checks,
                                uint64_t vram_free, std::string* err) = 0;
  virtual std::vector<LedgerMeasured> measured_rows(const std::string& hcs_fp) = 0;
  virtual int size() = 0;
  virtual int violation_count() = 0;
};

std::unique_ptr<Ledger> open_ledger(const std::string& path, std::string* err);

// Plan fields recorded in the placement text: "plan=<key> family=<n> variant=<n>[ shard_rows=<n>] | <why>"
// (shard_rows only for a streamed plan; rows written without it read back as resident).
std::string placement_of(const std::string& plan_key, int family, int variant, int shard_rows,
                         const std::string& why);
bool parse_placement(const std::string& placement, std::string* plan_key, int* family, int* variant,
                     int* shard_rows);
// shard_rows and the replayed mark of a placement text (0 / false when it has neither).
void placement_flags(const std::string& placement, int* shard_rows, bool* replayed);

}  // namespace uk
