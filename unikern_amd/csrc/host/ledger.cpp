// Kernel solution ledger: the text store and the SQLite store (see ledger.hpp).
#include "ledger.hpp"

#include <dlfcn.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <map>
#include <sstream>

namespace uk {

namespace {

constexpr char kSep = '\t';
constexpr const char* kViolation = "#VIOLATION";

std::vector<std::string> split_tabs(const std::string& line) {
  std::vector<std::string> f;
  size_t pos = 0;
  while (true) {
    const size_t tab = line.find(kSep, pos);
    f.push_back(line.substr(pos, tab == std::string::npos ? std::string::npos : tab - pos));
    if (tab == std::string::npos) break;
    pos = tab + 1;
  }
  return f;
}

bool to_double(const std::string& s, double* v) {
  try {
    size_t n = 0;
    *v = std::stod(s, &n);
    return n == s.size();
  } catch (...) {
    return false;
  }
}
bool to_int(const std::string& s, int* v) {
  try {
    size_t n = 0;
    *v = std::stoi(s, &n);
    return n == s.size();
  } catch (...) {
    return false;
  }
}

// ---------------------------------------------------------------------------------------
// Text ledger. Line formats (src/runtime.cpp:29-176):
//   key \t c_ms \t measured_ms \t kernel_ms \t tm \t tn \t placement   (7 fields, written here)
//   key \t c_ms \t measured_ms \t tm \t tn \t placement                (6 fields)
//   key \t c_ms \t measured_ms \t placement                            (4 fields, legacy)
//   #VIOLATION \t key \t rate \t threshold \t migrations \t checks \t vram_free
// Doubles are written with max_digits10 so they read back exactly.
class FileLedger : public Ledger {
 public:
  explicit FileLedger(std::string path) : path_(std::move(path)) {}

  std::optional<LedgerRow> lookup(const LedgerKey& key) override {
    const std::string want = key.composite();
    std::ifstream in(path_);
    std::string line;
    std::optional<LedgerRow> found;  // the latest line of the key wins
    while (std::getline(in, line)) {
      const auto f = split_tabs(line);
      if (f.size() < 4 || f[0] != want) continue;
      LedgerRow r;
      if (!to_double(f[1], &r.c_ms) || !to_double(f[2], &r.measured_ms)) continue;  // corrupt: skip
      if (f.size() >= 7) {
        if (!to_double(f[3], &r.kernel_ms) || !to_int(f[4], &r.tile_m) || !to_int(f[5], &r.tile_n)) continue;
        r.placement = f[6];
      } else if (f.size() >= 6) {
        if (!to_int(f[3], &r.tile_m) || !to_int(f[4], &r.tile_n)) continue;
        r.placement = f[5];
      } else {
        r.placement = f[3];
      }
      found = r;
    }
    return found;
  }

  bool commit(const LedgerKey& key, const LedgerRow& row, std::string* err) override {
    std::ostringstream os;
    os.precision(std::numeric_limits<double>::max_digits10);
    os << key.composite() << kSep << row.c_ms << kSep << row.measured_ms << kSep << row.kernel_ms << kSep
       << row.tile_m << kSep << row.tile_n << kSep << row.placement << "\n";
    return append(os.str(), err);
  }

  bool record_violation(const LedgerKey& key, double rate, double threshold, int migrations, int checks,
                        uint64_t vram_free, std::string* err) override {
    std::ostringstream os;
    os.precision(std::numeric_limits<double>::max_digits10);
    os << kViolation << kSep << key.composite() << kSep << rate << kSep << threshold << kSep << migrations << kSep
       << checks << kSep << vram_free << "\n";
    return append(os.str(), err);
  }

  std::vector<LedgerMeasured> measured_rows(const std::string& hcs_fp) override {
    // The latest line of each key, as lookup reads it (a replacement appends a new line).
    std::vector<std::string> order;
    std::map<std::string, LedgerMeasured> latest;
    std::ifstream in(path_);
    std::string line;
    while (std::getline(in, line)) {
      const auto f = split_tabs(line);
      if (f.size() < 4 || f[0].rfind(kViolation, 0) == 0) continue;
      const size_t p1 = f[0].find('|');
      const size_t p2 = p1 == std::string::npos ? p1 : f[0].find('|', p1 + 1);
      if (p2 == std::string::npos || f[0].substr(p1 + 1, p2 - p1 - 1) != hcs_fp) continue;
      LedgerMeasured m;
      m.op_sig = f[0].substr(0, p1);
      if (!to_double(f[1], &m.c_ms) || !to_double(f[2], &m.measured_ms)) continue;
      if (f.size() >= 7 && !to_double(f[3], &m.kernel_ms)) continue;
      placement_flags(f.size() >= 7 ? f[6] : f.size() >= 6 ? f[5] : f[3], &m.shard_rows, &m.replayed);
      if (!latest.count(f[0])) order.push_back(f[0]);
      latest[f[0]] = m;
    }
    std::vector<LedgerMeasured> out;
    for (const std::string& k : order)
      if (latest[k].measured_ms > 0) out.push_back(latest[k]);
    return out;
  }

  int size() override { return count(false); }
  int violation_count() override { return count(true); }

 private:
  // One write per record: the line is composed first and written with a single append, so an
  // interrupted process leaves at most a trailing partial line, which lookups skip as corrupt.
  bool append(const std::string& text, std::string* err) {
    std::FILE* f = std::fopen(path_.c_str(), "ab");
    if (!f) {
      if (err) *err = "cannot open ledger " + path_;
      return false;
    }
    const bool ok = std::fwrite(text.data(), 1, text.size(), f) == text.size() && std::fflush(f) == 0;
    std::fclose(f);
    if (!ok && err) *err = "write failed: " + path_;
    return ok;
  }
  int count(bool violations) {
    std::ifstream in(path_);
    std::string line;
    int n = 0;
    while (std::getline(in, line)) {
      if (line.empty()) continue;
      const bool v = line.rfind(kViolation, 0) == 0;
      if (v == violations) ++n;
    }
    return n;
  }
  std::string path_;
};

// ---------------------------------------------------------------------------------------
// SQLite ledger through the system library, resolved at run time (the image ships
// libsqlite3.so.0 without its header). Only the documented C API is used.
struct SqliteApi {
  using open_v2_t = int (*)(const char*, void**, int, const char*);
  using close_t = int (*)(void*);
  using errmsg_t = const char* (*)(void*);
  using exec_t = int (*)(void*, const char*, void*, void*, char**);
  using prepare_t = int (*)(void*, const char*, int, void**, const char**);
  using bind_text_t = int (*)(void*, int, const char*, int, void (*)(void*));
  using bind_double_t = int (*)(void*, int, double);
  using bind_int_t = int (*)(void*, int, int);
  using bind_int64_t = int (*)(void*, int, long long);
  using step_t = int (*)(void*);
  using col_double_t = double (*)(void*, int);
  using col_int_t = int (*)(void*, int);
  using col_text_t = const unsigned char* (*)(void*, int);
  using finalize_t = int (*)(void*);
  using free_t = void (*)(void*);
  using busy_timeout_t = int (*)(void*, int);

  static constexpr int kOk = 0, kRow = 100, kDone = 101;
  static constexpr int kOpenReadWrite = 0x2, kOpenCreate = 0x4;

  void* lib = nullptr;
  open_v2_t open_v2 = nullptr;
  close_t close = nullptr;
  errmsg_t errmsg = nullptr;
  exec_t exec = nullptr;
  prepare_t prepare = nullptr;
  bind_text_t bind_text = nullptr;
  bind_double_t bind_double = nullptr;
  bind_int_t bind_int = nullptr;
  bind_int64_t bind_int64 = nullptr;
  step_t step = nullptr;
  col_double_t col_double = nullptr;
  col_int_t col_int = nullptr;
  col_text_t col_text = nullptr;
  finalize_t finalize = nullptr;
  free_t free = nullptr;
  busy_timeout_t busy_timeout = nullptr;

  bool load(std::string* err) {
    if (lib) return true;
    for (const char* name : {"libsqlite3.so.0", "libsqlite3.so"}) {
      lib = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (lib) break;
    }
    if (!lib) {
      if (err) *err = "the SQLite ledger needs libsqlite3.so.0 (use a .jsonl ledger path instead)";
      return false;
    }
    bool ok = true;
    auto sym = [&](auto& fn, const char* name) {
      fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(lib, name));
      ok = ok && fn;
    };
    sym(open_v2, "sqlite3_open_v2");
    sym(close, "sqlite3_close");
    sym(errmsg, "sqlite3_errmsg");
    sym(exec, "sqlite3_exec");
    sym(prepare, "sqlite3_prepare_v2");
    sym(bind_text, "sqlite3_bind_text");
    sym(bind_double, "sqlite3_bind_double");
    sym(bind_int, "sqlite3_bind_int");
    sym(bind_int64, "sqlite3_bind_int64");
    sym(step, "sqlite3_step");
    sym(col_double, "sqlite3_column_double");
    sym(col_int, "sqlite3_column_int");
    sym(col_text, "sqlite3_column_text");
    sym(finalize, "sqlite3_finalize");
    sym(free, "sqlite3_free");
    sym(busy_timeout, "sqlite3_busy_timeout");
    if (!ok && err) *err = "libsqlite3 lacks a required symbol";
    return ok;
  }
};

SqliteApi& sqlite_api() {
  static SqliteApi api;
  return api;
}

// SQLITE_TRANSIENT: the library copies bound text before the call returns.
void (*const kTransient)(void*) = reinterpret_cast<void (*)(void*)>(-1);

class SqliteLedger : public Ledger {
 public:
  // Schema of the reference's store (src/sqlite_ledger.cpp:6-9, :44-66):
  //   solutions(key TEXT PRIMARY KEY, op_sig, hcs_fp, tree_hash, c_ms REAL, measured_ms REAL,
  //             tm INTEGER, tn INTEGER, placement TEXT, kernel_ms REAL)
  //   violations(id INTEGER PRIMARY KEY AUTOINCREMENT, key, rate, threshold, migrations, checks,
  //              vram_free, ts)
  static std::unique_ptr<SqliteLedger> open(const std::string& path, std::string* err) {
    SqliteApi& a = sqlite_api();
    if (!a.load(err)) return nullptr;
    void* db = nullptr;
    if (a.open_v2(path.c_str(), &db, SqliteApi::kOpenReadWrite | SqliteApi::kOpenCreate, nullptr) != SqliteApi::kOk) {
      if (err) *err = "sqlite ledger open failed (" + path + "): " + (db ? a.errmsg(db) : "no handle");
      if (db) a.close(db);
      return nullptr;
    }
    std::unique_ptr<SqliteLedger> l(new SqliteLedger(db));
    a.busy_timeout(db, 5000);
    if (!l->exec("CREATE TABLE IF NOT EXISTS solutions(key TEXT PRIMARY KEY, op_sig TEXT, hcs_fp TEXT, "
                 "tree_hash TEXT, c_ms REAL, measured_ms REAL, tm INTEGER, tn INTEGER, placement TEXT)",
                 err))
      return nullptr;
    bool has_kernel = false;
    void* st = nullptr;
    if (a.prepare(db, "PRAGMA table_info(solutions)", -1, &st, nullptr) == SqliteApi::kOk) {
      while (a.step(st) == SqliteApi::kRow) {
        const unsigned char* name = a.col_text(st, 1);
        if (name && std::string(reinterpret_cast<const char*>(name)) == "kernel_ms") has_kernel = true;
      }
      a.finalize(st);
    }
    if (!has_kernel && !l->exec("ALTER TABLE solutions ADD COLUMN kernel_ms REAL NOT NULL DEFAULT 0", err))
      return nullptr;
    if (!l->exec("CREATE TABLE IF NOT EXISTS violations(id INTEGER PRIMARY KEY AUTOINCREMENT, key TEXT, "
                 "rate REAL, threshold REAL, migrations INTEGER, checks INTEGER, vram_free INTEGER, ts TEXT)",
                 err))
      return nullptr;
    return l;
  }
  ~SqliteLedger() override { sqlite_api().close(db_); }

  std::optional<LedgerRow> lookup(const LedgerKey& key) override {
    SqliteApi& a = sqlite_api();
    void* st = nullptr;
    if (a.prepare(db_, "SELECT c_ms, measured_ms, kernel_ms, tm, tn, placement FROM solutions WHERE key = ?1", -1,
                  &st, nullptr) != SqliteApi::kOk)
      return std::nullopt;
    const std::string k = key.composite();
    a.bind_text(st, 1, k.c_str(), -1, kTransient);
    std::optional<LedgerRow> out;
    if (a.step(st) == SqliteApi::kRow) {
      LedgerRow r;
      r.c_ms = a.col_double(st, 0);
      r.measured_ms = a.col_double(st, 1);
      r.kernel_ms = a.col_double(st, 2);
      r.tile_m = a.col_int(st, 3);
      r.tile_n = a.col_int(st, 4);
      const unsigned char* p = a.col_text(st, 5);
      r.placement = p ? reinterpret_cast<const char*>(p) : "";
      out = r;
    }
    a.finalize(st);
    return out;
  }

  bool commit(const LedgerKey& key, const LedgerRow& row, std::string* err) override {
    SqliteApi& a = sqlite_api();
    if (!exec("BEGIN IMMEDIATE", err)) return false;  // all-or-nothing against interrupts
    void* st = nullptr;
    if (a.prepare(db_,
                  "INSERT OR REPLACE INTO solutions(key, op_sig, hcs_fp, tree_hash, c_ms, measured_ms, tm, tn, "
                  "placement, kernel_ms) VALUES(?1, ?2, ?3, ?4, ?5, ?6, ?7, ?8, ?9, ?10)",
                  -1, &st, nullptr) != SqliteApi::kOk)
      return rollback(err);
    const std::string k = key.composite();
    a.bind_text(st, 1, k.c_str(), -1, kTransient);
    a.bind_text(st, 2, key.op_sig.c_str(), -1, kTransient);
    a.bind_text(st, 3, key.hcs_fp.c_str(), -1, kTransient);
    a.bind_text(st, 4, key.tree_hash.c_str(), -1, kTransient);
    a.bind_double(st, 5, row.c_ms);
    a.bind_double(st, 6, row.measured_ms);
    a.bind_int(st, 7, row.tile_m);
    a.bind_int(st, 8, row.tile_n);
    a.bind_text(st, 9, row.placement.c_str(), -1, kTransient);
    a.bind_double(st, 10, row.kernel_ms);
    const int rc = a.step(st);
    a.finalize(st);
    if (rc != SqliteApi::kDone) return rollback(err);
    return exec("COMMIT", err);
  }

  bool record_violation(const LedgerKey& key, double rate, double threshold, int migrations, int checks,
                        uint64_t vram_free, std::string* err) override {
    SqliteApi& a = sqlite_api();
    if (!exec("BEGIN IMMEDIATE", err)) return false;
    void* st = nullptr;
    if (a.prepare(db_,
                  "INSERT INTO violations(key, rate, threshold, migrations, checks, vram_free, ts) "
                  "VALUES(?1, ?2, ?3, ?4, ?5, ?6, datetime('now'))",
                  -1, &st, nullptr) != SqliteApi::kOk)
      return rollback(err);
    const std::string k = key.composite();
    a.bind_text(st, 1, k.c_str(), -1, kTransient);
    a.bind_double(st, 2, rate);
    a.bind_double(st, 3, threshold);
    a.bind_int(st, 4, migrations);
    a.bind_int(st, 5, checks);
    a.bind_int64(st, 6, (long long)vram_free);
    const int rc = a.step(st);
    a.finalize(st);
    if (rc != SqliteApi::kDone) return rollback(err);
    return exec("COMMIT", err);
  }

  std::vector<LedgerMeasured> measured_rows(const std::string& hcs_fp) override {
    SqliteApi& a = sqlite_api();
    std::vector<LedgerMeasured> out;
    void* st = nullptr;
    if (a.prepare(db_,
                  "SELECT op_sig, c_ms, measured_ms, kernel_ms, placement FROM solutions WHERE hcs_fp = ?1 AND "
                  "measured_ms > 0 ORDER BY key",
                  -1, &st, nullptr) != SqliteApi::kOk)
      return out;
    a.bind_text(st, 1, hcs_fp.c_str(), -1, kTransient);
    while (a.step(st) == SqliteApi::kRow) {
      LedgerMeasured m;
      const unsigned char* s = a.col_text(st, 0);
      m.op_sig = s ? reinterpret_cast<const char*>(s) : "";
      m.c_ms = a.col_double(st, 1);
      m.measured_ms = a.col_double(st, 2);
      m.kernel_ms = a.col_double(st, 3);
      const unsigned char* pl = a.col_text(st, 4);
      placement_flags(pl ? reinterpret_cast<const char*>(pl) : "", &m.shard_rows, &m.replayed);
      out.push_back(m);
    }
    a.finalize(st);
    return out;
  }

  int size() override { return count("SELECT count(*) FROM solutions"); }
  int violation_count() override { return count("SELECT count(*) FROM violations"); }

 private:
  explicit SqliteLedger(void* db) : db_(db) {}
  bool exec(const char* sql, std::string* err) {
    SqliteApi& a = sqlite_api();
    char* msg = nullptr;
    if (a.exec(db_, sql, nullptr, nullptr, &msg) != SqliteApi::kOk) {
      if (err) *err = std::string("sqlite: ") + (msg ? msg : a.errmsg(db_)) + " (" + sql + ")";
      if (msg) a.free(msg);
      return false;
    }
    return true;
  }
  bool rollback(std::string* err) {
    if (err) *err = std::string("sqlite: ") + sqlite_api().errmsg(db_);
    exec("ROLLBACK", nullptr);
    return false;
  }
  int count(const char* sql) {
    SqliteApi& a = sqlite_api();
    void* st = nullptr;
    int n = -1;
    if (a.prepare(db_, sql, -1, &st, nullptr) == SqliteApi::kOk) {
      if (a.step(st) == SqliteApi::kRow) n = a.col_int(st, 0);
      a.finalize(st);
    }
    return n;
  }
  void* db_;
};

bool ends_with(const std::string& s, const std::string& suf) {
  return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

}  // namespace

std::unique_ptr<Ledger> open_ledger(const std::string& path, std::string* err) {
  if (path.empty()) {
    if (err) *err = "empty ledger path";
    return nullptr;
  }
  if (ends_with(path, ".jsonl")) return std::make_unique<FileLedger>(path);
  return SqliteLedger::open(path, err);
}

std::string placement_of(const std::string& plan_key, int family, int variant, int shard_rows,
                         const std::string& why) {
  std::string p = "plan=" + plan_key + " family=" + std::to_string(family) + " variant=" + std::to_string(variant);
  if (shard_rows > 0) p += " shard_rows=" + std::to_string(shard_rows);
  return p + " | " + why;
}

void placement_flags(const std::string& placement, int* shard_rows, bool* replayed) {
  std::string key;
  int family = 0, variant = 0;
  if (!parse_placement(placement, &key, &family, &variant, shard_rows)) *shard_rows = 0;
  const size_t bar = placement.find(" | ");
  *replayed = bar != std::string::npos && placement.compare(bar + 3, std::strlen(kReplayedTag), kReplayedTag) == 0;
}

bool parse_placement(const std::string& placement, std::string* plan_key, int* family, int* variant,
                     int* shard_rows) {
  if (placement.rfind("plan=", 0) != 0) return false;
  std::istringstream is(placement);
  std::string a, b, c, d;
  is >> a >> b >> c >> d;
  if (b.rfind("family=", 0) != 0 || c.rfind("variant=", 0) != 0) return false;
  if (!to_int(b.substr(7), family) || !to_int(c.substr(8), variant)) return false;
  *shard_rows = 0;
  if (d.rfind("shard_rows=", 0) == 0 && !to_int(d.substr(11), shard_rows)) return false;
  *plan_key = a.substr(5);
  return true;
}

}  // namespace uk
