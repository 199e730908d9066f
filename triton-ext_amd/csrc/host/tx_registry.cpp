// Op registry and the plugin table.
//
// Mirrors the reference's registration surface: ops register themselves at
// static-initialisation time (support/Export.cpp:38-42 exportOp, driven by
// static initialisers such as support/ExportPass.cpp:38-40), and
// txGetPluginInfo materialises the table (support/Export.cpp:58-97).  Two
// differences: the table is released by txReleasePluginInfo (the reference
// declares tritonReleasePluginInfo, support/Export.h:17, but never defines
// it), and entries are kept in registration order in a vector rather than an
// unordered map, so the table order is deterministic.
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "tx_ops.h"
#include "tx_runtime.h"

#ifndef TX_VERSION_STRING
#define TX_VERSION_STRING "0.1.0"
#endif

namespace tx {
namespace {

struct Entry {
  std::string name;
  tx_op_fn fn;
  std::string signature;
};

std::vector<Entry> &registry() {
  static std::vector<Entry> r;  // constructed on first use
  return r;
}

}  // namespace

bool register_op(const char *name, tx_op_fn fn, const char *signature) {
  for (auto &e : registry())
    if (e.name == name) {
      e.fn = fn;
      e.signature = signature;
      return true;
    }
  registry().push_back(Entry{name, fn, signature});
  return true;
}

}  // namespace tx

extern "C" {

TX_API const tx_plugin_info *txGetPluginInfo(void) {
  const auto &r = tx::registry();
  tx_op_info *ops = new (std::nothrow) tx_op_info[r.size() ? r.size() : 1];
  tx_plugin_info *info = new (std::nothrow) tx_plugin_info;
  if (!ops || !info) {
    delete[] ops;
    delete info;
    tx::fail(TX_GENERIC_FAILURE, "out of host memory building the op table");
    return nullptr;
  }
  for (size_t i = 0; i < r.size(); ++i)
    ops[i] = tx_op_info{r[i].name.c_str(), r[i].fn, r[i].signature.c_str()};
  *info = tx_plugin_info{TX_PLUGIN_API_VERSION, "txamd", TX_VERSION_STRING, ops,
                         r.size(), "gfx950"};
  return info;
}

TX_API void txReleasePluginInfo(const tx_plugin_info *info) {
  if (!info) return;
  delete[] info->ops;
  delete info;
}

TX_API const tx_op_info *txFindOp(const char *name) {
  if (!name) return nullptr;
  static thread_local tx_op_info found;
  for (const auto &e : tx::registry())
    if (e.name == name) {
      found = tx_op_info{e.name.c_str(), e.fn, e.signature.c_str()};
      return &found;
    }
  return nullptr;
}

TX_API tx_status txInvokeOp(const char *name, tx_value *operands,
                            size_t num_operands, tx_stream_t stream) {
  tx::clear_error();
  const tx_op_info *op = txFindOp(name);
  if (!op)
    return tx::fail(TX_UNKNOWN_OP, "no op named '%s' is registered",
                    name ? name : "(null)");
  return op->fn(operands, num_operands, stream);
}

TX_API const char *txVersion(void) { return TX_VERSION_STRING; }

}  // extern "C"
