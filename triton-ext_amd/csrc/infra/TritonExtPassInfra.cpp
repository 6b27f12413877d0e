// Extension registry and pass manager: libTritonExtPassInfra.so.
//
// Behaviour of the four plugin entry points follows
// R:infra/pass/TritonExtPassInfra.cpp:7-52 (return codes, two-call
// enumeration, unknown-name failure).  The registry here is one ordered table
// under a mutex instead of two hash maps plus a name vector, so the count and
// the table cannot disagree and enumeration fills every slot.

#include "triton_ext/TritonExtPassInfra.h"

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace {

struct Extension {
  const char *name; // borrowed from the extension's rodata
  TritonExtRegisterPassFunc registerFunc;
  TritonExtAddPassFunc addFunc;
};

struct PassArgument {
  std::string arg;
  TxPassRunFunc run;
};

std::mutex &registryMutex() {
  static std::mutex m;
  return m;
}
std::vector<Extension> &extensions() {
  static std::vector<Extension> v;
  return v;
}
std::vector<PassArgument> &passArguments() {
  static std::vector<PassArgument> v;
  return v;
}

bool lookup(const char *name, Extension *out) {
  std::lock_guard<std::mutex> lock(registryMutex());
  for (const Extension &e : extensions())
    if (std::strcmp(e.name, name) == 0) {
      *out = e;
      return true;
    }
  return false;
}

} // namespace

struct TxPassManager {
  std::vector<PassArgument> passes;
};

extern "C" {

TRITON_PLUGIN_API
TritonExtLoadPass(const char *passName, TritonExtRegisterPassFunc registerFunc,
                  TritonExtAddPassFunc addFunc) {
  if (!passName || !registerFunc || !addFunc)
    return TP_GENERIC_FAILURE;
  std::lock_guard<std::mutex> lock(registryMutex());
  for (Extension &e : extensions())
    if (std::strcmp(e.name, passName) == 0) {
      e = Extension{passName, registerFunc, addFunc};
      return TP_SUCCESS;
    }
  extensions().push_back(Extension{passName, registerFunc, addFunc});
  return TP_SUCCESS;
}

TRITON_PLUGIN_API
tritonAddPluginPass(TxPassManager *pm, const char *passName) {
  if (!pm || !passName)
    return TP_GENERIC_FAILURE;
  Extension e;
  if (!lookup(passName, &e))
    return TP_GENERIC_FAILURE;
  e.addFunc(pm); // called outside the lock: it may register arguments
  return TP_SUCCESS;
}

TRITON_PLUGIN_API
tritonRegisterPluginPass(const char *passName) {
  if (!passName)
    return TP_GENERIC_FAILURE;
  Extension e;
  if (!lookup(passName, &e))
    return TP_GENERIC_FAILURE;
  e.registerFunc();
  return TP_SUCCESS;
}

TRITON_PLUGIN_API
tritonEnumeratePluginPasses(uint32_t *passCount, const char **passNames) {
  if (!passCount)
    return TP_GENERIC_FAILURE;
  std::lock_guard<std::mutex> lock(registryMutex());
  *passCount = static_cast<uint32_t>(extensions().size());
  if (!passNames)
    return TP_SUCCESS;
  for (size_t i = 0; i < extensions().size(); ++i)
    passNames[i] = extensions()[i].name;
  return TP_SUCCESS;
}

TxPassManager *txPassManagerCreate(void) { return new TxPassManager(); }

void txPassManagerDestroy(TxPassManager *pm) { delete pm; }

int txPassManagerAddPass(TxPassManager *pm, const char *argName,
                         TxPassRunFunc run) {
  if (!pm || !argName || !run)
    return 1;
  pm->passes.push_back(PassArgument{argName, run});
  return 0;
}

uint32_t txPassManagerSize(const TxPassManager *pm) {
  return pm ? static_cast<uint32_t>(pm->passes.size()) : 0;
}

const char *txPassManagerPassName(const TxPassManager *pm, uint32_t i) {
  if (!pm || i >= pm->passes.size())
    return nullptr;
  return pm->passes[i].arg.c_str();
}

int txPassManagerRun(TxPassManager *pm, tx_dot_plan *plan) {
  if (!pm || !plan)
    return 1;
  for (const PassArgument &p : pm->passes) {
    int rc = p.run(plan);
    if (rc != 0)
      return rc;
  }
  return 0;
}

int txRegisterPassArgument(const char *argName, TxPassRunFunc run) {
  if (!argName || !run)
    return 1;
  std::lock_guard<std::mutex> lock(registryMutex());
  for (PassArgument &a : passArguments())
    if (a.arg == argName) {
      a.run = run;
      return 0;
    }
  passArguments().push_back(PassArgument{argName, run});
  return 0;
}

int txPassManagerParsePipeline(TxPassManager *pm, const char *pipeline) {
  if (!pm || !pipeline)
    return 1;
  std::vector<PassArgument> parsed;
  std::string text(pipeline);
  size_t pos = 0;
  while (pos <= text.size()) {
    size_t comma = text.find(',', pos);
    if (comma == std::string::npos)
      comma = text.size();
    std::string arg = text.substr(pos, comma - pos);
    // trim spaces and an optional leading '-' (as in "-triton-loop-split")
    size_t b = arg.find_first_not_of(" \t");
    size_t e = arg.find_last_not_of(" \t");
    arg = (b == std::string::npos) ? std::string() : arg.substr(b, e - b + 1);
    while (!arg.empty() && arg[0] == '-')
      arg.erase(0, 1);
    if (!arg.empty()) {
      bool found = false;
      std::lock_guard<std::mutex> lock(registryMutex());
      for (const PassArgument &a : passArguments())
        if (a.arg == arg) {
          parsed.push_back(a);
          found = true;
          break;
        }
      if (!found)
        return 1;
    }
    pos = comma + 1;
  }
  for (const PassArgument &a : parsed)
    pm->passes.push_back(a);
  return 0;
}

int txReadExtConf(const char *dir, char *name, uint32_t nameCap, char *status,
                  uint32_t statusCap, char *hash, uint32_t hashCap) {
  if (!dir || !name || nameCap == 0)
    return 1;
  const char *files[2] = {"triton-ext.conf", "triton_ext.conf"};
  FILE *f = nullptr;
  for (const char *fn : files) {
    std::string path = std::string(dir) + "/" + fn;
    f = std::fopen(path.c_str(), "r");
    if (f)
      break;
  }
  if (!f)
    return 1;
  std::string content;
  char buf[256];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0)
    content.append(buf, n);
  std::fclose(f);
  // CMake-list format `name;status;hash` (R:cmake/utils.cmake:104-121);
  // defaults: status "experimental", hash "".
  std::vector<std::string> fields;
  size_t pos = 0;
  while (pos <= content.size()) {
    size_t semi = content.find(';', pos);
    if (semi == std::string::npos)
      semi = content.size();
    std::string fld = content.substr(pos, semi - pos);
    size_t b = fld.find_first_not_of(" \t\r\n");
    size_t e = fld.find_last_not_of(" \t\r\n");
    fields.push_back(b == std::string::npos ? std::string()
                                            : fld.substr(b, e - b + 1));
    pos = semi + 1;
  }
  std::string nm = fields.size() > 0 ? fields[0] : "";
  std::string st = fields.size() > 1 && !fields[1].empty() ? fields[1]
                                                           : "experimental";
  std::string hs = fields.size() > 2 ? fields[2] : "";
  if (nm.empty())
    return 1;
  auto put = [](const std::string &s, char *dst, uint32_t cap) {
    if (!dst || cap == 0)
      return;
    size_t len = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(dst, s.data(), len);
    dst[len] = '\0';
  };
  put(nm, name, nameCap);
  put(st, status, statusCap);
  put(hs, hash, hashCap);
  return 0;
}

} // extern "C"
