// Backend plugin contract of YiRage restated for the MI355X build, with the
// `hip` backend registered as BT_HIP.
//
// Mirrors include/yirage/backend/backend_interface.h:40-212 (pure virtual
// interface), backend_registry.h:40-166 (singleton registry, REGISTER_BACKEND)
// and src/backend/backend_registry.cc:28-197.  Unlike the reference, name
// lookup and the default query do not re-enter the registry mutex
// (backend_registry.cc:74-82,135-156 lock it twice and deadlock); every
// public method locks once and calls unlocked helpers.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "yr_common.h"

namespace yirage {
namespace type {

enum BackendType {
  BT_CUDA = 0,
  BT_MPS = 1,
  BT_CUDNN = 2,
  BT_CUSPARSELT = 3,
  BT_ASCEND = 4,
  BT_MACA = 5,
  BT_HIP = YR_BT_HIP,  // AMD Instinct (gfx950) -- this build
  BT_CPU = 10,
  BT_UNKNOWN = 999,
};

enum DataType {
  DT_FLOAT16 = YR_DTYPE_F16,
  DT_BFLOAT16 = YR_DTYPE_BF16,
  DT_FLOAT32 = YR_DTYPE_F32,
  DT_INT32 = YR_DTYPE_I32,
  DT_INT64 = YR_DTYPE_I64,
  DT_UNKNOWN = 999,
};

struct BackendInfo {
  BackendType type = BT_UNKNOWN;
  std::string name, display_name;
  bool requires_gpu = false;
  std::vector<std::string> required_libs;
};

}  // namespace type

namespace backend {

struct CompileContext {
  std::string source_code;
  std::string output_path;
  std::vector<std::string> include_dirs;
  std::vector<std::string> compile_flags;
  bool debug_mode = false;
  int optimization_level = 2;
};

class BackendInterface {
 public:
  virtual ~BackendInterface() = default;
  virtual type::BackendType get_type() const = 0;
  virtual std::string get_name() const = 0;
  virtual std::string get_display_name() const = 0;
  virtual bool is_available() const = 0;
  virtual type::BackendInfo get_info() const = 0;
  virtual bool compile(CompileContext const& ctx) = 0;
  virtual std::string get_compile_flags() const = 0;
  virtual std::vector<std::string> get_include_dirs() const = 0;
  virtual std::vector<std::string> get_library_dirs() const = 0;
  virtual std::vector<std::string> get_link_libraries() const = 0;
  virtual void* allocate_memory(size_t size) = 0;
  virtual void free_memory(void* ptr) = 0;
  virtual bool copy_to_device(void* dst, void const* src, size_t size) = 0;
  virtual bool copy_to_host(void* dst, void const* src, size_t size) = 0;
  virtual bool copy_device_to_device(void* dst, void const* src, size_t size) = 0;
  virtual void synchronize() = 0;
  virtual size_t get_max_memory() const = 0;
  virtual size_t get_max_shared_memory() const = 0;
  virtual bool supports_data_type(type::DataType dt) const = 0;
  virtual int get_compute_capability() const = 0;
  virtual int get_num_compute_units() const = 0;
  virtual bool set_device(int device_id) = 0;
  virtual int get_device() const = 0;
  virtual int get_device_count() const = 0;
};

class BackendRegistry {
 public:
  static BackendRegistry& get_instance() {
    static BackendRegistry inst;
    return inst;
  }

  bool register_backend(std::unique_ptr<BackendInterface> b) {
    if (!b) return false;
    std::lock_guard<std::mutex> lk(mu_);
    type::BackendType t = b->get_type();
    if (backends_.count(t)) return false;
    name_to_type_[b->get_name()] = t;
    order_.push_back(t);
    backends_[t] = std::move(b);
    return true;
  }

  BackendInterface* get_backend(type::BackendType t) {
    std::lock_guard<std::mutex> lk(mu_);
    return find_unlocked(t);
  }

  BackendInterface* get_backend(std::string const& name) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = name_to_type_.find(name);
    return it == name_to_type_.end() ? nullptr : find_unlocked(it->second);
  }

  std::vector<type::BackendType> get_registered_backends() const {
    std::lock_guard<std::mutex> lk(mu_);
    return order_;
  }

  std::vector<type::BackendType> get_available_backends() const {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<type::BackendType> r;
    for (auto t : order_)
      if (backends_.at(t)->is_available()) r.push_back(t);
    return r;
  }

  // priority: hip first, then registration order
  type::BackendType get_default_backend() const {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = backends_.find(type::BT_HIP);
    if (it != backends_.end() && it->second->is_available()) return type::BT_HIP;
    for (auto t : order_)
      if (backends_.at(t)->is_available()) return t;
    return type::BT_UNKNOWN;
  }

  bool unregister_backend(type::BackendType t) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = backends_.find(t);
    if (it == backends_.end()) return false;
    name_to_type_.erase(it->second->get_name());
    backends_.erase(it);
    for (size_t i = 0; i < order_.size(); i++)
      if (order_[i] == t) { order_.erase(order_.begin() + i); break; }
    return true;
  }

 private:
  BackendInterface* find_unlocked(type::BackendType t) {
    auto it = backends_.find(t);
    return it == backends_.end() ? nullptr : it->second.get();
  }
  mutable std::mutex mu_;
  std::map<type::BackendType, std::unique_ptr<BackendInterface>> backends_;
  std::map<std::string, type::BackendType> name_to_type_;
  std::vector<type::BackendType> order_;
};

#define REGISTER_BACKEND(BackendClass)                                                   \
  namespace {                                                                            \
  struct BackendClass##Registrar {                                                       \
    BackendClass##Registrar() {                                                          \
      ::yirage::backend::BackendRegistry::get_instance().register_backend(               \
          std::unique_ptr<::yirage::backend::BackendInterface>(new BackendClass()));     \
    }                                                                                    \
  };                                                                                     \
  static BackendClass##Registrar g_##BackendClass##_registrar;                           \
  }

// ------------------------------------------------------------------ HIPBackend
class HIPBackend : public BackendInterface {
 public:
  type::BackendType get_type() const override { return type::BT_HIP; }
  std::string get_name() const override { return "hip"; }
  std::string get_display_name() const override { return "AMD HIP (MI355X / gfx950)"; }

  // available when a gfx950 device is visible; device queries never abort
  bool is_available() const override {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return false;
    for (int i = 0; i < n; i++) {
      hipDeviceProp_t p;
      if (hipGetDeviceProperties(&p, i) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0)
        return true;
    }
    return false;
  }

  type::BackendInfo get_info() const override {
    type::BackendInfo i;
    i.type = get_type();
    i.name = get_name();
    i.display_name = get_display_name();
    i.requires_gpu = true;
    i.required_libs = {"amdhip64"};
    return i;
  }

  // Compiles a HIP source string into a shared object with hipcc.
  bool compile(CompileContext const& ctx) override {
    if (ctx.output_path.empty()) return false;
    std::string src = ctx.output_path + ".hip";
    FILE* f = fopen(src.c_str(), "w");
    if (!f) return false;
    fwrite(ctx.source_code.data(), 1, ctx.source_code.size(), f);
    fclose(f);
    std::string cmd = hipcc() + " " + get_compile_flags() + " -O" + std::to_string(ctx.optimization_level);
    if (ctx.debug_mode) cmd += " -g";
    for (auto& d : ctx.include_dirs) cmd += " -I" + d;
    for (auto& fl : ctx.compile_flags) cmd += " " + fl;
    cmd += " -shared -fPIC -o " + ctx.output_path + " " + src;
    return system(cmd.c_str()) == 0;
  }

  std::string get_compile_flags() const override {
    return "--offload-arch=gfx950 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops";
  }
  std::vector<std::string> get_include_dirs() const override { return {rocm() + "/include"}; }
  std::vector<std::string> get_library_dirs() const override { return {rocm() + "/lib"}; }
  std::vector<std::string> get_link_libraries() const override { return {"amdhip64"}; }

  void* allocate_memory(size_t size) override {
    void* p = nullptr;
    return hipMalloc(&p, size) == hipSuccess ? p : nullptr;
  }
  void free_memory(void* p) override {
    if (p) (void)hipFree(p);
  }
  bool copy_to_device(void* d, void const* s, size_t n) override {
    return hipMemcpy(d, s, n, hipMemcpyHostToDevice) == hipSuccess;
  }
  bool copy_to_host(void* d, void const* s, size_t n) override {
    return hipMemcpy(d, s, n, hipMemcpyDeviceToHost) == hipSuccess;
  }
  bool copy_device_to_device(void* d, void const* s, size_t n) override {
    return hipMemcpy(d, s, n, hipMemcpyDeviceToDevice) == hipSuccess;
  }
  void synchronize() override { (void)hipDeviceSynchronize(); }

  size_t get_max_memory() const override {
    hipDeviceProp_t p;
    return prop(p) ? p.totalGlobalMem : 0;
  }
  size_t get_max_shared_memory() const override {
    hipDeviceProp_t p;
    return prop(p) ? p.sharedMemPerBlock : 160 * 1024;
  }
  bool supports_data_type(type::DataType dt) const override {
    return dt == type::DT_FLOAT16 || dt == type::DT_BFLOAT16 || dt == type::DT_FLOAT32 ||
           dt == type::DT_INT32 || dt == type::DT_INT64;
  }
  int get_compute_capability() const override { return 950; }
  int get_num_compute_units() const override {
    hipDeviceProp_t p;
    return prop(p) ? p.multiProcessorCount : 0;
  }
  bool set_device(int id) override { return hipSetDevice(id) == hipSuccess; }
  int get_device() const override {
    int d = -1;
    return hipGetDevice(&d) == hipSuccess ? d : -1;
  }
  int get_device_count() const override {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess ? n : 0;
  }

 private:
  static std::string rocm() {
    const char* r = getenv("ROCM_PATH");
    return r ? r : "/opt/rocm";
  }
  static std::string hipcc() { return rocm() + "/bin/hipcc"; }
  bool prop(hipDeviceProp_t& p) const {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return false;
    return hipGetDeviceProperties(&p, d) == hipSuccess;
  }
};

REGISTER_BACKEND(HIPBackend)

// string <-> type (src/backend/backend_utils.cc:27-87, plus "hip")
static type::BackendType string_to_backend_type(std::string const& n) {
  static const std::map<std::string, type::BackendType> m = {
      {"cuda", type::BT_CUDA}, {"mps", type::BT_MPS},   {"cudnn", type::BT_CUDNN},
      {"ascend", type::BT_ASCEND}, {"maca", type::BT_MACA}, {"hip", type::BT_HIP},
      {"cpu", type::BT_CPU}};
  auto it = m.find(n);
  return it == m.end() ? type::BT_UNKNOWN : it->second;
}

}  // namespace backend
}  // namespace yirage

using yirage::backend::BackendRegistry;

static int copy_out(std::string const& s, char* buf, size_t n) {
  if (!buf || n == 0) return YR_E_INVALID;
  size_t k = s.size() < n - 1 ? s.size() : n - 1;
  memcpy(buf, s.data(), k);
  buf[k] = 0;
  return YR_OK;
}

extern "C" {

int yr_backend_num_registered(void) {
  return (int)BackendRegistry::get_instance().get_registered_backends().size();
}

int yr_backend_registered_name(int i, char* buf, size_t n) {
  auto v = BackendRegistry::get_instance().get_registered_backends();
  if (i < 0 || i >= (int)v.size()) return yr::fail(YR_E_INVALID, "backend index %d out of range", i);
  auto* b = BackendRegistry::get_instance().get_backend(v[i]);
  copy_out(b->get_name(), buf, n);
  return (int)v[i];
}

int yr_backend_is_available(const char* name) {
  if (!name) return 0;
  auto* b = BackendRegistry::get_instance().get_backend(std::string(name));
  return b && b->is_available() ? 1 : 0;
}

int yr_backend_type_from_name(const char* name) {
  return name ? (int)yirage::backend::string_to_backend_type(name) : YR_BT_UNKNOWN;
}

int yr_backend_default(char* buf, size_t n) {
  auto& r = BackendRegistry::get_instance();
  auto t = r.get_default_backend();
  if (t == yirage::type::BT_UNKNOWN) return copy_out("", buf, n);
  return copy_out(r.get_backend(t)->get_name(), buf, n);
}

int yr_backend_compile_flags(const char* name, char* buf, size_t n) {
  if (!name) return yr::fail(YR_E_INVALID, "null backend name");
  auto* b = BackendRegistry::get_instance().get_backend(std::string(name));
  if (!b) return yr::fail(YR_E_INVALID, "backend '%s' not registered", name);
  return copy_out(b->get_compile_flags(), buf, n);
}

}  // extern "C"
