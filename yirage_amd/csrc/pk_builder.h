// Host task-graph builder of the persistent megakernel (see pk_builder.cc).
#pragma once
#include <map>
#include <string>
#include <vector>

#include "pk_types.h"
#include "yr_common.h"

struct yr_pk_graph;

namespace yr {
namespace pk {

// Attention split records: at least 16 query rows x (head_dim + 2) floats
// (one MFMA row block); multi-token ops size them for max_tokens * G rows,
// at most kAttnMaxRows (eight row blocks, one per wave).
constexpr int kAttnRecRows = 16;
constexpr int kAttnMaxRows = 128;
// cached 64-position blocks one attention compute wave streams per task
constexpr int kAttnBlocksPerWave = 3;

struct Tensor {
  std::string name;
  uint64_t ptr = 0;
  std::vector<int64_t> dims;
  int dtype = 0;
  bool ll = false;  // link tensor: [rows][cols] tagged words, 4 bytes per element
};

// Column range [c0, c1) of a tensor (all rows).  scope: 0 = whole op range,
// 1 = the task's own output rows, 2 = the task's kv-head group.
struct Access {
  int tensor;  // -2: batch metadata
  int c0, c1;
  int scope = 0;
};

// A weight segment: rows [row0, row0 + rows) of tensor `tensor`.
struct WSeg {
  int tensor;
  int64_t row0, rows;
};

struct OpInfo {
  std::string name;
  int first_task = 0, num_tasks = 0;
  std::vector<Access> reads, writes;
  int kv_group_width = 0, kv_groups = 0, group_reads_qkv = -1;
  // operand tensors (-1: none), for the task-graph export
  int x = -1, out = -1, res = -1, norm = -1, tok = -1, table = -1, tok_out = -1, kc = -1, vc = -1, cos = -1,
      sin = -1, knorm = -1;
  std::vector<WSeg> wsegs;
  int group = 0, col0 = 0;
};

struct EventInfo {
  int num_triggers;
  int consumer_op;
};

struct BuildConfig {
  int max_tokens = 1, max_requests = 1, page_size = 64, max_pages = 0, max_seq_len = 0, total_requests = 1;
  int64_t eos_token_id = -1;
  int online = 0;  // PersistentKernel(mode="online")
};

struct Graph {
  int num_workers = 0;
  BuildConfig cfg;
  std::vector<Tensor> tensors;
  std::map<std::string, int> tensor_index;
  std::map<std::string, std::string> meta_names;
  std::vector<OpDesc> ops;
  std::vector<OpInfo> op_info;
  std::vector<TaskDesc> tasks;
  std::vector<EventInfo> events;
  std::vector<std::vector<int>> queues;
  int num_tickets = 0;
  int64_t scratch_floats = 0;
  std::vector<std::pair<uint64_t, uint64_t>> link_buffers;  // (device address, bytes), cleared on epoch re-base

  void build(const char* json_text);
  int tensor_id(const std::string& name) const;
  const Tensor& t(const std::string& name) const;
  std::string simulate(uint64_t seed, int epochs) const;
  std::string check_races(int window) const;
  std::string export_json() const;

 private:
  void make_events();
  void assign_workers();
};

}  // namespace pk
}  // namespace yr
