// Host-side task-graph builder, CPU protocol simulator and race checker for
// the persistent megakernel.
//
// Restates the reference's task-graph construction (src/kernel/runtime.cc:
// 161-538 register_mugraph, 540-600 sanity_check, 847-1318 JSON schema)
// for this backend's op set:
//   * each op ("layer") expands into tasks covering disjoint output ranges;
//   * consecutive ops are joined by events: a barrier event (all producer
//     tasks) or, when a paged-attention op consumes the QKV projection,
//     one event per kv-head group (the reference's gcd partitioning,
//     runtime.cc:53-159, specialised to that edge);
//   * tasks go to per-worker queues in op order (round-robin with a rotating
//     start), which with co-resident workers makes the schedule deadlock-free.
// The simulator replays the queue/event protocol on the CPU with random
// interleavings; the race checker proves that every pair of conflicting
// tensor accesses is ordered by the event graph.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <random>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "json_min.h"
#include "pk_builder.h"

namespace yr {
namespace pk {

static int dtype_bytes(int dt) {
  switch (dt) {
    case YR_DTYPE_F16: case YR_DTYPE_BF16: return 2;
    case YR_DTYPE_F32: case YR_DTYPE_I32: return 4;
    case YR_DTYPE_I64: return 8;
  }
  return 0;
}

using Seg = WSeg;

static std::vector<Seg> read_segments(Graph& g, const json::Value& v) {
  std::vector<Seg> segs;
  if (v.kind == json::Value::Str) {
    int t = g.tensor_id(v.s());
    segs.push_back({t, 0, g.tensors[t].dims[0]});
    return segs;
  }
  for (size_t i = 0; i < v.size(); i++) {
    const json::Value& s = v[i];
    int t = g.tensor_id(s[0].s());
    Seg sg{t, s[1].i64(), s[2].i64()};
    if (sg.row0 < 0 || sg.row0 + sg.rows > g.tensors[t].dims[0])
      throw std::runtime_error("weight segment out of range for tensor " + g.tensors[t].name);
    segs.push_back(sg);
  }
  return segs;
}

// Device address of virtual weight rows [r, r + n) (must lie in one segment).
static const uint16_t* seg_rows(Graph& g, const std::vector<Seg>& segs, int64_t r, int64_t n, int64_t K) {
  int64_t base = 0;
  for (auto& s : segs) {
    if (r >= base && r < base + s.rows) {
      if (r + n > base + s.rows)
        throw std::runtime_error("task rows straddle two weight segments; choose rows_per_task dividing the segments");
      const Tensor& t = g.tensors[s.tensor];
      if (t.dims.size() != 2 || t.dims[1] != K) throw std::runtime_error("weight " + t.name + " is not [rows, K]");
      return (const uint16_t*)(t.ptr + (uint64_t)((s.row0 + (r - base)) * K * 2));
    }
    base += s.rows;
  }
  throw std::runtime_error("task rows beyond the weight segments");
}

// Rows left in the segment that holds virtual row r.
static int64_t seg_remaining(const std::vector<Seg>& segs, int64_t r) {
  int64_t base = 0;
  for (auto& s : segs) {
    if (r >= base && r < base + s.rows) return base + s.rows - r;
    base += s.rows;
  }
  throw std::runtime_error("row beyond the weight segments");
}

static int64_t seg_total(const std::vector<Seg>& segs) {
  int64_t n = 0;
  for (auto& s : segs) n += s.rows;
  return n;
}

int Graph::tensor_id(const std::string& name) const {
  auto it = tensor_index.find(name);
  if (it == tensor_index.end()) throw std::runtime_error("unknown tensor '" + name + "'");
  return it->second;
}

const Tensor& Graph::t(const std::string& name) const { return tensors[tensor_id(name)]; }

static void need_dtype(const Tensor& t, int dt, const char* what) {
  if (t.dtype != dt) throw std::runtime_error(std::string(what) + ": tensor " + t.name + " has the wrong dtype");
}

static int ptr_tensor(Graph& g, const json::Value& op, const char* key, bool optional = false) {
  if (!op.has(key)) {
    if (optional) return -1;
    throw std::runtime_error(std::string("op is missing '") + key + "'");
  }
  return g.tensor_id(op[key].s());
}

void Graph::build(const char* text) {
  json::Value root = json::parse(text);
  num_workers = (int)root["num_workers"].i64(0);
  if (num_workers <= 0 || num_workers > 4096) throw std::runtime_error("num_workers must be in 1..4096");
  cfg.max_tokens = (int)root["max_tokens"].i64(1);
  cfg.max_requests = (int)root["max_requests"].i64(1);
  cfg.page_size = (int)root["page_size"].i64(64);
  cfg.max_pages = (int)root["max_pages"].i64(0);
  cfg.max_seq_len = (int)root["max_seq_len"].i64(0);
  cfg.total_requests = (int)root["total_requests"].i64(cfg.max_requests);
  cfg.eos_token_id = root["eos_token_id"].i64(-1);
  cfg.online = (int)root["online"].i64(0);

  const json::Value& tv = root["tensors"];
  if (tv.kind != json::Value::Obj) throw std::runtime_error("'tensors' must be an object");
  for (auto& kv : tv.obj) {
    Tensor t;
    t.name = kv.first;
    t.ptr = (uint64_t)kv.second["ptr"].f64();
    for (size_t i = 0; i < kv.second["dims"].size(); i++) t.dims.push_back(kv.second["dims"][i].i64());
    t.dtype = (int)kv.second["dtype"].i64();
    t.ll = kv.second.has("ll") && kv.second["ll"].i64(0) != 0;
    if (!dtype_bytes(t.dtype)) throw std::runtime_error("tensor " + t.name + ": unsupported dtype");
    if (t.ll) {
      if (t.dtype != YR_DTYPE_BF16 || t.dims.size() != 2 || t.dims[1] % 4)
        throw std::runtime_error("link tensor " + t.name + " must be 2-D bf16 with columns % 4 == 0");
      link_buffers.push_back({t.ptr, (uint64_t)(t.dims[0] * t.dims[1] * 4)});
    }
    tensor_index[t.name] = (int)tensors.size();
    tensors.push_back(t);
  }
  const json::Value& mv = root["meta"];
  if (mv.kind == json::Value::Obj)
    for (auto& kv : mv.obj) meta_names[kv.first] = kv.second.s();

  const json::Value& opsv = root["ops"];
  if (opsv.kind != json::Value::Arr || opsv.size() == 0) throw std::runtime_error("'ops' must be a non-empty array");
  int ticket_next = 0;
  int64_t scratch_next = 0;
  if (opsv.size() > (size_t)kMaxLinkOps) throw std::runtime_error("too many ops for the link-tensor tag");
  // op that last wrote each link tensor (readers check its tag)
  std::vector<int> link_writer(tensors.size(), -1);
  auto link_read = [&](int tensor, int& src) -> bool {
    if (!tensors[tensor].ll) return false;
    if (link_writer[tensor] < 0)
      throw std::runtime_error("link tensor " + tensors[tensor].name + " is read before any op writes it");
    src = link_writer[tensor];
    return true;
  };
  for (size_t oi = 0; oi < opsv.size(); oi++) {
    const json::Value& o = opsv[oi];
    const std::string type = o["type"].s();
    OpDesc d;
    memset(&d, 0, sizeof(d));
    OpInfo info;
    info.name = type;
    int first_task = (int)tasks.size();
    auto add_task = [&](TaskDesc td) {
      td.op = (int)ops.size();
      td.wait_event = -1;
      td.trigger_event = -1;
      tasks.push_back(td);
    };
    if (type == "embed") {
      d.type = TASK_EMBED;
      int tok = ptr_tensor(*this, o, "tokens"), tab = ptr_tensor(*this, o, "table"), out = ptr_tensor(*this, o, "out");
      need_dtype(tensors[tok], YR_DTYPE_I64, "embed tokens");
      const Tensor& T = tensors[tab];
      d.K = (int)T.dims[1];
      d.N = d.K;
      d.vocab = (int)T.dims[0];
      d.out_ld = (int)tensors[out].dims[1];
      d.max_tokens = cfg.max_tokens;
      d.tokens_in = (const int64_t*)tensors[tok].ptr;
      d.table = (const uint16_t*)T.ptr;
      d.out = (uint16_t*)tensors[out].ptr;
      if (tensors[out].ll) {
        d.flags |= OPF_OUT_LL;
        link_writer[out] = (int)ops.size();
      }
      int nt = (int)o["tasks"].i64(1);
      int per = (d.N + nt - 1) / nt;
      per = (per + 7) & ~7;
      for (int r = 0; r < d.N; r += per) {
        TaskDesc td;
        memset(&td, 0, sizeof(td));
        td.row0 = r;
        td.rows = std::min(per, d.N - r);
        add_task(td);
      }
      info.writes.push_back({out, 0, d.N, 1});
      info.tok = tok;
      info.table = tab;
      info.out = out;
    } else if (type == "linear" || type == "rmsnorm_linear" || type == "rmsnorm_linear_silu" ||
               type == "rmsnorm_linear_argmax") {
      bool norm = type != "linear";
      bool silu = type == "rmsnorm_linear_silu";
      bool amax = type == "rmsnorm_linear_argmax";
      d.type = type == "linear" ? TASK_LINEAR : silu ? TASK_RMSNORM_LINEAR_SILU
                                             : amax ? TASK_RMSNORM_LINEAR_ARGMAX : TASK_RMSNORM_LINEAR;
      int x = ptr_tensor(*this, o, "x"), out = ptr_tensor(*this, o, "out");
      const Tensor& X = tensors[x];
      need_dtype(X, YR_DTYPE_BF16, "linear x");
      d.K = (int)X.dims[1];
      d.x_ld = d.K;
      d.x = (const uint16_t*)X.ptr;
      if (link_read(x, d.x_src)) d.flags |= OPF_X_LL;
      d.max_tokens = cfg.max_tokens;
      if (X.dims[0] < cfg.max_tokens) throw std::runtime_error("activation rows < max_tokens");
      std::vector<Seg> segs = read_segments(*this, o["weight"]);
      int64_t wrows = seg_total(segs);
      int group = (int)o["group"].i64(0);
      d.N = silu ? (int)(wrows / 2) : (int)wrows;
      if (silu && (group <= 0 || wrows % (2 * group))) throw std::runtime_error("silu op: bad 'group'");
      const Tensor& OT = tensors[out];
      d.out_ld = (int)OT.dims[1];
      int col0 = (int)o["out_col0"].i64(0);
      if (col0 + d.N > d.out_ld) throw std::runtime_error("linear output columns exceed the out tensor");
      d.out = (uint16_t*)(OT.ptr + (uint64_t)col0 * (OT.ll ? 4 : 2));
      if (OT.ll && amax) throw std::runtime_error("argmax logits must be a plain tensor");
      if (norm) {
        int nw = ptr_tensor(*this, o, "norm");
        d.norm = (const uint16_t*)tensors[nw].ptr;
        d.eps = (float)o["eps"].f64(1e-6);
        info.reads.push_back({nw, 0, d.K});
      }
      int res = ptr_tensor(*this, o, "residual", true);
      if (res >= 0) {
        d.flags |= OPF_RESIDUAL;
        if (link_read(res, d.res_src)) d.flags |= OPF_RES_LL;
        d.residual = (const uint16_t*)tensors[res].ptr;
        d.res_ld = (int)tensors[res].dims[1];
        info.reads.push_back({res, 0, d.N, 1});
      }
      if (amax) {
        int to = ptr_tensor(*this, o, "tokens_out");
        need_dtype(tensors[to], YR_DTYPE_I64, "argmax tokens_out");
        d.tokens_out = (int64_t*)tensors[to].ptr;
        d.vocab = (int)o["vocab"].i64(d.N);
        info.writes.push_back({to, 0, 1});
      }
      int rpt = (int)o["rows_per_task"].i64(16);
      if (rpt <= 0 || rpt % 2) throw std::runtime_error("rows_per_task must be even and > 0");
      if (cfg.max_tokens > 16) throw std::runtime_error("max_tokens must be <= 16");
      {
        // per-wave partial-sum slots of a task in LDS (8192 floats): [rows + 7]
        // at one token, [16-row tiles + 7] x 16 x (8 or 16) tokens; the argmax
        // epilogue keeps [tokens][rows] floats
        const int rt = silu ? 2 * rpt : rpt;
        const int tm = cfg.max_tokens == 1 ? 1 : (cfg.max_tokens <= 8 ? 8 : 16);
        const int64_t slots = tm == 1 ? (int64_t)rt + 7 : ((int64_t)(rt + 15) / 16 + 7) * 16 * tm;
        if (slots > 8192) throw std::runtime_error("rows_per_task too large for the partial-sum slots");
        if (amax && (int64_t)tm * rpt > 8192) throw std::runtime_error("argmax: rows_per_task x tokens > 8192");
      }
      if (col0 % 2 || d.out_ld % 2) throw std::runtime_error("linear output columns must be even-aligned");
      // the staged activation block holds all of K at <= 8 tokens (RMSNorm
      // needs the whole row there); 16-token batches normalize while staging
      if (norm && (cfg.max_tokens == 1 ? d.K > 32768 : cfg.max_tokens <= 8 ? d.K > 4096 : d.K > 16384))
        throw std::runtime_error("rmsnorm input too wide for the staged activation block");
      if (cfg.max_tokens > 1 && d.K > 4096 && rpt > 7 * 3 * (silu ? 1 : 1))
        throw std::runtime_error("batch > 1 with K > 4096: rows_per_task must be <= 21");
      if (silu && group % rpt) throw std::runtime_error("silu op: rows_per_task must divide 'group'");
      int ntasks = (d.N + rpt - 1) / rpt;
      int ordinal = 0;
      for (int r = 0; r < d.N; r += rpt) {
        TaskDesc td;
        memset(&td, 0, sizeof(td));
        td.row0 = r;
        td.rows = std::min(rpt, d.N - r);
        if (silu) {
          int64_t gi = r / group, j = r % group;
          td.w0 = seg_rows(*this, segs, gi * 2 * group + j, td.rows, d.K);
          td.w1 = seg_rows(*this, segs, gi * 2 * group + group + j, td.rows, d.K);
        } else {
          // a task may straddle one segment boundary (e.g. the q/k rows of a
          // per-kv-group shuffled QKV weight): rows [0, split_row) from w0
          int64_t in_first = seg_remaining(segs, r);
          if (in_first >= td.rows) {
            td.w0 = seg_rows(*this, segs, r, td.rows, d.K);
            td.split_row = td.rows;
          } else {
            td.w0 = seg_rows(*this, segs, r, in_first, d.K);
            td.w1 = seg_rows(*this, segs, r + in_first, td.rows - in_first, d.K);
            td.split_row = (int)in_first;
          }
        }
        td.i0 = ordinal++;
        td.i1 = ntasks;
        add_task(td);
      }
      if (amax) {
        d.ticket_base = ticket_next;
        ticket_next += 1;
        d.scratch_off = (int)scratch_next;
        scratch_next += (int64_t)ntasks * cfg.max_tokens * 2;
      }
      info.reads.push_back({x, 0, d.K});
      info.writes.push_back({out, col0, col0 + d.N, 1});
      info.x = x;
      info.out = out;
      info.res = res;
      info.norm = norm ? ptr_tensor(*this, o, "norm") : -1;
      info.tok_out = amax ? ptr_tensor(*this, o, "tokens_out") : -1;
      info.wsegs = segs;
      info.group = group;
      info.col0 = col0;
      if (OT.ll) {
        d.flags |= OPF_OUT_LL;
        link_writer[out] = (int)ops.size();
      }
    } else if (type == "attention") {
      d.type = TASK_ATTENTION;
      int qkv = ptr_tensor(*this, o, "qkv"), out = ptr_tensor(*this, o, "out");
      int kc = ptr_tensor(*this, o, "k_cache"), vc = ptr_tensor(*this, o, "v_cache");
      d.num_q_heads = (int)o["num_q_heads"].i64();
      d.num_kv_heads = (int)o["num_kv_heads"].i64();
      d.head_dim = (int)o["head_dim"].i64(128);
      d.splits = (int)o["splits"].i64(1);
      // a split holds at most 7 compute waves x blocks_per_wave x 64
      // cached positions
      // empty_merger: one more split than the cached positions need, which
      // reads none of them and only appends and merges -- kept only while
      // every attention task still gets a worker of its own
      bool empty_merger = o.has("empty_merger") && o["empty_merger"].i64(0) != 0 && d.splits > 1;
      const int bpw = (int)o["blocks_per_wave"].i64(kAttnBlocksPerWave);
      if (bpw < 1 || bpw > 64) throw std::runtime_error("attention: blocks_per_wave must be 1..64");
      d.attn_blocks = 7 * bpw;
      const int per_split = 7 * bpw * 64;
      const int min_cached = (cfg.max_seq_len + per_split - 1) / per_split;
      int cached = empty_merger ? d.splits - 1 : d.splits;
      if (cached < min_cached) cached = min_cached;
      if (empty_merger && (int64_t)(cached + 1) * cfg.max_requests * d.num_kv_heads > num_workers) empty_merger = false;
      d.splits = empty_merger ? cached + 1 : cached;
      d.page_size = cfg.page_size;
      if (d.head_dim != 128) throw std::runtime_error("attention: head_dim must be 128");
      if (d.num_kv_heads <= 0 || d.num_q_heads % d.num_kv_heads) throw std::runtime_error("attention: bad heads");
      int G = d.num_q_heads / d.num_kv_heads;
      if (G > 16) throw std::runtime_error("attention: group size > 16");
      if (d.splits <= 0 || d.splits > 256) throw std::runtime_error("attention: splits must be 1..256");
      const Tensor& Q = tensors[qkv];
      d.qkv_ld = (int)Q.dims[1];
      if (d.qkv_ld != (d.num_q_heads + 2 * d.num_kv_heads) * d.head_dim)
        throw std::runtime_error("attention: qkv width must be (Hq + 2 Hkv) * head_dim");
      d.x = (const uint16_t*)Q.ptr;
      if (link_read(qkv, d.x_src)) d.flags |= OPF_X_LL;
      d.out = (uint16_t*)tensors[out].ptr;
      d.out_ld = (int)tensors[out].dims[1];
      if (tensors[out].ll) {
        d.flags |= OPF_OUT_LL;
        link_writer[out] = (int)ops.size();
      }
      if (empty_merger) d.flags |= OPF_EMPTY_MERGER;
      const Tensor& KC = tensors[kc];
      if (cfg.page_size != 64) throw std::runtime_error("attention: page_size must be 64");
      if (KC.dims.size() != 4 || KC.dims[1] != cfg.page_size || KC.dims[2] != d.num_kv_heads || KC.dims[3] != d.head_dim)
        throw std::runtime_error("attention: cache must be [pages, page_size, Hkv, head_dim]");
      d.k_cache = (uint16_t*)KC.ptr;
      d.v_cache = (uint16_t*)tensors[vc].ptr;
      int ct = ptr_tensor(*this, o, "cos", true), st = ptr_tensor(*this, o, "sin", true);
      d.cos_t = ct >= 0 ? (const uint16_t*)tensors[ct].ptr : nullptr;
      d.sin_t = st >= 0 ? (const uint16_t*)tensors[st].ptr : nullptr;
      // qk-norm (paged_attention_layer(q_norm=..., k_norm=...)): both or neither, [head_dim] each, eps 1e-6
      // as the reference's task passes it (task_register.cc:294-295)
      int qn = ptr_tensor(*this, o, "q_norm", true), kn = ptr_tensor(*this, o, "k_norm", true);
      if ((qn >= 0) != (kn >= 0)) throw std::runtime_error("attention: q_norm and k_norm come together");
      if (qn >= 0) {
        for (int w : {qn, kn})
          if (tensors[w].dims.size() != 1 || tensors[w].dims[0] != d.head_dim)
            throw std::runtime_error("attention: q_norm / k_norm must be [head_dim]");
        d.flags |= OPF_QK_NORM;
        d.norm = (const uint16_t*)tensors[qn].ptr;
        d.k_norm = (const uint16_t*)tensors[kn].ptr;
        d.eps = 1e-6f;
      }
      info.norm = qn;
      info.knorm = kn;
      d.max_tokens = cfg.max_tokens;
      d.ticket_base = ticket_next;
      ticket_next += cfg.max_requests * d.num_kv_heads;
      // split records hold every query row of a request: up to max_tokens * G
      // (rows beyond one 16-row MFMA block go to the multi-token task body)
      d.rec_rows = std::max(kAttnRecRows, (cfg.max_tokens * G + 15) / 16 * 16);
      if (cfg.max_tokens * G > kAttnMaxRows)
        throw std::runtime_error("attention: max_tokens * (q heads per kv head) must be <= " +
                                 std::to_string(kAttnMaxRows));
      scratch_next = (scratch_next + 31) / 32 * 32;  // 16-byte loads of the records
      d.scratch_off = (int)scratch_next;
      // records of tagged 8-byte words {f32, tag}: 2 floats per value
      scratch_next += (int64_t)cfg.max_requests * d.num_kv_heads * d.splits * d.rec_rows * (d.head_dim + 2) * 2;
      if (scratch_next >= (1ll << 31)) throw std::runtime_error("attention: split records exceed 2^31 floats");
      // with an empty merger the merging splits come last, so they land on
      // consecutive workers (which the next linear op can leave free)
      const int S = d.splits, S0 = empty_merger ? S - 1 : S;
      for (int pass = 0; pass < (empty_merger ? 2 : 1); pass++)
        for (int r = 0; r < cfg.max_requests; r++)
          for (int h = 0; h < d.num_kv_heads; h++)
            for (int s = pass ? S0 : 0; s < (pass ? S : S0); s++) {
              TaskDesc td;
              memset(&td, 0, sizeof(td));
              td.i0 = r;
              td.i1 = h;
              td.i2 = s;
              td.row0 = h * (G + 2) * d.head_dim;
              td.rows = (G + 2) * d.head_dim;
              add_task(td);
            }
      info.reads.push_back({qkv, 0, d.qkv_ld, 2});
      info.writes.push_back({out, 0, d.num_q_heads * d.head_dim, 2});
      info.x = qkv;
      info.out = out;
      info.kc = kc;
      info.vc = vc;
      info.cos = ct;
      info.sin = st;
      info.kv_group_width = (G + 2) * d.head_dim;
      info.kv_groups = d.num_kv_heads;
      info.group_reads_qkv = qkv;
    } else if (type == "prepare_batch") {
      d.type = TASK_PREPARE_BATCH;
      TaskDesc td;
      memset(&td, 0, sizeof(td));
      add_task(td);
      info.writes.push_back({-2, 0, 1});  // batch metadata
    } else {
      throw std::runtime_error("unknown op type '" + type + "'");
    }
    info.first_task = first_task;
    info.num_tasks = (int)tasks.size() - first_task;
    if (info.num_tasks == 0) throw std::runtime_error("op '" + type + "' produced no tasks");
    ops.push_back(d);
    op_info.push_back(info);
  }
  num_tickets = ticket_next;
  scratch_floats = scratch_next;
  if (num_tickets > 16384) throw std::runtime_error("too many arrival tickets");
  // every op reads the batch metadata written by prepare_batch
  for (auto& oi : op_info)
    if (!(oi.writes.size() && oi.writes[0].tensor == -2)) oi.reads.push_back({-2, 0, 1});
  make_events();
  assign_workers();
}

void Graph::make_events() {
  events.clear();
  for (size_t i = 1; i < ops.size(); i++) {
    OpInfo& prod = op_info[i - 1];
    OpInfo& cons = op_info[i];
    bool grouped = false;
    if (ops[i].type == TASK_ATTENTION && prod.writes.size() && prod.writes[0].tensor == cons.group_reads_qkv) {
      // producer tasks must each fall inside one kv group of the qkv tensor
      grouped = true;
      int W = cons.kv_group_width;
      int col0 = prod.writes[0].c0;
      for (int t = prod.first_task; t < prod.first_task + prod.num_tasks; t++) {
        int a = col0 + tasks[t].row0, b = a + tasks[t].rows - 1;
        if (a / W != b / W) { grouped = false; break; }
      }
    }
    if (grouped) {
      int W = cons.kv_group_width;
      int col0 = prod.writes[0].c0;
      int base = (int)events.size();
      for (int g = 0; g < cons.kv_groups; g++) events.push_back(EventInfo{0, (int)i});
      for (int t = prod.first_task; t < prod.first_task + prod.num_tasks; t++) {
        int g = (col0 + tasks[t].row0) / W;
        tasks[t].trigger_event = base + g;
        events[base + g].num_triggers++;
      }
      for (int t = cons.first_task; t < cons.first_task + cons.num_tasks; t++) {
        int g = tasks[t].i1;
        if (events[base + g].num_triggers == 0) throw std::runtime_error("kv group without producer tasks");
        tasks[t].wait_event = base + g;
        tasks[t].wait_count = events[base + g].num_triggers;
      }
    } else {
      int e = (int)events.size();
      events.push_back(EventInfo{prod.num_tasks, (int)i});
      for (int t = prod.first_task; t < prod.first_task + prod.num_tasks; t++) tasks[t].trigger_event = e;
      for (int t = cons.first_task; t < cons.first_task + cons.num_tasks; t++) {
        tasks[t].wait_event = e;
        tasks[t].wait_count = prod.num_tasks;
      }
    }
  }
}

void Graph::assign_workers() {
  queues.assign(num_workers, {});
  int start = 0;
  for (auto& oi : op_info) {
    for (int j = 0; j < oi.num_tasks; j++) queues[(start + j) % num_workers].push_back(oi.first_task + j);
    start = (start + oi.num_tasks) % num_workers;
  }
}

// ------------------------------------------------------------------ simulator
std::string Graph::simulate(uint64_t seed, int epochs) const {
  std::mt19937_64 rng(seed);
  std::vector<int64_t> counters(events.size(), 0);
  std::vector<int> executed(tasks.size(), 0);
  for (int ep = 1; ep <= epochs; ep++) {
    std::vector<size_t> pos(num_workers, 0);
    size_t remaining = tasks.size();
    std::vector<int> ready;
    while (remaining) {
      ready.clear();
      for (int w = 0; w < num_workers; w++) {
        if (pos[w] >= queues[w].size()) continue;
        const TaskDesc& t = tasks[queues[w][pos[w]]];
        if (t.wait_event < 0 || counters[t.wait_event] >= (int64_t)t.wait_count * ep) ready.push_back(w);
      }
      if (ready.empty()) {
        std::ostringstream os;
        os << "deadlock in epoch " << ep << " with " << remaining << " tasks left";
        for (int w = 0; w < num_workers; w++)
          if (pos[w] < queues[w].size()) {
            const TaskDesc& t = tasks[queues[w][pos[w]]];
            os << "; worker " << w << " blocked on task " << queues[w][pos[w]] << " (event " << t.wait_event
               << ": " << counters[t.wait_event] << "/" << (int64_t)t.wait_count * ep << ")";
            break;
          }
        return os.str();
      }
      int w = ready[rng() % ready.size()];
      int tid = queues[w][pos[w]++];
      executed[tid]++;
      if (tasks[tid].trigger_event >= 0) {
        counters[tasks[tid].trigger_event]++;
        if (counters[tasks[tid].trigger_event] > (int64_t)events[tasks[tid].trigger_event].num_triggers * ep)
          return "event over-triggered: " + std::to_string(tasks[tid].trigger_event);
      }
      remaining--;
    }
    for (size_t e = 0; e < events.size(); e++)
      if (counters[e] != (int64_t)events[e].num_triggers * ep)
        return "event " + std::to_string(e) + " did not reach its trigger count";
  }
  for (size_t t = 0; t < tasks.size(); t++)
    if (executed[t] != epochs) return "task " + std::to_string(t) + " executed " + std::to_string(executed[t]) + " times";
  return "";
}

// ------------------------------------------------------------------ races
// For every pair of ops (a, b), a < b, whose tasks touch overlapping columns
// of one tensor with at least one write, every conflicting task pair must be
// ordered: b's task transitively waits for a's task through the events, or
// both run on the same worker with a first.  Reachability is propagated as
// per-task bitsets over the tasks of op a, within a window of ops.
std::string Graph::check_races(int window) const {
  auto overlap = [](const Access& x, const Access& y) {
    return x.tensor == y.tensor && x.c0 < y.c1 && y.c0 < x.c1;
  };
  // per-task access ranges (attention tasks touch one kv group; linear tasks
  // their own output columns)
  auto task_access = [&](int op, int t, std::vector<Access>& rd, std::vector<Access>& wr) {
    const OpInfo& oi = op_info[op];
    const TaskDesc& td = tasks[t];
    const OpDesc& od = ops[op];
    int G = od.type == TASK_ATTENTION ? od.num_q_heads / od.num_kv_heads : 0;
    auto fix = [&](std::vector<Access>& v, bool is_write) {
      for (auto& a : v) {
        if (a.scope == 1) {          // own output columns (base + row0 .. + rows)
          int base = a.c0;
          a.c0 = base + td.row0;
          a.c1 = a.c0 + td.rows;
        } else if (a.scope == 2) {   // kv-head group
          if (is_write) {
            a.c0 = td.i1 * G * od.head_dim;
            a.c1 = a.c0 + G * od.head_dim;
          } else {
            a.c0 = td.row0;
            a.c1 = td.row0 + td.rows;
          }
        }
      }
    };
    rd = oi.reads;
    wr = oi.writes;
    fix(rd, false);
    fix(wr, true);
  };
  // worker position of every task
  std::vector<int> worker(tasks.size()), qpos(tasks.size());
  for (int w = 0; w < num_workers; w++)
    for (size_t i = 0; i < queues[w].size(); i++) {
      worker[queues[w][i]] = w;
      qpos[queues[w][i]] = (int)i;
    }
  // producers of each event
  std::vector<std::vector<int>> producers(events.size());
  for (size_t t = 0; t < tasks.size(); t++)
    if (tasks[t].trigger_event >= 0) producers[tasks[t].trigger_event].push_back((int)t);

  int nops = (int)ops.size();
  int64_t checked = 0;
  for (int a = 0; a < nops; a++) {
    const OpInfo& A = op_info[a];
    // reach[t] (t in ops a+1 .. a+window): bitset over A's tasks already done
    int last = std::min(nops - 1, a + window);
    int na = A.num_tasks;
    int words = (na + 63) / 64;
    std::vector<std::vector<uint64_t>> reach(tasks.size());
    auto get = [&](int t) -> std::vector<uint64_t>& {
      if (reach[t].empty()) reach[t].assign(words, 0);
      return reach[t];
    };
    for (int b = a + 1; b <= last; b++) {
      const OpInfo& B = op_info[b];
      for (int t = B.first_task; t < B.first_task + B.num_tasks; t++) {
        std::vector<uint64_t>& r = get(t);
        if (qpos[t] > 0) {  // the worker's previous task finished first
          int p = queues[worker[t]][qpos[t] - 1];
          if (p >= A.first_task && p < A.first_task + na) {
            int k = p - A.first_task;
            r[k / 64] |= 1ull << (k % 64);
          } else if (!reach[p].empty()) {
            for (int i = 0; i < words; i++) r[i] |= reach[p][i];
          }
        }
        int e = tasks[t].wait_event;
        if (e >= 0)
          for (int p : producers[e]) {
            if (p >= A.first_task && p < A.first_task + na) {
              int k = p - A.first_task;
              r[k / 64] |= 1ull << (k % 64);
            } else if (!reach[p].empty()) {
              for (int i = 0; i < words; i++) r[i] |= reach[p][i];
            }
          }
      }
      // conflicts between op a and op b
      std::vector<Access> ra, wa, rb, wb;
      for (int tb = B.first_task; tb < B.first_task + B.num_tasks; tb++) {
        task_access(b, tb, rb, wb);
        for (int ta = A.first_task; ta < A.first_task + na; ta++) {
          task_access(a, ta, ra, wa);
          bool conflict = false;
          for (auto& x : wa) {
            for (auto& y : rb) conflict |= overlap(x, y);
            for (auto& y : wb) conflict |= overlap(x, y);
          }
          for (auto& x : ra)
            for (auto& y : wb) conflict |= overlap(x, y);
          if (!conflict) continue;
          checked++;
          int k = ta - A.first_task;
          bool ordered = (reach[tb][k / 64] >> (k % 64)) & 1;
          ordered |= worker[ta] == worker[tb] && qpos[ta] < qpos[tb];
          if (!ordered) {
            std::ostringstream os;
            os << "race: task " << ta << " (op " << a << " " << A.name << ") and task " << tb << " (op " << b << " "
               << B.name << ") conflict but are not ordered";
            return os.str();
          }
        }
      }
    }
  }
  (void)checked;
  return "";
}

// ------------------------------------------------------------------ export
// Task graph in the reference's JSON vocabulary (runtime.cc:847-1318):
// all_tasks / all_events / first_tasks.
// The task graph in the reference's task_graph.json schema
// (src/kernel/runtime.cc:847-1318): all_tasks[0] = TASK_TERMINATE,
// all_tasks[1] = TASK_BEGIN_TASK_GRAPH, then one entry per task with the
// reference's task type code, variant_id, inputs / outputs as {base_ptr
// (tensor name), offset (bytes), data_type, dims, strides}, trigger_event,
// dependent_event, request_id, expert_offset; all_events with event_type,
// num_triggers and the [first_task_id, last_task_id) range of the tasks the
// event launches; first_tasks.  Fused tasks of this backend use the code of
// the reference task they extend with a variant: TASK_RMS_NORM_LINEAR (102)
// variant 0 plain, 1 with the silu_mul epilogue over [gate | up] rows, 2 with
// the argmax_partial / argmax_reduce epilogue.  The offline batch manager,
// which the reference runs between iterations rather than as a task, is
// written as task type 1000.  Each task also carries "yr" = {op, split} (its
// op index, attention split and [gate | up] row group), which the
// reference's loader ignores.
namespace {
constexpr unsigned long long kEventInvalid = 0x7ffffffffffffffeull;
constexpr int kRefTerminate = 0, kRefBegin = 10, kRefEmbedding = 101, kRefRmsNormLinear = 102,
              kRefLinearResidual = 108, kRefPagedAttention = 116, kRefLinear = 120, kRefPrepareBatch = 1000;
constexpr int kRefEventLaunch = 901;

struct IoOut {
  std::ostringstream& os;
  bool first = true;
  void add(const Tensor& t, int64_t elem_off, std::vector<int64_t> dims, std::vector<int64_t> strides) {
    os << (first ? "" : ",") << "{\"base_ptr\":\"" << t.name << "\",\"offset\":" << elem_off * dtype_bytes(t.dtype)
       << ",\"data_type\":" << t.dtype << ",\"dims\":[";
    for (size_t i = 0; i < dims.size(); i++) os << (i ? "," : "") << dims[i];
    os << "],\"strides\":[";
    for (size_t i = 0; i < strides.size(); i++) os << (i ? "," : "") << strides[i];
    os << "]}";
    first = false;
  }
};

// pieces of virtual weight rows [r, r + n): (segment, row in its tensor, rows)
std::vector<WSeg> seg_pieces(const std::vector<WSeg>& segs, int64_t r, int64_t n) {
  std::vector<WSeg> out;
  int64_t base = 0;
  for (auto& s : segs) {
    const int64_t lo = std::max(r, base), hi = std::min(r + n, base + s.rows);
    if (lo < hi) out.push_back({s.tensor, s.row0 + (lo - base), hi - lo});
    base += s.rows;
  }
  return out;
}
}  // namespace

std::string Graph::export_json() const {
  std::ostringstream os;
  const int64_t T = cfg.max_tokens;
  os << "{\"all_tasks\":[";
  os << "{\"task_type\":" << kRefTerminate << ",\"variant_id\":0,\"inputs\":[],\"outputs\":[],\"trigger_event\":"
     << kEventInvalid << ",\"dependent_event\":" << kEventInvalid << ",\"request_id\":-1,\"expert_offset\":-1},";
  os << "{\"task_type\":" << kRefBegin << ",\"variant_id\":0,\"inputs\":[],\"outputs\":[],\"trigger_event\":"
     << kEventInvalid << ",\"dependent_event\":" << kEventInvalid << ",\"request_id\":-1,\"expert_offset\":-1}";
  for (size_t i = 0; i < tasks.size(); i++) {
    const TaskDesc& t = tasks[i];
    const OpDesc& d = ops[t.op];
    const OpInfo& inf = op_info[t.op];
    int code = 0, variant = 0;
    std::ostringstream ins, outs;
    IoOut I{ins}, Ot{outs};
    switch (d.type) {
      case TASK_EMBED: {
        code = kRefEmbedding;
        const Tensor& tab = tensors[inf.table];
        I.add(tensors[inf.tok], 0, {T, 1}, {1, 1});
        I.add(tab, t.row0, {tab.dims[0], t.rows}, {tab.dims[1], 1});
        Ot.add(tensors[inf.out], t.row0, {T, t.rows}, {tensors[inf.out].dims[1], 1});
        break;
      }
      case TASK_LINEAR:
      case TASK_RMSNORM_LINEAR:
      case TASK_RMSNORM_LINEAR_SILU:
      case TASK_RMSNORM_LINEAR_ARGMAX: {
        code = d.type == TASK_LINEAR ? (inf.res >= 0 ? kRefLinearResidual : kRefLinear) : kRefRmsNormLinear;
        variant = d.type == TASK_RMSNORM_LINEAR_SILU ? 1 : d.type == TASK_RMSNORM_LINEAR_ARGMAX ? 2 : 0;
        I.add(tensors[inf.x], 0, {T, d.K}, {d.K, 1});
        std::vector<WSeg> pieces;
        if (d.type == TASK_RMSNORM_LINEAR_SILU) {
          const int64_t g = inf.group, gi = t.row0 / g, j = t.row0 % g;
          for (auto& p : seg_pieces(inf.wsegs, gi * 2 * g + j, t.rows)) pieces.push_back(p);
          for (auto& p : seg_pieces(inf.wsegs, gi * 2 * g + g + j, t.rows)) pieces.push_back(p);
        } else {
          pieces = seg_pieces(inf.wsegs, t.row0, t.rows);
        }
        for (auto& p : pieces) I.add(tensors[p.tensor], p.row0 * d.K, {p.rows, d.K}, {d.K, 1});
        if (inf.norm >= 0) I.add(tensors[inf.norm], 0, {d.K}, {1});
        if (inf.res >= 0) I.add(tensors[inf.res], t.row0, {T, t.rows}, {d.res_ld, 1});
        const Tensor& ot = tensors[inf.out];
        Ot.add(ot, inf.col0 + t.row0, {T, t.rows}, {ot.dims[1], 1});
        if (inf.tok_out >= 0) Ot.add(tensors[inf.tok_out], 0, {T, 1}, {1, 1});
        break;
      }
      case TASK_ATTENTION: {
        code = kRefPagedAttention;
        const int G = d.num_q_heads / d.num_kv_heads, D = d.head_dim, h = t.i1;
        I.add(tensors[inf.x], (int64_t)h * (G + 2) * D, {T, (int64_t)(G + 2) * D}, {d.qkv_ld, 1});
        for (int c : {inf.kc, inf.vc}) {
          const Tensor& ct = tensors[c];
          I.add(ct, 0, ct.dims, {ct.dims[1] * ct.dims[2] * ct.dims[3], ct.dims[2] * ct.dims[3], ct.dims[3], 1});
        }
        // the reference's operand order: input, k_cache, v_cache, q_norm, k_norm, cos, sin
        for (int c : {inf.norm, inf.knorm})
          if (c >= 0) I.add(tensors[c], 0, {(int64_t)D}, {1});
        for (int c : {inf.cos, inf.sin})
          if (c >= 0) I.add(tensors[c], 0, tensors[c].dims, {tensors[c].dims[1], 1});
        Ot.add(tensors[inf.out], (int64_t)h * G * D, {T, (int64_t)G * D}, {tensors[inf.out].dims[1], 1});
        break;
      }
      case TASK_PREPARE_BATCH:
        code = kRefPrepareBatch;
        break;
      default:
        break;
    }
    os << ",{\"task_type\":" << code << ",\"variant_id\":" << variant << ",\"inputs\":[" << ins.str()
       << "],\"outputs\":[" << outs.str() << "],\"trigger_event\":"
       << (t.trigger_event >= 0 ? (unsigned long long)t.trigger_event : kEventInvalid) << ",\"dependent_event\":"
       << (t.wait_event >= 0 ? (unsigned long long)t.wait_event : kEventInvalid)
       << ",\"request_id\":" << (d.type == TASK_ATTENTION ? t.i0 : -1) << ",\"expert_offset\":-1,\"yr\":{\"op\":" << t.op
       << ",\"split\":" << (d.type == TASK_ATTENTION ? t.i2 : 0) << ",\"group\":" << inf.group << "}}";
  }
  os << "],\"all_events\":[";
  for (size_t e = 0; e < events.size(); e++) {
    int first = -1, last = -1;
    const OpInfo& ci = op_info[events[e].consumer_op];
    for (int t = ci.first_task; t < ci.first_task + ci.num_tasks; t++)
      if (tasks[t].wait_event == (int)e) {
        if (first < 0) first = t;
        last = t;
      }
    os << (e ? "," : "") << "{\"event_type\":" << kRefEventLaunch << ",\"num_triggers\":" << events[e].num_triggers
       << ",\"first_task_id\":" << (first < 0 ? -1 : first + 2) << ",\"last_task_id\":" << (last < 0 ? -1 : last + 3)
       << "}";
  }
  os << "],\"first_tasks\":[";
  for (int t = 0; t < op_info[0].num_tasks; t++) os << (t ? "," : "") << t + 2;
  os << "],\"yr_config\":{\"num_workers\":" << num_workers << ",\"max_tokens\":" << cfg.max_tokens
     << ",\"max_requests\":" << cfg.max_requests << ",\"page_size\":" << cfg.page_size << ",\"max_pages\":"
     << cfg.max_pages << ",\"max_seq_len\":" << cfg.max_seq_len << ",\"total_requests\":" << cfg.total_requests
     << ",\"eos_token_id\":" << cfg.eos_token_id << "}}";
  return os.str();
}

}  // namespace pk
}  // namespace yr

// ------------------------------------------------------------------ C ABI
using yr::pk::Graph;

extern "C" {

int yr_pk_graph_build(const char* json_text, yr_pk_graph** out) {
  if (!json_text || !out) return yr::fail(YR_E_INVALID, "yr_pk_graph_build: null argument");
  *out = nullptr;
  Graph* g = new Graph();
  try {
    g->build(json_text);
  } catch (std::exception& e) {
    delete g;
    return yr::fail(YR_E_GRAPH, "task graph: %s", e.what());
  }
  *out = reinterpret_cast<yr_pk_graph*>(g);
  return YR_OK;
}

void yr_pk_graph_free(yr_pk_graph* g) { delete reinterpret_cast<Graph*>(g); }

int yr_pk_graph_info(const yr_pk_graph* gp, int64_t* info, int n) {
  const Graph* g = reinterpret_cast<const Graph*>(gp);
  if (!g || !info || n < 8) return yr::fail(YR_E_INVALID, "yr_pk_graph_info: bad arguments");
  size_t maxq = 0;
  for (auto& q : g->queues) maxq = std::max(maxq, q.size());
  info[0] = (int64_t)g->ops.size();
  info[1] = (int64_t)g->tasks.size();
  info[2] = (int64_t)g->events.size();
  info[3] = g->num_workers;
  info[4] = g->num_tickets;
  info[5] = g->scratch_floats;
  info[6] = (int64_t)maxq;
  info[7] = 0;
  return YR_OK;
}

int yr_pk_graph_task(const yr_pk_graph* gp, int task, int64_t* rec, int n) {
  const Graph* g = reinterpret_cast<const Graph*>(gp);
  if (!g || !rec || n < 10 || task < 0 || task >= (int)g->tasks.size())
    return yr::fail(YR_E_INVALID, "yr_pk_graph_task: bad arguments");
  const yr::pk::TaskDesc& t = g->tasks[task];
  rec[0] = t.op;
  rec[1] = g->ops[t.op].type;
  rec[2] = t.wait_event;
  rec[3] = t.wait_count;
  rec[4] = t.trigger_event;
  rec[5] = t.row0;
  rec[6] = t.rows;
  rec[7] = t.i0;
  rec[8] = t.i1;
  rec[9] = t.i2;
  return YR_OK;
}

int yr_pk_graph_simulate(const yr_pk_graph* gp, uint64_t seed, int epochs, int race_window, char* report,
                         size_t report_len) {
  const Graph* g = reinterpret_cast<const Graph*>(gp);
  if (!g) return yr::fail(YR_E_INVALID, "yr_pk_graph_simulate: null graph");
  std::string r = g->simulate(seed, epochs > 0 ? epochs : 1);
  if (r.empty() && race_window > 0) r = g->check_races(race_window);
  if (report && report_len) {
    size_t k = std::min(report_len - 1, r.size());
    memcpy(report, r.data(), k);
    report[k] = 0;
  }
  return r.empty() ? YR_OK : yr::fail(YR_E_GRAPH, "%s", r.c_str());
}

int yr_pk_graph_export_json(const yr_pk_graph* gp, char* buf, size_t buf_len, size_t* needed) {
  const Graph* g = reinterpret_cast<const Graph*>(gp);
  if (!g) return yr::fail(YR_E_INVALID, "yr_pk_graph_export_json: null graph");
  std::string s = g->export_json();
  if (needed) *needed = s.size() + 1;
  if (buf && buf_len) {
    size_t k = std::min(buf_len - 1, s.size());
    memcpy(buf, s.data(), k);
    buf[k] = 0;
    if (buf_len < s.size() + 1) return yr::fail(YR_E_INVALID, "buffer too small");
  }
  return YR_OK;
}

}  // extern "C"
