// Host runtime of the gfx950 backend: the implementation of include/skyla_hip.h.
//
// It plays the role skyla-vk (Vulkan) and skyla-metal (Metal) play for skyla-engine
// (skyla-engine/src/backend.rs:1-19): contexts, buffers, pipelines, recordings.
//   * Kernels are compiled ahead of time for gfx950 into code objects that are linked
//     into this library and loaded with hipModuleLoadData; a pipeline resolves the
//     (shader name, spec constants) pair to the exported symbol name__s0_s1_.. with
//     hipModuleGetFunction, and launches it with hipModuleLaunchKernel.
//   * A recording is a launch list.  Replaying it launches one HIP graph (built once by
//     capturing the list on the context stream), so a decode step costs one submission
//     instead of one per kernel; a profiled recording replays eagerly with a HIP event
//     after every mark.
//   * Dispatches the engine records with no barrier between them are independent.  Runs of
//     such dispatches of one matvec pipeline (q/k/v, gate/up, an expert's gate/up) become
//     one launch over their combined rows: each kernel launch on MI355X carries ~1.7 us of
//     fixed cost and a ramp-up/drain, which dominate the small decode matrices.
//   * Buffers are HBM allocations with a host mirror that the caller synchronises
//     explicitly (the reference's buffers are host-coherent; a discrete GPU's are not).
#include "../../../include/skyla_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

// Code objects embedded by embed.S.
extern "C" const unsigned char skyla_co_matvec[], skyla_co_matvec_end[];
extern "C" const unsigned char skyla_co_matmul[], skyla_co_matmul_end[];
extern "C" const unsigned char skyla_co_moe[], skyla_co_moe_end[];
extern "C" const unsigned char skyla_co_util[], skyla_co_util_end[];
extern "C" const unsigned char skyla_co_attention[], skyla_co_attention_end[];

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

#define HIP_TRY(call)                                                                       \
  do {                                                                                      \
    hipError_t e_ = (call);                                                                 \
    if (e_ != hipSuccess)                                                                   \
      return fail(SKYLA_HIP_E_DEVICE, "%s failed: %s", #call, hipGetErrorString(e_));       \
  } while (0)

constexpr uint64_t kMaxBuffer = 4ull << 30;  // keeps u32 element offsets valid
constexpr uint32_t kMaxMarks = 2048;          // skyla-vk/src/record.rs:6
constexpr uint64_t kMaxPinned = 1ull << 30;   // host mirrors pinned up to this size

// Tactics: every choice the runtime makes between kernel forms that compute the same
// values, in one table.  The defaults are the forms measured fastest on MI355X; the
// environment variable SKYLA_HIP_TACTIC="key=value,key=value" overrides entries (for
// sweeps, and for the parity tests that run every compiled form).  Read when a pipeline is
// created or a recording ends.
struct Tactic {
  const char *key, *def, *what;
};
const Tactic kTactics[] = {
    {"fuse", "1", "independent dispatches of one kernel run as one segmented launch (0: one launch each)"},
    {"retile", "1", "dense matvec launches take the variant the size rule gives them (0: the engine's)"},
    {"variant", "", "W_R_L: every dense launch of a matvec kernel on that (waves, rows, lanes) variant"},
    {"q8_small", "4_1_64", "W_R_L: dense Q8_0 launches (plain and SiLU-folded) below 2048 rows on that variant "
                           "(empty: the engine's)"},
    {"q8_big", "4_1_16", "W_R_L: dense Q8_0 launches of 65536 rows or more (an output head) on that variant "
                         "(empty: the engine's)"},
    {"ks", "1", "K-split matvec forms for n_in 4096 (Q4_K) and 12288 (Q6_K); 0: none; R_G: Q4_K shape"},
    {"ks6", "", "R_G_D: the Q6_K K-split form on that (rows, groups, groups ahead) shape"},
    {"ks3", "1", "the Q4_K K-split form for n_in 12288 (0: LDS-staged form; R_G: that shape)"},
    {"ksnorm", "", "R_G: the Q4_K K-split form with the RMSNorm folded in on that shape"},
    {"ksglun", "1", "the norm-folded gate/up pair on its K-split form (0: LDS-staged form; R_G: shape)"},
    {"moe_fuse", "26", "bit mask of the MoE decode forms (2 gate/up pair, 8 down + combine, 16 route + pair)"},
    {"splitk", "1", "dense K-quant matmuls of at most 128 tiles split their super-blocks (0: never)"},
    {"split_slots", "256", "workgroup slots a matmul K split fills (64..2048)"},
    {"split_stages", "2", "fewest 256-value super-blocks per split of a matmul K split (1..16)"},
    {"seg_big", "512", "slots for a segmented matmul run past 128 tiles (gate and up at M = 128), 0: no such run"},
    {"xhalf", "1", "f16 row prepass for matmuls on f32 rows: 1 four-wave tile where it fits, 4 without "
                   "the balanced K halves, 8 eight-wave tile throughout, 0 the tile's own f32 staging"},
    {"xhalf_moe", "1", "expert-group matmuls on f32 rows take the f16 row prepass (0: the tile's own f32 staging)"},
    {"xhalf_join", "1", "a dense matmul's f16 row prepass runs in the rmsnorm or silu_mul launch that writes its "
                        "rows (0: a launch of its own)"},
    {"dl", "1", "matmul tiles with their operands loaded straight into LDS (0: register-staged)"},
    {"merge_t", "1", "batched attention merge as one wave per (head, token) (0: 1024-thread form)"},
    {"nograph", "0", "1: recordings replay as direct launches instead of one HIP graph (kernel traces)"},
};

// The value of tactic `key`: the last `key=value` entry of SKYLA_HIP_TACTIC, else the
// table's default.  An unknown key is a programming error and reads as "".
std::string tactic(const char *key) {
  std::string v;
  bool known = false;
  for (const Tactic &t : kTactics)
    if (std::strcmp(t.key, key) == 0) {
      v = t.def;
      known = true;
    }
  if (!known) return "";
  const char *env = std::getenv("SKYLA_HIP_TACTIC");
  if (!env) return v;
  const std::string all(env), k = std::string(key) + "=";
  size_t pos = 0;
  while (pos <= all.size()) {
    size_t end = all.find(',', pos);
    if (end == std::string::npos) end = all.size();
    const std::string item = all.substr(pos, end - pos);
    if (item.compare(0, k.size(), k) == 0) v = item.substr(k.size());
    pos = end + 1;
  }
  return v;
}
bool tactic_on(const char *key) {
  const std::string v = tactic(key);
  return !v.empty() && v != "0";
}

// Bindings, push words and workgroup shape of every kernel the engine creates
// (kernels.rs:170-205; workgroup shapes as skyla-metal/src/pipeline.rs:14-24).
struct KernelInfo {
  const char *name;
  uint32_t n_buffers;
  uint32_t push_words;
  uint32_t spec_len_min, spec_len_max;
  int threads_from_spec;  // -1: fixed (`threads`); k >= 0: 64 * spec[k] (matvec waves) or spec[k]
  bool waves;
  bool segmented;  // takes its push words as a segment table (kernels/common.h Segments)
  uint32_t threads = 256;
};

const KernelInfo kKernels[] = {
    {"matvec_q4k", 4, 9, 5, 5, 0, true, true},
    {"matvec_q6k", 5, 11, 5, 5, 0, true, true},
    {"matvec_q8_0", 5, 9, 5, 5, 0, true, true},
    // fused forms (kernels/matvec.hip): + the second vector's offset and eps
    {"matvec_q4k_norm", 4, 11, 5, 5, 0, true, true},
    {"matvec_q4k_silu", 4, 11, 5, 5, 0, true, true},
    {"matvec_q6k_norm", 5, 13, 5, 5, 0, true, true},
    {"matvec_q6k_silu", 5, 13, 5, 5, 0, true, true},
    {"matvec_q8_0_norm", 5, 11, 5, 5, 0, true, true},
    {"matvec_q8_0_silu", 5, 11, 5, 5, 0, true, true},
    {"matvec_q4k_glu", 4, 11, 5, 5, 0, true, true},  // gate + up -> silu(gate) * up
    {"matvec_q4k_glun", 4, 13, 5, 5, 0, true, true},  // the same after the FFN RMSNorm
    {"matmul", 5, 13, 3, 4, -1, false, false},
    {"moe_logits", 3, 5, 0, 0, -1, false, false},
    {"moe_route", 2, 5, 0, 0, -1, false, false, 256},  // one workgroup per token
    {"moe_sort", 1, 5, 0, 0, -1, false, false},
    {"moe_combine", 1, 6, 0, 0, -1, false, false},
    {"silu_mul", 2, 4, 0, 0, -1, false, false},
    {"to_half", 3, 6, 0, 0, -1, false, false},
    {"bandwidth", 2, 1, 1, 3, 0, false, false},  // [threads] or [threads, depth, nt]
    {"dequant", 3, 7, 1, 1, -1, false, false},
    // the decode step around the matvecs (kernels/attention.hip; kernels.rs:186-193)
    {"rmsnorm", 3, 6, 0, 0, -1, false, false},
    {"qkv_prep", 5, 16, 5, 5, -1, false, false, 64},       // one wave per (head, token)
    {"attention", 5, 11, 6, 6, -1, false, false, 256},     // four waves per (kv head, split, token)
    {"attention_merge", 2, 6, 2, 2, -1, false, false, 1024},
    {"attention_prep", 5, 18, 6, 6, -1, false, false, 256},  // qkv_prep + attention, one token
    {"attention_prep1", 5, 20, 6, 6, -1, false, false, 256},  // the same over one split, merged
    {"rope_table", 3, 3, 0, 0, -1, false, false, 64},         // a decode step's rope pairs
    {"take_last", 2, 4, 0, 0, -1, false, false},
    {"embed", 4, 8, 1, 1, -1, false, false},  // token rows from the HBM token_embd (util.hip)
};

const KernelInfo *find_kernel(const char *name) {
  for (const auto &k : kKernels)
    if (std::strcmp(k.name, name) == 0) return &k;
  return nullptr;
}

}  // namespace

// Layout of the static workspace `scratch` in the matmul code object (kernels/matmul.hip):
// SCRATCH_TILES f32 tiles of 128 x 128, then SCRATCH_COUNTERS u32 counters.
constexpr uint64_t kScratchTiles = 256;
constexpr uint64_t kScratchCounters = 1024;

struct skyla_hip_context {
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<hipModule_t> modules;
  std::string name;
  uint32_t warp = 64;
  // device address of this context's copy of `scratch` (looked up once, at context_new),
  // its size, and the fill kernel that clears its counters
  char *scratch = nullptr;
  size_t scratch_bytes = 0;
  hipFunction_t fill_u32 = nullptr;
  uint32_t n_cu = 256;  // compute units of the device (hipDeviceProp_t.multiProcessorCount)
  hipFunction_t x_half_rows = nullptr;  // f16 row prepass of dense K-quant matmuls (matmul.hip)
  hipFunction_t silu_half_rows = nullptr;  // silu_mul with the expert down projection's prepass
  hipFunction_t silu_mul = nullptr;        // (moe.hip): the launch it replaces
  hipFunction_t rmsnorm_half_rows = nullptr;  // rmsnorm with a dense matmul's prepass (matmul.hip)
  hipFunction_t rmsnorm = nullptr;            // (attention.hip): the launch it replaces
};

struct HostFree {
  bool pinned;
  HostFree(bool p = false) : pinned(p) {}
  void operator()(unsigned char *p) const {
    if (pinned)
      (void)hipHostFree(p);
    else
      delete[] p;
  }
};

struct skyla_hip_buffer {
  skyla_hip_context *ctx = nullptr;
  void *dev = nullptr;
  // host mirror: pinned (hipHostMalloc) up to kMaxPinned bytes, so the per-step copies
  // (control words up, logits down) are direct DMA; larger mirrors (weights, copied once)
  // are pageable
  std::unique_ptr<unsigned char[], HostFree> host;
  uint64_t size = 0;
};

// Alternative gfx950 variants of a dense matvec pipeline (same push layout, different
// rows per workgroup) and the launch sizes they serve best.  A launch of `rows` output
// rows in total uses the first alternative whose min_rows <= rows.
struct MatvecAlt {
  hipFunction_t fn;
  uint32_t rwg, threads;  // outputs per workgroup, threads per workgroup
  uint64_t min_rows;
  uint32_t n_in_req = 0;              // nonzero: every segment's n_in must equal it
  uint64_t max_rows = ~uint64_t{0};   // and the launch at most this many rows
};
struct Retile {
  uint32_t n_out_word;     // index of n_out in the push words
  uint32_t n_in_word = 4;  // index of n_in
  std::vector<MatvecAlt> alts;
};

struct skyla_hip_pipeline {
  skyla_hip_context *ctx = nullptr;
  std::string symbol;
  hipFunction_t fn = nullptr;
  uint32_t n_buffers = 0;
  uint32_t push_words = 0;
  uint32_t threads = 256;
  bool segmented = false;
  std::shared_ptr<const Retile> retile;  // matvec pipelines with a variant rule
  hipFunction_t split_fn = nullptr;      // dense K-quant matmul: the K-split variant
  hipFunction_t hx_fn = nullptr;         // and its variant on x_half_rows's f16 rows
  hipFunction_t hx4_fn = nullptr;        // the four-wave tile on those rows
  hipFunction_t hx4b_fn = nullptr;       // and over a balanced grid (some tiles in K halves)
  hipFunction_t hxs_fn = nullptr;        // the eight-wave tile over several matrices (segments)
  hipFunction_t hxm_fn = nullptr;        // expert groups (MOE = 1) on x_half_rows's f16 rows
  hipFunction_t hxms_fn = nullptr;       // and over several matrices on the same rows (segments)
  uint32_t split_threads = 0;
  hipFunction_t tok_fn = nullptr;        // batched form: a tok_per_wg x tok_per_wg_y block of
  uint32_t tok_per_wg = 0;               // grid.x and grid.y per workgroup
  uint32_t tok_per_wg_y = 0;
  uint32_t tok_threads = 0;              // its workgroup size (0: the pipeline's)
  std::string name;                      // shader name
  hipFunction_t moe_fn = nullptr;        // MoE decode forms (fuse_moe), Q4_K experts: the gate/up pair,
  hipFunction_t moe_fn3 = nullptr;       // the down projection with moe_combine,
  hipFunction_t moe_fn4 = nullptr;       // and the gate/up pair that routes for itself
  std::vector<std::vector<void *>> sets;
};

namespace {

struct Command {
  enum Kind { Dispatch, Barrier, Mark } kind;
  hipFunction_t fn = nullptr;
  uint32_t threads = 0;
  bool segmented = false;
  std::shared_ptr<const Retile> retile;
  hipFunction_t split_fn = nullptr;
  uint32_t split_threads = 0;
  hipFunction_t hx_fn = nullptr, hx4_fn = nullptr, hx4b_fn = nullptr, hxs_fn = nullptr, hxm_fn = nullptr,
                hxms_fn = nullptr;
  hipFunction_t tok_fn = nullptr;
  uint32_t tok_per_wg = 0, tok_per_wg_y = 0, tok_threads = 0;
  std::string name;                 // the pipeline's shader name
  hipFunction_t moe_fn = nullptr, moe_fn3 = nullptr, moe_fn4 = nullptr;
  uint32_t groups[3] = {0, 0, 0};
  std::vector<void *> bufs;
  std::vector<uint32_t> push;
  std::string label;
};

// One kernel launch (or a mark) of a recording.  `args` is the by-value argument after the
// binding pointers: the push words, or for segmented kernels the segment table
// {n, start[kMaxSeg], push[kMaxSeg][words]} of kernels/common.h.
struct Launch {
  bool mark = false;
  hipFunction_t fn = nullptr;
  uint32_t threads = 0;
  uint32_t groups[3] = {0, 0, 0};
  std::vector<void *> bufs;
  std::vector<uint32_t> args;
  // K split (matmul): S > 1 appends (workspace, counters, S) to the kernel arguments
  uint32_t split = 0;
  uint64_t ws_bytes = 0;  // partial tiles
  uint32_t n_cnt = 0;     // per-tile counters
  void *ws = nullptr;
  void *cnt = nullptr;
  std::vector<uint32_t> extra;  // trailing by-value u32 arguments (batched forms: the token count)
  // f16 row prepass: bufs[xh_buf] is replaced by the recording's f16-row buffer, which
  // holds xh_bytes for this launch
  int xh_buf = -1;
  uint64_t xh_bytes = 0;
};

constexpr uint32_t kMaxSeg = 4;  // MAXSEG in kernels/common.h
constexpr uint64_t kSplitTileBytes = 128 * 128 * 4;  // one f32 partial tile (kernels/matmul.hip)

// K split of a dense K-quant matmul launch (matmul.hip, matmul_tile128_w): launches of at
// most 128 tiles of 128 x 128 leave CUs idle (the tile keeps one workgroup per CU), so
// their super-blocks are split over up to 256 workgroups, keeping at least 4 per split.
// Measured on MI355X at M = 512: 4096 x 4096 68.6 -> 53.0 us, 4096 x 12288 191.6 -> 119.3 us.
// Workgroup slots a K split fills (the split_slots tactic, default 256: one eight-wave
// workgroup per CU).
uint64_t split_slots() {
  const long v = std::atol(tactic("split_slots").c_str());
  return v >= 64 && v <= 2048 ? (uint64_t)v : 256;
}

// Fewest super-blocks per split (the split_stages tactic, default 2: config-5 512-token
// prefill 15.93-15.94k tok/s against 15.82-15.86k with 4 and 15.81-15.82k with 3, two runs
// each on one box; at M = 128 the n_in-4096 launches of 32 and 48 tiles then split 8 and 5
// ways instead of 4).
uint32_t split_stages() {
  const long v = std::atol(tactic("split_stages").c_str());
  return v >= 1 && v <= 16 ? (uint32_t)v : 2u;
}

uint32_t split_of(const Command &a) {
  if (!a.split_fn || a.push.size() < 7) return 1;
  const uint64_t tiles = (uint64_t)a.groups[0] * a.groups[1] * a.groups[2];
  const uint32_t n_stage = a.push[6] / 256;  // MatmulPush.n_in
  if (tiles == 0 || tiles > 128) return 1;
  uint32_t S = (uint32_t)(split_slots() / tiles);
  S = std::min(S, n_stage / split_stages());
  S = std::min(S, 8u);
  return S < 2 ? 1 : S;
}

// Packs consecutive dispatches of one segmented kernel into one launch.
Launch pack(const Command *const *run, uint32_t n) {
  Launch l;
  const Command &a = *run[0];
  l.fn = a.fn;
  l.threads = a.threads;
  l.bufs = a.bufs;
  if (!a.segmented) {
    for (int i = 0; i < 3; i++) l.groups[i] = a.groups[i];
    l.args = a.push;
    if (a.tok_fn && a.groups[1] > 1) {  // grid (x, y) = (experts, tokens): blocks of both
      l.fn = a.tok_fn;
      l.groups[0] = (a.groups[0] + a.tok_per_wg - 1) / a.tok_per_wg;
      l.groups[1] = (a.groups[1] + a.tok_per_wg_y - 1) / a.tok_per_wg_y;
      if (a.tok_threads) l.threads = a.tok_threads;
      l.extra = {a.groups[0], a.groups[1]};
    }
    const uint32_t S = split_of(a);
    if (S > 1) {
      l.fn = a.split_fn;
      l.threads = a.split_threads;
      l.groups[2] = a.groups[2] * S;
      l.split = S;
      l.n_cnt = a.groups[0] * a.groups[2];
      l.ws_bytes = (uint64_t)l.n_cnt * S * kSplitTileBytes;
    }
    return l;
  }
  const size_t w = a.push.size();
  // a matvec launch may run on the variant that suits its total size; grid.x is then
  // recomputed from each segment's n_out (every row is still computed exactly once)
  const MatvecAlt *alt = nullptr;
  if (a.retile) {
    uint64_t rows = 0;
    for (uint32_t i = 0; i < n; i++) rows += run[i]->push[a.retile->n_out_word];
    for (const MatvecAlt &v : a.retile->alts) {
      if (rows < v.min_rows || rows > v.max_rows) continue;
      bool fits = true;
      for (uint32_t i = 0; i < n && v.n_in_req; i++) fits &= run[i]->push[a.retile->n_in_word] == v.n_in_req;
      if (fits) {
        alt = &v;
        break;
      }
    }
  }
  if (alt) {
    l.fn = alt->fn;
    l.threads = alt->threads;
  }
  l.args.assign(1 + kMaxSeg + kMaxSeg * w, 0u);
  l.args[0] = n;
  uint32_t x = 0;
  for (uint32_t i = 0; i < kMaxSeg; i++) {
    l.args[1 + i] = i < n ? x : 0xffffffffu;
    if (i < n) {
      std::copy(run[i]->push.begin(), run[i]->push.end(), l.args.begin() + 1 + kMaxSeg + i * w);
      x += alt ? (run[i]->push[a.retile->n_out_word] + alt->rwg - 1) / alt->rwg : run[i]->groups[0];
    }
  }
  l.groups[0] = x;
  l.groups[1] = a.groups[1];
  l.groups[2] = a.groups[2];
  return l;
}

// Can dispatch c join a fused launch that starts with dispatch a and holds `x` blocks?
// (Dispatches between two barriers are independent; same kernel, bindings and grid y/z.)
bool fusable(const Command &a, const Command &c, uint64_t x) {
  return a.segmented && c.kind == Command::Dispatch && c.fn == a.fn && c.bufs == a.bufs &&
         c.retile == a.retile &&
         c.threads == a.threads && c.groups[1] == a.groups[1] && c.groups[2] == a.groups[2] &&
         x + c.groups[0] <= 0x7fffffffu;
}

// Index of the next dispatch after i, skipping barriers; cmds.size() if a mark (a profiled
// stage boundary) or the end comes first.
size_t next_dispatch(const std::vector<Command> &cmds, size_t i) {
  for (size_t j = i + 1; j < cmds.size(); j++) {
    if (cmds[j].kind == Command::Barrier) continue;
    return cmds[j].kind == Command::Dispatch ? j : cmds.size();
  }
  return cmds.size();
}

// MoE decode forms.  graph/moe.rs:42-80 records a decode token's MoE layer as six
// dependent dispatches (logits, route, gate + up, silu, down, combine), and each launch on
// MI355X costs ~2.3 us before any work.  The runtime can replace runs of them with one
// launch each, computing the same values bit for bit (tests/test_gpu_moe.py compares every
// form with the six launches):
//   2: a Q4_K expert gate and up then silu_mul    -> matvec_q4k_glu__4_0_1_1_16 (writes
//      silu(gate) * up where silu_mul leaves it; the up rows are not stored)
//  16: moe_route, then form 2's three dispatches   -> matvec_q4k_glur__4_0_1_1_16 (every
//      workgroup runs the route selection itself, so it needs no other's result)
//   8: a Q4_K expert down then moe_combine        -> matvec_q4k_dcomb__8 (a workgroup owns
//      8 rows of every slot, so it combines its own rows: no handoff; n_used <= 8 and
//      n_in <= 1024)
// The expert forms keep the arithmetic of the launch shape the runtime's variant rule gives
// expert matvecs (four waves, one row, 16 lanes per row), so each row sums exactly as it
// would alone.  Config-4 decode, us per layer (graph replay, MI355X): six launches 25.9;
// form 2 24.0; 2 + 8 21.8; 2 + 8 + 16 (three launches: logits, route + gate/up, down +
// combine) 20.5-20.7.  Two forms that handed results from workgroup to workgroup inside
// the launch (a coherent store, its completion, a device-scope count, coherent reads) cost
// as much as the launch boundary they removed and were taken out.  The moe_fuse tactic
// selects the forms as a bit mask (0 keeps the six launches).
constexpr unsigned kMoeForms = 2 | 8 | 16;  // all built forms, and the default

// The experts' gate dispatch at i, their up dispatch right after it and silu_mul after a
// barrier (graph/moe.rs:63-72): the index of the silu_mul, or 0 when the pattern is not there.
size_t glu_run(const std::vector<Command> &cmds, size_t i) {
  const Command &a = cmds[i];
  if (a.kind != Command::Dispatch || !a.moe_fn || a.name != "matvec_q4k" || a.push.size() != 9 ||
      i + 1 >= cmds.size())
    return 0;
  const Command &b = cmds[i + 1];
  const size_t j = next_dispatch(cmds, i + 1);
  const bool ok = b.kind == Command::Dispatch && b.fn == a.fn && b.bufs == a.bufs && b.groups[1] == a.groups[1] &&
                  b.groups[2] == 1 && a.groups[2] == 1 && b.push[2] == a.push[2] && b.push[4] == a.push[4] &&
                  b.push[5] == a.push[5] && b.push[6] == a.push[6] && b.push[7] == a.push[7] &&
                  b.push[8] == a.push[8] && j < cmds.size() && cmds[j].name == "silu_mul" &&
                  cmds[j].groups[1] == 1 && cmds[j].push[0] == a.push[3] && cmds[j].push[1] == b.push[3] &&
                  cmds[j].push[3] == 0 && cmds[j].push[2] == a.groups[1] * a.push[8] && a.push[8] >= a.push[5];
  return ok ? j : 0;
}

// The gate/up pair launch of gate dispatch a and up dispatch b: the gate's words, then the
// up matrix's regions.
Command glu_command(const Command &a, const Command &b, hipFunction_t fn, const char *name) {
  Command f = a;
  f.fn = fn;
  f.name = name;
  f.threads = 256;
  f.retile = nullptr;
  f.groups[0] = (a.push[5] + 7) / 8;
  f.push.push_back(b.push[0]);
  f.push.push_back(b.push[1]);
  return f;
}
std::vector<Command> fuse_moe(const std::vector<Command> &cmds) {
  const unsigned forms = (unsigned)std::strtoul(tactic("moe_fuse").c_str(), nullptr, 0) & kMoeForms;
  if (!forms) return cmds;
  std::vector<Command> out;
  out.reserve(cmds.size());
  for (size_t i = 0; i < cmds.size();) {
    const Command &a = cmds[i];
    // moe_route, then the experts' gate and up and silu_mul -> the pair that routes itself
    if ((forms & 16) && a.kind == Command::Dispatch && a.name == "moe_route" && a.groups[0] == 1 &&
        a.groups[1] == 1 && a.groups[2] == 1) {
      const size_t jg = next_dispatch(cmds, i);
      const size_t js = jg < cmds.size() ? glu_run(cmds, jg) : 0;
      // the pair reads the logits and writes the weights through its y binding, the ids
      // through its ids binding: the route's arena and ids buffers
      if (js && cmds[jg].moe_fn4 && cmds[jg].push[6] == a.push[1] && a.bufs.size() == 2 &&
          cmds[jg].bufs[2] == a.bufs[0] && cmds[jg].bufs[3] == a.bufs[1]) {
        Command f = glu_command(cmds[jg], cmds[jg + 1], cmds[jg].moe_fn4, "matvec_q4k_glur");
        f.push.insert(f.push.end(), a.push.begin(), a.push.end());
        out.push_back(std::move(f));
        i = js + 1;
        continue;
      }
    }
    // expert matvec push: o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride
    if (a.kind == Command::Dispatch && a.moe_fn && a.name == "matvec_q4k" && a.push.size() == 9) {
      if (const size_t js = (forms & 2) ? glu_run(cmds, i) : 0) {
        out.push_back(glu_command(a, cmds[i + 1], a.moe_fn, "matvec_q4k_glu"));
        i = js + 1;
        continue;
      }
      const size_t j = next_dispatch(cmds, i);
      const bool comb = j < cmds.size() && cmds[j].name == "moe_combine" && cmds[j].groups[1] == 1 &&
                        a.groups[2] == 1 && cmds[j].push[1] == a.push[3] && cmds[j].push[4] == a.push[8] &&
                        cmds[j].push[3] == a.push[5] && cmds[j].push[5] == a.groups[1];
      if ((forms & 8) && comb && a.moe_fn3 && a.groups[1] <= 8 && a.push[4] <= 1024 && a.push[4] % 256 == 0) {
        Command f = a;
        f.fn = a.moe_fn3;
        f.name = "matvec_q4k_dcomb";
        f.threads = 256;
        f.retile = nullptr;
        f.groups[0] = (a.push[5] + 7) / 8;
        f.groups[1] = 1;
        f.push.push_back(cmds[j].push[0]);
        f.push.push_back(cmds[j].push[2]);
        f.push.push_back(cmds[j].push[5]);
        out.push_back(std::move(f));
        i = j + 1;
        continue;
      }
    }
    out.push_back(a);
    i++;
  }
  return out;
}

// f16 rows for a dense K-quant matmul with f32 inputs (matmul.hip, x_half_rows), and the
// matmul on them: the conversion the tile would do per stage, done once per launch with a
// per-row scale, lets the tile read f16 (config-3 GEMMs 14-19% faster).  One prepass serves
// every such matmul that reads the same rows before the next barrier (dispatches between
// barriers are independent: none of them writes those rows).  Buffer pointers are filled
// in by bind_workspace.  MatmulPush words: x_off 4, n_in 6, x_stride 8.
// rows: the most input rows the launch can read (groups[0] of the prepass, rows past
// ctl[2] x rows_per_token skip); the exponents come first, h_bytes_off bytes, then the rows.
Launch x_half_prepass(skyla_hip_context *ctx, const Command &a, uint64_t h_bytes_off, uint32_t rows,
                      uint32_t rows_per_token = 1) {
  Launch l;
  l.fn = ctx->x_half_rows;
  l.threads = 256;
  l.groups[0] = rows;
  l.groups[1] = l.groups[2] = 1;
  l.bufs = {a.bufs[2], nullptr, a.bufs[4]};
  l.args = {a.push[4], a.push[8], a.push[6], (uint32_t)(h_bytes_off / 4), rows_per_token};
  l.xh_buf = 1;
  l.xh_bytes = h_bytes_off + (uint64_t)l.groups[0] * a.push[6] * 2;
  return l;
}

// Can matmul c run as a further segment of a fused launch of matmul a on f16 rows?  The
// same kernel, bindings and token grid, and the same activation rows (x_off, n_in,
// x_stride); dispatches with no barrier between them are independent.
bool fusable_matmul(const Command &a, const Command &c) {
  return c.kind == Command::Dispatch && c.hx_fn == a.hx_fn && c.hxs_fn == a.hxs_fn && !c.segmented &&
         c.push.size() == 13 && c.bufs == a.bufs && c.groups[1] == 1 && c.groups[2] == a.groups[2] &&
         c.push[4] == a.push[4] && c.push[6] == a.push[6] && c.push[8] == a.push[8];
}

// The launch list of a recording.  Barriers need no command of their own: launches on one
// stream (and the nodes of a graph captured from it) run in order.  The fuse tactic 0 keeps
// one launch per dispatch; the xhalf tactic 0 keeps the matmuls' own f32 staging.
std::vector<Launch> build_launches(skyla_hip_context *ctx, const std::vector<Command> &recorded) {
  const std::vector<Command> cmds = fuse_moe(recorded);
  const bool fuse = tactic_on("fuse");
  const std::string xh = tactic("xhalf");
  const bool xhalf = ctx && ctx->x_half_rows && xh != "0";
  const bool x4 = xh != "8";       // 8: the eight-wave tile throughout
  const bool balance = xh != "4";  // 4: the plain grid
  const bool moe_xh = tactic_on("xhalf_moe");
  const bool join = tactic_on("xhalf_join");
  uint32_t moe_used = 0;  // experts used per token: the x_div of the last expert gate/up matmul
  std::vector<Launch> out;
  std::vector<uint32_t> xkey;  // the rows the last prepass converted, until a barrier
  for (size_t i = 0; i < cmds.size();) {
    const Command &a = cmds[i];
    if (a.kind == Command::Mark) {
      Launch m;
      m.mark = true;
      out.push_back(std::move(m));
      xkey.clear();
      i++;
      continue;
    }
    if (a.kind != Command::Dispatch) {
      xkey.clear();
      i++;
      continue;
    }
    // expert groups (graph/moe.rs:26-40: grid (row tiles, experts, token tiles of 32)) on
    // f16 rows: gate and up read the token rows (x_div = experts used per token), down the
    // slot rows (x_div = 1), as many as the tokens times the experts used, which the last
    // gate/up launch's x_div gives
    if (a.kind == Command::Dispatch && a.name == "matmul" && a.push.size() == 13 && a.groups[1] > 1 && a.push[12] > 1)
      moe_used = a.push[12];
    // (the tile map, 640 words before the table, exists only with table_off >= 640: moe.hip)
    if (xhalf && moe_xh && a.hxm_fn && !a.segmented && a.push.size() == 13 && a.bufs.size() == 5 && a.groups[1] > 1 &&
        a.push[6] % 256 == 0 && a.push[6] <= 12288 && a.push[4] % 4 == 0 && a.push[8] % 4 == 0 &&
        a.push[10] >= 640 && (a.push[12] > 1 || moe_used > 1)) {
      const uint32_t per_token = a.push[12] > 1 ? 1u : moe_used;
      const uint32_t rows = a.groups[2] * 32 * per_token;  // token tiles of 32: the chunk's tokens
      const uint64_t h_off = ((uint64_t)rows * 4 + 255) & ~(uint64_t)255;
      const std::vector<uint32_t> key = {(uint32_t)((uintptr_t)a.bufs[2] >> 32), (uint32_t)(uintptr_t)a.bufs[2],
                                         a.push[4], a.push[8], a.push[6], rows, 1u};
      // the down projection's rows come from silu_mul, the launch before it: one launch of
      // both (silu_half_rows: the same f32 rows and the same f16 rows) when it covers them
      // (g_off = the rows read, one flat region of at least rows x x_stride values)
      Launch *prev = out.empty() ? nullptr : &out.back();
      if (key != xkey && per_token > 1 && ctx->silu_half_rows && prev && !prev->mark && prev->fn == ctx->silu_mul &&
          prev->args.size() == 4 && prev->args[0] == a.push[4] && prev->args[3] == 0 &&
          (uint64_t)prev->args[2] >= (uint64_t)rows * a.push[8] && prev->groups[1] == 1 && prev->groups[2] == 1) {
        Launch f = x_half_prepass(ctx, a, h_off, rows, per_token);
        f.fn = ctx->silu_half_rows;
        f.bufs = {prev->bufs[0], nullptr, a.bufs[4]};
        f.args = {prev->args[0], prev->args[1], a.push[8], a.push[6], (uint32_t)(h_off / 4), per_token};
        *prev = std::move(f);
        xkey = key;
      }
      if (key != xkey) {
        out.push_back(x_half_prepass(ctx, a, h_off, rows, per_token));
        xkey = key;
      }
      // expert matmuls on the same rows with no barrier between them (gate and up) run as
      // one launch of segments: row tiles of segment s after those of s - 1
      uint32_t n_run = 1;
      uint64_t row_tiles = a.groups[0];
      while (fuse && a.hxms_fn && n_run < kMaxSeg && i + n_run < cmds.size()) {
        const Command &c = cmds[i + n_run];
        if (!(c.kind == Command::Dispatch && c.hxm_fn == a.hxm_fn && c.hxms_fn == a.hxms_fn && !c.segmented &&
              c.bufs == a.bufs && c.push.size() == 13 && c.groups[1] == a.groups[1] && c.groups[2] == a.groups[2] &&
              c.push[4] == a.push[4] && c.push[6] == a.push[6] && c.push[8] == a.push[8] &&
              c.push[10] == a.push[10] && c.push[11] == a.push[11] && c.push[12] == a.push[12]))
          break;
        row_tiles += c.groups[0];
        n_run++;
      }
      Launch l;
      l.bufs = a.bufs;
      l.threads = 256;
      l.split = 0;
      if (n_run > 1) {
        l.fn = a.hxms_fn;
        const size_t w = 13;
        l.args.assign(1 + kMaxSeg + kMaxSeg * w, 0u);
        l.args[0] = n_run;
        uint32_t start = 0;
        for (uint32_t sgi = 0; sgi < kMaxSeg; sgi++) {
          l.args[1 + sgi] = sgi < n_run ? start : 0xffffffffu;
          if (sgi < n_run) {
            const Command &c = cmds[i + sgi];
            uint32_t *dst = l.args.data() + 1 + kMaxSeg + sgi * w;
            std::copy(c.push.begin(), c.push.end(), dst);
            dst[4] = (uint32_t)(h_off / 2);  // f16 units
            dst[8] = a.push[6];
            start += c.groups[0];
          }
        }
        l.groups[0] = (uint32_t)row_tiles;
      } else {
        const Command *one[1] = {&a};
        l = pack(one, 1);
        l.fn = a.hxm_fn;
        l.threads = 256;
        l.split = 0;
        l.args[4] = (uint32_t)(h_off / 2);  // f16 units
        l.args[8] = a.push[6];
      }
      // grid.y over moe_sort's tile map: at most sum_e ceil(c_e / 32) <= (S + 31 k) / 32
      // pairs, S = the slots (the token tiles' 32 columns times the experts used per token)
      // and k <= min(experts, S) the experts with slots, and at most every expert's every
      // token tile (an expert takes a token at most once)
      const uint64_t used = a.push[12] > 1 ? a.push[12] : moe_used;
      const uint64_t slots = (uint64_t)a.groups[2] * 32 * used, experts = a.groups[1];
      // (at most 280 with 256 experts and 1024 slots, the engine's limits; the map's 640 words
      // hold 319 entries, which bounds what a workgroup reads in any case), rounded up to a
      // multiple of 8 for the tiles' XCD-aware order (the entries past the count return)
      const uint64_t bound = std::min(experts * a.groups[2], (slots + 31 * std::min(experts, slots)) / 32);
      l.groups[1] = (uint32_t)std::min<uint64_t>((bound + 7) & ~7ull, 312);
      l.groups[2] = 1;
      l.xh_buf = 2;
      l.xh_bytes = out.back().xh_bytes;
      out.push_back(std::move(l));
      i += n_run;
      continue;
    }
    if (xhalf && a.hx_fn && !a.segmented && a.push.size() == 13 && a.bufs.size() == 5 && a.groups[1] == 1 &&
        a.push[6] % 256 == 0 && a.push[6] <= 12288 && a.push[4] % 4 == 0 && a.push[8] % 4 == 0) {
      const uint32_t rows = a.groups[2] * 128;
      const uint64_t h_off = ((uint64_t)rows * 4 + 255) & ~(uint64_t)255;
      const std::vector<uint32_t> key = {(uint32_t)((uintptr_t)a.bufs[2] >> 32), (uint32_t)(uintptr_t)a.bufs[2],
                                         a.push[4], a.push[8], a.push[6], a.groups[2]};
      if (key != xkey) {
        // The rows usually come from the launch just before: rmsnorm (q, k, v; gate and up)
        // or silu_mul (down).  When it writes exactly these rows, one launch does both
        // (rmsnorm_half_rows, silu_half_rows: the same f32 rows and the same f16 rows).
        Launch f = x_half_prepass(ctx, a, h_off, rows);
        Launch *prev = out.empty() ? nullptr : &out.back();
        const bool plain = join && prev && !prev->mark && prev->split == 0 && prev->extra.empty() && prev->xh_buf < 0 &&
                           prev->groups[2] == 1 && prev->threads == 256;
        if (plain && ctx->rmsnorm_half_rows && prev->fn == ctx->rmsnorm && prev->args.size() == 6 &&
            prev->bufs.size() == 3 && prev->bufs[1] == a.bufs[2] && prev->bufs[2] == a.bufs[4] &&
            prev->groups[0] == 1 && prev->args[2] == a.push[4] && prev->args[5] == a.push[8] &&
            prev->args[3] == a.push[6] && prev->args[3] <= 4096 &&
            ((prev->args[0] | prev->args[1] | prev->args[2] | prev->args[3] | prev->args[5]) & 3u) == 0) {
          // NormPush {x_off, w_off, y_off, n, eps, stride} + h_off; rmsnorm's grid
          f.fn = ctx->rmsnorm_half_rows;
          f.bufs = {prev->bufs[0], prev->bufs[1], nullptr, prev->bufs[2]};
          f.xh_buf = 2;
          f.args = prev->args;
          f.args.push_back((uint32_t)(h_off / 4));
          for (int d = 0; d < 3; d++) f.groups[d] = prev->groups[d];
          *prev = std::move(f);
        } else if (plain && ctx->silu_half_rows && prev->fn == ctx->silu_mul && prev->args.size() == 4 &&
                   prev->bufs.size() == 2 && prev->bufs[0] == a.bufs[2] && prev->bufs[1] == a.bufs[4] &&
                   prev->args[0] == a.push[4] && prev->args[3] == a.push[8] && prev->args[2] == a.push[6] &&
                   prev->args[1] % 4 == 0) {
          // SiluPush {g_off, u_off, n, stride}, one row a token: the rows of the prepass's grid
          f.fn = ctx->silu_half_rows;
          f.bufs = {prev->bufs[0], nullptr, prev->bufs[1]};
          f.args = {prev->args[0], prev->args[1], a.push[8], a.push[6], (uint32_t)(h_off / 4), 1u};
          *prev = std::move(f);
        } else {
          out.push_back(std::move(f));
        }
        xkey = key;
      }
      // Matmuls on the same rows with no barrier between them (q, k, v of a prefill chunk)
      // run as one launch of segments while the run stays a K-split launch (at most 128
      // tiles: the split spreads the few tiles of each small matrix over more CUs).  A run
      // of up to 256 tiles (gate and up at M = 128: 2 x 96) is one launch too, split over
      // seg_big slots (512: two ways, 384 workgroups instead of two launches of 192):
      // config-5 prefill 15.74-15.77k -> 16.06-16.10k tok/s; three, four and five ways
      // (576, 768, 1024) ran 15.0-15.1k, 14.4k and 13.8-13.9k (one box).
      uint32_t n_run = 1;
      uint64_t row_tiles = a.groups[0];
      const long seg_big = std::atol(tactic("seg_big").c_str());
      const uint64_t max_tiles = seg_big > 0 ? 256 : 128;
      if (fuse && a.hxs_fn && a.split_fn) {
        while (n_run < kMaxSeg && i + n_run < cmds.size() && fusable_matmul(a, cmds[i + n_run]) &&
               (row_tiles + cmds[i + n_run].groups[0]) * a.groups[2] <= max_tiles) {
          row_tiles += cmds[i + n_run].groups[0];
          n_run++;
        }
      }
      if (n_run > 1) {
        const uint64_t tiles = row_tiles * a.groups[2];
        // split_of's rule on the fused tile count
        uint32_t S = (uint32_t)((tiles > 128 ? (uint64_t)seg_big : split_slots()) / tiles);
        S = std::min(std::min(S, a.push[6] / 256 / split_stages()), 8u);
        if (S < 2) S = 1;
        Launch l;
        l.fn = a.hxs_fn;
        l.threads = 512;
        l.bufs = a.bufs;
        const size_t w = 13;
        l.args.assign(1 + kMaxSeg + kMaxSeg * w, 0u);
        l.args[0] = n_run;
        uint32_t start = 0;
        for (uint32_t sgi = 0; sgi < kMaxSeg; sgi++) {
          l.args[1 + sgi] = sgi < n_run ? start : 0xffffffffu;
          if (sgi < n_run) {
            const Command &c = cmds[i + sgi];
            uint32_t *dst = l.args.data() + 1 + kMaxSeg + sgi * w;
            std::copy(c.push.begin(), c.push.end(), dst);
            dst[4] = (uint32_t)(h_off / 2);  // f16 units
            dst[8] = a.push[6];
            start += c.groups[0];
          }
        }
        l.groups[0] = (uint32_t)row_tiles;
        l.groups[1] = 1;
        l.groups[2] = a.groups[2] * S;
        l.split = S;
        l.n_cnt = S > 1 ? (uint32_t)tiles : 0;
        l.ws_bytes = S > 1 ? tiles * S * kSplitTileBytes : 0;
        l.xh_buf = 2;
        l.xh_bytes = out.back().xh_bytes;
        out.push_back(std::move(l));
        i += n_run;
        continue;
      }
      const Command *one[1] = {&a};
      Launch l = pack(one, 1);
      l.fn = a.hx_fn;
      l.threads = a.split_threads;
      // Launches of more than 128 tiles (no K split) run the four-wave tile, two workgroups
      // per CU: each dequantised fragment feeds four MFMAs (M = 512 gate: 124 -> 108 us).
      // K-split launches keep the eight-wave tile (the four-wave one split four ways
      // measured 1.2-1.7x slower, and in a later build made an illegal memory access at the
      // config-3 shapes whose cause was not found: it is never launched split more than
      // the balanced grid's two K halves).  Both give the same bits.
      if (!l.split && x4 && a.hx4_fn) {
        l.fn = a.hx4_fn;
        l.threads = 256;
        // More tiles than CUs but fewer than the two-per-CU slots: some CUs would run two
        // tiles and the rest one.  Balanced grid instead: hf tiles whole and the rest in two
        // K halves, hf + 2 (tiles - hf) = one workgroup per slot (M = 512 gate: 384 tiles,
        // 256 whole + 128 halved).  The xhalf tactic 4 keeps the plain grid.
        const uint64_t tiles = (uint64_t)a.groups[0] * a.groups[2];
        const uint64_t slots = 2ull * ctx->n_cu;
        if (balance && a.hx4b_fn && tiles > slots / 2 && tiles < slots && a.push[6] >= 2 * 256) {
          const uint32_t hf = (uint32_t)(2 * tiles - slots);
          l.fn = a.hx4b_fn;
          l.groups[0] = (uint32_t)slots;
          l.groups[1] = l.groups[2] = 1;
          l.split = 2;
          l.extra = {hf, a.groups[2]};
          l.n_cnt = (uint32_t)(tiles - hf);
          l.ws_bytes = (uint64_t)l.n_cnt * 2 * kSplitTileBytes;
        }
      }
      if (!l.split) l.split = 1;  // the K-split arguments, unsplit
      l.args[4] = (uint32_t)(h_off / 2);  // f16 units
      l.args[8] = a.push[6];
      l.xh_buf = 2;
      l.xh_bytes = out.back().xh_bytes;
      out.push_back(std::move(l));
      i++;
      continue;
    }
    const Command *run[kMaxSeg] = {&a};
    uint32_t n = 1;
    uint64_t x = a.groups[0];
    while (fuse && n < kMaxSeg && i + n < cmds.size() && fusable(a, cmds[i + n], x)) {
      run[n] = &cmds[i + n];
      x += cmds[i + n].groups[0];
      n++;
    }
    out.push_back(pack(run, n));
    i += n;
  }
  return out;
}

int launch(hipStream_t stream, const Launch &l) {
  // kernel parameters: binding pointers in order, then the push struct by value
  std::vector<void *> params;
  params.reserve(l.bufs.size() + 1);
  for (void *const &p : l.bufs) params.push_back(const_cast<void **>(&p));
  params.push_back(const_cast<uint32_t *>(l.args.data()));
  if (l.split) {
    params.push_back(const_cast<void **>(&l.ws));
    params.push_back(const_cast<void **>(&l.cnt));
    params.push_back(const_cast<uint32_t *>(&l.split));
  }
  for (const uint32_t &v : l.extra) params.push_back(const_cast<uint32_t *>(&v));
  HIP_TRY(hipModuleLaunchKernel(l.fn, l.groups[0], l.groups[1], l.groups[2], l.threads, 1, 1, 0,
                                stream, params.data(), nullptr));
  return SKYLA_HIP_OK;
}

// Gives the K-split launches of a list their workspace: one device allocation (partial
// tiles, then per-tile counters, then the f16 rows of the matmul prepass) sized for the
// largest, shared by all of them since the launches of a list run one after another on one
// stream.  The counters are zeroed here, outside any graph capture, and every launch leaves
// them zero.  *owned receives the allocation (nullptr when no launch needs one).
int bind_workspace(std::vector<Launch> &ls, void **owned) {
  *owned = nullptr;
  uint64_t ws = 0, n_cnt = 0, xh = 0;
  for (const Launch &l : ls) {
    if (l.split) {
      ws = std::max(ws, l.ws_bytes);
      n_cnt = std::max<uint64_t>(n_cnt, l.n_cnt);
    }
    if (l.xh_buf >= 0) xh = std::max(xh, l.xh_bytes);
  }
  if (!ws && !n_cnt && !xh) return SKYLA_HIP_OK;
  const uint64_t cnt_off = (ws + 255) & ~(uint64_t)255;
  const uint64_t xh_off = (cnt_off + n_cnt * 4 + 255) & ~(uint64_t)255;
  void *mem = nullptr;
  HIP_TRY(hipMalloc(&mem, xh_off + xh));
  hipError_t e = hipMemset((char *)mem + cnt_off, 0, n_cnt * 4);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    hipFree(mem);
    return fail(SKYLA_HIP_E_DEVICE, "K-split workspace: %s", hipGetErrorString(e));
  }
  for (Launch &l : ls) {
    if (l.split) {
      l.ws = mem;
      l.cnt = (char *)mem + cnt_off;
    }
    if (l.xh_buf >= 0) l.bufs[l.xh_buf] = (char *)mem + xh_off;
  }
  *owned = mem;
  return SKYLA_HIP_OK;
}

}  // namespace

struct skyla_hip_recorder {
  skyla_hip_context *ctx = nullptr;
  bool profile = false;
  std::vector<Command> cmds;
  int status = SKYLA_HIP_OK;
  std::string error;
  uint32_t marks = 0;
};

struct skyla_hip_recording {
  skyla_hip_context *ctx = nullptr;
  bool profile = false;
  std::vector<Command> cmds;
  std::vector<Launch> launches;
  void *workspace = nullptr;  // K-split partials and counters of the launches
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  std::vector<std::string> labels;
  std::vector<double> mark_ns;
  bool replayed = false;
  // device resources go with the recording, also when record_end fails half-way
  ~skyla_hip_recording() {
    if (ctx) {
      hipSetDevice(ctx->device);
      hipStreamSynchronize(ctx->stream);
    }
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    if (workspace) hipFree(workspace);
  }
};

namespace {

// The command a dispatch of pipeline p records: its kernel and every form the runtime
// may substitute for it (binding set `bufs`, grid `groups`, the push words).
Command dispatch_command(const skyla_hip_pipeline *p, const std::vector<void *> &bufs, const uint32_t *groups,
                         const uint32_t *push, uint32_t n_push) {
  Command c;
  c.kind = Command::Dispatch;
  c.fn = p->fn;
  c.threads = p->threads;
  c.segmented = p->segmented;
  c.retile = p->retile;
  c.split_fn = p->split_fn;
  c.hx_fn = p->hx_fn;
  c.hxm_fn = p->hxm_fn;
  c.hxms_fn = p->hxms_fn;
  c.hx4_fn = p->hx4_fn;
  c.hx4b_fn = p->hx4b_fn;
  c.hxs_fn = p->hxs_fn;
  c.split_threads = p->split_threads;
  c.tok_fn = p->tok_fn;
  c.tok_per_wg = p->tok_per_wg;
  c.tok_per_wg_y = p->tok_per_wg_y;
  c.tok_threads = p->tok_threads;
  c.name = p->name;
  c.moe_fn = p->moe_fn;
  c.moe_fn3 = p->moe_fn3;
  c.moe_fn4 = p->moe_fn4;
  for (int i = 0; i < 3; i++) c.groups[i] = groups[i];
  c.bufs = bufs;
  c.push.assign(push, push + n_push);
  return c;
}

hipFunction_t find_function(skyla_hip_context *ctx, const std::string &sym) {
  for (hipModule_t m : ctx->modules) {
    hipFunction_t fn = nullptr;
    if (hipModuleGetFunction(&fn, m, sym.c_str()) == hipSuccess && fn) return fn;
  }
  (void)hipGetLastError();  // lookups that missed leave a sticky error behind
  return nullptr;
}

// Variant choice for matvec launches, from sweeps on MI355X.  Dense rows (Qwen3-8B decode
// shapes, n_in 4096 and 12288): eight-wave workgroups (four for Q6_K launches of 12288 rows
// or more); large launches gain from fewer lanes per row (more pipelined load steps per
// lane, fewer workgroups staging the activations), small ones from more workgroups.
// Q6_K 12288 -> 4096 (the down projection, f32 arithmetic), us per launch over 36 layers:
// (8, 1, 64) 12.2, (8, 1, 32) 13.4-13.6, (4, 1, 32) 13.6, (4, 2, 64) 13.7, (4, 1, 16) 14.7.
// Expert rows (MOE = 1, grid.y = slots; config-4 gate/up n_in 2048 and down n_in 768 over
// 8 slots): 16 lanes per row, one row each, four waves.
// Each entry is (min_rows, waves, rows, lanes per row); grid.x follows from n_out.
struct VariantRule {
  const char *name;
  uint32_t moe;
  uint32_t n_out_word;
  struct { uint64_t min_rows; uint32_t waves, rows, lpr; } v[3];
  int n;
};
const VariantRule kVariantRules[] = {
    {"matvec_q4k", 0, 5, {{6144, 8, 1, 16}, {0, 8, 1, 64}}, 2},
    {"matvec_q6k", 0, 7, {{12288, 4, 1, 16}, {0, 8, 1, 64}}, 2},
    {"matvec_q4k", 1, 5, {{0, 4, 1, 16}}, 1},
    // the fused forms take the same variants (they are compiled for exactly these)
    {"matvec_q4k_norm", 0, 5, {{6144, 8, 1, 16}, {0, 8, 1, 64}}, 2},
    {"matvec_q4k_silu", 0, 5, {{6144, 8, 1, 16}, {0, 8, 1, 64}}, 2},
    {"matvec_q6k_norm", 0, 7, {{12288, 4, 1, 16}, {0, 8, 1, 32}}, 2},
    {"matvec_q6k_silu", 0, 7, {{12288, 4, 1, 16}, {0, 8, 1, 32}}, 2},
};

// K-split Q4_K forms for launches whose rows all have n_in = 4096 (matvec.hip,
// matvec_q4k_ks_body): (rows per slot, row-groups per workgroup) by launch size, from sweeps
// on MI355X.  A workgroup of 512 threads covers 4 * rpl * ng rows (half as many outputs for
// the gate/up pair).  Config-2 launches (us, K-split 4 x 1 against the LDS-staged forms):
// q+k+v 6.50 / 6.71, o 5.28 / 6.13; gate+up was 13.33 / 13.04 in an earlier build, and the
// whole config-2 step now measures 3385 against 3322 GB/s with gate+up on 4 x 1 too, so
// every plain launch takes it.  The gate/up pair (8192 outputs or more) stays on the
// LDS-staged pair form.  The ks tactic 0 keeps the LDS-staged forms everywhere; ks=R_G
// forces one shape (for sweeps).
struct KsRule {
  uint64_t min_rows, max_rows;  // rows of the launch (outputs for the gate/up pair)
  uint32_t rpl, ng;
  uint32_t pd = 1;              // Q6_K: row-groups loaded ahead
};
// (the launches of at most 8191 rows, q+k+v and o, on their own shape: config-2 step
// (4, 1) 3387-3397 GB/s, (2, 2) 3336, (2, 1) 3331-3340, (8, 1) 3247 on one box.)  Launches
// of 16384 rows or more (the fused gate+up, 24576 rows) take (4, 6), 1024 workgroups
// instead of 1536: config-2 step 3540-3547 against 3503-3510 GB/s, matvec_q4k 7.58-7.65
// against 7.71-7.77 us per launch (four runs each, one box); (8, 1) 3518-3538, (4, 3)
// 3469-3482, (4, 2), (8, 3), (2, 2), (2, 1) slower.  A row's sum does not depend on the
// shape, so every shape gives the same bits.
const KsRule kKsRules[] = {{0, 16383, 4, 1}, {16384, ~uint64_t{0}, 4, 6}};
const KsRule kKsPairRules[] = {{0, 8191, 4, 1}};
// the gate/up pair with the FFN norm folded in (MODE 4 of the K-split body).  Its 102 VGPRs
// (the norm weights held beside x) leave two 8-wave workgroups per CU, so the shape is the
// one whose workgroups all fit at once: config 5 at 1k context, device ms per token on one
// box, (4, 3) 1.854 and (4, 6) 1.855 against 1.877-1.882 for the LDS-staged pair form;
// (4, 2) 1.883, (8, 1) 1.894, (8, 3) 1.917, and (4, 1) 2.049 and (2, 2) 2.046 (three rounds
// of workgroups).  With the weights loaded non-temporal, (4, 6) 1.781-1.783 against (4, 3)
// 1.792-1.793 at 1k and 2.266-2.267 against 2.274-2.279 at 16k (two runs each, one box;
// (4, 2) 1.836, (8, 1) 1.855).  The ksglun tactic 0 keeps the LDS-staged pair, R_G forces a
// shape.
const KsRule kKsGlunRules[] = {{0, ~uint64_t{0}, 4, 6}};
// q/k/v with the attention norm folded in (MODE 2, the same 102 VGPRs): config 5 at 1k
// context, device ms per token on one box, (4, 2) 1.809 against 1.833-1.838 for (4, 1);
// (8, 1) 1.826, (2, 2) 1.850, (4, 3) 1.849, (2, 1) 1.900.  The ksnorm tactic R_G forces a shape.
const KsRule kKsNormRules[] = {{0, ~uint64_t{0}, 4, 2}};
// K-split Q6_K form (n_in = 12288; rows per slot, row-groups, row-groups loaded ahead).
// Config-2 down projection (4096 rows), us per launch over 36 layers on two boxes: (1, 8, 1)
// 11.75 / 11.89 against 12.25 / 12.48 for the LDS-staged (8, 1, 64); (1, 8, 2) 12.40,
// (1, 16, 2) 12.83, (2, 4, 2) 13.89, (8, 1, 1) 14.02, (1, 8, 7) 14.19.  The ks6 tactic R_G_D
// forces one shape (sweeps); ks=0 turns it off with the Q4_K forms.
const std::vector<KsRule> kKs6Rules = {{0, ~uint64_t{0}, 1, 8, 1}};
// K-split Q4_K form for n_in = 12288 (rows per slot, row-groups; matvec_q4k_ks3).  The ks3
// tactic R_G forces one shape, 0 keeps the LDS-staged form.
const KsRule kKs3Rules[] = {{0, ~uint64_t{0}, 2, 2}};

void add_ks(skyla_hip_context *ctx, const char *name, const uint32_t *spec, Retile &t) {
  const std::string ksv = tactic("ks");
  if (ksv == "0") return;
  uint32_t fr = 0, fg = 0, fd = 0;
  if (std::strcmp(name, "matvec_q6k") == 0 && spec[3] == 0) {
    // K-split Q6_K form for launches whose rows all have n_in = 12288 (matvec_q6k_ks_body):
    // three waves, RPL rows per row-group, NG row-groups per workgroup
    std::vector<KsRule> rules(std::begin(kKs6Rules), std::end(kKs6Rules));
    if (std::sscanf(tactic("ks6").c_str(), "%u_%u_%u", &fr, &fg, &fd) == 3) rules = {{0, ~uint64_t{0}, fr, fg, fd}};
    std::vector<MatvecAlt> alts;
    for (const KsRule &r : rules) {
      const std::string sym = "matvec_q6k_ks__" + std::to_string(spec[1]) + "_" + std::to_string(r.rpl) + "_" +
                              std::to_string(r.ng) + "_" + std::to_string(r.pd);
      hipFunction_t fn = find_function(ctx, sym);
      if (!fn) return;  // all or nothing
      alts.push_back({fn, r.rpl * r.ng, 192, r.min_rows, 12288, r.max_rows});
    }
    t.n_in_word = 6;  // MatvecPush4.n_in
    t.alts.insert(t.alts.end(), alts.begin(), alts.end());
    return;
  }
  std::string ks;
  bool pair = false, glun = false, norm = false;
  if (std::strcmp(name, "matvec_q4k") == 0 && spec[3] == 0)
    ks = "matvec_q4k_ks__" + std::to_string(spec[1]);
  else if (std::strcmp(name, "matvec_q4k_norm") == 0 && spec[1] == 0)
    ks = "matvec_q4k_ks_norm__0", norm = true;
  else if (std::strcmp(name, "matvec_q4k_glu") == 0)
    ks = "matvec_q4k_ks_glu__0", pair = true;
  else if (std::strcmp(name, "matvec_q4k_glun") == 0 && tactic("ksglun") != "0")
    ks = "matvec_q4k_ks_glun__0", pair = true, glun = true;
  else
    return;
  std::vector<KsRule> rules(glun ? std::begin(kKsGlunRules) : pair ? std::begin(kKsPairRules)
                            : norm ? std::begin(kKsNormRules) : std::begin(kKsRules),
                            glun ? std::end(kKsGlunRules) : pair ? std::end(kKsPairRules)
                            : norm ? std::end(kKsNormRules) : std::end(kKsRules));
  // forced shapes (sweeps and the parity tests of every compiled shape): ks=R_G for the plain
  // and pair forms, ksglun=R_G for the norm-folded pair, ksnorm=R_G for the norm-folded form
  const std::string forced = glun ? tactic("ksglun") : norm ? tactic("ksnorm") : ksv;
  if (std::sscanf(forced.c_str(), "%u_%u", &fr, &fg) == 2) rules = {{0, ~uint64_t{0}, fr, fg}};
  std::vector<MatvecAlt> alts;
  for (const KsRule &r : rules) {
    hipFunction_t fn = find_function(ctx, ks + "_" + std::to_string(r.rpl) + "_" + std::to_string(r.ng));
    if (!fn) return;  // all or nothing
    alts.push_back({fn, (pair ? 2u : 4u) * r.rpl * r.ng, 512, r.min_rows, 4096, r.max_rows});
  }
  // plain Q4_K launches whose rows all have n_in = 12288 (the down projection): the same
  // body with three 4096-value parts per row (matvec_q4k_ks3)
  if (!pair && !norm) {
    std::vector<KsRule> rules3(std::begin(kKs3Rules), std::end(kKs3Rules));
    if (std::sscanf(tactic("ks3").c_str(), "%u_%u", &fr, &fg) == 2) rules3 = {{0, ~uint64_t{0}, fr, fg}};
    for (const KsRule &r : rules3) {
      if (tactic("ks3") == "0") break;
      hipFunction_t fn = find_function(ctx, "matvec_q4k_ks3__" + std::to_string(spec[1]) + "_" +
                                                std::to_string(r.rpl) + "_" + std::to_string(r.ng));
      if (!fn) return;  // all or nothing
      alts.push_back({fn, 4u * r.rpl * r.ng, 512, r.min_rows, 12288, r.max_rows});
    }
  }
  t.alts.insert(t.alts.end(), alts.begin(), alts.end());
}

std::shared_ptr<const Retile> make_retile(skyla_hip_context *ctx, const char *name, const uint32_t *spec,
                                          uint32_t n_spec) {
  if (n_spec != 5) return nullptr;
  if (!tactic_on("retile")) return nullptr;
  auto t = std::make_shared<Retile>();
  t->n_out_word = 5;
  add_ks(ctx, name, spec, *t);
  std::vector<VariantRule> rules(std::begin(kVariantRules), std::end(kVariantRules));
  // Dense Q8_0 launches of 65536 rows or more (config 1's tied head, 151936 x 1024): the
  // engine's (4, 2, 64) variant stages the activations in a workgroup per 8 rows (72.7 us,
  // 2.1 TB/s); (4, 1, 16) covers 16 rows a workgroup with 16 lanes a row: config 1 0.852 ->
  // 0.817-0.820 ms per token (1090 -> 1137-1140 tok/s); (8, 1, 16) 0.818-0.821, (4, 2, 16)
  // 0.820-0.822, (4, 4, 64) 0.833-0.835, (8, 1, 32) 0.834-0.836, (8, 2, 64) 0.838, (2, 1,
  // 16) 0.861-0.862 (one box).  Launches below 2048 rows (config 1's o and SiLU-folded
  // down, 1024 rows: 128 workgroups of 8 rows) take (4, 1, 64), 4 rows a workgroup: 0.818 ->
  // 0.781-0.782 ms per token (1131-1135 -> 1183-1189 tok/s); (2, 1, 64) 0.832-0.833, (2, 2,
  // 64) 0.840-0.841, (1, 1, 64) 0.857-0.858 (one box).  The rest keep the engine's variant.
  if (std::strcmp(name, "matvec_q8_0") == 0 || std::strcmp(name, "matvec_q8_0_silu") == 0) {
    VariantRule q{name, 0, 5, {}, 0};
    unsigned bw = 0, br = 0, bl = 0, sw = 0, sr = 0, sl = 0;
    const bool big = std::strcmp(name, "matvec_q8_0") == 0 && spec[1] == 0 &&
                     std::sscanf(tactic("q8_big").c_str(), "%u_%u_%u", &bw, &br, &bl) == 3;
    const bool small = std::sscanf(tactic("q8_small").c_str(), "%u_%u_%u", &sw, &sr, &sl) == 3;
    if (big) q.v[q.n++] = {65536, bw, br, bl};
    q.v[q.n++] = {small ? 2048u : 0u, spec[0], spec[2], spec[4]};
    if (small) q.v[q.n++] = {0, sw, sr, sl};
    if (q.n > 1) rules.push_back(q);
  }
  for (VariantRule r : rules) {
    if (std::strcmp(r.name, name) != 0 || r.moe != spec[3]) continue;
    // the variant tactic W_R_L puts every dense launch of this kernel on one variant (sweeps)
    if (!spec[3]) {
      unsigned vw = 0, vr = 0, vl = 0;
      if (std::sscanf(tactic("variant").c_str(), "%u_%u_%u", &vw, &vr, &vl) == 3) {
        r.v[0] = {0, vw, vr, vl};
        r.n = 1;
      }
    }
    t->n_out_word = r.n_out_word;
    std::vector<MatvecAlt> alts;
    for (int i = 0; i < r.n; i++) {
      const auto &v = r.v[i];
      const std::string sym = std::string(name) + "__" + std::to_string(v.waves) + "_" +
                              std::to_string(spec[1]) + "_" + std::to_string(v.rows) + "_" +
                              std::to_string(spec[3]) + "_" + std::to_string(v.lpr);
      hipFunction_t fn = find_function(ctx, sym);
      if (!fn) {  // keep the engine's variant if any alternative is missing
        alts.clear();
        break;
      }
      alts.push_back({fn, v.waves * v.rows * (64 / v.lpr), 64 * v.waves, v.min_rows});
    }
    t->alts.insert(t->alts.end(), alts.begin(), alts.end());
    break;
  }
  if (t->alts.empty()) return nullptr;
  return t;
}

}  // namespace

extern "C" {

const char *skyla_hip_last_error(void) { return g_error.c_str(); }

int skyla_hip_context_new(int device, skyla_hip_context **out) {
  if (!out) return fail(SKYLA_HIP_E_ARG, "context_new: null output");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(SKYLA_HIP_E_DEVICE, "no HIP device available (%s)",
                e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  if (device < 0) {
    const char *env = std::getenv("SKYLA_DEVICE");  // skyla-vk/src/context.rs:50-55
    device = env ? std::atoi(env) : 0;
  }
  if (device < 0 || device >= count)
    return fail(SKYLA_HIP_E_ARG, "device %d out of range (%d devices)", device, count);
  auto ctx = std::make_unique<skyla_hip_context>();
  ctx->device = device;
  HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(SKYLA_HIP_E_DEVICE, "device %d is %s; this backend carries gfx950 code only",
                device, prop.gcnArchName);
  ctx->name = prop.name[0] ? prop.name : "AMD Instinct";
  ctx->name += std::string(" (") + prop.gcnArchName + ", " + std::to_string(prop.multiProcessorCount) + " CUs)";
  ctx->warp = (uint32_t)prop.warpSize;
  HIP_TRY(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
  const unsigned char *images[] = {skyla_co_matvec, skyla_co_matmul, skyla_co_moe, skyla_co_util,
                                   skyla_co_attention};
  for (const unsigned char *img : images) {
    hipModule_t m = nullptr;
    hipError_t le = hipModuleLoadData(&m, img);
    if (le != hipSuccess) {
      skyla_hip_context_free(ctx.release());
      return fail(SKYLA_HIP_E_DEVICE, "hipModuleLoadData: %s", hipGetErrorString(le));
    }
    ctx->modules.push_back(m);
  }
  // The allocation-free dispatch's workspace: the `scratch` array of the matmul code object
  // as loaded for this device.  The code objects are loaded with hipModuleLoadData rather
  // than registered with the runtime, so the module API's lookup (hipModuleGetGlobal) is
  // the one that resolves its address; host code uses only this pointer, never the name.
  {
    hipDeviceptr_t dp = nullptr;
    size_t bytes = 0;
    hipError_t ge = hipModuleGetGlobal(&dp, &bytes, ctx->modules[1], "scratch");
    if (ge != hipSuccess || !dp || bytes < kScratchTiles * 128 * 128 * 4 + kScratchCounters * 4) {
      (void)hipGetLastError();
      skyla_hip_context_free(ctx.release());
      return fail(SKYLA_HIP_E_DEVICE, "hipModuleGetGlobal(scratch): %s (%zu bytes)", hipGetErrorString(ge), bytes);
    }
    ctx->scratch = static_cast<char *>(dp);
    ctx->scratch_bytes = bytes;
    hipError_t fe = hipModuleGetFunction(&ctx->fill_u32, ctx->modules[1], "fill_u32");
    if (fe != hipSuccess || !ctx->fill_u32) {
      (void)hipGetLastError();
      skyla_hip_context_free(ctx.release());
      return fail(SKYLA_HIP_E_DEVICE, "hipModuleGetFunction(fill_u32): %s", hipGetErrorString(fe));
    }
  }
  ctx->x_half_rows = find_function(ctx.get(), "x_half_rows");
  ctx->silu_half_rows = find_function(ctx.get(), "silu_half_rows");
  ctx->silu_mul = find_function(ctx.get(), "silu_mul");
  ctx->rmsnorm_half_rows = find_function(ctx.get(), "rmsnorm_half_rows");
  ctx->rmsnorm = find_function(ctx.get(), "rmsnorm");
  if (prop.multiProcessorCount > 0) ctx->n_cu = (uint32_t)prop.multiProcessorCount;
  *out = ctx.release();
  return SKYLA_HIP_OK;
}

void skyla_hip_context_free(skyla_hip_context *ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  for (hipModule_t m : ctx->modules) hipModuleUnload(m);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
}

uint32_t skyla_hip_subgroup_size(const skyla_hip_context *ctx) { return ctx ? ctx->warp : 0; }

uint64_t skyla_hip_max_buffer(const skyla_hip_context *ctx) { return ctx ? kMaxBuffer : 0; }

int skyla_hip_device_name(const skyla_hip_context *ctx, char *out, size_t cap) {
  if (!ctx || !out || cap == 0) return fail(SKYLA_HIP_E_ARG, "device_name: bad argument");
  std::snprintf(out, cap, "%s", ctx->name.c_str());
  return SKYLA_HIP_OK;
}

int skyla_hip_alloc(skyla_hip_context *ctx, uint64_t size, skyla_hip_buffer **out) {
  if (!ctx || !out) return fail(SKYLA_HIP_E_ARG, "alloc: bad argument");
  *out = nullptr;
  if (size == 0) return fail(SKYLA_HIP_E_ARG, "alloc: zero-sized buffer");
  if (size > kMaxBuffer)
    return fail(SKYLA_HIP_E_OOM, "alloc: %llu bytes is above the %llu-byte buffer cap",
                (unsigned long long)size, (unsigned long long)kMaxBuffer);
  HIP_TRY(hipSetDevice(ctx->device));
  auto b = std::make_unique<skyla_hip_buffer>();
  b->ctx = ctx;
  b->size = size;
  hipError_t e = hipMalloc(&b->dev, size);
  if (e != hipSuccess)
    return fail(SKYLA_HIP_E_OOM, "hipMalloc(%llu): %s", (unsigned long long)size,
                hipGetErrorString(e));
  e = hipMemsetAsync(b->dev, 0, size, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    hipFree(b->dev);
    return fail(SKYLA_HIP_E_DEVICE, "clearing a new buffer: %s", hipGetErrorString(e));
  }
  *out = b.release();
  return SKYLA_HIP_OK;
}

void skyla_hip_buffer_free(skyla_hip_buffer *buf) {
  if (!buf) return;
  hipSetDevice(buf->ctx->device);
  hipStreamSynchronize(buf->ctx->stream);
  hipFree(buf->dev);
  delete buf;
}

uint64_t skyla_hip_buffer_size(const skyla_hip_buffer *buf) { return buf ? buf->size : 0; }

void *skyla_hip_buffer_host(skyla_hip_buffer *buf) {
  if (!buf) {
    fail(SKYLA_HIP_E_ARG, "buffer_host: null buffer");
    return nullptr;
  }
  if (!buf->host) {
    void *pinned = nullptr;
    if (buf->size <= kMaxPinned && hipHostMalloc(&pinned, buf->size, hipHostMallocDefault) == hipSuccess) {
      buf->host = std::unique_ptr<unsigned char[], HostFree>((unsigned char *)pinned, HostFree(true));
    } else {
      (void)hipGetLastError();  // a refused pinned allocation falls back to pageable memory
      buf->host.reset(new (std::nothrow) unsigned char[buf->size]);
    }
    if (!buf->host) {
      fail(SKYLA_HIP_E_OOM, "buffer_host: cannot allocate %llu host bytes",
           (unsigned long long)buf->size);
      return nullptr;
    }
    std::memset(buf->host.get(), 0, buf->size);
  }
  return buf->host.get();
}

static int check_range(const skyla_hip_buffer *buf, uint64_t off, uint64_t len, const char *what) {
  if (!buf) return fail(SKYLA_HIP_E_ARG, "%s: null buffer", what);
  if (off > buf->size || len > buf->size - off)
    return fail(SKYLA_HIP_E_ARG, "%s: range [%llu, +%llu) outside a %llu-byte buffer", what,
                (unsigned long long)off, (unsigned long long)len, (unsigned long long)buf->size);
  return SKYLA_HIP_OK;
}

int skyla_hip_buffer_upload(skyla_hip_buffer *buf, uint64_t off, uint64_t len) {
  int s = check_range(buf, off, len, "buffer_upload");
  if (s) return s;
  if (!skyla_hip_buffer_host(buf)) return SKYLA_HIP_E_OOM;
  HIP_TRY(hipSetDevice(buf->ctx->device));
  HIP_TRY(hipMemcpyAsync((char *)buf->dev + off, buf->host.get() + off, len,
                         hipMemcpyHostToDevice, buf->ctx->stream));
  HIP_TRY(hipStreamSynchronize(buf->ctx->stream));
  return SKYLA_HIP_OK;
}

int skyla_hip_buffer_download(skyla_hip_buffer *buf, uint64_t off, uint64_t len) {
  int s = check_range(buf, off, len, "buffer_download");
  if (s) return s;
  if (!skyla_hip_buffer_host(buf)) return SKYLA_HIP_E_OOM;
  HIP_TRY(hipSetDevice(buf->ctx->device));
  HIP_TRY(hipMemcpyAsync(buf->host.get() + off, (char *)buf->dev + off, len,
                         hipMemcpyDeviceToHost, buf->ctx->stream));
  HIP_TRY(hipStreamSynchronize(buf->ctx->stream));
  return SKYLA_HIP_OK;
}

void *skyla_hip_buffer_device(skyla_hip_buffer *buf) { return buf ? buf->dev : nullptr; }

int skyla_hip_buffer_copy(skyla_hip_buffer *dst, uint64_t dst_off, const skyla_hip_buffer *src,
                          uint64_t src_off, uint64_t len) {
  int s = check_range(dst, dst_off, len, "buffer_copy dst");
  if (s) return s;
  s = check_range(src, src_off, len, "buffer_copy src");
  if (s) return s;
  HIP_TRY(hipSetDevice(dst->ctx->device));
  HIP_TRY(hipMemcpyAsync((char *)dst->dev + dst_off, (const char *)src->dev + src_off, len,
                         hipMemcpyDeviceToDevice, dst->ctx->stream));
  HIP_TRY(hipStreamSynchronize(dst->ctx->stream));
  return SKYLA_HIP_OK;
}

int skyla_hip_pipeline_new(skyla_hip_context *ctx, const char *name, uint32_t n_buffers,
                           uint32_t push_size, const uint32_t *spec, uint32_t n_spec,
                           uint32_t n_sets, skyla_hip_pipeline **out) {
  if (!ctx || !name || !out || (n_spec && !spec))
    return fail(SKYLA_HIP_E_ARG, "pipeline_new: bad argument");
  *out = nullptr;
  const KernelInfo *k = find_kernel(name);
  if (!k) return fail(SKYLA_HIP_E_NO_KERNEL, "no gfx950 kernel named %s", name);
  if (n_spec < k->spec_len_min || n_spec > k->spec_len_max)
    return fail(SKYLA_HIP_E_NO_KERNEL, "%s takes %u..%u spec constants, got %u", name,
                k->spec_len_min, k->spec_len_max, n_spec);
  if (n_buffers != k->n_buffers)
    return fail(SKYLA_HIP_E_ARG, "%s binds %u buffers, pipeline asks for %u", name,
                k->n_buffers, n_buffers);
  if (push_size != 4 * k->push_words)
    return fail(SKYLA_HIP_E_ARG, "%s takes %u push bytes, pipeline asks for %u", name,
                4 * k->push_words, push_size);
  if (n_sets == 0) n_sets = 1;
  // symbol: name__s0_s1_...; matmul's trailing X_HALF = 0 is the plain variant
  uint32_t n_key = n_spec;
  if (std::strcmp(name, "matmul") == 0 && n_spec == 4 && spec[3] == 0) n_key = 3;
  std::string sym = name;
  for (uint32_t i = 0; i < n_key; i++) sym += (i ? "_" : "__") + std::to_string(spec[i]);
  uint32_t threads = k->threads;
  if (k->threads_from_spec >= 0)
    threads = k->waves ? 64 * spec[k->threads_from_spec] : spec[k->threads_from_spec];
  // matmul: dense tiles (MOE = 0) run eight waves, expert groups four (matmul.hip)
  if (std::strcmp(name, "matmul") == 0 && spec[2] == 0) threads = 512;
  auto p = std::make_unique<skyla_hip_pipeline>();
  p->ctx = ctx;
  p->symbol = sym;
  p->n_buffers = n_buffers;
  p->push_words = k->push_words;
  p->threads = threads;
  p->segmented = k->segmented;
  p->sets.assign(n_sets, std::vector<void *>(n_buffers, nullptr));
  HIP_TRY(hipSetDevice(ctx->device));
  for (hipModule_t m : ctx->modules) {
    hipFunction_t fn = nullptr;
    if (hipModuleGetFunction(&fn, m, sym.c_str()) == hipSuccess && fn) {
      p->fn = fn;
      break;
    }
  }
  (void)hipGetLastError();  // lookups that missed leave a sticky error behind
  if (!p->fn)
    return fail(SKYLA_HIP_E_NO_KERNEL, "no gfx950 kernel %s for this spec", sym.c_str());
  p->retile = make_retile(ctx, name, spec, n_spec);
  p->name = name;
  // MoE decode forms (fuse_moe): Q4_K expert matvecs whose launches the variant rule puts
  // on (4, 1, 16)
  if (std::strcmp(name, "matvec_q4k") == 0 && n_spec == 5 && spec[1] == 0 && spec[3] == 1 && p->retile &&
      p->retile->alts.size() == 1 && p->retile->alts[0].rwg == 16 && p->retile->alts[0].threads == 256) {
    p->moe_fn = find_function(ctx, "matvec_q4k_glu__4_0_1_1_16");
    p->moe_fn3 = find_function(ctx, "matvec_q4k_dcomb__8");
    p->moe_fn4 = find_function(ctx, "matvec_q4k_glur__4_0_1_1_16");
  }
  // router logits of a batch: 8 x 8 (expert, token) blocks per workgroup (moe.hip, moe_logits_t)
  if (std::strcmp(name, "moe_logits") == 0) {
    p->tok_fn = find_function(ctx, "moe_logits_t");
    p->tok_per_wg = p->tok_per_wg_y = 8;
  }
  // the attention merge of a batched step (grid (heads, tokens)): one wave per (head, token),
  // four heads per workgroup (attention.hip, attention_merge_t); the merge_t tactic 0 keeps
  // the 1024-thread form
  if (std::strcmp(name, "attention_merge") == 0 && n_spec == 2 && spec[0] == 128 && spec[1] == 0) {
    if (tactic_on("merge_t")) {
      p->tok_fn = find_function(ctx, "attention_merge_t__128_0");
      p->tok_per_wg = 4;
      p->tok_per_wg_y = 1;
      p->tok_threads = 256;
    }
  }
  // dense K-quant matmul (TYPE 1/2, MOE 0): its K-split variant, used for launches with few
  // tiles (split_of); the splitk tactic 0 keeps every launch on the engine's kernel
  if (std::strcmp(name, "matmul") == 0 && n_spec >= 3 && (spec[0] == 1 || spec[0] == 2) && spec[2] == 0) {
    if (tactic_on("splitk")) {
      const std::string ssym = "matmul_w8__" + std::to_string(spec[0]) + "_" + std::to_string(spec[1]) + "_" +
                               std::to_string(n_spec == 4 ? spec[3] : 0);
      p->split_fn = find_function(ctx, ssym);
      p->split_threads = 512;
    }
    // f32 inputs: the tile on x_half_rows's f16 rows (build_launches inserts the prepass),
    // by default the forms whose operands go straight into LDS (eight waves: x8d, x8ds; four
    // waves, Q4_K only: x4d, x4db); the dl tactic 0 keeps the register-staged tiles.
    if (!(n_spec == 4 && spec[3])) {
      const bool dl = tactic_on("dl");
      const bool dl4 = dl && spec[0] == 1;
      const std::string ts = std::to_string(spec[0]) + "_" + std::to_string(spec[1]);
      p->hx_fn = find_function(ctx, (dl ? "matmul_x8d__" : "matmul_x8__") + ts);
      p->hx4_fn = find_function(ctx, (dl4 ? "matmul_x4d__" : "matmul_x4__") + ts);
      p->hx4b_fn = find_function(ctx, (dl4 ? "matmul_x4db__" : "matmul_x4b__") + ts);
      p->hxs_fn = find_function(ctx, (dl ? "matmul_x8ds__" : "matmul_x8s__") + ts);
      p->split_threads = 512;
    }
  }
  // expert-group K-quant matmul (MOE = 1) on f32 inputs: the same tile on x_half_rows's f16
  // rows (build_launches inserts the prepass of the launch's input rows)
  if (std::strcmp(name, "matmul") == 0 && n_spec >= 3 && (spec[0] == 1 || spec[0] == 2) && spec[2] == 1 &&
      !(n_spec == 4 && spec[3]))
  {
    p->hxm_fn = find_function(ctx, "matmul_xm__" + std::to_string(spec[0]) + "_" + std::to_string(spec[1]));
    p->hxms_fn = find_function(ctx, "matmul_xms__" + std::to_string(spec[0]) + "_" + std::to_string(spec[1]));
  }
  if (p->tok_fn) {  // the batched form must take the workgroup it is launched with
    int tok_max = 0;
    const uint32_t want = p->tok_threads ? p->tok_threads : threads;
    if (hipFuncGetAttribute(&tok_max, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, p->tok_fn) != hipSuccess ||
        tok_max <= 0 || want > (uint32_t)tok_max)
      p->tok_fn = nullptr;
  }
  int max_threads = 0;
  if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, p->fn) ==
          hipSuccess &&
      max_threads > 0 && threads > (uint32_t)max_threads)
    return fail(SKYLA_HIP_E_NO_KERNEL, "%s: %u threads above its limit %d", sym.c_str(),
                threads, max_threads);
  *out = p.release();
  return SKYLA_HIP_OK;
}

void skyla_hip_pipeline_free(skyla_hip_pipeline *p) { delete p; }

int skyla_hip_pipeline_bind(skyla_hip_pipeline *p, uint32_t set, skyla_hip_buffer *const *bufs,
                            uint32_t n) {
  if (!p || (n && !bufs)) return fail(SKYLA_HIP_E_ARG, "pipeline_bind: bad argument");
  if (set >= p->sets.size())
    return fail(SKYLA_HIP_E_ARG, "pipeline_bind: set %u of %zu", set, p->sets.size());
  if (n != p->n_buffers)
    return fail(SKYLA_HIP_E_ARG, "pipeline_bind: %s binds %u buffers, got %u",
                p->symbol.c_str(), p->n_buffers, n);
  for (uint32_t i = 0; i < n; i++) {
    if (!bufs[i]) return fail(SKYLA_HIP_E_ARG, "pipeline_bind: binding %u is null", i);
    if (bufs[i]->ctx != p->ctx)
      return fail(SKYLA_HIP_E_ARG, "pipeline_bind: binding %u belongs to another context", i);
  }
  for (uint32_t i = 0; i < n; i++) p->sets[set][i] = bufs[i]->dev;
  return SKYLA_HIP_OK;
}

int skyla_hip_pipeline_threads(const skyla_hip_pipeline *p, uint32_t out[3]) {
  if (!p || !out) return fail(SKYLA_HIP_E_ARG, "pipeline_threads: bad argument");
  out[0] = p->threads;
  out[1] = 1;
  out[2] = 1;
  return SKYLA_HIP_OK;
}

int skyla_hip_record_begin(skyla_hip_context *ctx, int profile, skyla_hip_recorder **out) {
  if (!ctx || !out) return fail(SKYLA_HIP_E_ARG, "record_begin: bad argument");
  auto r = new (std::nothrow) skyla_hip_recorder();
  if (!r) return fail(SKYLA_HIP_E_OOM, "record_begin: out of memory");
  r->ctx = ctx;
  r->profile = profile != 0;
  *out = r;
  return SKYLA_HIP_OK;
}

static int record_fail(skyla_hip_recorder *r, int code) {
  if (r->status == SKYLA_HIP_OK) {
    r->status = code;
    r->error = g_error;
  }
  return code;
}

int skyla_hip_record_dispatch(skyla_hip_recorder *r, const skyla_hip_pipeline *p, uint32_t set,
                              const uint32_t groups[3], const uint32_t *push, uint32_t n_push) {
  if (!r) return fail(SKYLA_HIP_E_ARG, "record_dispatch: null recorder");
  if (!p || !groups || (n_push && !push))
    return record_fail(r, fail(SKYLA_HIP_E_ARG, "record_dispatch: bad argument"));
  if (p->ctx != r->ctx)
    return record_fail(r, fail(SKYLA_HIP_E_ARG, "record_dispatch: pipeline of another context"));
  if (set >= p->sets.size())
    return record_fail(r, fail(SKYLA_HIP_E_ARG, "record_dispatch: set %u of %zu", set,
                               p->sets.size()));
  if (n_push != p->push_words)
    return record_fail(r, fail(SKYLA_HIP_E_ARG, "record_dispatch: %s takes %u push words, got %u",
                               p->symbol.c_str(), p->push_words, n_push));
  for (void *b : p->sets[set])
    if (!b)
      return record_fail(r, fail(SKYLA_HIP_E_STATE, "record_dispatch: %s set %u is not bound",
                                 p->symbol.c_str(), set));
  Command c = dispatch_command(p, p->sets[set], groups, push, n_push);
  if (groups[0] && groups[1] && groups[2]) r->cmds.push_back(std::move(c));
  return SKYLA_HIP_OK;
}

int skyla_hip_record_barrier(skyla_hip_recorder *r) {
  if (!r) return fail(SKYLA_HIP_E_ARG, "record_barrier: null recorder");
  Command c;
  c.kind = Command::Barrier;
  r->cmds.push_back(std::move(c));
  return SKYLA_HIP_OK;
}

int skyla_hip_record_host_barrier(skyla_hip_recorder *r) {
  // replay waits for the stream, so host visibility needs no command of its own
  return skyla_hip_record_barrier(r);
}

int skyla_hip_record_mark(skyla_hip_recorder *r, const char *label) {
  if (!r) return fail(SKYLA_HIP_E_ARG, "record_mark: null recorder");
  if (!r->profile) return SKYLA_HIP_OK;
  if (r->marks + 1 >= kMaxMarks)
    return record_fail(r, fail(SKYLA_HIP_E_STATE, "too many profiling marks"));
  Command c;
  c.kind = Command::Mark;
  c.label = label ? label : "";
  r->cmds.push_back(std::move(c));
  r->marks++;
  return SKYLA_HIP_OK;
}

int skyla_hip_record_end(skyla_hip_recorder *r, skyla_hip_recording **out) {
  if (!r) return fail(SKYLA_HIP_E_ARG, "record_end: null recorder");
  std::unique_ptr<skyla_hip_recorder> own(r);
  if (!out) return fail(SKYLA_HIP_E_ARG, "record_end: null output");
  *out = nullptr;
  if (r->status != SKYLA_HIP_OK) {
    g_error = "recording failed earlier: " + r->error;
    return r->status;
  }
  auto rec = std::make_unique<skyla_hip_recording>();
  rec->ctx = r->ctx;
  rec->profile = r->profile;
  rec->cmds = std::move(r->cmds);
  for (const Command &c : rec->cmds)
    if (c.kind == Command::Mark) rec->labels.push_back(c.label);
  rec->launches = build_launches(rec->ctx, rec->cmds);
  rec->mark_ns.assign(rec->labels.size(), 0.0);
  HIP_TRY(hipSetDevice(rec->ctx->device));
  if (int s = bind_workspace(rec->launches, &rec->workspace)) return s;
  // the nograph tactic 1: replay the launch list as direct launches (kernel traces of the
  // exact launches a graph would hold, fused forms included)
  if (!rec->profile && skyla_hip_recording_len(rec.get()) > 0 && tactic("nograph") != "1") {
    // One graph for the whole recording, captured from the launch list on the stream.
    skyla_hip_context *ctx = rec->ctx;
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    int s = SKYLA_HIP_OK;
    for (const Launch &l : rec->launches)
      if (!l.mark && (s = launch(ctx->stream, l)) != SKYLA_HIP_OK) break;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (s != SKYLA_HIP_OK) {
      if (graph) hipGraphDestroy(graph);
      return s;
    }
    if (e != hipSuccess)
      return fail(SKYLA_HIP_E_DEVICE, "hipStreamEndCapture: %s", hipGetErrorString(e));
    rec->graph = graph;
    if (graph) {
      e = hipGraphInstantiate(&rec->exec, graph, nullptr, nullptr, 0);
      if (e != hipSuccess) {
        hipGraphDestroy(graph);
        rec->graph = nullptr;
        return fail(SKYLA_HIP_E_DEVICE, "hipGraphInstantiate: %s", hipGetErrorString(e));
      }
    }
  }
  *out = rec.release();
  return SKYLA_HIP_OK;
}

void skyla_hip_recording_free(skyla_hip_recording *rec) { delete rec; }

uint32_t skyla_hip_recording_len(const skyla_hip_recording *rec) {
  if (!rec) return 0;
  uint32_t n = 0;
  for (const Command &c : rec->cmds) n += c.kind == Command::Dispatch;
  return n;
}

uint32_t skyla_hip_recording_launches(const skyla_hip_recording *rec) {
  if (!rec) return 0;
  uint32_t n = 0;
  for (const Launch &l : rec->launches) n += !l.mark;
  return n;
}

namespace {

// Launches a recording on the context stream.  With `events`, one event is recorded at
// the start and one at every mark.
static int submit(skyla_hip_context *ctx, const skyla_hip_recording *rec, std::vector<hipEvent_t> *events) {
  if (rec->exec && !events) {
    HIP_TRY(hipGraphLaunch(rec->exec, ctx->stream));
    return SKYLA_HIP_OK;
  }
  if (events) HIP_TRY(hipEventRecord((*events)[0], ctx->stream));
  size_t m = 1;
  for (const Launch &l : rec->launches) {
    if (!l.mark) {
      int s = launch(ctx->stream, l);
      if (s) return s;
    } else if (events) {
      HIP_TRY(hipEventRecord((*events)[m++], ctx->stream));
    }
  }
  return SKYLA_HIP_OK;
}

struct Events {
  std::vector<hipEvent_t> ev;
  ~Events() {
    for (hipEvent_t e : ev) hipEventDestroy(e);
  }
  int make(size_t n) {
    ev.assign(n, nullptr);
    for (auto &e : ev) HIP_TRY(hipEventCreate(&e));
    return SKYLA_HIP_OK;
  }
};

}  // namespace

int skyla_hip_replay(skyla_hip_context *ctx, const skyla_hip_recording *rec) {
  if (!ctx || !rec) return fail(SKYLA_HIP_E_ARG, "replay: bad argument");
  if (rec->ctx != ctx) return fail(SKYLA_HIP_E_ARG, "replay: recording of another context");
  HIP_TRY(hipSetDevice(ctx->device));
  if (!rec->profile) {
    int s = submit(ctx, rec, nullptr);
    if (s) return s;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return SKYLA_HIP_OK;
  }
  Events e;
  int s = e.make(rec->labels.size() + 1);
  if (s) return s;
  s = submit(ctx, rec, &e.ev);
  if (s) return s;
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  auto *mut = const_cast<skyla_hip_recording *>(rec);
  for (size_t i = 0; i < rec->labels.size(); i++) {
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e.ev[i], e.ev[i + 1]));
    mut->mark_ns[i] = (double)ms * 1e6;
  }
  mut->replayed = true;
  return SKYLA_HIP_OK;
}

int skyla_hip_replay_timed(skyla_hip_context *ctx, const skyla_hip_recording *rec, double *ns) {
  if (!ctx || !rec || !ns) return fail(SKYLA_HIP_E_ARG, "replay_timed: bad argument");
  if (rec->ctx != ctx) return fail(SKYLA_HIP_E_ARG, "replay_timed: recording of another context");
  HIP_TRY(hipSetDevice(ctx->device));
  Events e;
  int s = e.make(2);
  if (s) return s;
  HIP_TRY(hipEventRecord(e.ev[0], ctx->stream));
  s = submit(ctx, rec, nullptr);
  if (s) return s;
  HIP_TRY(hipEventRecord(e.ev[1], ctx->stream));
  HIP_TRY(hipEventSynchronize(e.ev[1]));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, e.ev[0], e.ev[1]));
  *ns = (double)ms * 1e6;
  return SKYLA_HIP_OK;
}

int skyla_hip_marks(skyla_hip_context *ctx, const skyla_hip_recording *rec, const char **labels,
                    double *ns, uint32_t cap, uint32_t *count) {
  if (!ctx || !rec || !count) return fail(SKYLA_HIP_E_ARG, "marks: bad argument");
  if (!rec->profile) return fail(SKYLA_HIP_E_STATE, "recording was not profiled");
  if (!rec->replayed) return fail(SKYLA_HIP_E_STATE, "profiled recording was not replayed");
  *count = (uint32_t)rec->labels.size();
  for (uint32_t i = 0; i < cap && i < rec->labels.size(); i++) {
    if (labels) labels[i] = rec->labels[i].c_str();
    if (ns) ns[i] = rec->mark_ns[i];
  }
  return SKYLA_HIP_OK;
}

int skyla_hip_time_dispatch(skyla_hip_context *ctx, const skyla_hip_pipeline *p,
                            const uint32_t groups[3], const uint32_t *push, uint32_t n_push,
                            uint32_t reps, double *ns_out) {
  if (!ctx || !p || !groups || !ns_out || reps == 0)
    return fail(SKYLA_HIP_E_ARG, "time_dispatch: bad argument");
  if (n_push != p->push_words)
    return fail(SKYLA_HIP_E_ARG, "time_dispatch: %s takes %u push words, got %u",
                p->symbol.c_str(), p->push_words, n_push);
  for (void *b : p->sets[0])
    if (!b) return fail(SKYLA_HIP_E_STATE, "time_dispatch: %s is not bound", p->symbol.c_str());
  HIP_TRY(hipSetDevice(ctx->device));
  const Command c = dispatch_command(p, p->sets[0], groups, push, n_push);
  const Command *one[1] = {&c};
  std::vector<Launch> ls{pack(one, 1)};
  void *workspace = nullptr;
  if (int s = bind_workspace(ls, &workspace)) return s;
  struct FreeWs {
    void *p;
    ~FreeWs() {
      if (p) hipFree(p);
    }
  } free_ws{workspace};
  const Launch &l = ls[0];
  Events e;
  int s = e.make(reps + 1);
  if (s) return s;
  HIP_TRY(hipEventRecord(e.ev[0], ctx->stream));
  for (uint32_t i = 0; i < reps; i++) {
    s = launch(ctx->stream, l);
    if (s) return s;
    HIP_TRY(hipEventRecord(e.ev[i + 1], ctx->stream));
  }
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  for (uint32_t i = 0; i < reps; i++) {
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, e.ev[i], e.ev[i + 1]));
    ns_out[i] = (double)ms * 1e6;
  }
  return SKYLA_HIP_OK;
}

int skyla_hip_dispatch_noalloc(skyla_hip_context *ctx, const skyla_hip_pipeline *p, const uint32_t groups[3],
                               const uint32_t *push, uint32_t n_push) {
  if (!ctx || !p || !groups || (n_push && !push)) return fail(SKYLA_HIP_E_ARG, "dispatch_noalloc: bad argument");
  if (p->ctx != ctx) return fail(SKYLA_HIP_E_ARG, "dispatch_noalloc: pipeline of another context");
  if (n_push != p->push_words)
    return fail(SKYLA_HIP_E_ARG, "dispatch_noalloc: %s takes %u push words, got %u", p->symbol.c_str(),
                p->push_words, n_push);
  for (void *b : p->sets[0])
    if (!b) return fail(SKYLA_HIP_E_STATE, "dispatch_noalloc: %s is not bound", p->symbol.c_str());
  if (!ctx->scratch || !ctx->fill_u32) return fail(SKYLA_HIP_E_STATE, "dispatch_noalloc: no scratch on this context");
  HIP_TRY(hipSetDevice(ctx->device));
  const Command c = dispatch_command(p, p->sets[0], groups, push, n_push);
  const Command *one[1] = {&c};
  Launch l = pack(one, 1);
  if (l.split) {  // the K split's partials and counters live in the static scratch array
    const uint64_t tile_cap = kScratchTiles * kSplitTileBytes;
    if (l.ws_bytes > tile_cap || l.n_cnt > kScratchCounters)
      return fail(SKYLA_HIP_E_OOM,
                  "dispatch_noalloc: %s needs %llu B of partial tiles and %u counters; the static scratch holds "
                  "%llu B and %llu",
                  p->symbol.c_str(), (unsigned long long)l.ws_bytes, l.n_cnt, (unsigned long long)tile_cap,
                  (unsigned long long)kScratchCounters);
    l.ws = ctx->scratch;
    l.cnt = ctx->scratch + tile_cap;
    // counters start at zero: every K-split launch leaves them so, but the array keeps
    // whatever the last call on this device left
    void *cp = l.cnt;
    uint32_t n = l.n_cnt, zero = 0;
    void *fp[] = {&cp, &n, &zero};
    HIP_TRY(hipModuleLaunchKernel(ctx->fill_u32, (n + 255) / 256, 1, 1, 256, 1, 1, 0, ctx->stream, fp, nullptr));
  }
  if (int s = launch(ctx->stream, l)) return s;
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return SKYLA_HIP_OK;
}

}  // extern "C"
