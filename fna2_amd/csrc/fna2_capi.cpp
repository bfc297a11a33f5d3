// fna2_capi.cpp — the extern "C" boundary: validation, workspace layout and
// kernel dispatch.  Host code only; every GPU launch goes through the
// launch_* wrappers of the .hip files.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "fna2.h"
#include "fna2_kernels.h"
#include "fna2_sched.h"

namespace {

using fna2::kDqBM;
using fna2::kDqBN;
using fna2::kFwdBM;
using fna2::kFwdBN;
using fna2::kKvBM;

constexpr size_t kAlign = 256;
constexpr int64_t kMaxGrid = (int64_t)1 << 24;  // workgroups per launch

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Rows of the query / key side (dense: B * S, varlen: tokens).
int64_t rows_q(const fna2_problem& p) {
  return p.varlen ? (int64_t)p.total_q : (int64_t)p.batch * p.seqlen_q;
}
int64_t rows_k(const fna2_problem& p) {
  return p.varlen ? (int64_t)p.total_k : (int64_t)p.batch * p.seqlen_k;
}

int check_problem(const fna2_problem& p) {
  if (p.dtype != FNA2_BF16 && p.dtype != FNA2_F16) return FNA2_E_DTYPE;
  if (p.head_dim != 64 && p.head_dim != 128) return FNA2_E_HEAD_DIM;
  if (p.heads <= 0 || p.heads_kv <= 0 || p.heads % p.heads_kv != 0) return FNA2_E_HEADS;
  if (p.heads_graph < 0 || p.heads_graph > p.heads) return FNA2_E_HEADS;
  if (p.heads_graph > 0 && (p.rank < 8 || p.rank > 64 || p.rank % 8 != 0)) return FNA2_E_RANK;
  if (p.batch < 0) return FNA2_E_SHAPE;
  if (p.varlen) {
    if (p.total_q < 0 || p.total_k < 0) return FNA2_E_SHAPE;
    if (p.batch > 0 && (!p.cu_seqlens_q || !p.cu_seqlens_k)) return FNA2_E_SEQLENS;
  } else {
    if (p.seqlen_q < 0 || p.seqlen_k < 0) return FNA2_E_SHAPE;
  }
  if (!std::isfinite(p.softmax_scale)) return FNA2_E_SCALE;
  return FNA2_OK;
}

// feat: elements per row (16-byte vectors) or 0 for an fp32 scalar view.
int check_view(const fna2_tensor& t, const fna2_problem& p, bool required, bool vec,
               size_t esize) {
  if (!required) return FNA2_OK;
  if (!t.ptr) return FNA2_E_NULL;
  const size_t a = vec ? 16 : esize;
  if (!aligned(t.ptr, a)) return FNA2_E_STRIDE;
  const int64_t ss = t.stride_s, sh = t.stride_h, sb = p.varlen ? 0 : t.stride_b;
  const int64_t unit = vec ? (int64_t)(16 / esize) : 1;
  if (ss % unit || sh % unit || sb % unit) return FNA2_E_STRIDE;
  return FNA2_OK;
}

#define FNA2_TRY(x)              \
  do {                           \
    int _s = (x);                \
    if (_s != FNA2_OK) return _s; \
  } while (0)

struct Grids {
  int64_t fwd_bound = 0;  // varlen tile-list capacity
  int64_t fwd_grid = 0;
  int64_t dq_bound = 0, dq_grid = 0;
  int64_t kv_bound = 0, kv_grid = 0;
  int64_t kv_tiles = 0;   // key tiles (varlen: bound)
  int64_t q_tiles = 0;    // dQ query tiles (varlen: bound)
};

// Keys per dK/dV item of the problem.
int kv_tile(const fna2_problem& p) {
  return fna2::kv_bn(p.head_dim, fna2::padded_rank32(p.heads_graph, p.rank));
}

Grids grids(const fna2_problem& p) {
  Grids g;
  if (p.batch <= 0) return g;
  const int kbn = kv_tile(p);
  if (p.varlen) {
    g.fwd_bound = fna2::tile_bound(p.total_q, p.batch, kFwdBM);
    g.fwd_grid = g.fwd_bound * p.heads;
    g.dq_bound = fna2::tile_bound(p.total_q, p.batch, kDqBM);
    g.dq_grid = g.dq_bound * p.heads;
    g.kv_bound = fna2::tile_bound(p.total_k, p.batch, kbn);
    g.kv_grid = g.kv_bound * p.heads_kv;
    g.kv_tiles = g.kv_bound;
    g.q_tiles = g.dq_bound;
  } else {
    g.fwd_grid = (int64_t)p.batch * cdiv64(p.seqlen_q, kFwdBM) * p.heads;
    g.dq_grid = (int64_t)p.batch * cdiv64(p.seqlen_q, kDqBM) * p.heads;
    g.kv_grid = (int64_t)p.batch * cdiv64(p.seqlen_k, kbn) * p.heads_kv;
    g.kv_tiles = (int64_t)p.batch * cdiv64(p.seqlen_k, kbn);
    g.q_tiles = (int64_t)p.batch * cdiv64(p.seqlen_q, kDqBM);
  }
  return g;
}

int check_grids(const fna2_problem& p) {
  const Grids g = grids(p);
  if (g.fwd_grid > kMaxGrid || g.dq_grid > kMaxGrid || g.kv_grid > kMaxGrid) return FNA2_E_SHAPE;
  if (rows_q(p) > INT32_MAX || rows_k(p) > INT32_MAX) return FNA2_E_SHAPE;
  return FNA2_OK;
}

// Workspace layouts (byte offsets), all 256-byte aligned.
struct FwdWs {
  size_t tiles = 0, count = 0, bytes = 0;
};
FwdWs fwd_ws(const fna2_problem& p) {
  FwdWs w;
  const Grids g = grids(p);
  if (p.varlen && g.fwd_bound > 0) {
    w.tiles = 0;
    w.count = align_up(sizeof(fna2::TileRec) * g.fwd_bound);
    w.bytes = w.count + kAlign;
  }
  return w;
}

struct BwdWs {
  size_t tiles_q = 0, count_q = 0, tiles_k = 0, count_k = 0, partial = 0, nlse = 0;
  size_t bytes = 0;
};
BwdWs bwd_ws(const fna2_problem& p) {
  BwdWs w;
  const Grids g = grids(p);
  size_t off = 0;
  if (p.varlen && g.dq_bound > 0) {
    w.tiles_q = off;
    off += align_up(sizeof(fna2::TileRec) * g.dq_bound);
    w.count_q = off;
    off += kAlign;
    w.tiles_k = off;
    off += align_up(sizeof(fna2::TileRec) * g.kv_bound);
    w.count_k = off;
    off += kAlign;
  }
  w.partial = off;
  // d_gs partials: [query tiles][4 waves][H_G]
  off += align_up(sizeof(float) * 4u * (size_t)(g.q_tiles > 0 ? g.q_tiles : 1) *
                  (size_t)(p.heads_graph > 0 ? p.heads_graph : 1));
  // -LSE log2(e), fp32 [H][rows_q] (per batch)
  w.nlse = off;
  off += align_up((size_t)rows_q(p) * (size_t)p.heads * 4u);
  w.bytes = off;
  return w;
}

// Plan (varlen): the query-tile list the forward and the dQ kernel share
// (the same tile shape) and the dK/dV key-tile list.
static_assert(kFwdBM == kDqBM && kFwdBN == kDqBN, "the forward and dQ share their tile list");
struct PlanLayout {
  size_t tiles_q = 0, count_q = 0, tiles_k = 0, count_k = 0, bytes = 0;
};
PlanLayout plan_layout(const fna2_problem& p) {
  PlanLayout L;
  if (!p.varlen || p.batch <= 0) return L;
  const Grids g = grids(p);
  size_t off = 0;
  L.tiles_q = off;
  off += align_up(sizeof(fna2::TileRec) * (size_t)g.fwd_bound);
  L.count_q = off;
  off += kAlign;
  L.tiles_k = off;
  off += align_up(sizeof(fna2::TileRec) * (size_t)g.kv_bound);
  L.count_k = off;
  off += kAlign;
  L.bytes = off;
  return L;
}

bool use_plan(const void* plan, const fna2_problem& p) { return plan && p.varlen && p.batch > 0; }

// Plans that fna2_fwd filled, by address, with the problem each was built
// for.  The tile records carry extents clamped to that problem's token
// counts and lists sized by its sequence count, so a backward may only read
// a plan built for the same sequences: fna2_bwd uses a plan found here with
// a matching key, and otherwise builds its own lists (as without a plan).
// A small ring: an address reused by a later forward is re-registered.  The
// key-tile size (head_dim and padded rank pick it) shapes the key list, so
// it is part of the key: a plan built for another tile size is not used.
uint64_t plan_key(const fna2_problem& p) {
  const uint64_t f[] = {(uint64_t)p.batch,          (uint64_t)p.total_q,
                        (uint64_t)p.total_k,        (uint64_t)p.causal,
                        (uint64_t)(uintptr_t)p.cu_seqlens_q,
                        (uint64_t)(uintptr_t)p.cu_seqlens_k,
                        (uint64_t)kv_tile(p)};
  uint64_t h = 1469598103934665603ull;  // FNV-1a over the words
  for (uint64_t w : f) {
    for (int i = 0; i < 8; ++i) {
      h ^= (w >> (8 * i)) & 0xffu;
      h *= 1099511628211ull;
    }
  }
  return h;
}
struct PlanEntry {
  const void* plan;
  uint64_t key;
};
constexpr int kPlanSlots = 256;
std::mutex g_plan_mu;
PlanEntry g_plans[kPlanSlots];
int g_plan_next = 0;

void plan_register(const void* plan, const fna2_problem& p) {
  std::lock_guard<std::mutex> lk(g_plan_mu);
  const uint64_t key = plan_key(p);
  for (PlanEntry& e : g_plans) {
    if (e.plan == plan) {
      e.key = key;
      return;
    }
  }
  g_plans[g_plan_next] = PlanEntry{plan, key};
  g_plan_next = (g_plan_next + 1) % kPlanSlots;
}

bool plan_filled_for(const void* plan, const fna2_problem& p) {
  std::lock_guard<std::mutex> lk(g_plan_mu);
  const uint64_t key = plan_key(p);
  for (const PlanEntry& e : g_plans)
    if (e.plan == plan) return e.key == key;
  return false;
}

fna2::Problem make_problem(const fna2_problem& p) {
  fna2::Problem P;
  std::memset(&P, 0, sizeof(P));
  P.varlen = p.varlen;
  P.nseq = p.batch;
  P.sq = p.varlen ? 0 : p.seqlen_q;
  P.sk = p.varlen ? 0 : p.seqlen_k;
  P.total_q = p.varlen ? p.total_q : 0;
  P.total_k = p.varlen ? p.total_k : 0;
  P.H = p.heads;
  P.H_KV = p.heads_kv;
  P.H_G = p.heads_graph;
  P.D = p.head_dim;
  P.R = p.heads_graph > 0 ? p.rank : 0;
  P.causal = p.causal ? 1 : 0;
  P.f16 = p.dtype == FNA2_F16 ? 1 : 0;
  P.group = p.heads / p.heads_kv;
  const float s = p.softmax_scale;
  if (s > 0.f) {
    P.c = s;
    P.qa = 1.f;
  } else if (s < 0.f) {
    P.c = -s;
    P.qa = -1.f;
  } else {
    P.c = 1.f;
    P.qa = 0.f;
  }
  P.c2 = P.c * fna2::kLog2e;
  P.cu_q = p.cu_seqlens_q;
  P.cu_k = p.cu_seqlens_k;
  return P;
}

// Records caller-owned event i on the stream when events are requested.
bool mark(void* const* events, int i, hipStream_t stream) {
  if (!events || !events[i]) return true;
  return hipEventRecord((hipEvent_t)events[i], stream) == hipSuccess;
}

fna2::TView view(const fna2_tensor& t) {
  fna2::TView v;
  v.ptr = t.ptr;
  v.sb = t.stride_b;
  v.ss = t.stride_s;
  v.sh = t.stride_h;
  return v;
}

// Kernels exist for gfx950 only; cache the answer (and the CU count, which
// sizes the persistent grids) per device.
int check_device(int* num_cus = nullptr) {
  static std::mutex mu;
  static int state[64] = {0};  // 0 unknown, 1 ok, -1 wrong arch
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FNA2_E_DEVICE;
  if (dev < 0 || dev >= 64) return FNA2_E_DEVICE;
  std::lock_guard<std::mutex> lk(mu);
  if (state[dev] == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return FNA2_E_DEVICE;
    state[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    cus[dev] = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;
  }
  if (num_cus) *num_cus = cus[dev];
  return state[dev] == 1 ? FNA2_OK : FNA2_E_DEVICE;
}

}  // namespace

extern "C" {

int fna2_version(void) { return FNA2_ABI_VERSION; }

const char* fna2_status_string(int s) {
  switch (s) {
    case FNA2_OK: return "ok";
    case FNA2_E_NULL: return "a required pointer is NULL";
    case FNA2_E_DTYPE: return "unsupported dtype (attention: bf16 or fp16)";
    case FNA2_E_HEAD_DIM: return "head_dim must be 64 or 128";
    case FNA2_E_RANK: return "rank must be a multiple of 8 in [8, 64]";
    case FNA2_E_HEADS: return "heads must be a multiple of heads_kv and heads_graph <= heads";
    case FNA2_E_SHAPE: return "negative extent or problem too large";
    case FNA2_E_STRIDE: return "pointer or stride breaks 16-byte row alignment";
    case FNA2_E_SEQLENS: return "varlen mode needs cu_seqlens_q and cu_seqlens_k";
    case FNA2_E_WORKSPACE: return "workspace missing or too small";
    case FNA2_E_LAUNCH: return "kernel launch failed";
    case FNA2_E_DEVICE: return "current device is not gfx950";
    case FNA2_E_SCALE: return "softmax_scale must be finite";
    case FNA2_E_ALIAS: return "an output overlaps its input without being equal to it";
    case FNA2_E_SCRATCH:
      return "the problem needs more than the allocation-free entry point's static scratch "
             "(fna2_fwd_noalloc_max_bytes); use fna2_fwd with a workspace";
  }
  return "unknown status";
}

int fna2_check_fwd(const fna2_fwd_args* a) {
  if (!a) return FNA2_E_NULL;
  const fna2_problem& p = a->p;
  FNA2_TRY(check_problem(p));
  FNA2_TRY(check_grids(p));
  const bool qw = rows_q(p) > 0, kw = rows_k(p) > 0;
  const bool g = p.heads_graph > 0;
  FNA2_TRY(check_view(a->q, p, qw, true, 2));
  FNA2_TRY(check_view(a->out, p, qw, true, 2));
  FNA2_TRY(check_view(a->lse, p, qw, false, 4));
  FNA2_TRY(check_view(a->k, p, qw && kw, true, 2));
  FNA2_TRY(check_view(a->v, p, qw && kw, true, 2));
  FNA2_TRY(check_view(a->r_q, p, qw && g, true, 2));
  FNA2_TRY(check_view(a->r_k, p, qw && kw && g, true, 2));
  if (qw && g && !a->graph_scale) return FNA2_E_NULL;
  if (use_plan(a->plan, p)) {
    if (a->plan_bytes < plan_layout(p).bytes || !aligned(a->plan, 32)) return FNA2_E_WORKSPACE;
  } else if (a->workspace_bytes < fwd_ws(p).bytes || (fwd_ws(p).bytes && !a->workspace)) {
    return FNA2_E_WORKSPACE;
  }
  return FNA2_OK;
}

int fna2_check_bwd(const fna2_bwd_args* a) {
  if (!a) return FNA2_E_NULL;
  const fna2_problem& p = a->p;
  FNA2_TRY(check_problem(p));
  FNA2_TRY(check_grids(p));
  const bool qw = rows_q(p) > 0, kw = rows_k(p) > 0;
  const bool g = p.heads_graph > 0;
  FNA2_TRY(check_view(a->q, p, qw, true, 2));
  FNA2_TRY(check_view(a->out, p, qw, true, 2));
  FNA2_TRY(check_view(a->dout, p, qw, true, 2));
  FNA2_TRY(check_view(a->dq, p, qw, true, 2));
  FNA2_TRY(check_view(a->lse, p, qw, false, 4));
  FNA2_TRY(check_view(a->delta, p, qw, false, 4));
  FNA2_TRY(check_view(a->k, p, kw, true, 2));
  FNA2_TRY(check_view(a->v, p, kw, true, 2));
  FNA2_TRY(check_view(a->dk, p, kw, true, 2));
  FNA2_TRY(check_view(a->dv, p, kw, true, 2));
  FNA2_TRY(check_view(a->r_q, p, qw && g, true, 2));
  FNA2_TRY(check_view(a->dr_q, p, qw && g, true, 2));
  FNA2_TRY(check_view(a->r_k, p, kw && g, true, 2));
  FNA2_TRY(check_view(a->dr_k, p, kw && g, true, 2));
  if (g && (!a->graph_scale || !a->d_graph_scale)) return FNA2_E_NULL;
  // The dK/dV kernel addresses one sequence's query rows of a head with
  // 32-bit byte offsets.  In varlen mode seqlen_q is only a scheduling hint:
  // total_q bounds every sequence's length.
  const uint64_t span_rows =
      (uint64_t)(p.varlen ? std::max(p.total_q, p.seqlen_q) : p.seqlen_q);
  auto span_ok = [&](const fna2_tensor& t, uint64_t esize) {
    const uint64_t ss = (uint64_t)(t.stride_s < 0 ? -t.stride_s : t.stride_s);
    return span_rows * ss * esize < (1ull << 31);
  };
  if (qw && !(span_ok(a->q, 2) && span_ok(a->dout, 2) && span_ok(a->delta, 4)))
    return FNA2_E_SHAPE;
  // (the workspace copy of bf16(b Rq), one padded-rank row per query row)
  if (qw && g && span_rows * (uint64_t)fna2::padded_rank32(p.heads_graph, p.rank) * 2u >=
                     (1ull << 31))
    return FNA2_E_SHAPE;
  const BwdWs w = bwd_ws(p);
  if (a->workspace_bytes < w.bytes || !a->workspace) return FNA2_E_WORKSPACE;
  if (use_plan(a->plan, p) && (a->plan_bytes < plan_layout(p).bytes || !aligned(a->plan, 32)))
    return FNA2_E_WORKSPACE;
  return FNA2_OK;
}

size_t fna2_fwd_workspace_bytes(const fna2_problem* p) {
  if (!p || check_problem(*p) != FNA2_OK) return 0;
  return fwd_ws(*p).bytes;
}

size_t fna2_bwd_workspace_bytes(const fna2_problem* p) {
  if (!p || check_problem(*p) != FNA2_OK) return 0;
  return bwd_ws(*p).bytes;
}

size_t fna2_plan_bytes(const fna2_problem* p) {
  if (!p || check_problem(*p) != FNA2_OK) return 0;
  return plan_layout(*p).bytes;
}

}  // extern "C"

namespace {

// The forward, with its varlen tile list in `ws` (at least fwd_ws(p).bytes;
// unused with a plan or in dense mode).  `a` has been checked.
int fwd_launch(const fna2_fwd_args* a, void* ws, hipStream_t stream) {
  const fna2_problem& p = a->p;
  // A plan is filled even without query rows: the backward relies on it.
  if (p.batch == 0 || (rows_q(p) == 0 && !use_plan(a->plan, p))) return FNA2_OK;
  FNA2_TRY(check_device());
  fna2::FwdParams K;
  std::memset(&K, 0, sizeof(K));
  K.p = make_problem(p);
  K.q = view(a->q);
  K.k = view(a->k);
  K.v = view(a->v);
  K.rq = view(a->r_q);
  K.rk = view(a->r_k);
  K.o = view(a->out);
  K.lse = view(a->lse);
  K.gs = a->graph_scale;
  const Grids g = grids(p);
  if (p.varlen && use_plan(a->plan, p)) {
    // One launch builds this call's list and the backward's key-tile list,
    // unless the caller vouches that an earlier forward of this problem
    // filled the plan (and our record of it agrees).
    const PlanLayout L = plan_layout(p);
    char* pl = (char*)a->plan;
    fna2::TileRec* tiles = (fna2::TileRec*)(pl + L.tiles_q);
    int* count = (int*)(pl + L.count_q);
    if (!(a->plan_filled && plan_filled_for(a->plan, p))) {
      const fna2::TileList lq{{0, kFwdBM, kFwdBN, 1}, tiles, count, (int)g.fwd_bound};
      const fna2::TileList lk{{1, kv_tile(p), kKvBM, 0}, (fna2::TileRec*)(pl + L.tiles_k),
                              (int*)(pl + L.count_k), (int)g.kv_bound};
      if (fna2::launch_build_tiles(K.p, lq, &lk, nullptr, stream) != hipSuccess)
        return FNA2_E_LAUNCH;
      plan_register(a->plan, p);
    }
    if (rows_q(p) == 0) return FNA2_OK;
    K.tiles = tiles;
    K.n_tiles = count;
  } else if (p.varlen) {
    const FwdWs w = fwd_ws(p);
    fna2::TileRec* tiles = (fna2::TileRec*)((char*)ws + w.tiles);
    int* count = (int*)((char*)ws + w.count);
    const fna2::TileList list{{0, kFwdBM, kFwdBN, 1}, tiles, count, (int)g.fwd_bound};
    if (fna2::launch_build_tiles(K.p, list, nullptr, nullptr, stream) != hipSuccess)
      return FNA2_E_LAUNCH;
    K.tiles = tiles;
    K.n_tiles = count;
  }
  const int rpl = fna2::padded_rank32(K.p.H_G, K.p.R);
  if (!mark(a->events, 0, stream)) return FNA2_E_LAUNCH;
  if (fna2::launch_fwd(K, rpl, (int)g.fwd_grid, stream) != hipSuccess) return FNA2_E_LAUNCH;
  if (!mark(a->events, 1, stream)) return FNA2_E_LAUNCH;
  return FNA2_OK;
}

// Device memory of the allocation-free forward: the varlen tile list (and
// its count) that fna2_fwd keeps in the caller's workspace.  Every GPU the
// library runs on holds its own copy until the process ends.  In host code
// `scratch` names a host-side stand-in, never its device address: that is
// resolved per device (hipGetSymbolAddress, with the device current) and
// only the resolved pointer is handed to kernels.
constexpr size_t kScratchBytes = (size_t)1 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

int scratch_ptr(void** out) {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return FNA2_E_DEVICE;
  std::lock_guard<std::mutex> lk(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
      return FNA2_E_DEVICE;
    ptrs[dev] = ptr;
  }
  *out = ptrs[dev];
  return FNA2_OK;
}

}  // namespace

extern "C" {

int fna2_fwd(const fna2_fwd_args* a, void* stream_ptr) {
  FNA2_TRY(fna2_check_fwd(a));
  return fwd_launch(a, a->workspace, (hipStream_t)stream_ptr);
}

size_t fna2_fwd_noalloc_max_bytes(void) { return kScratchBytes; }

int fna2_fwd_noalloc(const fna2_fwd_args* a, void* stream_ptr) {
  if (!a) return FNA2_E_NULL;
  // Validate as fna2_fwd would with a workspace of the scratch's size (the
  // caller's workspace fields are ignored).
  fna2_fwd_args b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  FNA2_TRY(check_problem(b.p));
  if (!use_plan(b.plan, b.p) && fwd_ws(b.p).bytes > kScratchBytes) return FNA2_E_SCRATCH;
  void* ws = nullptr;
  if (!use_plan(b.plan, b.p) && fwd_ws(b.p).bytes > 0) {
    FNA2_TRY(scratch_ptr(&ws));
    b.workspace = ws;
    b.workspace_bytes = kScratchBytes;
  }
  FNA2_TRY(fna2_check_fwd(&b));
  return fwd_launch(&b, ws, (hipStream_t)stream_ptr);
}

int fna2_bwd(const fna2_bwd_args* a, void* stream_ptr) {
  FNA2_TRY(fna2_check_bwd(a));
  const fna2_problem& p = a->p;
  int n_cu = 1;
  FNA2_TRY(check_device(&n_cu));
  hipStream_t stream = (hipStream_t)stream_ptr;
  fna2::BwdParams K;
  std::memset(&K, 0, sizeof(K));
  K.p = make_problem(p);
  K.q = view(a->q);
  K.k = view(a->k);
  K.v = view(a->v);
  K.rq = view(a->r_q);
  K.rk = view(a->r_k);
  K.o = view(a->out);
  K.lse = view(a->lse);
  K.dout = view(a->dout);
  K.delta = view(a->delta);
  K.dq = view(a->dq);
  K.dk = view(a->dk);
  K.dv = view(a->dv);
  K.drq = view(a->dr_q);
  K.drk = view(a->dr_k);
  K.gs = a->graph_scale;
  K.dgs = a->d_graph_scale;
  const BwdWs w = bwd_ws(p);
  const Grids g = grids(p);
  K.dgs_partial = (float*)((char*)a->workspace + w.partial);
  K.q_tiles = (int)g.q_tiles;
  K.k_tiles = (int)g.kv_tiles;
  const int rpl = fna2::padded_rank32(K.p.H_G, K.p.R);
  // Head-major (a head's rows are contiguous): the dK/dV kernel reads it per
  // head, 32 rows at a time.
  const int64_t seq_rows = p.varlen ? (int64_t)p.total_q : (int64_t)p.seqlen_q;
  K.nlse.ptr = (char*)a->workspace + w.nlse;
  K.nlse.ss = 1;
  K.nlse.sh = seq_rows;
  K.nlse.sb = p.varlen ? 0 : (int64_t)p.heads * seq_rows;

  if (p.batch > 0 && (rows_q(p) > 0 || rows_k(p) > 0)) {
    if (p.varlen && use_plan(a->plan, p) && rows_q(p) > 0 && plan_filled_for(a->plan, p)) {
      // The forward built both lists; the dQ kernel's spare workgroups zero
      // the rows no sequence covers.  (Without query rows no dQ kernel runs:
      // the lists are then built, and the rows zeroed, below.)
      const PlanLayout L = plan_layout(p);
      const char* pl = (const char*)a->plan;
      K.tiles_q = (const fna2::TileRec*)(pl + L.tiles_q);
      K.n_tiles_q = (const int*)(pl + L.count_q);
      K.tiles_k = (const fna2::TileRec*)(pl + L.tiles_k);
      K.n_tiles_k = (const int*)(pl + L.count_k);
      K.zero_uncovered = 1;
    } else if (p.varlen) {
      fna2::TileRec* tq = (fna2::TileRec*)((char*)a->workspace + w.tiles_q);
      int* cq = (int*)((char*)a->workspace + w.count_q);
      fna2::TileRec* tk = (fna2::TileRec*)((char*)a->workspace + w.tiles_k);
      int* ck = (int*)((char*)a->workspace + w.count_k);
      const fna2::TileList lq{{0, kDqBM, kDqBN, 1}, tq, cq, (int)g.dq_bound};
      const fna2::TileList lk{{1, kv_tile(p), kKvBM, 0}, tk, ck, (int)g.kv_bound};
      const fna2::ZeroRows zero{K.dq, K.drq, K.dk, K.dv, K.drk,
                                (int)std::max(p.total_q, p.total_k)};
      if (fna2::launch_build_tiles(K.p, lq, &lk, &zero, stream) != hipSuccess)
        return FNA2_E_LAUNCH;
      K.tiles_q = tq;
      K.n_tiles_q = cq;
      K.tiles_k = tk;
      K.n_tiles_k = ck;
    }
    // dQ first: it also stores delta, which the dK/dV kernel reads.
    if (!mark(a->events, 0, stream)) return FNA2_E_LAUNCH;
    // (with a plan, one more row of workgroups than tiles can fill, so that
    // spare workgroups exist for the zeroing whatever the lengths)
    const int dq_grid = (int)g.dq_grid + (K.zero_uncovered ? p.heads : 0);
    if (rows_q(p) > 0 && fna2::launch_bwd_dq(K, rpl, dq_grid, stream) != hipSuccess)
      return FNA2_E_LAUNCH;
    if (!mark(a->events, 1, stream) || !mark(a->events, 2, stream)) return FNA2_E_LAUNCH;
    // persistent: one workgroup per CU walks the (key tile, KV head) items
    const int kv_grid = (int)std::min<int64_t>(g.kv_grid, n_cu);
    if (rows_k(p) > 0 && fna2::launch_bwd_dkdv(K, rpl, kv_grid, stream) != hipSuccess)
      return FNA2_E_LAUNCH;
    if (!mark(a->events, 3, stream)) return FNA2_E_LAUNCH;
  } else if (p.varlen && p.batch == 0 && (rows_q(p) > 0 || rows_k(p) > 0)) {
    // No sequences: every token lies outside them and gets zero gradients.
    const fna2::ZeroRows zero{K.dq, K.drq, K.dk, K.dv, K.drk,
                              (int)std::max(p.total_q, p.total_k)};
    if (fna2::launch_zero_rows(K.p, zero, stream) != hipSuccess) return FNA2_E_LAUNCH;
  }
  // The dK/dV kernel reduces d_gs when it runs.
  const bool dkdv_ran = p.batch > 0 && rows_k(p) > 0 && g.kv_grid > 0;
  if (!dkdv_ran && fna2::launch_bwd_dgs(K, stream) != hipSuccess) return FNA2_E_LAUNCH;
  return FNA2_OK;
}

}  // extern "C"

namespace {

// Byte range [lo, hi) a [T, heads, D] view covers.
void rope_extent(const fna2_tensor& t, int T, int heads, int D, size_t es, uintptr_t& lo,
                 uintptr_t& hi) {
  int64_t a = 0, b = D;
  const int64_t ds = (int64_t)(T - 1) * t.stride_s, dh = (int64_t)(heads - 1) * t.stride_h;
  (ds < 0 ? a : b) += ds;
  (dh < 0 ? a : b) += dh;
  lo = (uintptr_t)t.ptr + (uintptr_t)(a * (int64_t)es);
  hi = (uintptr_t)t.ptr + (uintptr_t)(b * (int64_t)es);
}

int rope_pair(const fna2_tensor& in, const fna2_tensor& out, int T, int heads, int D,
              size_t es) {
  if (!in.ptr || !out.ptr) return FNA2_E_NULL;
  for (const fna2_tensor* t : {&in, &out}) {
    if ((uintptr_t)t->ptr % 16 || (t->stride_s * (int64_t)es) % 16 ||
        (t->stride_h * (int64_t)es) % 16)
      return FNA2_E_STRIDE;
  }
  if (in.ptr == out.ptr)
    return in.stride_s == out.stride_s && in.stride_h == out.stride_h ? FNA2_OK : FNA2_E_ALIAS;
  uintptr_t l0, h0, l1, h1;
  rope_extent(in, T, heads, D, es, l0, h0);
  rope_extent(out, T, heads, D, es, l1, h1);
  return (l0 < h1 && l1 < h0) ? FNA2_E_ALIAS : FNA2_OK;
}

// Checks shared by the forward and the backward (no tensors).
int rope_common(const fna2_rope_args* a) {
  if (!a) return FNA2_E_NULL;
  if (a->dtype != FNA2_BF16 && a->dtype != FNA2_F16 && a->dtype != FNA2_F32) return FNA2_E_DTYPE;
  const int D = a->head_dim;
  if (D < 16 || D > 512 || (D & (D - 1)) != 0) return FNA2_E_HEAD_DIM;
  if (a->total_tokens < 0 || a->heads_q < 0 || a->heads_k < 0 || a->nseq < 0 ||
      (a->sign != 1 && a->sign != -1))
    return FNA2_E_SHAPE;
  if ((a->norm_q || a->norm_k) && !(std::isfinite(a->norm_eps) && a->norm_eps >= 0.f))
    return FNA2_E_SCALE;
  if (a->total_tokens == 0 || a->heads_q + a->heads_k == 0) return FNA2_OK;
  if (!a->cu_seqlens) return FNA2_E_SEQLENS;
  if (!a->inv_freq) return FNA2_E_NULL;
  return FNA2_OK;
}

bool rope_empty(const fna2_rope_args* a) {
  return a->total_tokens == 0 || a->heads_q + a->heads_k == 0;
}

size_t rope_esize(const fna2_rope_args* a) { return a->dtype == FNA2_F32 ? 4 : 2; }

fna2::RopeParams rope_params(const fna2_rope_args* a) {
  fna2::RopeParams P;
  std::memset(&P, 0, sizeof(P));
  P.dtype = a->dtype == FNA2_BF16 ? fna2::kRopeBF16
            : a->dtype == FNA2_F16 ? fna2::kRopeF16
                                   : fna2::kRopeF32;
  P.T = a->total_tokens;
  P.Hq = a->heads_q;
  P.Hk = a->heads_k;
  P.D = a->head_dim;
  P.nseq = a->nseq;
  P.sign = a->sign;
  P.cu = a->cu_seqlens;
  P.inv_freq = a->inv_freq;
  P.q = a->q.ptr;
  P.k = a->k.ptr;
  P.q_ss = a->q.stride_s;
  P.q_sh = a->q.stride_h;
  P.k_ss = a->k.stride_s;
  P.k_sh = a->k.stride_h;
  P.wq = a->heads_q > 0 ? a->norm_q : nullptr;
  P.wk = a->heads_k > 0 ? a->norm_k : nullptr;
  P.eps = a->norm_eps;
  return P;
}

void rope_out(fna2::RopeParams& P, const fna2_tensor& qo, const fna2_tensor& ko) {
  P.q_out = qo.ptr;
  P.k_out = ko.ptr;
  P.qo_ss = qo.stride_s;
  P.qo_sh = qo.stride_h;
  P.ko_ss = ko.stride_s;
  P.ko_sh = ko.stride_h;
}

size_t rope_ws(const fna2_rope_args* a) {
  if (!(a->norm_q || a->norm_k) || rope_empty(a)) return 0;
  return align_up(sizeof(float) * 2u * (size_t)fna2::rope_blocks(a->total_tokens) *
                  (size_t)a->head_dim);
}

}  // namespace

extern "C" {

int fna2_check_rope(const fna2_rope_args* a) {
  FNA2_TRY(rope_common(a));
  if (rope_empty(a)) return FNA2_OK;
  const int T = a->total_tokens, D = a->head_dim;
  const size_t es = rope_esize(a);
  if (a->heads_q > 0) FNA2_TRY(rope_pair(a->q, a->q_out, T, a->heads_q, D, es));
  if (a->heads_k > 0) FNA2_TRY(rope_pair(a->k, a->k_out, T, a->heads_k, D, es));
  return FNA2_OK;
}

int fna2_rope_varlen(const fna2_rope_args* a, void* stream) {
  FNA2_TRY(fna2_check_rope(a));
  if (rope_empty(a)) return FNA2_OK;
  FNA2_TRY(check_device());
  fna2::RopeParams P = rope_params(a);
  rope_out(P, a->q_out, a->k_out);
  if (fna2::launch_rope(P, (hipStream_t)stream) != hipSuccess) return FNA2_E_LAUNCH;
  return FNA2_OK;
}

size_t fna2_rope_bwd_workspace_bytes(const fna2_rope_args* a) {
  if (!a || rope_common(a) != FNA2_OK) return 0;
  return rope_ws(a);
}

int fna2_check_rope_bwd(const fna2_rope_bwd_args* b) {
  if (!b) return FNA2_E_NULL;
  const fna2_rope_args* a = &b->fwd;
  FNA2_TRY(rope_common(a));
  if (rope_empty(a)) return FNA2_OK;
  const int T = a->total_tokens, D = a->head_dim;
  const size_t es = rope_esize(a);
  const bool norm = a->norm_q || a->norm_k;
  if (a->heads_q > 0) {
    FNA2_TRY(rope_pair(b->dq_out, b->dq, T, a->heads_q, D, es));
    if (norm) FNA2_TRY(rope_pair(a->q, b->dq, T, a->heads_q, D, es));
    if (a->norm_q && !b->dnorm_q) return FNA2_E_NULL;
  }
  if (a->heads_k > 0) {
    FNA2_TRY(rope_pair(b->dk_out, b->dk, T, a->heads_k, D, es));
    if (norm) FNA2_TRY(rope_pair(a->k, b->dk, T, a->heads_k, D, es));
    if (a->norm_k && !b->dnorm_k) return FNA2_E_NULL;
  }
  const size_t need = rope_ws(a);
  if (need && (!b->workspace || b->workspace_bytes < need)) return FNA2_E_WORKSPACE;
  return FNA2_OK;
}

int fna2_rope_bwd(const fna2_rope_bwd_args* b, void* stream) {
  FNA2_TRY(fna2_check_rope_bwd(b));
  const fna2_rope_args* a = &b->fwd;
  if (rope_empty(a)) return FNA2_OK;
  FNA2_TRY(check_device());
  fna2::RopeParams P = rope_params(a);
  rope_out(P, b->dq, b->dk);
  if (!(P.wq || P.wk)) {  // the inverse rotation of the gradients
    P.q = b->dq_out.ptr;
    P.k = b->dk_out.ptr;
    P.q_ss = b->dq_out.stride_s;
    P.q_sh = b->dq_out.stride_h;
    P.k_ss = b->dk_out.stride_s;
    P.k_sh = b->dk_out.stride_h;
    P.sign = -a->sign;
    if (fna2::launch_rope(P, (hipStream_t)stream) != hipSuccess) return FNA2_E_LAUNCH;
    return FNA2_OK;
  }
  P.gq = b->dq_out.ptr;
  P.gk = b->dk_out.ptr;
  P.gq_ss = b->dq_out.stride_s;
  P.gq_sh = b->dq_out.stride_h;
  P.gk_ss = b->dk_out.stride_s;
  P.gk_sh = b->dk_out.stride_h;
  P.part = (float*)b->workspace;
  P.dwq = P.wq ? b->dnorm_q : nullptr;
  P.dwk = P.wk ? b->dnorm_k : nullptr;
  if (fna2::launch_rope_norm_bwd(P, (hipStream_t)stream) != hipSuccess) return FNA2_E_LAUNCH;
  return FNA2_OK;
}

}  // extern "C"

namespace {

// Work units of a decode launch are sized for MI355X's 256 compute units
// (a fixed figure, so that the split count and the workspace size are a
// function of the arguments alone).
constexpr int kDecodeCUs = 256;
constexpr int64_t kOff31 = ((int64_t)1 << 31) - 16;  // buffer-offset bound

int dec_group(const fna2_decode_args& a) { return a.heads / a.heads_kv; }

// Graph heads of the widest KV-head group and their rank chunks.
int dec_graph_heads(const fna2_decode_args& a) {
  return a.heads_graph > 0 ? std::min(dec_group(a), a.heads_graph) : 0;
}
int dec_rc(const fna2_decode_args& a) {
  return fna2::decode_rank_chunks(dec_graph_heads(a) * (a.heads_graph > 0 ? a.rank / 8 : 0));
}

int check_bf16_rows(const fna2_tensor& t) {
  if (!t.ptr) return FNA2_E_NULL;
  if (!aligned(t.ptr, 16)) return FNA2_E_STRIDE;
  if (t.stride_b < 0 || t.stride_s < 0 || t.stride_h < 0) return FNA2_E_STRIDE;
  if (t.stride_b % 8 || t.stride_s % 8 || t.stride_h % 8) return FNA2_E_STRIDE;
  return FNA2_OK;
}

struct DecSplit {
  int n = 1, keys = 32;
};

DecSplit dec_split(const fna2_decode_args& a) {
  DecSplit s;
  const int64_t L = a.max_seqlen_k;
  if (L <= 0) return s;
  int64_t n = a.num_splits;
  if (n <= 0) {
    const int64_t units = std::max<int64_t>((int64_t)a.batch * a.heads_kv, 1);
    const int rc = std::max(dec_rc(a), 0);
    const int per_cu = std::max(1, (160 * 1024) / (fna2::kDecodeStages *
                                                   fna2::decode_stage_bytes(a.head_dim, rc)));
    const int64_t target = 2ll * kDecodeCUs * per_cu;  // two rounds of resident waves
    n = std::min<int64_t>(cdiv64(target, units), cdiv64(L, 128));  // >= 4 steps a split
    n = std::max<int64_t>(std::min<int64_t>(n, 64), 1);
  }
  n = std::min<int64_t>(n, cdiv64(L, 32));
  s.keys = (int)(cdiv64(cdiv64(L, n), 32) * 32);
  s.n = (int)cdiv64(L, s.keys);
  return s;
}

}  // namespace

extern "C" {

int fna2_check_decode(const fna2_decode_args* a) {
  if (!a) return FNA2_E_NULL;
  if (a->head_dim != 64 && a->head_dim != 128) return FNA2_E_HEAD_DIM;
  if (a->heads <= 0 || a->heads_kv <= 0 || a->heads % a->heads_kv != 0) return FNA2_E_HEADS;
  if (dec_group(*a) > 32) return FNA2_E_HEADS;
  if (a->heads_graph < 0 || a->heads_graph > a->heads) return FNA2_E_HEADS;
  const bool graph = a->heads_graph > 0;
  if (graph && (a->rank < 8 || a->rank > 64 || a->rank % 8 != 0)) return FNA2_E_RANK;
  if (graph && dec_rc(*a) < 0) return FNA2_E_RANK;
  if (a->batch < 0 || a->max_seqlen_k < 0) return FNA2_E_SHAPE;
  if (a->num_splits < 0 || a->num_splits > 64) return FNA2_E_SHAPE;
  if (!std::isfinite(a->softmax_scale)) return FNA2_E_SCALE;
  if (a->batch == 0) return FNA2_OK;
  FNA2_TRY(check_bf16_rows(a->q));
  FNA2_TRY(check_bf16_rows(a->out));
  const bool rows = a->max_seqlen_k > 0;  // an empty cache is never read
  if (rows) {
    FNA2_TRY(check_bf16_rows(a->k_cache));
    FNA2_TRY(check_bf16_rows(a->v_cache));
  }
  if (graph) {
    FNA2_TRY(check_bf16_rows(a->r_q));
    if (rows) FNA2_TRY(check_bf16_rows(a->rk_cache));
    if (!a->graph_scale) return FNA2_E_NULL;
  }
  if (a->lse.ptr) {
    if (!aligned(a->lse.ptr, 4) || a->lse.stride_b < 0 || a->lse.stride_h < 0)
      return FNA2_E_STRIDE;
  }
  const int64_t g = dec_group(*a), D = a->head_dim;
  if ((g - 1) * a->q.stride_h * 2 + D * 2 > kOff31) return FNA2_E_SHAPE;
  if (32 * a->k_cache.stride_s * 2 > kOff31 || 32 * a->v_cache.stride_s * 2 > kOff31)
    return FNA2_E_SHAPE;
  if (graph) {
    const int64_t gg = dec_graph_heads(*a), R = a->rank;
    if ((gg - 1) * a->r_q.stride_h * 2 + R * 2 > kOff31) return FNA2_E_SHAPE;
    if ((gg - 1) * a->rk_cache.stride_h * 2 + 31 * a->rk_cache.stride_s * 2 + R * 2 > kOff31)
      return FNA2_E_SHAPE;
  }
  const DecSplit s = dec_split(*a);
  if ((int64_t)a->batch * a->heads_kv * s.n > kMaxGrid) return FNA2_E_SHAPE;
  return FNA2_OK;
}

int fna2_decode_num_splits(const fna2_decode_args* a) {
  FNA2_TRY(fna2_check_decode(a));
  return dec_split(*a).n;
}

size_t fna2_decode_workspace_bytes(const fna2_decode_args* a) {
  if (fna2_check_decode(a) != FNA2_OK) return 0;
  const DecSplit s = dec_split(*a);
  if (s.n <= 1) return 0;
  const size_t rows = (size_t)s.n * (size_t)a->batch * (size_t)a->heads;
  return align_up(rows * (size_t)a->head_dim * 4u) + align_up(rows * 8u);
}

int fna2_decode(const fna2_decode_args* a, void* stream_ptr) {
  FNA2_TRY(fna2_check_decode(a));
  if (a->batch == 0) return FNA2_OK;
  FNA2_TRY(check_device());
  const DecSplit s = dec_split(*a);
  const size_t need = fna2_decode_workspace_bytes(a);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need || !aligned(a->workspace, 16)))
    return FNA2_E_WORKSPACE;
  hipStream_t stream = (hipStream_t)stream_ptr;
  fna2::DecodeParams K;
  std::memset(&K, 0, sizeof(K));
  K.B = a->batch;
  K.H = a->heads;
  K.H_KV = a->heads_kv;
  K.H_G = a->heads_graph;
  K.D = a->head_dim;
  K.R = a->heads_graph > 0 ? a->rank : 0;
  K.group = dec_group(*a);
  K.nsplit = s.n;
  K.split_keys = s.keys;
  K.max_len = a->max_seqlen_k;
  const float sc = a->softmax_scale;
  K.c = sc > 0.f ? sc : sc < 0.f ? -sc : 1.f;
  K.qa = sc > 0.f ? 1.f : sc < 0.f ? -1.f : 0.f;
  K.c2 = K.c * fna2::kLog2e;
  K.seqlens = a->seqlens_k;
  K.q = view(a->q);
  K.rq = view(a->r_q);
  K.k = view(a->k_cache);
  K.v = view(a->v_cache);
  K.rk = view(a->rk_cache);
  K.o = view(a->out);
  K.lse = view(a->lse);
  K.gs = a->graph_scale;
  if (s.n > 1) {
    const size_t rows = (size_t)s.n * (size_t)a->batch * (size_t)a->heads;
    K.acc = (float*)a->workspace;
    K.ml = (float*)((char*)a->workspace + align_up(rows * (size_t)a->head_dim * 4u));
  }
  const int rc = a->heads_graph > 0 ? dec_rc(*a) : 0;
  if (!mark(a->events, 0, stream)) return FNA2_E_LAUNCH;
  if (fna2::launch_decode(K, rc, stream) != hipSuccess) return FNA2_E_LAUNCH;
  if (!mark(a->events, 1, stream)) return FNA2_E_LAUNCH;
  if (fna2::launch_decode_merge(K, stream) != hipSuccess) return FNA2_E_LAUNCH;
  return FNA2_OK;
}

}  // extern "C"
